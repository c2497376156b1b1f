// router_dev.h -- device bodies of the router-logit row dot, the shared-expert gate and the top-k router, shared
// by the per-operation kernels (vector_ops.hip) and the fused decode-layer kernel (fused_decode.hip) so that
// both produce the same bits. All take a 256-thread workgroup; part is 4 floats of LDS.
#ifndef ROUTER_DEV_H
#define ROUTER_DEV_H

#include "moe_common.h"

#define ROUTER_MAX_E 1024

__device__ __forceinline__ float block256_sum(float v, float* part) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
    __syncthreads();
    const float s = (part[0] + part[1]) + (part[2] + part[3]);
    __syncthreads();
    return s;
}

// W[row] . x over K values: 16-byte loads, per-thread fma chain, then the workgroup sum
__device__ __forceinline__ float f32_row_dot(const float* wr, const float* x, int K, float* part) {
    const int tid = threadIdx.x;
    float acc = 0.0f;
    if ((K & 3) == 0 && (((uintptr_t)wr | (uintptr_t)x) & 15) == 0) {
        const float4* w4 = (const float4*)wr;
        const float4* x4 = (const float4*)x;
#pragma unroll 4
        for (int i = tid; i < K / 4; i += 256) {
            const float4 a = w4[i], b = x4[i];
            acc = fmaf(a.x, b.x, acc);
            acc = fmaf(a.y, b.y, acc);
            acc = fmaf(a.z, b.z, acc);
            acc = fmaf(a.w, b.w, acc);
        }
    } else {
        for (int i = tid; i < K; i += 256) acc = fmaf(wr[i], x[i], acc);
    }
    return block256_sum(acc, part);
}

// W[row] . x[t] for tokens t < T (T <= TMAX; x rows ldx apart), the router row read once: per token the same fma
// chain and workgroup sum as f32_row_dot, so the same bits. y[t] is valid in every thread.
template <int TMAX>
__device__ __forceinline__ void f32_row_dot_multi(const float* wr, const float* x, long long ldx, int T, int K,
                                                  float (*part)[4], float y[TMAX]) {
    const int tid = threadIdx.x;
    float acc[TMAX];
#pragma unroll
    for (int t = 0; t < TMAX; ++t) acc[t] = 0.0f;
    const bool vec = (K & 3) == 0 && (ldx & 3) == 0 && (((uintptr_t)wr | (uintptr_t)x) & 15) == 0;
    if (vec) {
        const float4* w4 = (const float4*)wr;
        for (int i = tid; i < K / 4; i += 256) {
            const float4 a = w4[i];
            float4 b[TMAX];
#pragma unroll
            for (int t = 0; t < TMAX; ++t) b[t] = ((const float4*)(x + (size_t)min(t, T - 1) * ldx))[i];
#pragma unroll
            for (int t = 0; t < TMAX; ++t)
                if (t < T) {
                    acc[t] = fmaf(a.x, b[t].x, acc[t]);
                    acc[t] = fmaf(a.y, b[t].y, acc[t]);
                    acc[t] = fmaf(a.z, b[t].z, acc[t]);
                    acc[t] = fmaf(a.w, b[t].w, acc[t]);
                }
        }
    } else {
        for (int i = tid; i < K; i += 256) {
            const float a = wr[i];
#pragma unroll
            for (int t = 0; t < TMAX; ++t)
                if (t < T) acc[t] = fmaf(a, x[(size_t)t * ldx + i], acc[t]);
        }
    }
#pragma unroll
    for (int t = 0; t < TMAX; ++t) {
        const float v = wave_sum(acc[t]);
        if ((threadIdx.x & 63) == 0) part[t][threadIdx.x >> 6] = v;
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < TMAX; ++t) y[t] = (part[t][0] + part[t][1]) + (part[t][2] + part[t][3]);
    __syncthreads();
}

// sigmoid(x . w) over n values (the shared expert's gate)
__device__ __forceinline__ float shexp_gate(const float* xr, const float* w, int n, float* part) {
    const int tid = threadIdx.x;
    float d = 0.0f;
    if ((n & 3) == 0 && (((uintptr_t)xr | (uintptr_t)w) & 15) == 0) {
        for (int i = tid; i < n / 4; i += 256) {
            const float4 a = ((const float4*)xr)[i], b = ((const float4*)w)[i];
            d += a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
        }
    } else {
        for (int i = tid; i < n; i += 256) d += xr[i] * w[i];
    }
    d = block256_sum(d, part);
    return 1.0f / (1.0f + expf(-d));
}

// Order-preserving map of a float onto uint32 (larger float, larger key; keys of real floats are >= 0x007fffff)
__device__ __forceinline__ uint32_t f32_order_key(float v) {
    const uint32_t u = __float_as_uint(v);
    return u ^ ((u >> 31) ? 0xffffffffu : 0x80000000u);
}
__device__ __forceinline__ float f32_from_order_key(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? k ^ 0x80000000u : ~k);
}

// Wave-wide unsigned max / min, read out of lane 63 as a wave-uniform value: the row steps (quad, half-row and row
// mirrors leave every lane of a 16-lane row with the row's result), then row_bcast:15 and row_bcast:31 carry rows
// 0..2 into lane 63. Each step is one DPP-operand VALU op (the operation's identity fills lanes a step skips).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v, uint32_t identity) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)identity, (int)v, CTRL, ROW_MASK, 0xf, false);
}
__device__ __forceinline__ uint32_t wave_max_u32_uniform(uint32_t v) {
    v = max(v, dpp_u<0xb1, 0xf>(v, 0u));
    v = max(v, dpp_u<0x4e, 0xf>(v, 0u));
    v = max(v, dpp_u<0x141, 0xf>(v, 0u));
    v = max(v, dpp_u<0x140, 0xf>(v, 0u));
    v = max(v, dpp_u<0x142, 0xa>(v, 0u));
    v = max(v, dpp_u<0x143, 0xc>(v, 0u));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
__device__ __forceinline__ uint32_t wave_min_u32_uniform(uint32_t v) {
    v = min(v, dpp_u<0xb1, 0xf>(v, 0xffffffffu));
    v = min(v, dpp_u<0x4e, 0xf>(v, 0xffffffffu));
    v = min(v, dpp_u<0x141, 0xf>(v, 0xffffffffu));
    v = min(v, dpp_u<0x140, 0xf>(v, 0xffffffffu));
    v = min(v, dpp_u<0x142, 0xa>(v, 0xffffffffu));
    v = min(v, dpp_u<0x143, 0xc>(v, 0xffffffffu));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Selection on one wave; lane l holds logits l, l + 64, ... (NPL of them) as order keys (0: taken or absent, below
// every real key; -0 is keyed as +0). Each of the nu rounds takes the largest remaining key (a max reduction), then
// the lowest index holding it (a min reduction), so ties go to the lower index. Lane r keeps round r's logit and
// index; the probabilities and their sum in rank order follow the rounds.
template <int NPL>
__device__ __forceinline__ void router_select_wave(const float* lg, int ne, int nu, int* id_row, float* wts) {
    const int lane = threadIdx.x & 63;
    float v[NPL];
    uint32_t key[NPL];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < NPL; ++j) v[j] = lg[min(lane + 64 * j, ne - 1)];  // (all loads in flight at once)
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
        const int e = lane + 64 * j;
        if (e >= ne) v[j] = -INFINITY;
        key[j] = e < ne ? f32_order_key(v[j] == 0.0f ? 0.0f : v[j]) : 0u;
        mx = fmaxf(mx, v[j]);
    }
    mx = wave_max(mx);
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < NPL; ++j)
        if (lane + 64 * j < ne) sum += expf(v[j] - mx);
    sum = wave_sum(sum);
    const float inv = 1.0f / sum;
    uint32_t mykey = 0;
    int myid = 0;
    for (int r = 0; r < nu; ++r) {
        uint32_t lk = key[0];
#pragma unroll
        for (int j = 1; j < NPL; ++j) lk = max(lk, key[j]);
        const uint32_t best = wave_max_u32_uniform(lk);
        uint32_t li = 0xffffffffu;
#pragma unroll
        for (int j = NPL - 1; j >= 0; --j)
            if (key[j] == best) li = lane + 64 * j;
        const uint32_t e = wave_min_u32_uniform(li);
#pragma unroll
        for (int j = 0; j < NPL; ++j)
            if (lane + 64 * j == (int)e) key[j] = 0u;
        if (lane == r) {
            mykey = best;
            myid = (int)e;
        }
    }
    const float p = expf(f32_from_order_key(mykey) - mx) * inv;
    float ws = 0.0f;
    for (int r = 0; r < nu; ++r) ws += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), r));  // rank order
    ws = fmaxf(ws, 6.103515625e-5f);
    if (lane < nu) {
        id_row[lane] = myid;
        wts[lane] = p / ws;
    }
}

// Softmax over ne (<= ROUTER_MAX_E) logits, the nu (<= 64) largest in descending order (ties to the lower index),
// weights renormalised by max(sum, 6.103515625e-5). router_select: wave 0 of the workgroup selects; it writes
// id_row[0..nu) and wts[0..nu) (any memory), visible to the whole workgroup on return. router_select_one_wave:
// the calling wave selects (no workgroup barrier).
__device__ __forceinline__ void router_select_one_wave(const float* lg, int ne, int nu, int* id_row, float* wts) {
    if (ne <= 128)
        router_select_wave<2>(lg, ne, nu, id_row, wts);
    else if (ne <= 256)
        router_select_wave<4>(lg, ne, nu, id_row, wts);
    else if (ne <= 512)
        router_select_wave<8>(lg, ne, nu, id_row, wts);
    else
        router_select_wave<16>(lg, ne, nu, id_row, wts);
}
__device__ __forceinline__ void router_select(const float* lg, int ne, int nu, int* id_row, float* wts) {
    if (threadIdx.x < 64) router_select_one_wave(lg, ne, nu, id_row, wts);
    __syncthreads();
}

#endif  // ROUTER_DEV_H
