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
            const float4 a = ld_w4(w4 + i), b = x4[i];
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
            const float4 a = ld_w4(w4 + i);
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
            const float4 a = ((const float4*)xr)[i], b = ld_w4((const float4*)w + i);
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

// The softmax's normalisation on one wave: lane l's logits l, l + 64, ... (NPL of them; -inf past ne) into v, the
// maximum mx and 1 / (sum of exp(logit - mx)), the sum in lane order and then over the wave (the router's bits)
template <int NPL>
__device__ __forceinline__ void router_softmax_norm(const float* lg, int ne, float (&v)[NPL], float& mx, float& inv) {
    const int lane = threadIdx.x & 63;
    mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < NPL; ++j) v[j] = lg[min(lane + 64 * j, ne - 1)];  // (all loads in flight at once)
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
        if (lane + 64 * j >= ne) v[j] = -INFINITY;
        mx = fmaxf(mx, v[j]);
    }
    mx = wave_max(mx);
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < NPL; ++j)
        if (lane + 64 * j < ne) sum += expf(v[j] - mx);
    sum = wave_sum(sum);
    inv = 1.0f / sum;
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
    float mx, inv;
    router_softmax_norm<NPL>(lg, ne, v, mx, inv);
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
        const int e = lane + 64 * j;
        key[j] = e < ne ? f32_order_key(v[j] == 0.0f ? 0.0f : v[j]) : 0u;
    }
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

// The nu selected experts by rank, by a whole workgroup of NT threads (up to 256 experts). Keys: 64 bits, the order
// key of the logit, then nep - 1 - index (all distinct; nep the power of two >= max(ne, 32); padding keys 0), so the
// selection order (larger logit; on equal logits the lower index) is the keys' descending order. A key's rank is the
// number of larger keys, counted by G threads (two keys a read). Two stages, to keep the LDS reads few: the rank of
// every key within its group of 32, then, over the nu' = min(nu, 32) best of each group (which hold the nu best
// overall), the rank among those. The same ids, in the same order, as router_select (nu rounds of reductions on
// one wave). s_ids[0..nu) on return (visible to the workgroup); s_pk, s_pk2: 256 8-byte words of LDS each,
// 16-byte aligned.
template <int G>
__device__ __forceinline__ int keys_above(const uint64_t* seg, int per, uint64_t pc) {
    int cnt = 0;
    for (int j = 0; j < per; j += 2) {
        const ulonglong2 q = *(const ulonglong2*)(seg + j);
        cnt += q.x > pc ? 1 : 0;
        cnt += q.y > pc ? 1 : 0;
    }
    return group_sum_i<G>(cnt);
}

// Stage 1, G threads a key: rank within the key's group of 32; the nu' best of group k go to s_pk2[k nu' + rank]
template <int G>
__device__ __forceinline__ void rank_in_groups(const uint64_t* s_pk, int nep, int nu1, uint64_t* s_pk2) {
    const int tid = threadIdx.x, c = tid / G, g = tid - c * G, cc = min(c, nep - 1);  // (no early exit: DPP sums)
    const uint64_t pc = s_pk[cc];
    const int r = keys_above<G>(s_pk + (cc & ~31) + g * (32 / G), 32 / G, pc);
    if (g == 0 && c < nep && r < nu1) s_pk2[(c >> 5) * nu1 + r] = pc;
}

// Stage 2, G threads a key of s_pk2[0..n2) (n2p: a power of two >= n2, zero-padded): the rank among them
template <int G>
__device__ __forceinline__ void rank_survivors(const uint64_t* s_pk2, int n2, int n2p, int nep, int ne, int nu,
                                               int* s_ids) {
    const int tid = threadIdx.x, c = tid / G, g = tid - c * G;
    const uint64_t pc = s_pk2[min(c, n2 - 1)];
    const int r = keys_above<G>(s_pk2 + g * (n2p / G), n2p / G, pc);
    const int idx = nep - 1 - (int)(uint32_t)pc;
    if (g == 0 && c < n2 && r < nu && idx < ne) s_ids[r] = idx;
}

template <int NT>
__device__ __forceinline__ void router_rank_select(const float* lg, int ne, int nu, int* s_ids, uint64_t* s_pk,
                                                   uint64_t* s_pk2) {
    static_assert(NT >= 4 * 256, "at least 4 threads for each of up to 256 keys");
    const int tid = threadIdx.x;
    int nep = 32;
    while (nep < ne) nep <<= 1;
    const int nu1 = min(nu, 32), n2 = (nep >> 5) * nu1;
    int n2p = 32;
    while (n2p < n2) n2p <<= 1;
    for (int i = tid; i < nep; i += NT) {
        const float v = lg[min(i, ne - 1)];
        const uint32_t key = i < ne ? f32_order_key(v == 0.0f ? 0.0f : v) : 0u;
        s_pk[i] = (uint64_t)key << 32 | (uint32_t)(nep - 1 - i);
    }
    for (int i = n2 + tid; i < n2p; i += NT) s_pk2[i] = 0;  // (disjoint from stage 1's writes)
    __syncthreads();
    // G threads a key, each over 32 / G keys two at a time: G <= 16
    switch (min(NT / nep, 16)) {  // (uniform)
    case 16: rank_in_groups<16>(s_pk, nep, nu1, s_pk2); break;
    case 8: rank_in_groups<8>(s_pk, nep, nu1, s_pk2); break;
    default: rank_in_groups<4>(s_pk, nep, nu1, s_pk2); break;
    }
    __syncthreads();
    switch (min(NT / n2p, 16)) {  // (uniform) n2p / G >= 2
    case 16: rank_survivors<16>(s_pk2, n2, n2p, nep, ne, nu, s_ids); break;
    case 8: rank_survivors<8>(s_pk2, n2, n2p, nep, ne, nu, s_ids); break;
    default: rank_survivors<4>(s_pk2, n2, n2p, nep, ne, nu, s_ids); break;
    }
    __syncthreads();
}

// The renormalised weights of the selected experts ids[0..nu) (selection order) on one wave, with router_select's
// expressions: p = exp(logit - mx) / sum over every expert, then p / max(sum of the selected p in rank order,
// 6.103515625e-5). Lanes < nu write wts[lane].
__device__ __forceinline__ void router_weights_one_wave(const float* lg, int ne, int nu, const int* ids, float* wts) {
    const int lane = threadIdx.x & 63;
    float mx, inv;
    if (ne <= 128) {
        float v[2];
        router_softmax_norm<2>(lg, ne, v, mx, inv);
    } else if (ne <= 256) {
        float v[4];
        router_softmax_norm<4>(lg, ne, v, mx, inv);
    } else if (ne <= 512) {
        float v[8];
        router_softmax_norm<8>(lg, ne, v, mx, inv);
    } else {
        float v[16];
        router_softmax_norm<16>(lg, ne, v, mx, inv);
    }
    const float l = lane < nu ? lg[ids[lane]] : 0.0f;
    const float p = expf((l == 0.0f ? 0.0f : l) - mx) * inv;
    float ws = 0.0f;
    for (int r = 0; r < nu; ++r) ws += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), r));  // rank order
    ws = fmaxf(ws, 6.103515625e-5f);
    if (lane < nu) wts[lane] = p / ws;
}

#endif  // ROUTER_DEV_H
