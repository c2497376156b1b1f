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

// Order-preserving map of a float onto uint32 (larger float, larger key; -0 below +0)
__device__ __forceinline__ uint32_t f32_order_key(float v) {
    const uint32_t u = __float_as_uint(v);
    return u ^ ((u >> 31) ? 0xffffffffu : 0x80000000u);
}

__device__ __forceinline__ float f32_from_order_key(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? k ^ 0x80000000u : ~k);
}

// Largest 64-bit key over the wave, in every lane
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t k) {
#define RS_STEP(S)                                                                              \
    {                                                                                           \
        const uint32_t lo = (uint32_t)partner_i<S>((int)(uint32_t)k);                           \
        const uint32_t hi = (uint32_t)partner_i<S>((int)(uint32_t)(k >> 32));                   \
        const uint64_t o = ((uint64_t)hi << 32) | lo;                                           \
        k = o > k ? o : k;                                                                      \
    }
    RS_STEP(1) RS_STEP(2) RS_STEP(4) RS_STEP(8) RS_STEP(16) RS_STEP(32)
#undef RS_STEP
    return k;
}

// Selection on one wave; lane l holds logits l, l + 64, ... (NPL of them). Key: the logit's order key above the
// complement of its index, so the largest key is the largest logit, ties to the lower index; a taken (or absent)
// entry has key 0, below every real one.
template <int NPL>
__device__ __forceinline__ void router_select_wave(const float* lg, int ne, int nu, int* id_row, float* wts) {
    const int lane = threadIdx.x & 63;
    float v[NPL];
    uint64_t key[NPL];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
        const int e = lane + 64 * j;
        v[j] = e < ne ? lg[e] : -INFINITY;
        key[j] = e < ne ? ((uint64_t)f32_order_key(v[j]) << 32) | (0xffffffffu - (uint32_t)e) : 0;
        mx = fmaxf(mx, v[j]);
    }
    mx = wave_max(mx);
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < NPL; ++j)
        if (lane + 64 * j < ne) sum += expf(v[j] - mx);
    sum = wave_sum(sum);
    const float inv = 1.0f / sum;
    float ws = 0.0f, myp = 0.0f;
    int myid = 0;
    for (int r = 0; r < nu; ++r) {
        uint64_t best = key[0];
#pragma unroll
        for (int j = 1; j < NPL; ++j) best = key[j] > best ? key[j] : best;
        best = wave_max_u64(best);
#pragma unroll
        for (int j = 0; j < NPL; ++j)
            if (key[j] == best) key[j] = 0;
        const int e = (int)(0xffffffffu - (uint32_t)best);
        const float p = expf(f32_from_order_key((uint32_t)(best >> 32)) - mx) * inv;
        ws += p;  // the sum in rank order
        if (lane == r) {
            myp = p;
            myid = e;
        }
    }
    ws = fmaxf(ws, 6.103515625e-5f);
    if (lane < nu) {
        id_row[lane] = myid;
        wts[lane] = myp / ws;
    }
}

// Softmax over ne (<= ROUTER_MAX_E) logits, the nu (<= 64) largest in descending order (ties to the lower index),
// weights renormalised by max(sum, 6.103515625e-5). Wave 0 of the 256-thread workgroup selects; it writes
// id_row[0..nu) and wts[0..nu) (any memory), visible to the whole workgroup on return.
__device__ __forceinline__ void router_select(const float* lg, int ne, int nu, int* id_row, float* wts) {
    if (threadIdx.x < 64) {
        if (ne <= 128)
            router_select_wave<2>(lg, ne, nu, id_row, wts);
        else if (ne <= 256)
            router_select_wave<4>(lg, ne, nu, id_row, wts);
        else if (ne <= 512)
            router_select_wave<8>(lg, ne, nu, id_row, wts);
        else
            router_select_wave<16>(lg, ne, nu, id_row, wts);
    }
    __syncthreads();
}

#endif  // ROUTER_DEV_H
