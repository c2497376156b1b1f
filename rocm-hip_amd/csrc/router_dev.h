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

// Softmax over ne logits, the nu largest in descending order (ties to the lower index), weights renormalised by
// max(sum, 6.103515625e-5). sl: LDS of ROUTER_MAX_E floats; sel_p: LDS of 64. Writes id_row[0..nu) (any memory)
// and, from thread 0, wts[0..nu). Selection by rank counting: an expert's rank is the number of experts with a
// larger logit or an equal one at a lower index (softmax is strictly monotonic, so this is the probability order).
__device__ __forceinline__ void router_select(const float* lg, int ne, int nu, float* sl, float* part, float* sel_p,
                                              int* id_row, float* wts) {
    const int tid = threadIdx.x;
    for (int e = tid; e < ne; e += 256) sl[e] = lg[e];
    const int ne4 = (ne + 3) & ~3;
    for (int e = ne + tid; e < ne4; e += 256) sl[e] = -INFINITY;  // pad: never beats a real expert
    float mx = -INFINITY;
    for (int e = tid; e < ne; e += 256) mx = fmaxf(mx, lg[e]);
    mx = wave_max(mx);
    if ((tid & 63) == 0) part[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
    __syncthreads();
    float sum = 0.0f;
    for (int e = tid; e < ne; e += 256) sum += expf(sl[e] - mx);
    sum = block256_sum(sum, part);
    const float inv = 1.0f / sum;
    for (int e = tid; e < ne; e += 256) {
        const float v = sl[e];
        int rank = 0;
        for (int k = 0; k < ne4; k += 4) {
            const float4 c = *(const float4*)(sl + k);
            rank += (c.x > v || (c.x == v && k < e)) + (c.y > v || (c.y == v && k + 1 < e)) +
                    (c.z > v || (c.z == v && k + 2 < e)) + (c.w > v || (c.w == v && k + 3 < e));
        }
        if (rank < nu) {
            id_row[rank] = e;
            sel_p[rank] = expf(v - mx) * inv;
        }
    }
    __syncthreads();
    if (tid == 0) {
        float ws = 0.0f;
        for (int r = 0; r < nu; ++r) ws += sel_p[r];
        ws = fmaxf(ws, 6.103515625e-5f);
        for (int r = 0; r < nu; ++r) wts[r] = sel_p[r] / ws;
    }
}

#endif  // ROUTER_DEV_H
