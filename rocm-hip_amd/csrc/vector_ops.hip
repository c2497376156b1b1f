// vector_ops.hip -- the per-token kernels of the MoE FFN path on gfx950 (wave64) and their C-ABI launchers:
// activation quantizer, router logits (F32 matvec), router (softmax / top-k / renormalisation), SwiGLU,
// combine, and the quantizing RMSNorm producer. Semantics: src/gpu_ops.hip and src/matvec_q.hip of the
// reference; the code is laid out for 64-lane waves.

#include <math.h>

#include "gpu_ops.h"
#include "host_common.h"
#include "moe_common.h"
#include "fused_common.h"
#include "q8_quant.h"
#include "qmatvec.h"
#include "router_dev.h"

static Q8Out q8_out(const qmatvec_q8* q) {
    Q8Out o = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0};
    if (q) {
        o.q0 = q->q0;
        o.d0 = q->d0;
        o.qK = q->qK;
        o.dK = q->dK;
        o.bsK = q->bsK;
        o.s0 = q->s0;
        o.xh = q->xh;
        o.xh_bf16 = q->xh_bf16;
    }
    return o;
}

__device__ __forceinline__ void half_copy(const Q8Out& o, long long i, float v) {
    if (!o.xh) return;
    if (o.xh_bf16) {
        const uint32_t u = __float_as_uint(v);
        o.xh[i] = (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    } else {
        o.xh[i] = __half_as_ushort(__float2half(v));
    }
}

// ------------------------------------------------------------------ quantizer (src/matvec_q.hip:1245-1250)

__global__ void __launch_bounds__(256) k_quantize_q8(const float* x, int n, Q8Out o) {
    __shared__ Q8Smem sh;
    const int t = threadIdx.x;
    const long long i = (long long)blockIdx.x * 256 + t;
    const bool act = i < n;
    const float v = act ? x[i] : 0.0f;
    if (act) half_copy(o, i, v);
    q8_quantize_256(v, act, blockIdx.x, t, sh, o);
}

// The same bundle for n % 256 == 0 and 16-byte aligned x: one wave per 256-value block (q8_quantize_256_wave),
// four blocks a workgroup, 16-byte loads
__global__ void __launch_bounds__(256) k_quantize_q8_w(const float* x, long long nblk, Q8Out o) {
    const long long blk = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= nblk) return;  // (whole waves)
    const int lane = threadIdx.x & 63;
    const float4 p = *(const float4*)(x + blk * 256 + 4 * lane);
    const float v[4] = {p.x, p.y, p.z, p.w};
    if (o.xh)
#pragma unroll
        for (int j = 0; j < 4; ++j) half_copy(o, blk * 256 + 4 * lane + j, v[j]);
    q8_quantize_256_wave(v, blk, lane, o);
}

// Q8_0 values and scales only (the Q8_0-activation types need no Q8_1 sums or Q8_K): 2,048 values per
// workgroup, the quantizer's expressions (the same bits as k_quantize_q8's Q8_0 part)
__global__ void __launch_bounds__(256) k_quantize_q8_0(const float* x, int n, int8_t* q0, float* d0) {
    const int base = blockIdx.x * 2048;
    quantize_row_q8_0(x + base, min(2048, n - base), q0 + base, d0 + base / 32);
}

// ------------------------------------------------------------------ SwiGLU (src/gpu_ops.hip:103-114)

__global__ void __launch_bounds__(256) k_swiglu(const float* g, const float* u, float* out, int n, Q8Out o) {
    __shared__ Q8Smem sh;
    const int t = threadIdx.x;
    const long long i = (long long)blockIdx.x * 256 + t;
    float v = 0.0f;
    if (i < n) {
        const float a = g[i];
        v = a / (1.0f + __expf(-a)) * u[i];
        if (out) out[i] = v;
        half_copy(o, i, v);
    }
    q8_quantize_256(v, i < n, blockIdx.x, t, sh, o);
}

// The same for n % 256 == 0 and 16-byte aligned rows: a wave per 256-value block (q8_quantize_256_wave); out may be
// null (the layer's own SwiGLU, whose fp32 values nothing reads)
__global__ void __launch_bounds__(256) k_swiglu_w(const float* g, const float* u, float* out, long long nblk, Q8Out o) {
    const long long blk = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= nblk) return;  // (whole waves)
    const int lane = threadIdx.x & 63;
    const long long i0 = blk * 256 + 4 * lane;
    const float4 g4 = *(const float4*)(g + i0), u4 = *(const float4*)(u + i0);
    const float gg[4] = {g4.x, g4.y, g4.z, g4.w}, uu[4] = {u4.x, u4.y, u4.z, u4.w};
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = gg[j] / (1.0f + __expf(-gg[j])) * uu[j];
    if (out) *(float4*)(out + i0) = make_float4(v[0], v[1], v[2], v[3]);
    if (o.xh)
#pragma unroll
        for (int j = 0; j < 4; ++j) half_copy(o, i0 + j, v[j]);
    q8_quantize_256_wave(v, blk, lane, o);
}

// ------------------------------------------------------------------ combine (src/gpu_ops.hip:245-264)

// out = w0 d0 + w1 d1 + ... in slot order (each expert's output first times exp_scale[id] when set), then the
// shared expert (times sg when set)
// V consecutive values per thread (V = 4: 16-byte loads and stores, n % 4 == 0 and 16-byte aligned rows); every
// value takes the same expression in the same order either way
template <int V>
__global__ void __launch_bounds__(256) k_combine(const float* down, const float* wts, const float* shared,
                                                 const float* sg, const int* ids, const float* exp_scale, float* out,
                                                 int nu, int n) {
    typedef float vec __attribute__((ext_vector_type(V)));
    const int t = blockIdx.y;
    const int i = (blockIdx.x * 256 + threadIdx.x) * V;
    if (i >= n) return;
    const float* d = down + (size_t)t * nu * n + i;
    const float* w = wts ? wts + (size_t)t * nu : nullptr;
    auto ld = [&](const float* p) { return *(const vec*)p; };
    vec acc;
    if (nu <= 16) {  // every slot's row loaded at once (a load per loop trip waited for the previous one)
        vec v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = ld(d + (size_t)min(j, nu - 1) * n);
        if (!wts) {
            acc = v[0];
#pragma unroll
            for (int j = 1; j < 16; ++j)
                if (j < nu) acc += v[j];
        } else if (exp_scale) {
            const int* e = ids + (size_t)t * nu;
            acc = (v[0] * exp_scale[e[0]]) * w[0];
#pragma unroll
            for (int j = 1; j < 16; ++j)
                if (j < nu) acc += (v[j] * exp_scale[e[j]]) * w[j];
        } else {
            acc = w[0] * v[0];
#pragma unroll
            for (int j = 1; j < 16; ++j)
                if (j < nu) acc += w[j] * v[j];
        }
    } else if (!wts) {  // weight 1 per expert
        acc = ld(d);
        for (int j = 1; j < nu; ++j) acc += ld(d + (size_t)j * n);
    } else if (exp_scale) {
        const int* e = ids + (size_t)t * nu;
        acc = (ld(d) * exp_scale[e[0]]) * w[0];
        for (int j = 1; j < nu; ++j) acc += (ld(d + (size_t)j * n) * exp_scale[e[j]]) * w[j];
    } else {
        acc = w[0] * ld(d);
        for (int j = 1; j < nu; ++j) acc += w[j] * ld(d + (size_t)j * n);
    }
    if (shared) acc += sg ? ld(shared + (size_t)t * n + i) * sg[t] : ld(shared + (size_t)t * n + i);
    *(vec*)(out + (size_t)t * n + i) = acc;
}

// ------------------------------------------------------------------ RMSNorm producer (src/gpu_ops.hip:24-56)

// One row per workgroup: x_out = x_in + add; y = x_out / sqrt(mean(x_out^2) + eps) * w, quantized per 256
__global__ void __launch_bounds__(256) k_add_rmsnorm(const float* x_in, const float* add, float* x_out,
                                                     const float* w, float* y, int n, float eps, Q8Out o,
                                                     int wave_blocks) {
    __shared__ Q8Smem sh;
    __shared__ float part[4];
    const int t = threadIdx.x, row = blockIdx.x;
    const float* xr = x_in + (size_t)row * n;
    const float* ar = add ? add + (size_t)row * n : nullptr;
    // rows of up to 4096 values stay in registers between the two passes (one read of x and add)
    constexpr int KEEP = 16;
    float keep[KEEP];
    const bool kept = n <= 256 * KEEP;
    float inv;
    float wn[KEEP];  // kept rows: the weights, loaded with x and add
    if (kept && rms_rows4(xr, ar, n) && n % 256 == 0 && wave_blocks) {
        // rms_first_pass4's layout is already the wave quantizer's: thread t's piece k is values 4 (t % 64) .. + 3 of
        // 256-value block 4 k + t / 64, so each wave takes its blocks from registers (16-byte stores, no LDS)
        const int lane = t & 63, wv = t >> 6, nb4 = n / 256;
        float4 wq[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            wq[k] = w ? ((const float4*)w)[min(t + 256 * k, n / 4 - 1)] : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
        float4 keep4[4];
        inv = rms_first_pass4(xr, ar, n, eps, keep4, part);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int b = 4 * k + wv;
            if (b >= nb4) break;  // (uniform per wave)
            const long long i = (long long)row * n + 256 * b + 4 * lane;
            const float4 xv = keep4[k];
            const float v[4] = {xv.x * inv * wq[k].x, xv.y * inv * wq[k].y, xv.z * inv * wq[k].z, xv.w * inv * wq[k].w};
            if (ar) *(float4*)(x_out + i) = xv;
            *(float4*)(y + i) = make_float4(v[0], v[1], v[2], v[3]);
#pragma unroll
            for (int j = 0; j < 4; ++j) half_copy(o, i + j, v[j]);
            q8_quantize_256_wave(v, (long long)row * nb4 + b, lane, o);
        }
        return;
    }
    if (kept && rms_rows4(xr, ar, n)) {
        // the squares in the 16-byte layout (rms_first_pass4, shared with the fused layer), then the values moved
        // through LDS into this kernel's layout (t + 256 k: one per thread and 256-value block for the quantizer)
        __shared__ __align__(16) float row4[256 * KEEP];
#pragma unroll
        for (int k = 0; k < KEEP; ++k) wn[k] = w ? w[min(t + 256 * k, n - 1)] : 1.0f;
        float4 keep4[4];
        inv = rms_first_pass4(xr, ar, n, eps, keep4, part);
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (t + 256 * k < n / 4) ((float4*)row4)[t + 256 * k] = keep4[k];
        __syncthreads();
#pragma unroll
        for (int k = 0; k < KEEP; ++k) keep[k] = t + 256 * k < n ? row4[t + 256 * k] : 0.0f;
    } else if (kept) {
#pragma unroll
        for (int k = 0; k < KEEP; ++k) wn[k] = w ? w[min(t + 256 * k, n - 1)] : 1.0f;
        inv = rms_first_pass(xr, ar, n, eps, keep, part);
    } else {
        float ss = 0.0f;
        for (int i = t; i < n; i += 256) {
            const float v = ar ? xr[i] + ar[i] : xr[i];
            ss += v * v;
        }
        ss = wave_sum(ss);
        if ((t & 63) == 0) part[t >> 6] = ss;
        __syncthreads();
        const float tot = (part[0] + part[1]) + (part[2] + part[3]);
        inv = 1.0f / sqrtf(tot / (float)n + eps);
    }
    const int nb = (n + 255) / 256;
    auto block = [&](int b, float xv, float wv) {  // block b of 256 values: outputs, then the quantizer (uniform call)
        const int i = b * 256 + t;
        const bool act = i < n;
        float v = 0.0f;
        if (act) {
            if (ar) x_out[(size_t)row * n + i] = xv;
            v = xv * inv * wv;
            y[(size_t)row * n + i] = v;
            half_copy(o, (long long)row * n + i, v);
        }
        q8_quantize_256(v, act, (long long)row * nb + b, t, sh, o);
    };
    if (kept) {
#pragma unroll
        for (int b = 0; b < KEEP; ++b)
            if (b < nb) block(b, keep[b], wn[b]);
    } else {
        for (int b = 0; b < nb; ++b) {
            const int i = b * 256 + t;
            block(b, i < n ? (ar ? xr[i] + ar[i] : xr[i]) : 0.0f, w && i < n ? w[i] : 1.0f);
        }
    }
}

// ------------------------------------------------------------------ router logits: F32 matvec

// Decode: one 256-thread workgroup per row and token, 16-byte loads (K / 1024 per thread), x re-read from L1 /
// L2. y[row] = W[row] . x
__global__ void __launch_bounds__(256) k_matvec_f32(const float* W, long long ldw, const float* x, float* y, int N,
                                                   int K) {
    __shared__ float part[4];
    const int row = blockIdx.x;
    const float acc = f32_row_dot(W + (size_t)row * ldw, x + (size_t)blockIdx.y * K, K, part);
    if (threadIdx.x == 0) y[(size_t)blockIdx.y * N + row] = acc;
}

// Prefill: tiles of 32 tokens x 32 rows (enough workgroups to fill the chip at a few thousand tokens), K staged
// through LDS in chunks of 64; each thread 2 x 2 outputs.
#define MF_TT 32
#define MF_TR 32
#define MF_KC 64
__global__ void __launch_bounds__(256) k_matmul_f32(const float* W, long long ldw, const float* X, float* Y, int N,
                                                   int K, int T) {
    __shared__ float sw[MF_KC][MF_TR + 1];
    __shared__ float sx[MF_KC][MF_TT + 1];
    const int tid = threadIdx.x;
    const int r0 = blockIdx.x * MF_TR, t0 = blockIdx.y * MF_TT;
    const int tr = (tid & 15) * 2, tt = (tid >> 4) * 2;
    float acc[2][2] = {};
    for (int k0 = 0; k0 < K; k0 += MF_KC) {
        for (int i = tid; i < MF_TR * MF_KC; i += 256) {
            const int r = i / MF_KC, k = i % MF_KC;
            sw[k][r] = (r0 + r < N && k0 + k < K) ? W[(size_t)(r0 + r) * ldw + k0 + k] : 0.0f;
            sx[k][r] = (t0 + r < T && k0 + k < K) ? X[(size_t)(t0 + r) * K + k0 + k] : 0.0f;
        }
        __syncthreads();
#pragma unroll 16
        for (int k = 0; k < MF_KC; ++k) {
            const float a0 = sx[k][tt], a1 = sx[k][tt + 1], b0 = sw[k][tr], b1 = sw[k][tr + 1];
            acc[0][0] = fmaf(a0, b0, acc[0][0]);
            acc[0][1] = fmaf(a0, b1, acc[0][1]);
            acc[1][0] = fmaf(a1, b0, acc[1][0]);
            acc[1][1] = fmaf(a1, b1, acc[1][1]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
            if (t0 + tt + i < T && r0 + tr + j < N) Y[(size_t)(t0 + tt + i) * N + r0 + tr + j] = acc[i][j];
}

// Prefill on fp32 MFMA (v_mfma_f32_32x32x2f32, exact fp32 products): one 32-token x 32-row output tile per
// workgroup, its MF_KS waves each 1 / MF_KS of K (more waves in flight to cover the loads' latency), summed through
// LDS in a fixed order. Both operands are rows along K; lane l holds 16 consecutive values (64 bytes) of token /
// weight row l % 32 per 32-value chunk (its half l / 32 of the chunk), and MFMA q of the chunk pairs value q of
// both lanes' runs: k = chunk + 16 h + q on both sides. K % (32 MF_KS) == 0.
// Each wave stages its chunks through its own 8 KB of LDS with LDS-direct loads (eight lanes per 128-byte row
// segment: 8 cache lines per load instead of the 32 of loads in MFMA layout), the 16-byte pieces of row r stored
// XOR-swizzled by (r / 2) % 8 so that the MFMA-layout reads of 16 lanes at a time hit 16 distinct bank groups.
// Per chunk: its operands to registers, the next chunk's loads into the same LDS, then the 16 MFMAs.
// Workgroups go to the 8 XCDs in turn (linear id L on XCD L % 8), so the grid is one-dimensional and L = 8 j + c
// takes token tile 8 (j / nx) + c, row tile j % nx: the nx workgroups of a token tile share one XCD's L2, which
// then fetches the tile's 32 token rows once (a row tile per grid column had spread them over all 8).
typedef float mf_v16f __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void mf_lds_void;
#ifndef MF_KS
#define MF_KS 8
#endif
__global__ void __launch_bounds__(64 * MF_KS) k_matmul_f32_mfma(const float* W, long long ldw, const float* X,
                                                               float* Y, int N, int K, int T) {
    __shared__ __align__(16) float stage[MF_KS][2][32 * 32];  // [wave][tokens / rows][row * 32 + value]
    static_assert((MF_KS - 1) * 16 * 64 <= MF_KS * 2 * 32 * 32, "the partial sums reuse the stage buffers");
    float (*red)[16][64] = (float (*)[16][64])&stage[0][0][0];  // after the loop: waves 1.. partial sums
    const int tid = threadIdx.x, l = tid & 63, w = tid >> 6, h = l >> 5, r = l & 31;
    const int nx = (N + 31) / 32, xc = blockIdx.x & 7, j = blockIdx.x >> 3;
    const int r0 = (j % nx) * 32, t0 = (8 * (j / nx) + xc) * 32;
    if (t0 >= T) return;  // (the last round of token tiles on some XCDs; uniform)
    const int kq = K / MF_KS, kb = w * kq;  // this wave's share of K
    // load i of a chunk: lane l brings row 8 i + l / 8, piece (l % 8) ^ swz(row) of the row's 128 bytes
    const float* gx[4];
    const float* gw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = 8 * i + (l >> 3), piece = (l & 7) ^ ((row >> 1) & 7);
        gx[i] = X + (size_t)min(t0 + row, T - 1) * K + kb + 4 * piece;  // (rows past the end: the last row,
        gw[i] = W + (size_t)min(r0 + row, N - 1) * ldw + kb + 4 * piece;  //  results unused)
    }
    float* sx = stage[w][0];
    float* sw = stage[w][1];
    auto issue = [&](int c) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_global_load_lds(gx[i] + c, (mf_lds_void*)(sx + 256 * i), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(gw[i] + c, (mf_lds_void*)(sw + 256 * i), 16, 0, 0);
        }
    };
    issue(0);
    mf_v16f acc = {};
    for (int c = 0; c < kq; c += 32) {
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this chunk's pieces are in LDS
        float4 xa[4], wa[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {  // piece 4 h + q of row r, where the swizzle put it
            const int at = 32 * r + 4 * ((4 * h + q) ^ ((r >> 1) & 7));
            xa[q] = *(const float4*)(sx + at);
            wa[q] = *(const float4*)(sw + at);
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the reads are done before the next loads overwrite
        if (c + 32 < kq) issue(c + 32);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[q].x, wa[q].x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[q].y, wa[q].y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[q].z, wa[q].z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[q].w, wa[q].w, acc, 0, 0, 0);
        }
    }
    __syncthreads();  // every wave is past its stage buffer
    if (w > 0)
#pragma unroll
        for (int i = 0; i < 16; ++i) red[w - 1][i][l] = acc[i];
    __syncthreads();
    if (w == 0) {  // acc[i]: token 8 (i / 4) + 4 h + i % 4, row l % 32 of the tile
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float v = acc[i];
#pragma unroll
            for (int q = 0; q < MF_KS - 1; ++q) v += red[q][i][l];
            const int t = t0 + 8 * (i >> 2) + 4 * h + (i & 3), rr = r0 + (l & 31);
            if (t < T && rr < N) Y[(size_t)t * N + rr] = v;
        }
    }
}

// ------------------------------------------------------------------ router (src/gpu_ops.hip:185-241)

// One 256-thread workgroup per token: the shared-expert gate, then router_select (router_dev.h). QX (the layer's
// prefill): waves 1..3 also quantize the token's row of x (n % 256 == 0) into o while wave 0 selects -- the wave
// quantizer's expressions, so the bits of k_quantize_q8_w / k_quantize_q8_0 -- which saves the quantizer's launch.
template <bool QX>
__global__ void __launch_bounds__(256) k_router(const float* logits, const float* x, const float* w_shexp, int* ids,
                                                float* wts, float* sg, int ne, int nu, int n, int ids_stride, Q8Out o) {
    __shared__ float part[4];
    const int t = blockIdx.x, tid = threadIdx.x;
    if (w_shexp) {  // (uniform branch)
        const float g = shexp_gate(x + (size_t)t * n, w_shexp, n, part);
        if (tid == 0) sg[t] = g;
    }
    if (QX && tid >= 64) {
        const int nb = n / 256, lane = tid & 63;
        for (int b = (tid >> 6) - 1; b < nb; b += 3) {
            const long long blk = (long long)t * nb + b;
            const float4 p = *(const float4*)(x + blk * 256 + 4 * lane);
            const float v[4] = {p.x, p.y, p.z, p.w};
            q8_quantize_256_wave(v, blk, lane, o);
        }
    }
    int* id_row = ids + (size_t)t * ids_stride;
    router_select(logits + (size_t)t * ne, ne, nu, id_row, wts + (size_t)t * nu);
    if (tid == 0 && ids_stride > nu) id_row[nu] = -1;
}

// ------------------------------------------------------------------ C ABI

extern "C" size_t qmatvec_q8_bytes(int max_k) {
    const size_t k = (size_t)max_k;
    auto a16 = [](size_t v) { return (v + 15) & ~(size_t)15; };
    return 2 * a16(k) + 2 * a16(k / 32 * 4) + a16(k / 256 * 4) + a16(k / 16 * 4);
}

extern "C" void qmatvec_q8_bind(qmatvec_q8* q, void* mem, int max_k) {
    const size_t k = (size_t)max_k;
    auto a16 = [](size_t v) { return (v + 15) & ~(size_t)15; };
    char* p = (char*)mem;
    q->q0 = (int8_t*)p;
    p += a16(k);
    q->qK = (int8_t*)p;
    p += a16(k);
    q->d0 = (float*)p;
    p += a16(k / 32 * 4);
    q->dK = (float*)p;
    p += a16(k / 256 * 4);
    q->bsK = (int32_t*)p;
    p += a16(k / 16 * 4);
    q->s0 = (int32_t*)p;
    q->max_k = max_k;
    q->xh = nullptr;
    q->xh_bf16 = 0;
}

extern "C" hipError_t qmatvec_quantize(const float* x, int K, const qmatvec_q8* q, hipStream_t stream) {
    if (!moe_lib_ready()) return hipErrorNotInitialized;
    if (!q || K <= 0 || K % 32 != 0 || K > q->max_k) return hipErrorInvalidValue;
    if (K % 256 == 0 && aligned(x, 16) && aligned(q->q0, 4) && aligned(q->qK, 4))
        return launch_kernel(k_quantize_q8_w, dim3((K / 256 + 3) / 4), dim3(256), 0, stream, x, (long long)K / 256,
                             q8_out(q));
    return launch_kernel(k_quantize_q8, dim3((K + 255) / 256), dim3(256), 0, stream, x, K, q8_out(q));
}

extern "C" int qmatvec_supported(int type) { return type == QT_F32; }

extern "C" hipError_t qmatvec_launch(int type, const void* W, size_t row_bytes, const float* x, float* y, int N, int K,
                                     hipStream_t stream) {
    if (!moe_lib_ready()) return hipErrorNotInitialized;
    if (type != QT_F32) return hipErrorInvalidDeviceFunction;
    if (N <= 0 || K <= 0 || row_bytes != (size_t)K * 4) return hipErrorInvalidValue;
    return launch_kernel(k_matvec_f32, dim3(N), dim3(256), 0, stream, (const float*)W, (long long)K, x, y, N, K);
}

extern "C" hipError_t qmatvec_launch_batch(int type, const void* W, size_t row_bytes, const float* x, float* y, int N,
                                           int K, int T, hipStream_t stream) {
    if (!moe_lib_ready()) return hipErrorNotInitialized;
    if (type != QT_F32) return hipErrorInvalidDeviceFunction;
    if (N <= 0 || K <= 0 || T <= 0 || row_bytes != (size_t)K * 4) return hipErrorInvalidValue;
    if (T <= 16)  // a few tokens: the decode kernel per token (the same sums as T single-token launches)
        return launch_kernel(k_matvec_f32, dim3(N, T), dim3(256), 0, stream, (const float*)W, (long long)K, x, y, N, K);
    if (K % (32 * MF_KS) == 0 && (((uintptr_t)W | (uintptr_t)x) & 15) == 0)
        return launch_kernel(k_matmul_f32_mfma, dim3(8 * ((N + 31) / 32) * ((T + 255) / 256)), dim3(64 * MF_KS), 0,
                             stream, (const float*)W, (long long)K, x, y, N, K, T);
    return launch_kernel(k_matmul_f32, dim3((N + MF_TR - 1) / MF_TR, (T + MF_TT - 1) / MF_TT), dim3(256), 0, stream,
                         (const float*)W, (long long)K, x, y, N, K, T);
}

extern "C" hipError_t gpu_add_rmsnorm(const float* x_in, const float* add, float* x_out, const float* w, float* y,
                                      int n, int T, float eps, const qmatvec_q8* q8, hipStream_t stream) {
    if (!moe_lib_ready()) return hipErrorNotInitialized;
    if (T <= 0 || n <= 0 || (q8 && (n % 256 != 0 || (long long)n * T > q8->max_k)) || (add && x_out == x_in))
        return hipErrorInvalidValue;
    // whole 256-value blocks on the wave quantizer where every row and output is aligned for its 16 / 4-byte stores
    const int wave_blocks = n % 256 == 0 && aligned(y, 16) && (!add || aligned(x_out, 16)) && (!w || aligned(w, 16)) &&
                            (!q8 || (aligned(q8->q0, 4) && aligned(q8->qK, 4)));
    return launch_kernel(k_add_rmsnorm, dim3(T), dim3(256), 0, stream, x_in, add, x_out, w, y, n, eps, q8_out(q8),
                         wave_blocks);
}

extern "C" hipError_t gpu_swiglu(const float* g, const float* u, float* out, int n, const qmatvec_q8* q8,
                                 hipStream_t stream) {
    if (!moe_lib_ready()) return hipErrorNotInitialized;
    if (n <= 0 || (q8 && (n % 32 != 0 || n > q8->max_k))) return hipErrorInvalidValue;
    return moe_swiglu_q8(g, u, out, n, q8, stream, 3);
}

// The bundle with only the formats in parts (1: Q8_0 + Q8_1 sums, 2: Q8_K) on the wave-per-block path
static Q8Out q8_out_parts(const qmatvec_q8* q, int parts) {
    Q8Out o = q8_out(q);
    if (!(parts & 1)) o.q0 = nullptr;
    if (!(parts & 2)) o.qK = nullptr;
    return o;
}

hipError_t moe_swiglu_q8(const float* g, const float* u, float* out, int n, const qmatvec_q8* q8, hipStream_t stream,
                         int parts) {
    if (n % 256 == 0 && (((uintptr_t)g | (uintptr_t)u | (uintptr_t)out) & 15) == 0 &&
        (!q8 || (aligned(q8->q0, 4) && aligned(q8->qK, 4))))
        return launch_kernel(k_swiglu_w, dim3((n / 256 + 3) / 4), dim3(256), 0, stream, g, u, out, (long long)n / 256,
                             q8_out_parts(q8, parts));
    return launch_kernel(k_swiglu, dim3((n + 255) / 256), dim3(256), 0, stream, g, u, out, n, q8_out(q8));
}

extern "C" hipError_t gpu_moe_router(const float* logits, const float* x, const float* w_shexp, int* ids, float* wts,
                                     float* sg, int n_expert, int n_used, int n, int T, hipStream_t stream,
                                     int ids_stride) {
    if (!moe_lib_ready()) return hipErrorNotInitialized;
    if (n_expert <= 0 || n_expert > 1024 || n_used <= 0 || n_used > 64 || n_used > n_expert || T <= 0)
        return hipErrorInvalidValue;
    if (ids_stride == 0) ids_stride = n_used;
    if (ids_stride < n_used || (w_shexp && (!x || !sg || n <= 0))) return hipErrorInvalidValue;
    return launch_kernel(k_router<false>, dim3(T), dim3(256), 0, stream, logits, x, w_shexp, ids, wts, sg, n_expert,
                         n_used, n, ids_stride, Q8Out{});
}

// Internal (moe_layer_forward): gpu_moe_router with x [T][n] quantized into q8 (the formats in parts) by the same
// launch; n % 256 == 0, x 16-byte and the values 4-byte aligned
hipError_t moe_router_quantize(const float* logits, const float* x, const float* w_shexp, int* ids, float* wts,
                               float* sg, int n_expert, int n_used, int n, int T, int ids_stride, const qmatvec_q8* q8,
                               int parts, hipStream_t stream) {
    if (!moe_lib_ready()) return hipErrorNotInitialized;
    if (n_expert <= 0 || n_expert > 1024 || n_used <= 0 || n_used > 64 || n_used > n_expert || T <= 0 || n <= 0 ||
        n % 256 || !x || !q8 || q8->xh || (long long)n * T > q8->max_k || !aligned(x, 16) || !aligned(q8->q0, 4) ||
        !aligned(q8->qK, 4))
        return hipErrorInvalidValue;
    if (ids_stride == 0) ids_stride = n_used;
    if (ids_stride < n_used || (w_shexp && !sg)) return hipErrorInvalidValue;
    return launch_kernel(k_router<true>, dim3(T), dim3(256), 0, stream, logits, x, w_shexp, ids, wts, sg, n_expert,
                         n_used, n, ids_stride, q8_out_parts(q8, parts));
}

// Internal (moe_layer_forward_norm): gpu_add_rmsnorm with y's quantized bundle (the formats in parts) written by the
// same launch, on its wave path only (rows of at most 4,096 values, a multiple of 256, every row and output
// aligned), which returns hipErrorInvalidValue where that path does not apply
hipError_t moe_add_rmsnorm_q8(const float* x_in, const float* add, float* x_out, const float* w, float* y, int n,
                              int T, float eps, const qmatvec_q8* q8, int parts, hipStream_t stream) {
    if (!moe_lib_ready()) return hipErrorNotInitialized;
    if (T <= 0 || n <= 0 || n > 4096 || n % 256 || !q8 || q8->xh || (long long)n * T > q8->max_k ||
        (add && x_out == x_in) || !aligned(x_in, 16) || (add && !aligned(add, 16)) || !aligned(y, 16) ||
        (add && !aligned(x_out, 16)) || (w && !aligned(w, 16)) || !aligned(q8->q0, 4) || !aligned(q8->qK, 4))
        return hipErrorInvalidValue;
    return launch_kernel(k_add_rmsnorm, dim3(T), dim3(256), 0, stream, x_in, add, x_out, w, y, n, eps,
                         q8_out_parts(q8, parts), 1);
}

extern "C" hipError_t gpu_moe_combine_scaled(const float* down, const float* wts, const float* shared, const float* sg,
                                             const int* ids, const float* exp_scale, float* out, int n_used, int n,
                                             int T, hipStream_t stream) {
    if (!moe_lib_ready()) return hipErrorNotInitialized;
    if (n_used <= 0 || n <= 0 || T <= 0 || (exp_scale && (!ids || !wts))) return hipErrorInvalidValue;
    if (n % 4 == 0 && aligned(down, 16) && aligned(out, 16) && (!shared || aligned(shared, 16)))
        return launch_kernel(k_combine<4>, dim3((n / 4 + 255) / 256, T), dim3(256), 0, stream, down, wts, shared, sg,
                             ids, exp_scale, out, n_used, n);
    return launch_kernel(k_combine<1>, dim3((n + 255) / 256, T), dim3(256), 0, stream, down, wts, shared, sg, ids,
                         exp_scale, out, n_used, n);
}

extern "C" hipError_t gpu_moe_combine(const float* down, const float* wts, const float* shared, const float* sg,
                                      float* out, int n_used, int n, int T, hipStream_t stream) {
    return gpu_moe_combine_scaled(down, wts, shared, sg, nullptr, nullptr, out, n_used, n, T, stream);
}

// Internal (moe_layer_forward, Q4_K): x's Q8_K part only (n % 256 == 0, n <= q->max_k); qmatvec_quantize's
// kernels and bits
hipError_t moe_quantize_q8k(const float* x, int n, const qmatvec_q8* q, hipStream_t stream) {
    if (!moe_lib_ready()) return hipErrorNotInitialized;
    if (n <= 0 || n % 256 || !q || n > q->max_k) return hipErrorInvalidValue;
    if (aligned(x, 16) && aligned(q->qK, 4))
        return launch_kernel(k_quantize_q8_w, dim3((n / 256 + 3) / 4), dim3(256), 0, stream, x, (long long)n / 256,
                             q8_out_parts(q, 2));
    return launch_kernel(k_quantize_q8, dim3((n + 255) / 256), dim3(256), 0, stream, x, n, q8_out(q));
}

// Internal (moe_layer_forward): Q8_0 values and scales of x [n] into q (n % 32 == 0, n <= q->max_k)
hipError_t moe_quantize_q8_0(const float* x, int n, const qmatvec_q8* q, hipStream_t stream) {
    if (!moe_lib_ready()) return hipErrorNotInitialized;
    if (n <= 0 || n % 32 || !q || n > q->max_k) return hipErrorInvalidValue;
    return launch_kernel(k_quantize_q8_0, dim3((n + 2047) / 2048), dim3(256), 0, stream, x, n, q->q0, q->d0);
}
