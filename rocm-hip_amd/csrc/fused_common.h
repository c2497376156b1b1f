// fused_common.h -- device pieces shared by the fused decode-layer kernels (fused_decode.hip: one token;
// fused_multi.hip: 2..7 tokens). Each restates a per-operation kernel's expressions, so the fused layers produce
// the per-operation path's bits.
#ifndef FUSED_COMMON_H
#define FUSED_COMMON_H

#include "expert_units.h"
#include "moe_layer.h"
#include "qmatvec.h"
#include "q8_quant.h"
#include "router_dev.h"

#define FD_MAX_E 4096  // largest E the fused kernels take
#define FD_MAX_T 7     // largest token count of the multi-token fused kernels (T >= 8 is the grouped path)

// Arguments of the fused kernels (T = 1: fused_decode.hip; T = 2..FD_MAX_T: fused_multi.hip)
struct FArgs {
    const float* x;          // [T][E]
    const float* logits_in;  // [T][NE] or nullptr
    const float* w_router;   // [NE][E]
    const float* w_shexp;    // [E] or nullptr
    const uint8_t* v[6];     // value planes: gate, up, down (stacked experts), shared gate, up, down
    const uint8_t* s[6];     // scale planes
    long long vrb_in, srb_in, vrb_out, srb_out;  // plane row bytes for K = E and K = FE
    float* out;              // [T][E]
    int* ids_out;            // [T][NU] or nullptr
    float* wts_out;          // [T][NU] or nullptr
    float* logits;           // scratch [T][NE]
    float* sg;               // scratch [T]
    int8_t* xq;              // scratch: x quantized, Q8_0 values [T][E] and scales [T][E / 32]
    float* xd;
    int* ids;                // scratch: the routing [T][ids_ld] (ids_ld: NU, or NS when the router kernel wrote it)
    float* wts;
    int8_t* act_q;           // scratch [T][NS][FE]
    float* act_d;            // scratch [T][NS][FE / 32]
    // Q4_K (T = 1): x's Q8_K bundle (written by kernel 1 through xo), the gate / up outputs in fp32, and down's
    // input bundle (written by the SwiGLU kernel between kernels 2 and 3)
    Q8Out xo;
    float* g;                // scratch [NS][FE]
    float* u;
    float* act;
    int8_t* aqk;             // down's input: Q8_K values [NS][FE], scales [NS][FE / 256], sums [NS][FE / 16]
    float* adk;
    int32_t* absk;
    unsigned long long* stamps;  // optional timestamps (profiling, one token): [workgroup][8], nullptr: none
    // norm set (T = 1): the layer's input is RMSNorm(x + add) * w_norm, formed by kernel 1 (gpu_add_rmsnorm's
    // expressions); x_out (when add is set) receives x + add
    const float* add;
    const float* w_norm;
    float* x_out;
    float eps;
    int norm;
    int T, E, NE, NU, FE, NS, has_gate, ids_ld;
    // T = 1 (set by the launcher): kernel 2 routes by rank counting over the whole workgroup and publishes only the
    // ids; kernel 3 has one more wave that forms the renormalised weights from the logits
    int rank_route;
};

// The RMSNorm producer fused into the layer (moe_layer_forward_norm): its arguments
struct FNorm {
    const float* add;
    const float* w;
    float* x_out;
    float eps;
};

// The RMSNorm producer's first pass (src/gpu_ops.hip:24-56, gpu_add_rmsnorm): thread t's values t + 256 k (k < 16,
// n <= 4096) of x (+ add) into keep, and the row's 1 / sqrt(mean(v^2) + eps). Every caller shares these expressions.
__device__ __forceinline__ float rms_first_pass(const float* xr, const float* ar, int n, float eps, float (&keep)[16],
                                                float* part) {
    const int t = threadIdx.x;
    float ss = 0.0f;
    // every load unconditional (past the end: the last value, unused) so that all of them are in flight at once;
    // a load under a per-value branch had each pair wait for the previous one
    float xv[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) xv[k] = xr[min(t + 256 * k, n - 1)];
    if (ar) {
        float av[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) av[k] = ar[min(t + 256 * k, n - 1)];
#pragma unroll
        for (int k = 0; k < 16; ++k) keep[k] = t + 256 * k < n ? xv[k] + av[k] : 0.0f;
    } else {
#pragma unroll
        for (int k = 0; k < 16; ++k) keep[k] = t + 256 * k < n ? xv[k] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) ss += keep[k] * keep[k];
    ss = wave_sum(ss);
    if ((t & 63) == 0) part[t >> 6] = ss;
    __syncthreads();
    const float tot = (part[0] + part[1]) + (part[2] + part[3]);
    return 1.0f / sqrtf(tot / (float)n + eps);
}

// Whether a row (and its addend) can take rms_first_pass4: n % 4 == 0, 16-byte aligned
__device__ __forceinline__ bool rms_rows4(const float* xr, const float* ar, int n) {
    return (n & 3) == 0 && (((uintptr_t)xr | (uintptr_t)(ar ? ar : xr)) & 15) == 0;
}

// The first pass for rows that rms_rows4 admits (n <= 4096): thread t's values 4 t + 1024 k + j (k < 4, j < 4) --
// the layout of the F32 row dot's 16-byte loads (f32_row_dot), so that a router-row dot can use them in place --
// loaded as 16-byte pieces (every load unconditional, past the end the last piece, unused), into keep; returns the
// row's 1 / sqrt(mean(v^2) + eps), the squares summed in (k, j) order per thread, then over the workgroup. The
// producer kernel (gpu_add_rmsnorm) and the fused layer share it, so they give the same bits.
__device__ __forceinline__ float rms_first_pass4(const float* xr, const float* ar, int n, float eps, float4 (&keep)[4],
                                                 float* part) {
    const int t = threadIdx.x, n4 = n >> 2;
    float4 xv[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) xv[k] = ((const float4*)xr)[min(t + 256 * k, n4 - 1)];
    if (ar) {
        float4 av[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) av[k] = ((const float4*)ar)[min(t + 256 * k, n4 - 1)];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const bool in = t + 256 * k < n4;
            keep[k] = in ? make_float4(xv[k].x + av[k].x, xv[k].y + av[k].y, xv[k].z + av[k].z, xv[k].w + av[k].w)
                         : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) keep[k] = t + 256 * k < n4 ? xv[k] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        ss += keep[k].x * keep[k].x;
        ss += keep[k].y * keep[k].y;
        ss += keep[k].z * keep[k].z;
        ss += keep[k].w * keep[k].w;
    }
    ss = wave_sum(ss);
    if ((t & 63) == 0) part[t >> 6] = ss;
    __syncthreads();
    const float tot = (part[0] + part[1]) + (part[2] + part[3]);
    return 1.0f / sqrtf(tot / (float)n + eps);
}

// Timestamp k of this workgroup (the 100 MHz wall clock), when stamps are requested: kernel 1 uses slots 0, 1,
// kernel 2 slots 2..4 and 7, kernel 3 slots 5, 6 of row blockIdx.x of a [max grid][8] table
__device__ __forceinline__ void stamp(const FArgs& a, int k) {
    if (a.stamps && threadIdx.x == 0) a.stamps[blockIdx.x * 8 + k] = wall_clock64();
}

// Host side, fused_decode.hip: whether the fused kernels take this layer (type, shapes, every expert matrix
// registered) with the planes and row bytes filled in; the scratch bytes of T tokens and its carve-up; the lane
// shapes (gate / up K = E: lanes li, units ni; down K = FE: lo, no)
bool moe_fused_prepare(const moe_layer_desc* d, FArgs& a);
size_t moe_fused_scratch_bytes(const moe_layer_desc* d, int T);
char* moe_fused_carve(FArgs& a, void* scratch);
// Q4_K's pieces, from the common part's end (qx: x's Q8_K bundle, when wanted)
void moe_fused_carve_q4k(FArgs& a, char* p, qmatvec_q8* qa, qmatvec_q8* qx = nullptr);
hipError_t moe_fused_launch_down(int type, const FArgs& a, hipStream_t st);  // kernel 3 for a.T tokens
// Q4_K kernel 3 for a.T tokens from the fp32 gate / up: SwiGLU and the Q8_K input formed inside when FE allows,
// else the SwiGLU kernel (into qa) and then kernel 3
hipError_t moe_fused_launch_down_q8k(const FArgs& a, const qmatvec_q8* qa, hipStream_t st);
void moe_mv_shape(int type, int K, int* lanes, int* units_per_lane);
unsigned long long* moe_fused_stamps_ptr();  // the table moe_layer_fused_stamps set, or nullptr

// Row dots of R rows per lane group of L lanes, each with its own weight row and input row (split-plane weights):
// all loads first, then the units in ascending order per row (rows_dot's order), then the group sums. Only rows
// r < nvalid are loaded; the others' results are undefined.
template <int TYPE, int L, int R, int NUPL>
__device__ __forceinline__ void rows_dot_multi(const uint8_t* const vr[R], const uint8_t* const sr[R],
                                               const int8_t* const xq[R], const float* const xd[R],
                                               const int* const xbs[R], int nu, int gl, int nvalid, float acc[R]) {
    WUnit<TYPE> w[R][NUPL];
    XUnit<TYPE> x[R][NUPL];
#pragma unroll
    for (int r = 0; r < R; ++r)
        if (r < nvalid)
#pragma unroll
            for (int i = 0; i < NUPL; ++i) load_packed<TYPE>(vr[r], sr[r], gl + i * L, nu, w[r][i]);
#pragma unroll
    for (int r = 0; r < R; ++r)
        if (r < nvalid)
#pragma unroll
            for (int i = 0; i < NUPL; ++i) load_x<TYPE>(xq[r], xd[r], xbs[r], gl + i * L, x[r][i]);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        acc[r] = 0.0f;
#pragma unroll
        for (int i = 0; i < NUPL; ++i) acc[r] += term<TYPE>(w[r][i], x[r][i], gl + i * L);
        acc[r] = group_sum<L>(acc[r]);
    }
}

// Q8_0 of one row of E values by a 256-thread workgroup, 8 values per thread (4 threads per block of 32): the
// activation quantizer's expressions (amax, id = 127 / amax, rint, d = F16(amax / 127))
__device__ __forceinline__ void quantize_row_q8_0(const float* x, int E, int8_t* xq, float* xd) {
    const int tid = threadIdx.x;
    for (int base = 0; base < E; base += 2048) {
        const int i0 = base + 8 * tid;
        float v[8];
        if (i0 + 8 <= E && ((uintptr_t)(x + i0) & 15) == 0) {  // two 16-byte loads
            const float4 p = ((const float4*)(x + i0))[0], q = ((const float4*)(x + i0))[1];
            v[0] = p.x, v[1] = p.y, v[2] = p.z, v[3] = p.w, v[4] = q.x, v[5] = q.y, v[6] = q.z, v[7] = q.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = i0 + j < E ? x[i0 + j] : 0.0f;
        }
        float am = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) am = fmaxf(am, fabsf(v[j]));
        am = group_max<4>(am);
        const float id = am != 0.0f ? 127.0f / am : 0.0f;
        if (i0 < E) {
            int q[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) q[j] = (int)rintf(v[j] * id);
            *(uint2*)(xq + i0) = make_uint2((q[0] & 0xff) | ((q[1] & 0xff) << 8) | ((q[2] & 0xff) << 16) |
                                                ((uint32_t)q[3] << 24),
                                            (q[4] & 0xff) | ((q[5] & 0xff) << 8) | ((q[6] & 0xff) << 16) |
                                                ((uint32_t)q[7] << 24));
            if ((tid & 3) == 0) xd[i0 / 32] = __half2float(__float2half(am / 127.0f));
        }
    }
}

// The same Q8_0 blocks from values in rms_first_pass4's layout (thread t's float4 k: values 4 (t + 256 k) ..): a
// block of 32 is eight lanes; the same expressions as quantize_row_q8_0, so the same bits. E % 32 == 0.
__device__ __forceinline__ void quantize_row4_q8_0(const float4 (&y4)[4], int E, int8_t* xq, float* xd) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int c = tid + 256 * k;  // this thread's 16-byte piece
        if (256 * k >= E / 4) break;  // (uniform)
        const bool in = c < E / 4;
        const float4 v = in ? y4[k] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        float am = fmaxf(fmaxf(fmaxf(fmaxf(0.0f, fabsf(v.x)), fabsf(v.y)), fabsf(v.z)), fabsf(v.w));
        am = group_max<8>(am);
        const float id = am != 0.0f ? 127.0f / am : 0.0f;
        if (in) {
            const int q0 = (int)rintf(v.x * id), q1 = (int)rintf(v.y * id), q2 = (int)rintf(v.z * id),
                      q3 = (int)rintf(v.w * id);
            *(uint32_t*)(xq + 4 * c) = (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | ((uint32_t)q3 << 24);
            if ((tid & 7) == 0) xd[c / 8] = __half2float(__float2half(am / 127.0f));
        }
    }
}

// One wave: SwiGLU of 32 gate / up values (the swiglu kernel's expression) and their Q8_0 block; lanes 0..31 write
// the 32 codes to q[0..32), lane 0 the scale to *d
__device__ __forceinline__ void swiglu_q8_block(const float* g32, const float* u32, int8_t* q, float* d) {
    const int lane = threadIdx.x & 63, t = lane & 31;
    const float g = g32[t], uu = u32[t];
    const float act = g / (1.0f + __expf(-g)) * uu;
    const float am = group_max<32>(fabsf(act));
    const float id = am != 0.0f ? 127.0f / am : 0.0f;
    if (lane < 32) {
        q[t] = (int8_t)(int)rintf(act * id);
        if (t == 0) *d = __half2float(__float2half(am / 127.0f));
    }
}

#endif  // FUSED_COMMON_H
