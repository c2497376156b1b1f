// fused_multi.hip -- 2..7 tokens of one MoE FFN layer (speculative verify, small batches) in three kernels, each
// distinct expert's rows read once for every token that chose it (gfx950, wave64).
//
// The per-operation path at these T reads each token's experts per token (the per-token launches of the
// reference's moe_core for T < 8, src/qwen_model.cpp:904-937). Here:
//   1  one workgroup per router-logit row (every token's dot with it), one per token quantizing x, one per token
//      for the shared-expert gate;
//   2  a persistent workgroup per CU: it routes all T tokens (wave t routes token t, the router's own code) and
//      forms the union of the chosen experts in ascending expert order (then the shared expert) once, then takes
//      units (union slot, 32-row block of FE) two at a time: the slot expert's 32 gate and 32 up rows against
//      each token that chose it, then each such token's SwiGLU and Q8_0 block of down's input; workgroup 0
//      publishes the routing;
//   3  one workgroup per 64 / L output rows (L: the down row dot's lanes): the (token, slot) pairs' down rows,
//      then the combine per token in slot order.
// Each row dot has the per-operation kernel's lane shape and order for its K, the router, quantizer, SwiGLU and
// combine are the per-operation expressions, so the layer equals the per-operation path bit for bit.

#include "fused_common.h"
#include "host_common.h"
#include "qmatvec.h"

#define FM_MAX_U 65  // union slots: at most FD_MAX_T * NU (<= 64) experts and the shared one

#ifndef FM_HALVES
#define FM_HALVES 1  // units per round of the persistent gate / up kernel (2: halves of 8 waves, 8 rows each)
#endif

// ---- kernel 1: logits (workgroups 0 .. NE - 1), x quantized (NE .. NE + T - 1), shared gates (then T more)
__global__ void __launch_bounds__(256) k_fm_logits(FArgs a) {
    __shared__ float part[4];
    const int b = blockIdx.x, tid = threadIdx.x, E = a.E, T = a.T;
    stamp(a, 0);
    if (b < a.NE) {  // the per-token F32 matvec's sums, one token after the other
        for (int t = 0; t < T; ++t) {
            const float y = f32_row_dot(a.w_router + (size_t)b * E, a.x + (size_t)t * E, E, part);
            if (tid == 0) a.logits[(size_t)t * a.NE + b] = y;
        }
    } else if (b < a.NE + T) {
        const int t = b - a.NE;
        quantize_row_q8_0(a.x + (size_t)t * E, E, a.xq + (size_t)t * E, a.xd + (size_t)t * (E / 32));
    } else {
        const int t = b - a.NE - T;
        const float g = shexp_gate(a.x + (size_t)t * E, a.w_shexp, E, part);
        if (tid == 0) a.sg[t] = g;
    }
    stamp(a, 1);
}

// The union of the routed experts (set bits of an NE-bit map, ascending) and the shared expert (-1) after them:
// slot u's expert, or -2 past the end. One thread.
__device__ __forceinline__ int union_expert(const uint32_t* bits, int ne, int u, bool shared) {
    int count = 0;
    for (int wd = 0; wd < (ne + 31) / 32; ++wd) {
        const uint32_t m = bits[wd];
        const int c = __popc(m);
        if (u < count + c) {
            uint32_t mm = m;
            for (int k = 0; k < u - count; ++k) mm &= mm - 1;  // drop the lower set bits
            return 32 * wd + __ffs(mm) - 1;
        }
        count += c;
    }
    return shared && u == count ? -1 : -2;
}

// Token t's slot holding expert e (e = -1: the shared slot NU), -1 if t did not choose e
__device__ __forceinline__ int slot_of(const int* ids_t, int nu, int e) {
    if (e == -1) return nu;
    for (int j = 0; j < nu; ++j)
        if (ids_t[j] == e) return j;
    return -1;
}

// ---- kernel 2 (persistent: a workgroup per CU): routing of every token and the union, once per workgroup; then
// units (union slot, 32-row block of FE) two at a time (one per half of the workgroup: 4 waves of 8 gate rows, 4 of
// 8 up rows; one at a time over 16 waves of 4 rows when a lane holds two units of a row), the unit's weights
// loaded once and dotted with every token that chose the slot's expert, then those tokens' SwiGLU and Q8_0 blocks
// of down's input
template <int TYPE, int NUPL_IN>
__global__ void __launch_bounds__(1024) k_fm_gate_up(FArgs a) {
    // NUPL_IN == 1: two units at a time (halves of 8 waves, 8 rows per wave); 2: one unit (16 waves, 4 rows)
    constexpr int HALVES = FM_HALVES, WPU = 16 / HALVES, RW = 64 / WPU, WPM = 32 / RW, TB = NUPL_IN == 1 ? 2 : 1;
    __shared__ int s_ids[FD_MAX_T][64];
    __shared__ float s_wts[FD_MAX_T][64];
    __shared__ uint32_t bits[ROUTER_MAX_E / 32];
    __shared__ int ulist[FM_MAX_U], s_nu;
    __shared__ int s_slot[2][FD_MAX_T];
    __shared__ float gu[2][2][FD_MAX_T][32];  // [half][gate / up][token][row]
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int h = w / WPU, hw = w - h * WPU;  // unit of the round, wave within it
    const int T = a.T, FE = a.FE, NU = a.NU, NE = a.NE, nbf = FE / 32, nu_in = fmt_units(TYPE, a.E);
    stamp(a, 2);
    for (int i = tid; i < (NE + 31) / 32; i += 1024) bits[i] = 0u;
    const float* lg = a.logits_in ? a.logits_in : a.logits;
    if (w < T) router_select_one_wave(lg + (size_t)w * NE, NE, NU, s_ids[w], s_wts[w]);
    __syncthreads();
    if (tid < T * NU) {
        const int t = tid / NU, j = tid - t * NU;
        const int e = s_ids[t][j];
        atomicOr(&bits[e >> 5], 1u << (e & 31));
        if (blockIdx.x == 0) {  // the routing for kernel 3 and the caller
            a.ids[tid] = e;
            a.wts[tid] = s_wts[t][j];
            if (a.ids_out) a.ids_out[tid] = e;
            if (a.wts_out) a.wts_out[tid] = s_wts[t][j];
        }
    }
    __syncthreads();
    if (tid == 0) {  // the union: routed experts ascending, then the shared one
        int n = 0;
        for (int wd = 0; wd < (NE + 31) / 32; ++wd)
            for (uint32_t m = bits[wd]; m; m &= m - 1) ulist[n++] = 32 * wd + __ffs(m) - 1;
        if (a.NS > NU) ulist[n++] = -1;
        s_nu = n;
    }
    __syncthreads();
    stamp(a, 3);
    const int units = s_nu * nbf, step = HALVES * gridDim.x;
    const int mat = hw / WPM;
    // this wave's weight units of unit k (RW rows of gate or up): issued a round ahead of their use
    auto load_w = [&](int k, WUnit<TYPE> (&wu)[NUPL_IN][RW]) {
        const int u = k / nbf, b = k - u * nbf, e = ulist[u];
        const int mi = e >= 0 ? mat : 3 + mat;
        const long long rbase = (e >= 0 ? (long long)e * FE : 0) + 32 * b + RW * (hw % WPM);
        const uint8_t* vb = a.v[mi] + rbase * a.vrb_in;
        const uint8_t* sb = a.s[mi] + rbase * a.srb_in;
#pragma unroll
        for (int i = 0; i < NUPL_IN; ++i)
#pragma unroll
            for (int r = 0; r < RW; ++r)
                load_unit<TYPE, true>(vb + (long long)r * a.vrb_in, sb + (long long)r * a.srb_in, lane + i * 64,
                                      nu_in, wu[i][r]);
    };
    WUnit<TYPE> wu[NUPL_IN][RW];
    if (HALVES * blockIdx.x + h < units) load_w(HALVES * blockIdx.x + h, wu);
    for (int k0 = HALVES * blockIdx.x; k0 < units; k0 += step) {  // (uniform over the workgroup)
        const int unit = k0 + h;
        const bool live = unit < units;  // (uniform per half)
        const int u = live ? unit / nbf : 0, b = live ? unit - u * nbf : 0;
        const int e = live ? ulist[u] : -2;
        __syncthreads();  // the previous round's gu / s_slot are consumed
        if (tid - h * 64 * WPU < T) s_slot[h][tid - h * 64 * WPU] = live ? slot_of(s_ids[tid - h * 64 * WPU], NU, e) : -1;
        __syncthreads();
        if (live) {
            for (int t0 = 0; t0 < T; t0 += TB) {
                XUnit<TYPE> x[TB][NUPL_IN];
#pragma unroll
                for (int q = 0; q < TB; ++q) {  // the batch's participating tokens' x, issued together
                    const int t = t0 + q;
                    if (t < T && s_slot[h][t] >= 0)
#pragma unroll
                        for (int i = 0; i < NUPL_IN; ++i)
                            load_x<TYPE>(a.xq + (size_t)t * a.E, a.xd + (size_t)t * (a.E / 32), nullptr,
                                         lane + i * 64, x[q][i]);
                }
#pragma unroll
                for (int q = 0; q < TB; ++q) {
                    const int t = t0 + q;
                    if (t >= T || s_slot[h][t] < 0) continue;  // (uniform)
                    float acc[RW];
#pragma unroll
                    for (int r = 0; r < RW; ++r) {
                        acc[r] = 0.0f;
#pragma unroll
                        for (int i = 0; i < NUPL_IN; ++i) acc[r] += term<TYPE>(wu[i][r], x[q][i], lane + i * 64);
                        acc[r] = group_sum<64>(acc[r]);
                    }
                    if (lane == 0)
#pragma unroll
                        for (int r = 0; r < RW; ++r) gu[h][mat][t][RW * (hw % WPM) + r] = acc[r];
                }
            }
        }
        if (unit + step < units) load_w(unit + step, wu);  // the next round's weights, in flight from here on
        __syncthreads();
        stamp(a, 7);
        if (live && hw < T && s_slot[h][hw] >= 0) {  // token hw's SwiGLU and Q8_0 block for its slot of e
            const long long sl = (long long)hw * a.NS + s_slot[h][hw];
            swiglu_q8_block(gu[h][0][hw], gu[h][1][hw], a.act_q + sl * FE + 32 * b, a.act_d + sl * nbf + b);
        }
    }
    stamp(a, 4);
}

// ---- kernel 3: down rows i0 .. i0 + RB - 1 for every (token, slot) pair -- the items, a flat list, taken by the
// waves IB at a time with all their loads issued together -- then the combine per token in slot order (the
// combine kernel's expression)
template <int TYPE, int L_OUT, int NUPL_OUT>
__global__ void __launch_bounds__(1024) k_fm_down(FArgs a) {
    constexpr int RB = 64 / L_OUT, IB = NUPL_OUT == 1 ? 4 : 2;
    __shared__ int s_e[FD_MAX_T * 17];
    __shared__ float s_wts[FD_MAX_T][64];
    __shared__ float downv[FD_MAX_T][17][RB];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int T = a.T, E = a.E, FE = a.FE, NU = a.NU, NS = a.NS;
    const int gl = lane & (L_OUT - 1), i = lane / L_OUT, i0 = blockIdx.x * RB, nu_out = fmt_units(TYPE, FE);
    stamp(a, 5);
    const int nitems = T * NS;
    if (tid < nitems) {  // item tid: token tid / NS, slot tid % NS (slot NU: the shared expert)
        const int t = tid / NS, j = tid - t * NS;
        s_e[tid] = j < NU ? a.ids[t * NU + j] : -1;
        if (j < NU) s_wts[t][j] = a.wts[t * NU + j];
    }
    __syncthreads();
    for (int k0 = w * IB; k0 < nitems; k0 += 16 * IB) {  // (uniform per wave)
        WUnit<TYPE> wu[IB][NUPL_OUT];
        XUnit<TYPE> x[IB][NUPL_OUT];
#pragma unroll
        for (int q = 0; q < IB; ++q) {
            const int k = k0 + q;
            if (k < nitems) {
                const int e = s_e[k];
                const long long row = e >= 0 ? (long long)e * E + i0 + i : i0 + i;
                const int mi = e >= 0 ? 2 : 5;
                const uint8_t* vr = a.v[mi] + row * a.vrb_out;
                const uint8_t* sr = a.s[mi] + row * a.srb_out;
#pragma unroll
                for (int c = 0; c < NUPL_OUT; ++c) load_packed<TYPE>(vr, sr, gl + c * L_OUT, nu_out, wu[q][c]);
#pragma unroll
                for (int c = 0; c < NUPL_OUT; ++c)
                    load_x<TYPE>(a.act_q + (long long)k * FE, a.act_d + (long long)k * (FE / 32), nullptr,
                                 gl + c * L_OUT, x[q][c]);
            }
        }
#pragma unroll
        for (int q = 0; q < IB; ++q) {
            const int k = k0 + q;
            if (k >= nitems) continue;  // (uniform)
            float acc = 0.0f;
#pragma unroll
            for (int c = 0; c < NUPL_OUT; ++c) acc += term<TYPE>(wu[q][c], x[q][c], gl + c * L_OUT);
            acc = group_sum<L_OUT>(acc);
            const int t = k / NS;
            if (gl == 0) downv[t][k - t * NS][i] = acc;
        }
    }
    __syncthreads();
    if (tid < T * RB) {
        const int t = tid / RB, r = tid - t * RB;
        float o = s_wts[t][0] * downv[t][0][r];
        for (int j = 1; j < NU; ++j) o += s_wts[t][j] * downv[t][j][r];
        if (NS > NU) o += a.has_gate ? downv[t][NU][r] * a.sg[t] : downv[t][NU][r];
        a.out[(size_t)t * E + i0 + r] = o;
    }
    stamp(a, 6);
}

// ------------------------------------------------------------------ host side

namespace {

template <int TYPE, int NI, int LO, int NO>
hipError_t launch_multi(const FArgs& a, int kernels, hipStream_t st) {
    const int nsu = (a.T * a.NU < a.NE ? a.T * a.NU : a.NE) + (a.NS > a.NU ? 1 : 0);  // union slots, at most
    const int per = FM_HALVES;                                                        // units per round
    const int pairs = (nsu * (a.FE / 32) + per - 1) / per, cus = moe_device_cus();
    hipError_t e = hipSuccess;
    if (kernels & 1) e = launch_kernel(k_fm_logits, dim3(a.NE + a.T * (1 + a.has_gate)), dim3(256), 0, st, a);
    if (e == hipSuccess && (kernels & 2))
        e = launch_kernel(k_fm_gate_up<TYPE, NI>, dim3(pairs < cus ? pairs : cus), dim3(1024), 0, st, a);
    if (e == hipSuccess && (kernels & 4))
        e = launch_kernel(k_fm_down<TYPE, LO, NO>, dim3(a.E / (64 / LO)), dim3(1024), 0, st, a);
    return e;
}

template <int TYPE>
hipError_t launch_multi_t(const FArgs& a, int ni, int lo, int no, int kernels, hipStream_t st) {
#define FM_CASE(I, L, O) \
    if (ni == I && lo == L && no == O) return launch_multi<TYPE, I, L, O>(a, kernels, st);
    FM_CASE(1, 16, 1) FM_CASE(1, 8, 3) FM_CASE(1, 32, 1) FM_CASE(1, 16, 3) FM_CASE(1, 64, 1)
    FM_CASE(2, 16, 1) FM_CASE(2, 8, 3) FM_CASE(2, 32, 1) FM_CASE(2, 16, 3) FM_CASE(2, 64, 1)
#undef FM_CASE
    return hipErrorInvalidDeviceFunction;
}

}  // namespace

// T = 2..FD_MAX_T tokens through the multi-token kernels, when moe_fused_prepare takes the layer
bool moe_fused_multi_try(const moe_layer_desc* d, const float* x, const float* logits, int T, float* out,
                         int* ids_out, float* wts_out, void* scratch, int kernels, hipStream_t st, hipError_t* err) {
    if (T < 2 || T > FD_MAX_T || d->type == QT_Q4_K) return false;  // (Q4_K: the per-operation path)
    FArgs a = {};
    if (!moe_fused_prepare(d, a)) return false;
    if (a.NS > 17 || T * a.NU > 64) return false;  // (the union and the per-token slot tables' sizes)
    a.T = T;
    a.x = x;
    a.logits_in = logits;
    a.out = out;
    a.ids_out = ids_out;
    a.wts_out = wts_out;
    a.stamps = moe_fused_stamps_ptr();
    moe_fused_carve(a, scratch);
    int li, ni, lo, no;
    moe_mv_shape(d->type, a.E, &li, &ni);
    moe_mv_shape(d->type, a.FE, &lo, &no);
    switch (d->type) {
    case QT_Q8_0: *err = launch_multi_t<QT_Q8_0>(a, ni, lo, no, kernels, st); break;
    case QT_ROCMFP4: *err = launch_multi_t<QT_ROCMFP4>(a, ni, lo, no, kernels, st); break;
    default: *err = launch_multi_t<QT_ROCMFP4_FAST>(a, ni, lo, no, kernels, st); break;
    }
    return true;
}
