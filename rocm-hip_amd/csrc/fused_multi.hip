// fused_multi.hip -- 2..7 tokens of one MoE FFN layer (speculative verify, small batches) in three kernels, each
// distinct expert's rows read once for every token that chose it (gfx950, wave64).
//
// The per-operation path at these T reads each token's experts per token (the per-token launches of the
// reference's moe_core for T < 8, src/qwen_model.cpp:904-937). Here:
//   1  one workgroup per router-logit row (every token's dot with it), one per token quantizing x, one per token
//      for the shared-expert gate;
//   2  gate / up / SwiGLU over units (union slot, 32-row block of FE), the union being the chosen experts in
//      ascending order (then the shared expert): each unit's rows are dotted with every token that chose the
//      slot's expert, then each such token's SwiGLU and Q8_0 block of down's input. Two forms: a workgroup per
//      unit (every workgroup routes all T tokens, one wave each, and forms the union itself) when the grid fits
//      one round of resident workgroups; otherwise a persistent workgroup per CU that routes once and takes
//      units round after round;
//   3  down + combine: per token (the T = 1 kernel, one wave per slot, over T rows of workgroups), or the
//      item-list form (one workgroup per 64 / L output rows takes every (token, slot) pair, then combines per
//      token in slot order).
// Each row dot has the per-operation kernel's lane shape and order for its K, the router, quantizer, SwiGLU and
// combine are the per-operation expressions, so the layer equals the per-operation path bit for bit.

#include <atomic>

#include "fused_common.h"
#include "gpu_ops.h"
#include "host_common.h"
#include "qmatvec.h"

#define FM_MAX_U 65  // union slots: at most FD_MAX_T * NU (<= 64) experts and the shared one

#ifndef FM_HALVES
#define FM_HALVES 1  // units per round of the persistent gate / up kernel (2: halves of 8 waves, 8 rows each)
#endif

// ---- kernel 1: logits (workgroups 0 .. NE - 1), x quantized (the next nq: one per token, Q4_K one per token and
// 256-value block, the activation quantizer itself), shared gates (then T more)
__global__ void __launch_bounds__(256) k_fm_logits(FArgs a) {
    __shared__ float part[4];
    const int b = blockIdx.x, tid = threadIdx.x, E = a.E, T = a.T;
    const int nq = a.xo.qK ? T * (E / 256) : T;
    stamp(a, 0);
    if (b < a.NE) {  // the per-token F32 matvec's sums, every token in one pass over the router row
        __shared__ float tpart[FD_MAX_T][4];
        float y[FD_MAX_T];
        const float* wr = a.w_router + (size_t)b * E;
        if (T <= 2)  // (uniform: as many token registers as the batch needs)
            f32_row_dot_multi<2>(wr, a.x, E, T, E, tpart, y);
        else if (T <= 4)
            f32_row_dot_multi<4>(wr, a.x, E, T, E, tpart, y);
        else
            f32_row_dot_multi<FD_MAX_T>(wr, a.x, E, T, E, tpart, y);
        if (tid == 0)
#pragma unroll
            for (int t = 0; t < FD_MAX_T; ++t)
                if (t < T) a.logits[(size_t)t * a.NE + b] = y[t];
    } else if (b < a.NE + nq) {
        if (a.xo.qK) {  // block blk of the [T][E] bundle: token blk / (E / 256)
            __shared__ Q8Smem sh;
            const int blk = b - a.NE;
            q8_quantize_256(a.x[(size_t)blk * 256 + tid], true, blk, tid, sh, a.xo);
        } else {
            const int t = b - a.NE;
            quantize_row_q8_0(a.x + (size_t)t * E, E, a.xq + (size_t)t * E, a.xd + (size_t)t * (E / 32));
        }
    } else {
        const int t = b - a.NE - nq;
        const float g = shexp_gate(a.x + (size_t)t * E, a.w_shexp, E, part);
        if (tid == 0) a.sg[t] = g;
    }
    stamp(a, 1);
}

// Token t's slot holding expert e (e = -1: the shared slot NU), -1 if t did not choose e
__device__ __forceinline__ int slot_of(const int* ids_t, int nu, int e) {
    if (e == -1) return nu;
    for (int j = 0; j < nu; ++j)
        if (ids_t[j] == e) return j;
    return -1;
}

// The union of the T tokens' chosen experts (ids[t][0..nu), row stride 64), ascending, then the shared expert (-1)
// when there is one: ulist[0..n), *count = n. One wave, in LDS byte flags (flag[ne], 4-byte aligned): the flags
// cleared, every id's flag set (lanes 0 .. T nu - 1, one id each; a wave's LDS operations complete in order), then
// lane l reads the flags of experts l, l + 64, ... and a ballot gives each chosen expert its place among the
// chosen below it. (LDS atomics from T nu threads onto a bit map and one thread walking it took ~1.3 µs at T = 4;
// a loop testing every id lane by lane, ~1.5 µs of dependent scalar steps.)
__device__ __forceinline__ void form_union(const int (*ids)[64], int T, int nu, int ne, bool shared, uint8_t* flag,
                                           int* ulist, int* count) {
    const int lane = threadIdx.x & 63, tn = T * nu;
    for (int i = lane; i < (ne + 3) / 4; i += 64) ((uint32_t*)flag)[i] = 0u;
    if (lane < tn) flag[ids[lane / nu][lane % nu]] = 1;
    int n = 0;
    for (int e0 = 0; e0 < ne; e0 += 64) {  // (uniform)
        const int e = e0 + lane;
        const bool hit = e < ne && flag[e] != 0;
        const uint64_t m = __ballot(hit);
        if (hit) ulist[n + __popcll(m & ((1ull << lane) - 1))] = e;
        n += __popcll(m);
    }
    if (lane == 0) {
        if (shared) ulist[n] = -1;
        *count = n + (shared ? 1 : 0);
    }
}

// ---- kernel 2 (persistent: a workgroup per CU): routing of every token and the union, once per workgroup; then
// units (union slot, 32-row block of FE) two at a time (one per half of the workgroup: 4 waves of 8 gate rows, 4 of
// 8 up rows; one at a time over 16 waves of 4 rows when a lane holds two units of a row), the unit's weights
// loaded once and dotted with every token that chose the slot's expert, then those tokens' SwiGLU and Q8_0 blocks
// of down's input. A row is one group of L_IN lanes with NUPL_IN units per lane (the per-operation shape for
// K = E), so a wave holds 64 / L_IN groups of RW L_IN / 64 rows. Q4_K writes gate / up in fp32 instead (its down
// input is Q8_K, one scale per 256 values: the SwiGLU kernel between kernels 2 and 3 quantizes it).
template <int TYPE, int L_IN, int NUPL_IN>
__global__ void __launch_bounds__(1024) k_fm_gate_up(FArgs a) {
    // NUPL_IN == 1: two units at a time (halves of 8 waves, 8 rows per wave); 2: one unit (16 waves, 4 rows)
    constexpr int HALVES = FM_HALVES, WPU = 16 / HALVES, RW = 64 / WPU, WPM = 32 / RW;
    constexpr int G = 64 / L_IN, R = RW / G;  // lane groups per wave, rows per group
    static_assert(R >= 1, "a wave's rows must cover its lane groups");
    constexpr bool Q8K = Fmt<TYPE>::Q8K;
    __shared__ int s_ids[FD_MAX_T][64];
    __shared__ float s_wts[FD_MAX_T][64];
    __shared__ int ulist[FM_MAX_U], s_nu;
    __shared__ __align__(4) uint8_t s_flag[ROUTER_MAX_E];
    __shared__ int s_slot[2][FD_MAX_T];
    __shared__ float gu[2][2][FD_MAX_T][32];  // [half][gate / up][token][row]
    // every token's quantized x, staged once: Q8_0 values [T][E] and scales [T][E / 32], or Q8_K values, scales
    // [T][E / 256] and sums of 16 [T][E / 16]
    __shared__ __align__(16) int8_t s_xq[FD_MAX_T * FD_MAX_E];
    __shared__ float s_xd[FD_MAX_T * FD_MAX_E / 32];
    __shared__ __align__(16) int s_xbs[Q8K ? FD_MAX_T * FD_MAX_E / 16 : 4];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, gl = lane & (L_IN - 1), grp = lane / L_IN;
    const int h = w / WPU, hw = w - h * WPU;  // unit of the round, wave within it
    const int T = a.T, FE = a.FE, NU = a.NU, NE = a.NE, nbf = FE / 32, nu_in = fmt_units(TYPE, a.E);
    stamp(a, 2);
    const float* lg = a.logits_in ? a.logits_in : a.logits;
    if (w < T) {
        router_select_one_wave(lg + (size_t)w * NE, NE, NU, s_ids[w], s_wts[w]);
    } else {  // the other waves stage x meanwhile
        const int i0 = tid - 64 * T, n = 1024 - 64 * T, TE = T * a.E;
        const int8_t* gq = Q8K ? a.xo.qK : a.xq;
        const float* gd = Q8K ? a.xo.dK : a.xd;
        for (int i = i0; i < TE / 16; i += n) ((uint4*)s_xq)[i] = ((const uint4*)gq)[i];
        for (int i = i0; i < TE / (Q8K ? 256 : 32); i += n) s_xd[i] = gd[i];
        if constexpr (Q8K)
            for (int i = i0; i < TE / 64; i += n) ((int4*)s_xbs)[i] = ((const int4*)a.xo.bsK)[i];
    }
    __syncthreads();
    if (blockIdx.x == 0 && tid < T * NU) {  // the routing for kernel 3 and the caller
        const int t = tid / NU, j = tid - t * NU;
        a.ids[tid] = s_ids[t][j];
        a.wts[tid] = s_wts[t][j];
        if (a.ids_out) a.ids_out[tid] = s_ids[t][j];
        if (a.wts_out) a.wts_out[tid] = s_wts[t][j];
    }
    if (w == 0) form_union(s_ids, T, NU, NE, a.NS > NU, s_flag, ulist, &s_nu);  // routed ascending, then the shared one
    __syncthreads();
    stamp(a, 3);
    const int units = s_nu * nbf, step = HALVES * gridDim.x;
    const int mat = hw / WPM, r0 = RW * (hw % WPM) + grp * R;  // gate or up; this group's first row of the unit's 32
    // this group's weight units of unit k (R rows of gate or up): issued a round ahead of their use
    auto load_w = [&](int k, WUnit<TYPE> (&wu)[NUPL_IN][R]) {
        const int u = k / nbf, b = k - u * nbf, e = ulist[u];
        const int mi = e >= 0 ? mat : 3 + mat;
        const long long rbase = (e >= 0 ? (long long)e * FE : 0) + 32 * b + r0;
        const uint8_t* vb = pick_opaque(a.v, mi) + rbase * a.vrb_in;
        const uint8_t* sb = pick_opaque(a.s, mi) + rbase * a.srb_in;
#pragma unroll
        for (int i = 0; i < NUPL_IN; ++i)
#pragma unroll
            for (int r = 0; r < R; ++r)
                load_unit<TYPE, true>(vb + (long long)r * a.vrb_in, sb + (long long)r * a.srb_in, gl + i * L_IN,
                                      nu_in, wu[i][r]);
    };
    // one round: unit k0 + h from the registers wu, then the next round's weights issued into them (in flight
    // during the SwiGLU and the next round's slot tables). (Two register sets in turn, the next round's loads
    // issued first, measured slower: 45.7 against 41.7 µs at config 1 T = 4.)
    WUnit<TYPE> wu[NUPL_IN][R];
    auto round = [&](int k0) {
        const int unit = k0 + h;
        const bool live = unit < units;  // (uniform per half)
        const int u = live ? unit / nbf : 0, b = live ? unit - u * nbf : 0;
        const int e = live ? ulist[u] : -2;
        __syncthreads();  // the previous round's gu / s_slot are consumed
        if (tid - h * 64 * WPU < T) s_slot[h][tid - h * 64 * WPU] = live ? slot_of(s_ids[tid - h * 64 * WPU], NU, e) : -1;
        __syncthreads();
        if (live) {
            for (int t = 0; t < T; ++t) {
                if (s_slot[h][t] < 0) continue;  // (uniform)
                XUnit<TYPE> x[NUPL_IN];
                float acc[R];
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
                for (int i = 0; i < NUPL_IN; ++i) {
                    if constexpr (Q8K)
                        load_x<TYPE>(s_xq + t * a.E, s_xd + t * (a.E / 256), s_xbs + t * (a.E / 16), gl + i * L_IN,
                                     x[i]);
                    else
                        load_x<TYPE>(s_xq + t * a.E, s_xd + t * (a.E / 32), nullptr, gl + i * L_IN, x[i]);
#pragma unroll
                    for (int r = 0; r < R; ++r) acc[r] += term<TYPE>(wu[i][r], x[i], gl + i * L_IN);
                }
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r] = group_sum<L_IN>(acc[r]);
                if (gl == 0) {
                    if constexpr (Q8K) {  // row (token t, its slot of e) of the fp32 gate / up
                        float* o = (mat ? a.u : a.g) + ((long long)t * a.NS + s_slot[h][t]) * FE + 32 * b + r0;
#pragma unroll
                        for (int r = 0; r < R; ++r) o[r] = acc[r];
                    } else {
#pragma unroll
                        for (int r = 0; r < R; ++r) gu[h][mat][t][r0 + r] = acc[r];
                    }
                }
            }
        }
        if (unit + step < units) load_w(unit + step, wu);
        __syncthreads();
        stamp(a, 7);
        if (!Q8K && live && hw < T && s_slot[h][hw] >= 0) {  // token hw's SwiGLU and Q8_0 block for its slot of e
            const long long sl = (long long)hw * a.NS + s_slot[h][hw];
            swiglu_q8_block(gu[h][0][hw], gu[h][1][hw], a.act_q + sl * FE + 32 * b, a.act_d + sl * nbf + b);
        }
    };
    if (HALVES * blockIdx.x + h < units) load_w(HALVES * blockIdx.x + h, wu);
    for (int k0 = HALVES * blockIdx.x; k0 < units; k0 += step) round(k0);  // (uniform over the workgroup)
    stamp(a, 4);
}

// ---- kernel 2, one workgroup per unit (union slot, 32-row block of FE), the grid sized for the largest union:
// every workgroup routes all T tokens (wave t routes token t) while its other waves stage every token's quantized
// x in LDS, forms the union (routed experts ascending, then the shared one) and leaves when its unit is past the
// union's end; then 8 waves of 8 rows (4 waves of gate rows, 4 of up) of the slot expert, all loaded at once and
// dotted with each token that chose the expert, then those tokens' SwiGLU and Q8_0 blocks of down's input (Q4_K:
// fp32 gate / up for the SwiGLU kernel). The workgroups of a launch load their units together, instead of a
// persistent workgroup's units one round (and one memory latency) after the other.
template <int TYPE, int L_IN, int NUPL_IN>
__global__ void __launch_bounds__(512) k_fm_gate_up_unit(FArgs a) {
    constexpr int RW = 8, WPM = 4;            // rows per wave, waves per matrix
    constexpr int G = 64 / L_IN, R = RW / G;  // lane groups per wave, rows per group
    static_assert(R >= 1, "a wave's rows must cover its lane groups");
    constexpr bool Q8K = Fmt<TYPE>::Q8K;
    __shared__ int s_ids[FD_MAX_T][64];
    __shared__ float s_wts[FD_MAX_T][64];
    __shared__ int ulist[FM_MAX_U], s_nu;
    __shared__ __align__(4) uint8_t s_flag[ROUTER_MAX_E];
    __shared__ int s_slot[FD_MAX_T];
    __shared__ float gu[2][FD_MAX_T][32];  // [gate / up][token][row]
    __shared__ __align__(16) int8_t s_xq[FD_MAX_T * FD_MAX_E];
    __shared__ float s_xd[FD_MAX_T * FD_MAX_E / 32];
    __shared__ __align__(16) int s_xbs[Q8K ? FD_MAX_T * FD_MAX_E / 16 : 4];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, gl = lane & (L_IN - 1), grp = lane / L_IN;
    const int T = a.T, FE = a.FE, NU = a.NU, NE = a.NE, nbf = FE / 32, nu_in = fmt_units(TYPE, a.E);
    stamp(a, 2);
    const float* lg = a.logits_in ? a.logits_in : a.logits;
    if (w < T) {
        router_select_one_wave(lg + (size_t)w * NE, NE, NU, s_ids[w], s_wts[w]);
    } else {  // the other waves stage x meanwhile
        const int i0 = tid - 64 * T, n = 512 - 64 * T, TE = T * a.E;
        const int8_t* gq = Q8K ? a.xo.qK : a.xq;
        const float* gd = Q8K ? a.xo.dK : a.xd;
        for (int i = i0; i < TE / 16; i += n) ((uint4*)s_xq)[i] = ((const uint4*)gq)[i];
        for (int i = i0; i < TE / (Q8K ? 256 : 32); i += n) s_xd[i] = gd[i];
        if constexpr (Q8K)
            for (int i = i0; i < TE / 64; i += n) ((int4*)s_xbs)[i] = ((const int4*)a.xo.bsK)[i];
    }
    __syncthreads();
    if (blockIdx.x == 0 && tid < T * NU) {  // the routing for kernel 3 and the caller
        const int t = tid / NU, j = tid - t * NU;
        a.ids[tid] = s_ids[t][j];
        a.wts[tid] = s_wts[t][j];
        if (a.ids_out) a.ids_out[tid] = s_ids[t][j];
        if (a.wts_out) a.wts_out[tid] = s_wts[t][j];
    }
    if (w == 0) form_union(s_ids, T, NU, NE, a.NS > NU, s_flag, ulist, &s_nu);  // routed ascending, then the shared one
    __syncthreads();
    stamp(a, 3);
    const int u = blockIdx.x / nbf, b = blockIdx.x - u * nbf;
    if (u >= s_nu) return;  // (uniform) past the union's end
    const int e = wave_uniform(ulist[u]);
    const int mat = wave_uniform(w / WPM), r0 = RW * (w % WPM) + grp * R;  // gate or up; this group's first row
    {
        const int mi = e >= 0 ? mat : 3 + mat;
        const long long rbase = (e >= 0 ? (long long)e * FE : 0) + 32 * b + r0;
        const uint8_t* vb = pick(a.v, mi) + rbase * a.vrb_in;
        const uint8_t* sb = pick(a.s, mi) + rbase * a.srb_in;
        WUnit<TYPE> wu[NUPL_IN][R];
#pragma unroll
        for (int i = 0; i < NUPL_IN; ++i)
#pragma unroll
            for (int r = 0; r < R; ++r)
                load_unit<TYPE, true>(vb + (long long)r * a.vrb_in, sb + (long long)r * a.srb_in, gl + i * L_IN,
                                      nu_in, wu[i][r]);
        if (tid < T) s_slot[tid] = slot_of(s_ids[tid], NU, e);
        __syncthreads();
        for (int t = 0; t < T; ++t) {
            if (s_slot[t] < 0) continue;  // (uniform)
            XUnit<TYPE> x[NUPL_IN];
#pragma unroll
            for (int i = 0; i < NUPL_IN; ++i) {
                if constexpr (Q8K)
                    load_x<TYPE>(s_xq + t * a.E, s_xd + t * (a.E / 256), s_xbs + t * (a.E / 16), gl + i * L_IN, x[i]);
                else
                    load_x<TYPE>(s_xq + t * a.E, s_xd + t * (a.E / 32), nullptr, gl + i * L_IN, x[i]);
            }
            float acc[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                acc[r] = 0.0f;
#pragma unroll
                for (int i = 0; i < NUPL_IN; ++i) acc[r] += term<TYPE>(wu[i][r], x[i], gl + i * L_IN);
                acc[r] = group_sum<L_IN>(acc[r]);
            }
            if (gl == 0) {
                if constexpr (Q8K) {  // row (token t, its slot of e) of the fp32 gate / up
                    float* o = (mat ? a.u : a.g) + ((long long)t * a.NS + s_slot[t]) * FE + 32 * b + r0;
#pragma unroll
                    for (int r = 0; r < R; ++r) o[r] = acc[r];
                } else {
#pragma unroll
                    for (int r = 0; r < R; ++r) gu[mat][t][r0 + r] = acc[r];
                }
            }
        }
    }
    stamp(a, 7);
    if constexpr (!Q8K) {
        __syncthreads();
        if (w < T && s_slot[w] >= 0) {  // token w's SwiGLU and Q8_0 block for its slot of e
            const long long sl = (long long)w * a.NS + s_slot[w];
            swiglu_q8_block(gu[0][w], gu[1][w], a.act_q + sl * FE + 32 * b, a.act_d + sl * nbf + b);
        }
    }
    stamp(a, 4);
}

// ---- kernel 3: down rows i0 .. i0 + RB - 1 for every (token, slot) pair -- the items, a flat list, taken by the
// waves IB at a time with all their loads issued together -- then the combine per token in slot order (the
// combine kernel's expression)
template <int TYPE, int L_OUT, int NUPL_OUT>
__global__ void __launch_bounds__(1024) k_fm_down(FArgs a) {
    constexpr int RB = 64 / L_OUT, IB = NUPL_OUT == 1 && !Fmt<TYPE>::Q8K ? 4 : 2;  // (128 VGPRs at 1024 threads)
    __shared__ int s_e[FD_MAX_T * 17];
    __shared__ float s_wts[FD_MAX_T][64];
    __shared__ float downv[FD_MAX_T][17][RB];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int T = a.T, E = a.E, FE = a.FE, NU = a.NU, NS = a.NS;
    const int gl = lane & (L_OUT - 1), i = lane / L_OUT, i0 = blockIdx.x * RB, nu_out = fmt_units(TYPE, FE);
    stamp(a, 5);
    const float sgv = a.has_gate && tid < T * RB ? a.sg[tid / RB] : 0.0f;  // (read now: kernel 1 wrote it)
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
                const uint8_t* vr = pick_opaque(a.v, mi) + row * a.vrb_out;
                const uint8_t* sr = pick_opaque(a.s, mi) + row * a.srb_out;
#pragma unroll
                for (int c = 0; c < NUPL_OUT; ++c) load_packed<TYPE>(vr, sr, gl + c * L_OUT, nu_out, wu[q][c]);
#pragma unroll
                for (int c = 0; c < NUPL_OUT; ++c) {
                    if constexpr (Fmt<TYPE>::Q8K)
                        load_x<TYPE>(a.aqk + (long long)k * FE, a.adk + (long long)k * (FE / 256),
                                     a.absk + (long long)k * (FE / 16), gl + c * L_OUT, x[q][c]);
                    else
                        load_x<TYPE>(a.act_q + (long long)k * FE, a.act_d + (long long)k * (FE / 32), nullptr,
                                     gl + c * L_OUT, x[q][c]);
                }
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
        if (NS > NU) o += a.has_gate ? downv[t][NU][r] * sgv : downv[t][NU][r];
        a.out[(size_t)t * E + i0 + r] = o;
    }
    stamp(a, 6);
}

// ------------------------------------------------------------------ host side

namespace {

template <int TYPE, int LI, int NI, int LO, int NO>
hipError_t launch_multi(const FArgs& a, const qmatvec_q8* qa, int kernels, hipStream_t st) {
    const int nsu = (a.T * a.NU < a.NE ? a.T * a.NU : a.NE) + (a.NS > a.NU ? 1 : 0);  // union slots, at most
    const int per = FM_HALVES;                                                        // units per round
    const int pairs = (nsu * (a.FE / 32) + per - 1) / per, cus = moe_device_cus();
    hipError_t e = hipSuccess;
    const int nq = Fmt<TYPE>::Q8K ? a.T * (a.E / 256) : a.T;  // quantizing workgroups of kernel 1
    if (kernels & 1) e = launch_kernel(k_fm_logits, dim3(a.NE + nq + a.T * a.has_gate), dim3(256), 0, st, a);
    // gate / up: a workgroup per unit when the grid fits two 512-thread workgroups per CU (one round: each pays its
    // own routing once), else the persistent form (routing once per CU, then rounds of units). Measured at
    // config 1 (µs per layer, persistent / per unit): T = 2 28.7 / 26.8, T = 3 39.2 / 39.7, T = 7 67.7 / 76.5.
    const int units = nsu * (a.FE / 32);
    if (e == hipSuccess && (kernels & 2)) {
        if (units <= 2 * cus)
            e = launch_kernel(k_fm_gate_up_unit<TYPE, LI, NI>, dim3(units), dim3(512), 0, st, a);
        else
            e = launch_kernel(k_fm_gate_up<TYPE, LI, NI>, dim3(pairs < cus ? pairs : cus), dim3(1024), 0, st, a);
    }
    if (Fmt<TYPE>::Q8K && e == hipSuccess && (kernels & 2))
        e = moe_swiglu_q8(a.g, a.u, nullptr, a.T * a.NS * a.FE, qa, st, 2);  // (Q4_K: Q8_K only)
    // down + combine: per token (the T = 1 kernel over T rows of workgroups, one wave per slot) for Q8_0 and up to
    // T = 3; the item-list kernel for the 4-bit types from T = 4 (its 8-row workgroups share an expert's rows among
    // the tokens that chose it: config 1 T = 4 43.6 against 44.4 µs, T = 7 65.5 against 67.7). Q8_0's units
    // need more registers than the item-list kernel's batches have at 1,024 threads (config 0 T = 2: 29 against
    // 43 µs).
    if (e == hipSuccess && (kernels & 4)) {
        if (TYPE == QT_Q8_0 || a.T <= 3)
            e = moe_fused_launch_down(TYPE, a, st);
        else
            e = launch_kernel(k_fm_down<TYPE, LO, NO>, dim3(a.E / (64 / LO)), dim3(1024), 0, st, a);
    }
    return e;
}

template <int TYPE>
hipError_t launch_multi_t(const FArgs& a, const qmatvec_q8* qa, int li, int ni, int lo, int no, int kernels,
                          hipStream_t st) {
#define FM_CASE(I, L, O) \
    if (li == 64 && ni == I && lo == L && no == O) return launch_multi<TYPE, 64, I, L, O>(a, qa, kernels, st);
    if constexpr (TYPE == QT_Q4_K) {
        if (li == 16 && ni == 3 && lo == 16 && no == 1) return launch_multi<TYPE, 16, 3, 16, 1>(a, qa, kernels, st);
    } else {
        FM_CASE(1, 16, 1) FM_CASE(1, 8, 3) FM_CASE(1, 32, 1) FM_CASE(1, 16, 3) FM_CASE(1, 64, 1)
        FM_CASE(2, 16, 1) FM_CASE(2, 8, 3) FM_CASE(2, 32, 1) FM_CASE(2, 16, 3) FM_CASE(2, 64, 1)
    }
#undef FM_CASE
    return hipErrorInvalidDeviceFunction;
}

size_t q4k_row_bytes(int k) { return (size_t)k / 256 * 144; }

// Q4_K, T = 2..7, per token: kernel 1 (logits, x's Q8_K bundle, shared gates), the router kernel (ids with stride
// NS, slot NU = -1 when there is a shared expert), the per-operation id launch of gate and up (fp32 [T][NS][FE]),
// then kernel 3 with the SwiGLU, the Q8_K input and the combine per token
hipError_t launch_q4k_by_token(const moe_layer_desc* d, FArgs& a, const qmatvec_q8* qx, const qmatvec_q8* qa,
                               int kernels, hipStream_t st) {
    hipError_t e = hipSuccess;
    const int T = a.T, nq = T * (a.E / 256);
    if (kernels & 1) e = launch_kernel(k_fm_logits, dim3(a.NE + nq + T * a.has_gate), dim3(256), 0, st, a);
    a.ids_ld = a.NS;
    if (e == hipSuccess && (kernels & 2)) {
        const float* lg = a.logits_in ? a.logits_in : a.logits;
        e = gpu_moe_router(lg, a.x, a.has_gate ? a.w_shexp : nullptr, a.ids, a.wts, a.sg, a.NE, a.NU, a.E, T, st, a.NS);
        const size_t rb = q4k_row_bytes(a.E);
        if (e == hipSuccess) {
            if (a.NS > a.NU)
                e = qmatvec_launch_q8_id_x(QT_Q4_K, d->w_gate, d->w_up, d->s_gate, d->s_up, rb, a.ids, a.NS, 0, qx,
                                           a.g, a.u, a.FE, a.E, T, st);
            else
                e = qmatvec_launch_q8_id_pair(QT_Q4_K, d->w_gate, d->w_up, rb, a.ids, a.NS, 0, qx, a.g, a.u, a.FE,
                                              a.E, T, st);
        }
    }
    if (e == hipSuccess && (kernels & 4)) e = moe_fused_launch_down_q8k(a, qa, st);
    if (e == hipSuccess && (kernels & 2) && a.ids_out)
        e = hipMemcpy2DAsync(a.ids_out, (size_t)a.NU * 4, a.ids, (size_t)a.NS * 4, (size_t)a.NU * 4, T,
                             hipMemcpyDeviceToDevice, st);
    if (e == hipSuccess && (kernels & 2) && a.wts_out)
        e = hipMemcpyAsync(a.wts_out, a.wts, (size_t)T * a.NU * 4, hipMemcpyDeviceToDevice, st);
    return e;
}

}  // namespace

static std::atomic<bool> g_fm_q4k{false};  // Q4_K through the multi-token kernels (the parity tests turn it on)
extern "C" void moe_layer_fused_multi_q4k(int on) { g_fm_q4k.store(on != 0, std::memory_order_relaxed); }

// T = 2..FD_MAX_T tokens through the multi-token kernels, when moe_fused_prepare takes the layer
bool moe_fused_multi_try(const moe_layer_desc* d, const float* x, const float* logits, int T, float* out,
                         int* ids_out, float* wts_out, void* scratch, int kernels, hipStream_t st, hipError_t* err) {
    if (T < 2 || T > FD_MAX_T) return false;
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
    char* p = moe_fused_carve(a, scratch);
    qmatvec_q8 qa = {}, qx = {};
    if (d->type == QT_Q4_K) moe_fused_carve_q4k(a, p, &qa, &qx);
    // Q4_K: with 256 experts few rows are shared between tokens and the per-operation id launches read each
    // token's rows faster than the union kernels (config-3 shape, T = 4: 55 us per layer against 65.6), so by
    // default, up to T = 4, kernel 1, the router kernel, the id launch of gate / up (the shared expert as slot NU)
    // and the Q4_K kernel 3 -- four launches for the per-operation path's seven, the same bits (config-3 shape:
    // T = 2 39.5 -> 35.7 us, T = 4 54.7 -> 53.6); from T = 5 the per-operation path (its kernel 3 forms each
    // token's SwiGLU and Q8_K input in every workgroup: T = 7 76.4 us against 74.5)
    if (d->type == QT_Q4_K && !g_fm_q4k.load(std::memory_order_relaxed)) {
        if (T > 4) return false;
        *err = launch_q4k_by_token(d, a, &qx, &qa, kernels, st);
        return true;
    }
    int li, ni, lo, no;
    moe_mv_shape(d->type, a.E, &li, &ni);
    moe_mv_shape(d->type, a.FE, &lo, &no);
    switch (d->type) {
    case QT_Q8_0: *err = launch_multi_t<QT_Q8_0>(a, &qa, li, ni, lo, no, kernels, st); break;
    case QT_ROCMFP4: *err = launch_multi_t<QT_ROCMFP4>(a, &qa, li, ni, lo, no, kernels, st); break;
    case QT_ROCMFP4_FAST: *err = launch_multi_t<QT_ROCMFP4_FAST>(a, &qa, li, ni, lo, no, kernels, st); break;
    default: *err = launch_multi_t<QT_Q4_K>(a, &qa, li, ni, lo, no, kernels, st); break;
    }
    return true;
}
