// fused_decode.hip -- one batch-1 MoE FFN layer in three kernels (gfx950, wave64).
//
// The per-operation layer (router logits, router, quantize, gate/up, SwiGLU, down, combine) costs seven launches,
// each with ~2.5 us of ramp and tail on MI355X, while the layer's ~25-40 MB of weights take 3-5 us at HBM speed.
// Here the layer is three launches with no grid-wide synchronisation inside any of them:
//   1  one workgroup per router-logit row, one that quantizes x (the activation quantizer's expressions) and
//      one for the shared-expert gate;
//   2  one workgroup per (slot, 32-row block of FE): it routes (every workgroup for itself; workgroup 0 also
//      publishes the ids), then computes the slot expert's 32 gate and 32 up rows, SwiGLU, and the Q8_0
//      quantization of those 32 values (one Q8_0 block of down's input). The top-k is a rank count over the
//      whole workgroup (router_rank_select: the router's ids, in its order, in two LDS passes where the router's
//      one-wave selection takes nu rounds of wave reductions: -0.85 us on the critical path at 128 experts);
//   3  one workgroup per 64 / L output rows (L: the down row dot's lanes), one wave per slot: their down rows,
//      then the combine in slot order; one more wave forms the renormalised weights from the logits and the ids
//      (the router's expressions) while the slots' rows load.
// Every sum is formed in the same order as the per-operation kernels (rows_dot's lane groups and DPP group sums,
// the same router, quantizer and combine), so the layer's output equals the per-operation path bit for bit.
// (A single persistent kernel with two grid barriers was measured slower: each barrier's cross-XCD fences and
// 256-way atomic arrival cost ~10 us on MI355X, more than a kernel boundary.)

#include <atomic>

#include "fused_common.h"
#include "gpu_ops.h"
#include "host_common.h"
#include "moe_layer.h"
#include "qmatvec.h"

#ifndef FD_SHARED_NO_ROUTE
#define FD_SHARED_NO_ROUTE 1  // the shared expert's units skip the routing (config 1: 18.75 -> 18.59 us per layer)
#endif
#ifndef FD_GU_RW
#define FD_GU_RW 4              // gate / up rows per wave in kernel 2 (64 / FD_GU_RW waves per workgroup)
#endif



#ifndef FD_RANK_MAX_NE
#define FD_RANK_MAX_NE 256  // the largest expert count routed by rank counting over the workgroup, else by one
                            // wave (128, i.e. one wave at 256 experts: config 4 1,555 -> 1,447 tokens/s)
#endif

// ---- kernel 1: router logits (workgroups 0 .. NE - 1), x quantized (workgroup NE; Q4_K: E / 256 workgroups),
// the shared gate (the last workgroup)
__global__ void __launch_bounds__(256) k_fd_logits(FArgs a) {
    __shared__ float part[4];
    __shared__ __align__(16) float ys[FD_MAX_E];
    const int tid = threadIdx.x, E = a.E;
    stamp(a, 0);
    const float* xv = a.x;
    // router-row workgroups with the norm: the row's loads are issued first (they do not wait for the norm), then
    // the dot takes f32_row_dot's order (16-byte loads, lane i, i + 256, ... of the row) and sums
    const float* wrow = a.w_router + (size_t)blockIdx.x * E;
    const bool pre = a.norm && (int)blockIdx.x < a.NE && (E & 3) == 0 && ((uintptr_t)wrow & 15) == 0;
    // the shared expert's gate workgroup with the norm: its gate vector loaded the same way
    const bool gate_wg = (int)blockIdx.x == a.NE + (a.xo.qK ? E / 256 : 1);
    const bool pre_gate = a.norm && gate_wg && a.w_shexp && (E & 3) == 0 && ((uintptr_t)a.w_shexp & 15) == 0;
    float4 wpre[FD_MAX_E / 1024];
    if (pre || pre_gate)
#pragma unroll
        for (int k = 0; k < FD_MAX_E / 1024; ++k)
            if (tid + 256 * k < E / 4) wpre[k] = ld_w4((const float4*)(pre ? wrow : a.w_shexp) + tid + 256 * k);
    if (a.norm && rms_rows4(a.x, a.add, E)) {
        // every workgroup forms the normalized input itself (E <= 4096 values, from L2) in the 16-byte layout of the
        // router-row dot (rms_first_pass4): a router workgroup dots it in place, with f32_row_dot's order; the
        // others stage it in LDS
        float4 wn4[4];  // the norm weights, loaded with x and add (16-byte pieces when the weights are aligned)
        const bool wa = ((uintptr_t)a.w_norm & 15) == 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int c = min(tid + 256 * k, E / 4 - 1);
            if (!a.w_norm)
                wn4[k] = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
            else if (wa)
                wn4[k] = ((const float4*)a.w_norm)[c];
            else
                wn4[k] = make_float4(a.w_norm[4 * c], a.w_norm[4 * c + 1], a.w_norm[4 * c + 2], a.w_norm[4 * c + 3]);
        }
        float4 keep4[4];
        const float inv = rms_first_pass4(a.x, a.add, E, a.eps, keep4, part);
        float4 y4[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            y4[k] = make_float4(keep4[k].x * inv * wn4[k].x, keep4[k].y * inv * wn4[k].y, keep4[k].z * inv * wn4[k].z,
                                keep4[k].w * inv * wn4[k].w);
        if (blockIdx.x == 0 && a.add && a.x_out)  // workgroup 0 writes the residual
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (tid + 256 * k < E / 4) ((float4*)a.x_out)[tid + 256 * k] = keep4[k];
        if (pre) {  // a router row: f32_row_dot's expressions on the values in registers
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < FD_MAX_E / 1024; ++k)
                if (tid + 256 * k < E / 4) {
                    const float4 w4 = wpre[k], b = y4[k];
                    acc = fmaf(w4.x, b.x, acc);
                    acc = fmaf(w4.y, b.y, acc);
                    acc = fmaf(w4.z, b.z, acc);
                    acc = fmaf(w4.w, b.w, acc);
                }
            const float y = block256_sum(acc, part);
            if (tid == 0) a.logits[blockIdx.x] = y;
            stamp(a, 1);
            return;
        }
        if (pre_gate) {  // the shared expert's gate: shexp_gate's expressions on the values in registers
            float d = 0.0f;
#pragma unroll
            for (int k = 0; k < FD_MAX_E / 1024; ++k)
                if (tid + 256 * k < E / 4) {
                    const float4 p = y4[k], q = wpre[k];
                    d += p.x * q.x + p.y * q.y + p.z * q.z + p.w * q.w;
                }
            d = block256_sum(d, part);
            if (tid == 0) a.sg[0] = 1.0f / (1.0f + expf(-d));
            stamp(a, 1);
            return;
        }
        if (!a.xo.qK && !gate_wg && (int)blockIdx.x >= a.NE) {  // x quantized for gate / up, from the registers
            quantize_row4_q8_0(y4, E, a.xq, a.xd);
            stamp(a, 1);
            return;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (tid + 256 * k < E / 4) ((float4*)ys)[tid + 256 * k] = y4[k];
        __syncthreads();
        xv = ys;
    } else if (a.norm) {  // rows the 16-byte layout does not take: the producer kernel's other first pass
        float wn[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) wn[k] = a.w_norm ? a.w_norm[min(tid + 256 * k, E - 1)] : 1.0f;
        float keep[16];
        const float inv = rms_first_pass(a.x, a.add, E, a.eps, keep, part);
        const bool res = blockIdx.x == 0 && a.add && a.x_out;  // workgroup 0 writes the residual
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int i = tid + 256 * k;
            if (i < E) {
                ys[i] = keep[k] * inv * wn[k];
                if (res) a.x_out[i] = keep[k];
            }
        }
        __syncthreads();
        xv = ys;
    }
    if ((int)blockIdx.x < a.NE) {
        float y;
        if (pre) {  // (ys is 16-byte aligned LDS)
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < FD_MAX_E / 1024; ++k)
                if (tid + 256 * k < E / 4) {
                    const float4 w4 = wpre[k], b = ((const float4*)xv)[tid + 256 * k];
                    acc = fmaf(w4.x, b.x, acc);
                    acc = fmaf(w4.y, b.y, acc);
                    acc = fmaf(w4.z, b.z, acc);
                    acc = fmaf(w4.w, b.w, acc);
                }
            y = block256_sum(acc, part);
        } else {
            y = f32_row_dot(wrow, xv, E, part);
        }
        if (tid == 0) a.logits[blockIdx.x] = y;
        stamp(a, 1);
        return;
    }
    if (a.xo.qK) {  // Q4_K: one workgroup per 256-value block, the activation quantizer itself (Q8_0 and Q8_K)
        __shared__ Q8Smem sh;
        const int blk = blockIdx.x - a.NE;
        if (blk < E / 256) {
            q8_quantize_256(xv[blk * 256 + tid], true, blk, tid, sh, a.xo);
            stamp(a, 1);
            return;
        }
    }
    if ((int)blockIdx.x == a.NE + (a.xo.qK ? E / 256 : 1)) {  // the shared expert's gate
        const float g = shexp_gate(xv, a.w_shexp, E, part);
        if (tid == 0) a.sg[0] = g;
        stamp(a, 1);
        return;
    }
    quantize_row_q8_0(xv, E, a.xq, a.xd);  // x quantized for gate / up
    stamp(a, 1);
}

// ---- kernel 2: routing, then gate / up / SwiGLU / quantize of unit (slot, 32-row block). 16 waves of 4 rows
// (8 waves per matrix); a row is one group of L_IN lanes with NUPL_IN units per lane (the per-op shape for K = E),
// so a wave holds 64 / L_IN groups of 4 L_IN / 64 rows. Q4_K writes gate / up in fp32 instead (its down input is
// Q8_K, one scale per 256 values: the SwiGLU kernel between kernels 2 and 3 quantizes it).
template <int TYPE, int L_IN, int NUPL_IN>
__global__ void __launch_bounds__(64 * (64 / FD_GU_RW)) k_fd_gate_up(FArgs a) {
    constexpr int RW = FD_GU_RW, WPM = 32 / RW;  // rows per wave, waves per matrix
    constexpr int G = 64 / L_IN, R = RW / G;     // lane groups per wave, rows per group
    static_assert(R >= 1, "a wave's rows must cover its lane groups");
    __shared__ int s_ids[65];
    __shared__ float s_wts[64];
    __shared__ __align__(16) uint64_t s_pk[256];
    __shared__ __align__(16) uint64_t s_pk2[256];
    __shared__ float gu[2][32];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, gl = lane & (L_IN - 1), grp = lane / L_IN;
    const int FE = a.FE, NU = a.NU, nbf = FE / 32;
    const int slot = blockIdx.x / nbf, b = blockIdx.x - slot * nbf;
    stamp(a, 2);
    const float* lg = a.logits_in ? a.logits_in : a.logits;
#if FD_SHARED_NO_ROUTE
    // the shared expert's units need no routing: their loads start at once (workgroup 0, a routed unit, publishes)
    if (slot < NU) {
        if (a.rank_route)  // (uniform) every thread counts ranks; kernel 3 forms the weights
            router_rank_select<64 * (64 / FD_GU_RW)>(lg, a.NE, NU, s_ids, s_pk, s_pk2);
        else
            router_select(lg, a.NE, NU, s_ids, s_wts);
    }
#else
    if (a.rank_route)
        router_rank_select<64 * (64 / FD_GU_RW)>(lg, a.NE, NU, s_ids, s_pk, s_pk2);
    else
        router_select(lg, a.NE, NU, s_ids, s_wts);
#endif
    if (blockIdx.x == 0 && tid < NU) {  // the routing for kernel 3 and the caller
        a.ids[tid] = s_ids[tid];
        if (a.ids_out) a.ids_out[tid] = s_ids[tid];
        if (!a.rank_route) {
            a.wts[tid] = s_wts[tid];
            if (a.wts_out) a.wts_out[tid] = s_wts[tid];
        }
    }
    stamp(a, 3);
    const int e = wave_uniform(slot < NU ? s_ids[slot] : -1);
    const int mat = wave_uniform(w / WPM);  // the first WPM waves: gate rows; the next WPM: up rows
    const int mi = e >= 0 ? mat : 3 + mat;
    const long long rbase = e >= 0 ? (long long)e * FE : 0;
    const uint8_t* vb = pick(a.v, mi) + rbase * a.vrb_in;
    const uint8_t* sb = pick(a.s, mi) + rbase * a.srb_in;
    const int r0 = RW * (w % WPM) + grp * R;  // this group's first row of the unit's 32
    constexpr bool Q8K = Fmt<TYPE>::Q8K;
    float acc[R];
    rows_dot<TYPE, true, L_IN, R, NUPL_IN>(vb, sb, a.vrb_in, a.srb_in, 32 * b + r0, 1, FE, Q8K ? a.xo.qK : a.xq,
                                           Q8K ? a.xo.dK : a.xd, Q8K ? a.xo.bsK : nullptr, a.E, gl, acc);
    if constexpr (Q8K) {
        if (gl == 0)
#pragma unroll
            for (int r = 0; r < R; ++r) (mat ? a.u : a.g)[(long long)slot * FE + 32 * b + r0 + r] = acc[r];
        stamp(a, 7);
    } else {
        if (gl == 0)
#pragma unroll
            for (int r = 0; r < R; ++r) gu[mat][r0 + r] = acc[r];
        __syncthreads();
        stamp(a, 7);
        if (w == 0)  // SwiGLU and the Q8_0 block of these 32 values
            swiglu_q8_block(gu[0], gu[1], a.act_q + (long long)slot * FE + 32 * b,
                            a.act_d + (long long)slot * nbf + b);
    }
    stamp(a, 4);
}

// ---- kernel 3: down rows of every slot for RB = 64 / L_OUT output rows, then the combine in slot order. One wave
// per slot, one lane group of L_OUT lanes (NUPL_OUT units each) per output row: the per-operation down kernel's
// shape for this K, so the same sums. Token blockIdx.y (T = 1: 0; the multi-token layer launches T rows of
// workgroups over the same row blocks).
template <int TYPE, int L_OUT, int NUPL_OUT>
__global__ void __launch_bounds__(1024) k_fd_down(FArgs a) {
    constexpr int RB = 64 / L_OUT;
    __shared__ float downv[16][RB];
    __shared__ float s_wts[64];
    const int tid = threadIdx.x, E = a.E, FE = a.FE, NU = a.NU, NS = a.NS, t = blockIdx.y;
    const int slot = tid >> 6, lane = tid & 63, gl = lane & (L_OUT - 1), i = lane / L_OUT;
    const int i0 = blockIdx.x * RB;
    stamp(a, 5);
    const float sgv = a.has_gate && tid < RB ? a.sg[t] : 0.0f;  // (read now: kernel 1 wrote it)
    if (slot < NS) {
        const int e = wave_uniform(slot < NU ? a.ids[t * a.ids_ld + slot] : -1);
        const long long row = e >= 0 ? (long long)e * E + i0 + i : i0 + i;
        const int mi = e >= 0 ? 2 : 5;
        const uint8_t* vr[1] = {pick(a.v, mi) + row * a.vrb_out};
        const uint8_t* sr[1] = {pick(a.s, mi) + row * a.srb_out};
        constexpr bool Q8K = Fmt<TYPE>::Q8K;
        const long long sl = (long long)t * NS + slot;  // this (token, slot) pair's row of down's input
        const int8_t* xq[1] = {Q8K ? a.aqk + sl * FE : a.act_q + sl * FE};
        const float* xd[1] = {Q8K ? a.adk + sl * (FE / 256) : a.act_d + sl * (FE / 32)};
        const int* xbs[1] = {Q8K ? a.absk + sl * (FE / 16) : nullptr};
        float acc[1];
        rows_dot_multi<TYPE, L_OUT, 1, NUPL_OUT>(vr, sr, xq, xd, xbs, fmt_units(TYPE, FE), gl, 1, acc);
        if (gl == 0) downv[slot][i] = acc[0];
    } else {  // (rank_route: the wave after the slots) the renormalised weights, while the slots' rows load
        const float* lg = (a.logits_in ? a.logits_in : a.logits) + (size_t)t * a.NE;
        router_weights_one_wave(lg, a.NE, NU, a.ids + t * a.ids_ld, s_wts);
        if (blockIdx.x == 0 && a.wts_out && lane < NU) a.wts_out[t * NU + lane] = s_wts[lane];
    }
    __syncthreads();
    if (tid < RB) {  // the combine kernel's expression
        const float* wts = a.rank_route ? s_wts : a.wts + t * NU;
        float o = wts[0] * downv[0][tid];
        for (int j = 1; j < NU; ++j) o += wts[j] * downv[j][tid];
        if (NS > NU) o += a.has_gate ? downv[NU][tid] * sgv : downv[NU][tid];
        a.out[(size_t)t * E + i0 + tid] = o;
    }
    stamp(a, 6);
}

// ---- kernel 3 for Q4_K, token blockIdx.y (T = 1, or up to 4 tokens after the per-operation id launch of gate / up):
// down's Q8_K input formed here instead of by a SwiGLU launch before it. Each slot's wave reads its slot's fp32
// gate / up rows (FE = 1024: 16 consecutive values a lane, 16 lanes per 256-value block), forms SiLU(g) u (the SwiGLU kernel's expression) and the Q8_K blocks (the quantizer's: the
// signed value of largest |x| with the lowest index on ties, iscale = -127 / it, q = min(127, rint(iscale x)),
// d = 1 / iscale, sums of 16), into its own LDS; its weight loads are issued first. Then RS sets of 64 / L_OUT
// output rows with the per-operation down shape (L_OUT lanes, NUPL_OUT units a lane), and the combine in slot order.
// The same bits as the SwiGLU kernel and kernel 3; RS row sets a workgroup keep the workgroups' redundant reads of
// the gate / up rows at E / (RS 64 / L_OUT) x NS x 8 KB per token (RS = 4: 2 and 8 measured slower at T = 1, 8
// and 16 at T = 2..7).
#define FD_Q8K_FE 1024
template <int L_OUT, int NUPL_OUT, int RS>
__global__ void __launch_bounds__(1024) k_fd_down_q8k(FArgs a) {
    constexpr int RB = 64 / L_OUT;
    static_assert(L_OUT * NUPL_OUT * 64 == FD_Q8K_FE, "FE: one unit of 64 values a lane and unit");
    __shared__ float downv[16][RB * RS];
    __shared__ __align__(16) int8_t aq[16][FD_Q8K_FE];
    __shared__ float adk[16][FD_Q8K_FE / 256];
    __shared__ __align__(16) int abk[16][FD_Q8K_FE / 16];
    __shared__ float s_wts[64];
    const int tid = threadIdx.x, E = a.E, FE = a.FE, NU = a.NU, NS = a.NS, t = blockIdx.y;
    const int slot = tid >> 6, lane = tid & 63, gl = lane & (L_OUT - 1), i = lane / L_OUT;
    const int i0 = blockIdx.x * RB * RS;
    const long long sl = (long long)t * NS + slot;  // this (token, slot) pair's gate / up row
    stamp(a, 5);
    const float sgv = a.has_gate && tid < RB * RS ? a.sg[t] : 0.0f;  // (read now: kernel 1 wrote it)
    if (slot < NS) {
        const int e = wave_uniform(slot < NU ? a.ids[t * a.ids_ld + slot] : -1);
        const int mi = e >= 0 ? 2 : 5;
        const long long rbase = e >= 0 ? (long long)e * E : 0;
        const uint8_t* vb = pick(a.v, mi) + rbase * a.vrb_out;
        const uint8_t* sb = pick(a.s, mi) + rbase * a.srb_out;
        const int nu_out = fmt_units(QT_Q4_K, FE);
        WUnit<QT_Q4_K> wu[RS][NUPL_OUT];
#pragma unroll
        for (int r = 0; r < RS; ++r) {
            const long long row = i0 + RB * r + i;
#pragma unroll
            for (int c = 0; c < NUPL_OUT; ++c)
                load_packed<QT_Q4_K>(vb + row * a.vrb_out, sb + row * a.srb_out, gl + c * L_OUT, nu_out, wu[r][c]);
        }
        {  // this slot's SwiGLU and Q8_K blocks
            const float4* g4 = (const float4*)(a.g + sl * FE + 16 * lane);
            const float4* u4 = (const float4*)(a.u + sl * FE + 16 * lane);
            float v[16];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float4 g = g4[k], u = u4[k];
                const float gg[4] = {g.x, g.y, g.z, g.w}, uu[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) v[4 * k + j] = gg[j] / (1.0f + __expf(-gg[j])) * uu[j];
            }
            float ba = fabsf(v[0]), bv = v[0];
            int bi = 16 * (lane & 15);  // index within the 256-value block
#pragma unroll
            for (int k = 1; k < 16; ++k)
                if (fabsf(v[k]) > ba) {
                    ba = fabsf(v[k]);
                    bv = v[k];
                    bi = 16 * (lane & 15) + k;
                }
            argmax_step<1>(ba, bv, bi);
            argmax_step<2>(ba, bv, bi);
            argmax_step<4>(ba, bv, bi);
            argmax_step<8>(ba, bv, bi);
            const float iscale = ba != 0.0f ? -127.0f / bv : 0.0f;
            int q[16], s16 = 0;
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                q[k] = ba != 0.0f ? min(127, (int)rintf(iscale * v[k])) : 0;
                s16 += q[k];
            }
            uint32_t pk[4];
#pragma unroll
            for (int k = 0; k < 4; ++k)
                pk[k] = (q[4 * k] & 0xff) | ((q[4 * k + 1] & 0xff) << 8) | ((q[4 * k + 2] & 0xff) << 16) |
                        ((uint32_t)q[4 * k + 3] << 24);
            *(uint4*)&aq[slot][16 * lane] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
            if ((lane & 15) == 0) adk[slot][lane >> 4] = ba != 0.0f ? 1.0f / iscale : 0.0f;
            abk[slot][lane] = s16;
        }
        // (the slot's own wave reads what it wrote: LDS operations of a wave complete in order)
        XUnit<QT_Q4_K> x[NUPL_OUT];
#pragma unroll
        for (int c = 0; c < NUPL_OUT; ++c) load_x<QT_Q4_K>(aq[slot], adk[slot], abk[slot], gl + c * L_OUT, x[c]);
#pragma unroll
        for (int r = 0; r < RS; ++r) {
            float acc = 0.0f;
#pragma unroll
            for (int c = 0; c < NUPL_OUT; ++c) acc += term<QT_Q4_K>(wu[r][c], x[c], gl + c * L_OUT);
            acc = group_sum<L_OUT>(acc);
            if (gl == 0) downv[slot][RB * r + i] = acc;
        }
    } else {  // (rank_route: the wave after the slots) the renormalised weights, while the slots' rows load
        const float* lg = (a.logits_in ? a.logits_in : a.logits) + (size_t)t * a.NE;
        router_weights_one_wave(lg, a.NE, NU, a.ids + t * a.ids_ld, s_wts);
        if (blockIdx.x == 0 && a.wts_out && lane < NU) a.wts_out[t * NU + lane] = s_wts[lane];
    }
    __syncthreads();
    if (tid < RB * RS) {  // the combine kernel's expression
        const float* wts = a.rank_route ? s_wts : a.wts + t * NU;
        float o = wts[0] * downv[0][tid];
        for (int j = 1; j < NU; ++j) o += wts[j] * downv[j][tid];
        if (NS > NU) o += a.has_gate ? downv[NU][tid] * sgv : downv[NU][tid];
        a.out[(long long)t * E + i0 + tid] = o;
    }
    stamp(a, 6);
}

// ------------------------------------------------------------------ host side

bool moe_packed_planes(const void* W, int type, int K, size_t row_bytes, const uint8_t** v, const uint8_t** s);

namespace {

#ifndef FD_Q8K_RS
#define FD_Q8K_RS 4
#endif

// Q4_K kernel 3 over a.T rows of workgroups: k_fd_down_q8k. fused_shape_ok admits Q4_K only with down's lane shape
// 16 x 1 unit of 64 values, i.e. FE == FD_Q8K_FE, and E is a multiple of 256 (every caller has passed
// moe_fused_prepare); any other shape returns hipErrorInvalidValue rather than run a path no test covers.
template <int LO, int NO>
hipError_t launch_down_q8k(const FArgs& a, const qmatvec_q8* qa, hipStream_t st) {
    (void)qa;
    constexpr int RS = FD_Q8K_RS;  // row sets a workgroup
    if (a.FE != FD_Q8K_FE || a.E % (RS * (64 / LO)) != 0 || LO * NO * 64 != FD_Q8K_FE) return hipErrorInvalidValue;
    return launch_kernel(k_fd_down_q8k<LO, NO, RS>, dim3(a.E / (RS * (64 / LO)), a.T),
                         dim3(64 * (a.NS + a.rank_route)), 0, st, a);
}

// kernels: bit 0, 1, 2 launch kernel 1, 2 (with Q4_K's SwiGLU), 3 (7 in normal use; a subset only for profiling)
template <int TYPE, int LI, int NI, int LO, int NO>
hipError_t launch_fused(const FArgs& a, const qmatvec_q8* qa, int kernels, hipStream_t st) {
    hipError_t e = hipSuccess;
    const int nq = Fmt<TYPE>::Q8K ? a.E / 256 : 1;  // quantizing workgroups of kernel 1
    if (kernels & 1) e = launch_kernel(k_fd_logits, dim3(a.NE + nq + a.has_gate), dim3(256), 0, st, a);
    if (e == hipSuccess && (kernels & 2))
        e = launch_kernel(k_fd_gate_up<TYPE, LI, NI>, dim3(a.NS * (a.FE / 32)), dim3(64 * (64 / FD_GU_RW)), 0, st,
                          a);
    if constexpr (Fmt<TYPE>::Q8K) {  // down's Q8_K input formed by kernel 3 itself
        if (e == hipSuccess && (kernels & 4)) e = launch_down_q8k<LO, NO>(a, qa, st);
        return e;
    }
    if (e == hipSuccess && (kernels & 4))
        e = launch_kernel(k_fd_down<TYPE, LO, NO>, dim3(a.E / (64 / LO)), dim3(64 * (a.NS + a.rank_route)), 0, st,
                          a);
    return e;
}

// Gate / up: the per-operation (lanes, units) for K = E: 2048 -> (64, 1), 4096 -> (64, 2); Q4_K 3072 -> (16, 3).
// Down, for K = FE: 512 -> (16, 1), 768 -> (8, 3), 1024 -> (32, 1), 1536 -> (16, 3), 2048 -> (64, 1); Q4_K 1024
// -> (16, 1).
template <int TYPE>
hipError_t launch_fused_t(const FArgs& a, const qmatvec_q8* qa, int li, int ni, int lo, int no, int kernels,
                          hipStream_t st) {
#define FD_CASE(I, L, O) \
    if (li == 64 && ni == I && lo == L && no == O) return launch_fused<TYPE, 64, I, L, O>(a, qa, kernels, st);
    if constexpr (TYPE == QT_Q4_K) {
        if (li == 16 && ni == 3 && lo == 16 && no == 1) return launch_fused<TYPE, 16, 3, 16, 1>(a, qa, kernels, st);
    } else {
        FD_CASE(1, 16, 1) FD_CASE(1, 8, 3) FD_CASE(1, 32, 1) FD_CASE(1, 16, 3) FD_CASE(1, 64, 1)
        FD_CASE(2, 16, 1) FD_CASE(2, 8, 3) FD_CASE(2, 32, 1) FD_CASE(2, 16, 3) FD_CASE(2, 64, 1)
    }
#undef FD_CASE
    return hipErrorInvalidDeviceFunction;
}

template <int TYPE>
hipError_t launch_down_t(const FArgs& a, int lo, int no, hipStream_t st) {
    const dim3 g(a.E / (64 / lo), a.T), b(64 * a.NS);
#define FD_DOWN(L, O) \
    if (lo == L && no == O) return launch_kernel(k_fd_down<TYPE, L, O>, g, b, 0, st, a);
    if constexpr (TYPE == QT_Q4_K) {
        FD_DOWN(16, 1)
    } else {
        FD_DOWN(16, 1) FD_DOWN(8, 3) FD_DOWN(32, 1) FD_DOWN(16, 3) FD_DOWN(64, 1)
    }
#undef FD_DOWN
    return hipErrorInvalidDeviceFunction;
}

bool fused_shape_ok(int type, int li, int ni, int lo, int no) {
    if (type == QT_Q4_K) return li == 16 && ni == 3 && lo == 16 && no == 1;
    if (li != 64 || (ni != 1 && ni != 2)) return false;
    return (lo == 16 && no == 1) || (lo == 8 && no == 3) || (lo == 32 && no == 1) || (lo == 16 && no == 3) ||
           (lo == 64 && no == 1);
}

}  // namespace

namespace {
size_t fa256(size_t v) { return (v + 255) & ~(size_t)255; }
}

// Scratch bytes of the three kernels for T tokens: logits, gates, quantized x, routing, the quantized down input;
// Q4_K also x's activation bundle, gate / up / SwiGLU in fp32 and down's input bundle (T rows each)
size_t moe_fused_scratch_bytes(const moe_layer_desc* d, int T) {
    const size_t NS = d->n_used + (d->s_gate ? 1 : 0), E = d->n_embd, t = T;
    size_t n = fa256(t * d->n_expert * 4) + fa256(t * 4) + fa256(t * E) + fa256(t * E / 32 * 4) +
               2 * fa256(t * 64 * 4) + fa256(t * NS * d->n_ff) + fa256(t * NS * d->n_ff / 32 * 4);
    if (d->type == QT_Q4_K)
        n += fa256(qmatvec_q8_bytes((int)(t * ((E + 255) / 256 * 256)))) +
             fa256(qmatvec_q8_bytes((int)(t * NS * d->n_ff))) + 3 * fa256(t * NS * d->n_ff * 4);
    return n;
}

// Q4_K's pieces after the common part (a.T tokens): x's Q8_K bundle [T][E] (kernel 1), gate / up / SwiGLU in
// fp32 [T][NS][FE] (kernel 2, then the SwiGLU kernel) and down's input bundle [T][NS][FE]; qa receives the latter
void moe_fused_carve_q4k(FArgs& a, char* p, qmatvec_q8* qa, qmatvec_q8* qx_out) {
    qmatvec_q8 qx = {};
    const int kx = a.T * ((a.E + 255) / 256 * 256), ka = a.T * a.NS * a.FE;
    qmatvec_q8_bind(&qx, p, kx);
    p += fa256(qmatvec_q8_bytes(kx));
    qmatvec_q8_bind(qa, p, ka);
    p += fa256(qmatvec_q8_bytes(ka));
    a.xo = {qx.q0, qx.d0, qx.qK, qx.dK, qx.bsK, qx.s0, nullptr, 0};
    if (qx_out) *qx_out = qx;
    a.g = (float*)p;
    p += fa256((size_t)ka * 4);
    a.u = (float*)p;
    p += fa256((size_t)ka * 4);
    a.act = (float*)p;
    a.aqk = qa->qK;
    a.adk = qa->dK;
    a.absk = qa->bsK;
}

// The scratch pieces of a.T tokens (the layout moe_fused_scratch_bytes sizes); returns the end of the common part
char* moe_fused_carve(FArgs& a, void* scratch) {
    char* p = (char*)scratch;
    const size_t t = a.T;
    a.logits = (float*)p;
    p += fa256(t * a.NE * 4);
    a.sg = (float*)p;
    p += fa256(t * 4);
    a.xq = (int8_t*)p;
    p += fa256(t * a.E);
    a.xd = (float*)p;
    p += fa256(t * a.E / 32 * 4);
    a.ids = (int*)p;
    p += fa256(t * 64 * 4);
    a.wts = (float*)p;
    p += fa256(t * 64 * 4);
    a.act_q = (int8_t*)p;
    p += fa256(t * a.NS * a.FE);
    a.act_d = (float*)p;
    p += fa256(t * a.NS * a.FE / 32 * 4);
    return p;
}

// Whether the fused kernels take this layer: a supported type, every expert matrix registered in split-plane
// form, and shapes the instantiations cover. Fills the kernel arguments.
bool moe_fused_prepare(const moe_layer_desc* d, FArgs& a) {
    const int type = d->type, E = d->n_embd, FE = d->n_ff, NU = d->n_used;
    if (type != QT_Q8_0 && type != QT_ROCMFP4 && type != QT_ROCMFP4_FAST && type != QT_Q4_K) return false;
    if (E % 256 || E > FD_MAX_E || FE % 256 || NU > 64 || d->n_expert > ROUTER_MAX_E) return false;
    int li, ni, lo, no;
    moe_mv_shape(type, E, &li, &ni);
    moe_mv_shape(type, FE, &lo, &no);
    if (!fused_shape_ok(type, li, ni, lo, no)) return false;
    const int NS = NU + (d->s_gate ? 1 : 0);
    if (NS > 16) return false;
    auto native_row = [type](size_t k) {
        return type == QT_Q4_K ? k / 256 * 144 : k / 32 * (type == QT_Q8_0 ? 34 : type == QT_ROCMFP4 ? 18 : 17);
    };
    const size_t rb_in = native_row(E), rb_out = native_row(FE);
    const void* W[6] = {d->w_gate, d->w_up, d->w_down, d->s_gate, d->s_up, d->s_down};
    for (int i = 0; i < 6; ++i) {
        a.v[i] = a.s[i] = nullptr;
        if (!W[i]) {
            if (i < 3 || d->s_gate) return false;
            continue;
        }
        if (!moe_packed_planes(W[i], type, i % 3 == 2 ? FE : E, i % 3 == 2 ? rb_out : rb_in, &a.v[i], &a.s[i]))
            return false;
    }
    a.vrb_in = fmt_value_row(type, E);
    a.srb_in = fmt_scale_row(type, E);
    a.vrb_out = fmt_value_row(type, FE);
    a.srb_out = fmt_scale_row(type, FE);
    a.E = E;
    a.NE = d->n_expert;
    a.NU = NU;
    a.FE = FE;
    a.NS = NS;
    a.ids_ld = NU;
    a.w_router = d->w_router;
    a.w_shexp = d->w_shexp;
    a.has_gate = d->s_gate && d->w_shexp ? 1 : 0;
    return true;
}

hipError_t moe_fused_launch(const moe_layer_desc* d, FArgs& a, void* scratch, int kernels, hipStream_t st) {
    a.T = 1;
    char* p = moe_fused_carve(a, scratch);
    qmatvec_q8 qa = {};
    if (d->type == QT_Q4_K) moe_fused_carve_q4k(a, p, &qa);
    int li, ni, lo, no;
    moe_mv_shape(d->type, a.E, &li, &ni);
    moe_mv_shape(d->type, a.FE, &lo, &no);
    switch (d->type) {
    case QT_Q8_0: return launch_fused_t<QT_Q8_0>(a, &qa, li, ni, lo, no, kernels, st);
    case QT_ROCMFP4: return launch_fused_t<QT_ROCMFP4>(a, &qa, li, ni, lo, no, kernels, st);
    case QT_ROCMFP4_FAST: return launch_fused_t<QT_ROCMFP4_FAST>(a, &qa, li, ni, lo, no, kernels, st);
    default: return launch_fused_t<QT_Q4_K>(a, &qa, li, ni, lo, no, kernels, st);
    }
}

hipError_t moe_fused_launch_down_q8k(const FArgs& a, const qmatvec_q8* qa, hipStream_t st) {
    int lo, no;
    moe_mv_shape(QT_Q4_K, a.FE, &lo, &no);
    if (lo == 16 && no == 1) return launch_down_q8k<16, 1>(a, qa, st);
    return hipErrorInvalidDeviceFunction;
}

// Kernel 3 for a.T tokens (grid: row blocks x tokens), the multi-token layer's down + combine
hipError_t moe_fused_launch_down(int type, const FArgs& a, hipStream_t st) {
    int lo, no;
    moe_mv_shape(type, a.FE, &lo, &no);
    switch (type) {
    case QT_Q8_0: return launch_down_t<QT_Q8_0>(a, lo, no, st);
    case QT_ROCMFP4: return launch_down_t<QT_ROCMFP4>(a, lo, no, st);
    case QT_ROCMFP4_FAST: return launch_down_t<QT_ROCMFP4_FAST>(a, lo, no, st);
    default: return launch_down_t<QT_Q4_K>(a, lo, no, st);
    }
}

static std::atomic<unsigned long long*> g_stamps{nullptr};

// Profiling: every later fused layer writes timestamps to stamps (device memory of 8 words per workgroup of the
// largest of the three grids; nullptr: stop)
extern "C" void moe_layer_fused_stamps(void* stamps) {
    g_stamps.store((unsigned long long*)stamps, std::memory_order_relaxed);
}
unsigned long long* moe_fused_stamps_ptr() { return g_stamps.load(std::memory_order_relaxed); }

bool moe_fused_try(const moe_layer_desc* d, const float* x, const float* logits, float* out, int* ids_out,
                   float* wts_out, void* scratch, int kernels, hipStream_t st, hipError_t* err, const FNorm* norm) {
    FArgs a = {};
    a.stamps = g_stamps;
    if (!moe_fused_prepare(d, a)) return false;
    a.x = x;
    if (norm) {
        a.norm = 1;
        a.add = norm->add;
        a.w_norm = norm->w;
        a.x_out = norm->x_out;
        a.eps = norm->eps;
    }
    a.logits_in = logits;
    a.out = out;
    a.ids_out = ids_out;
    a.wts_out = wts_out;
    // Top-k by rank counting in kernel 2, the weights in an extra wave of kernel 3 (s_pk holds 256 keys; the
    // extra wave needs a 17th wave of room)
    a.rank_route = a.NE <= FD_RANK_MAX_NE && a.NS < 16 ? 1 : 0;
    *err = moe_fused_launch(d, a, scratch, kernels, st);
    return true;
}
