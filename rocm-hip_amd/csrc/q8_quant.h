// q8_quant.h -- the activation quantizer every producer of an expert-matvec input shares (gfx950, wave64).
//
// One 256-value block per 256-thread workgroup (four waves), value t of the block in thread t, into both of
// ggml's activation formats (src/q8_device.h:54-104):
//   Q8_0 per 32 values: amax, q = round-half-even(x * (127 / amax)) with the unrounded 127 / amax,
//        d = F16(amax / 127), and the Q8_1 sum s = F16(amax / 127 * sum q) kept as float bits.
//   Q8_K per 256 values: mx = the signed value of largest |x| (lowest index on ties), iscale = -127 / mx,
//        q = min(127, round-half-even(iscale * x)), d = 1 / iscale, and the sums of each 16 q.
// A Q8_0 block is half a wave, so its reductions stay inside the half (xor offsets below 32); the Q8_K
// arg-max runs over the wave and then over the four waves through LDS.
#ifndef Q8_QUANT_H
#define Q8_QUANT_H

#include "moe_common.h"

struct Q8Smem {
    float a[4];
    float v[4];
    int i[4];
};

__device__ __forceinline__ float fp16_round(float x) { return __half2float(__float2half(x)); }

// One step of the Q8_K arg-max: the larger |x|, the lower index on ties (a total order, so the result does not
// depend on the pairing pattern)
template <int S>
__device__ __forceinline__ void argmax_step(float& ba, float& bv, int& bi) {
    const float oa = partner_f<S>(ba), ov = partner_f<S>(bv);
    const int oi = partner_i<S>(bi);
    if (oa > ba || (oa == ba && oi < bi)) {
        ba = oa;
        bv = ov;
        bi = oi;
    }
}

// Every thread of the 256-thread workgroup calls this the same number of times (it holds barriers);
// threads past the end of the data pass active = false. blk: the 256-value block index in the output.
__device__ __forceinline__ void q8_quantize_256(float v, bool active, long long blk, int t, Q8Smem& sh,
                                                const Q8Out& o) {
    if (!o.qK) return;  // uniform: no int8 output wanted
    const int lane = t & 63, w = t >> 6;
    const long long i = blk * 256 + t;
    const float a = active ? fabsf(v) : 0.0f;

    const float am = group_max<32>(a);
    const float id = am != 0.0f ? 127.0f / am : 0.0f;
    const int q0 = active ? (int)rintf(v * id) : 0;
    const int s = group_sum_i<32>(q0);
    if (active) {
        o.q0[i] = (int8_t)q0;
        if ((t & 31) == 0) {
            const float d = am / 127.0f;
            o.d0[blk * 8 + (t >> 5)] = fp16_round(d);
            o.s0[blk * 8 + (t >> 5)] = __float_as_int(fp16_round(d * (float)s));
        }
    }

    float ba = a, bv = v;
    int bi = t;
    argmax_step<1>(ba, bv, bi);
    argmax_step<2>(ba, bv, bi);
    argmax_step<4>(ba, bv, bi);
    argmax_step<8>(ba, bv, bi);
    argmax_step<16>(ba, bv, bi);
    argmax_step<32>(ba, bv, bi);
    if (lane == 0) {
        sh.a[w] = ba;
        sh.v[w] = bv;
        sh.i[w] = bi;
    }
    __syncthreads();
    float fa = sh.a[0], fv = sh.v[0];
    int fi = sh.i[0];
#pragma unroll
    for (int k = 1; k < 4; ++k)
        if (sh.a[k] > fa || (sh.a[k] == fa && sh.i[k] < fi)) {
            fa = sh.a[k];
            fv = sh.v[k];
            fi = sh.i[k];
        }
    __syncthreads();  // sh is reused by the next block
    int q = 0;
    float iscale = 0.0f;
    if (fa != 0.0f) {
        iscale = -127.0f / fv;
        q = min(127, (int)rintf(iscale * v));
    }
    if (!active) q = 0;
    const int s16 = group_sum_i<16>(q);
    if (active) {
        o.qK[i] = (int8_t)q;
        if (t == 0) o.dK[blk] = fa != 0.0f ? 1.0f / iscale : 0.0f;
        if ((t & 15) == 0) o.bsK[blk * 16 + (t >> 4)] = s16;
    }
}

// The Q8_0 part of q8_quantize_256_wave (values, scales, Q8_1 sums)
__device__ __forceinline__ void q8_0_256_wave(const float (&v)[4], long long blk, int lane, long long i0, const Q8Out& o) {
    float a = fabsf(v[0]);
#pragma unroll
    for (int j = 1; j < 4; ++j) a = fmaxf(a, fabsf(v[j]));
    const float am = group_max<8>(a);
    const float id = am != 0.0f ? 127.0f / am : 0.0f;
    int q0[4], s = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        q0[j] = (int)rintf(v[j] * id);
        s += q0[j];
    }
    s = group_sum_i<8>(s);
    *(uint32_t*)(o.q0 + i0) =
        (q0[0] & 0xff) | ((q0[1] & 0xff) << 8) | ((q0[2] & 0xff) << 16) | ((uint32_t)q0[3] << 24);
    if ((lane & 7) == 0) {
        const float d = am / 127.0f;
        o.d0[blk * 8 + (lane >> 3)] = fp16_round(d);
        o.s0[blk * 8 + (lane >> 3)] = __float_as_int(fp16_round(d * (float)s));
    }
}

// The Q8_K part of q8_quantize_256_wave (values, scale, sums of 16)
__device__ __forceinline__ void q8_k_256_wave(const float (&v)[4], long long blk, int lane, long long i0, const Q8Out& o) {
    float ba = fabsf(v[0]), bv = v[0];
    int bi = 4 * lane;
#pragma unroll
    for (int j = 1; j < 4; ++j)  // (strictly larger: the lower index stays on ties)
        if (fabsf(v[j]) > ba) {
            ba = fabsf(v[j]);
            bv = v[j];
            bi = 4 * lane + j;
        }
    argmax_step<1>(ba, bv, bi);
    argmax_step<2>(ba, bv, bi);
    argmax_step<4>(ba, bv, bi);
    argmax_step<8>(ba, bv, bi);
    argmax_step<16>(ba, bv, bi);
    argmax_step<32>(ba, bv, bi);
    int q[4] = {0, 0, 0, 0}, s16 = 0;
    float iscale = 0.0f;
    if (ba != 0.0f) {
        iscale = -127.0f / bv;
#pragma unroll
        for (int j = 0; j < 4; ++j) q[j] = min(127, (int)rintf(iscale * v[j]));
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) s16 += q[j];
    s16 = group_sum_i<4>(s16);
    *(uint32_t*)(o.qK + i0) = (q[0] & 0xff) | ((q[1] & 0xff) << 8) | ((q[2] & 0xff) << 16) | ((uint32_t)q[3] << 24);
    if (lane == 0) o.dK[blk] = ba != 0.0f ? 1.0f / iscale : 0.0f;
    if ((lane & 3) == 0) o.bsK[blk * 16 + (lane >> 2)] = s16;
}

// The same outputs from one wave per 256-value block, the whole block valid: lane l holds values 4 l .. 4 l + 3, so
// a Q8_0 block is eight lanes and the Q8_K block the wave, with no LDS and no barrier. The expressions are
// q8_quantize_256's, and every reduction gives the same result in any pairing (maxima, the arg-max's total order,
// integer sums), so the outputs are the same bits; the stores are four bytes a lane. A null o.q0 / o.qK skips that
// format (uniform).
__device__ __forceinline__ void q8_quantize_256_wave(const float (&v)[4], long long blk, int lane, const Q8Out& o) {
    const long long i0 = blk * 256 + 4 * lane;
    if (o.q0) q8_0_256_wave(v, blk, lane, i0, o);
    if (o.qK) q8_k_256_wave(v, blk, lane, i0, o);
}

#endif  // Q8_QUANT_H
