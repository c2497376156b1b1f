// expert_units.h -- weight "units" of the int8 expert kernels: loading one unit of a weight row (from the
// native GGUF blocks or from the split-plane copy) and its integer dot with the quantized activation.
//
// A unit is 32 values for Q8_0 / ROCmFP4 / ROCmFP4_FAST (one block) and 64 values for Q4_K (chunk c of a
// super-block: 32 value bytes, sub-blocks 2c and 2c + 1). Its value bytes are held as dwords q[], its scale
// bytes as dwords s[]: Q8_0 s[0] = FP16 d; ROCmFP4 s[0] = e0 | e1 << 8; FAST s[0] = e; Q4_K s[0..3] = the
// super-block's 16-byte head (d | dmin << 16, then the 12 scale bytes).
//
// Split-plane layout of one row (built once by qmatvec_pack_weights): a value plane and a scale plane.
//   Q8_0, Q4_K (32 value bytes per unit, nu units): value bytes 0..15 of unit u at 16 u, bytes 16..31 at
//     16 (nu + u), so lane-consecutive units are lane-consecutive 16-byte loads in both halves.
//   ROCmFP4, FAST (16 value bytes per unit): unit u at 16 u.
//   Scale plane: Q8_0 2 bytes per unit, ROCmFP4 2 (e0, e1), FAST 1, Q4_K 16 per super-block (per 4 units).
// Row sizes: values K (Q8_0) or K / 2; scales K / 16 (Q8_0, ROCmFP4, Q4_K) or K / 32 (FAST). Plane sizes
// add up to the native row size.
#ifndef EXPERT_UNITS_H
#define EXPERT_UNITS_H

#include "moe_common.h"

template <int TYPE>
struct Fmt;
template <>
struct Fmt<QT_Q8_0> {
    static constexpr int UV = 32, QW = 8, SW = 1, BLOCK_BYTES = 34;
    static constexpr bool Q8K = false;
};
template <>
struct Fmt<QT_ROCMFP4> {
    static constexpr int UV = 32, QW = 4, SW = 1, BLOCK_BYTES = 18;
    static constexpr bool Q8K = false;
};
template <>
struct Fmt<QT_ROCMFP4_FAST> {
    static constexpr int UV = 32, QW = 4, SW = 1, BLOCK_BYTES = 17;
    static constexpr bool Q8K = false;
};
template <>
struct Fmt<QT_Q4_K> {
    static constexpr int UV = 64, QW = 8, SW = 4, BLOCK_BYTES = 144;
    static constexpr bool Q8K = true;
};

__host__ __device__ constexpr int fmt_value_row(int type, int K) { return type == QT_Q8_0 ? K : K / 2; }
__host__ __device__ constexpr int fmt_scale_row(int type, int K) { return type == QT_ROCMFP4_FAST ? K / 32 : K / 16; }
// Bytes per row in the MFMA operand tiles. Values: Q8_0 its int8 values; the FP4 types and Q4_K their codes
// re-encoded as FP6 E2M3 (6 bits each: every codebook value / 2, and every 4-bit Q4_K quant / 2, is exact in E2M3,
// which the hardware decodes 32 at a time). Scales: Q8_0 its FP16 d (2 per block); the FP4 types each block's
// (e0, e1) UE4M3 half-scales decoded to an FP16 pair (FAST: (e, e)), 4 per block; Q4_K per super-block of 256 a
// 32-byte slot (Q4K_TILE_SLOT), 16 bytes per 128-value half: its four 6-bit sub-block scales and four mins as
// bytes, then the super-block's FP16 d and dmin, 4 bytes of zeros (one 16-byte load a lane and half). The FP4 and
// Q4_K value tiles are stage-major: the 48 bytes of a lane's codes for four consecutive blocks in three 16-byte
// chunks, chunk i of the stage at 1024 i + 16 lane.
#define Q4K_TILE_SLOT 32
__host__ __device__ constexpr int tile_value_row(int type, int K) { return type == QT_Q8_0 ? K : K / 4 * 3; }
__host__ __device__ constexpr int tile_scale_row(int type, int K) {
    return type == QT_Q8_0 ? K / 16 : type == QT_Q4_K ? K / 256 * Q4K_TILE_SLOT : K / 8;
}
__host__ __device__ constexpr int fmt_units(int type, int K) { return type == QT_Q4_K ? K / 64 : K / 32; }

template <int TYPE>
struct WUnit {
    uint32_t q[Fmt<TYPE>::QW];
    uint32_t s[Fmt<TYPE>::SW];
};

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) { return *(const uint16_t*)p; }
// A scale-plane load (2 bytes), nontemporal when EU_NT_S is set (config 1 decode 16.7 -> 16.5 us, config 0 17.75 ->
// 17.35, config 4's stack 1,510 -> 1,555 tokens/s)
#ifndef EU_NT_S
#define EU_NT_S 1
#endif
__device__ __forceinline__ uint32_t ld_s16(const uint8_t* p, bool nt = true) {
#if EU_NT_S
    if (nt) return __builtin_nontemporal_load((const uint16_t*)p);
#endif
    (void)nt;
    return *(const uint16_t*)p;
}__device__ __forceinline__ uint32_t ld_u32(const uint8_t* p) { return *(const uint32_t*)p; }
// The 16-byte weight loads of the row dots as nontemporal loads (each weight byte is read once per launch). Measured
// per decode layer (us): config 1 17.4-17.9 -> 16.7, config 0 18.8 -> 17.7, config 3 22.5 -> 21.8, config 3 at
// T = 4 54.6 -> 52.3; config 4's 40-layer stack 1,430 -> 1,517 tokens/s.
#ifndef EU_NT
#define EU_NT 1
#endif
typedef unsigned int eu_v4u __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_u128(const uint8_t* p, bool nt = true) {
#if EU_NT
    if (nt) {
        const eu_v4u v = __builtin_nontemporal_load((const eu_v4u*)p);
        return make_uint4(v.x, v.y, v.z, v.w);
    }
#endif
    (void)nt;
    return *(const uint4*)p;
}
// ---- native GGUF rows (row pointer 4-byte aligned, as the reference's launchers require)
template <int TYPE>
__device__ __forceinline__ void load_native(const uint8_t* row, int u, WUnit<TYPE>& w);

template <>
__device__ __forceinline__ void load_native<QT_Q8_0>(const uint8_t* row, int u, WUnit<QT_Q8_0>& w) {
    const uint8_t* b = row + (size_t)u * 34;  // 2-byte aligned
    w.s[0] = ld_u16(b);
#pragma unroll
    for (int k = 0; k < 8; ++k) w.q[k] = ld_u16(b + 2 + 4 * k) | (ld_u16(b + 4 + 4 * k) << 16);
}
template <>
__device__ __forceinline__ void load_native<QT_ROCMFP4>(const uint8_t* row, int u, WUnit<QT_ROCMFP4>& w) {
    const uint8_t* b = row + (size_t)u * 18;  // 2-byte aligned
#pragma unroll
    for (int k = 0; k < 4; ++k) w.q[k] = ld_u16(b + 4 * k) | (ld_u16(b + 2 + 4 * k) << 16);
    w.s[0] = ld_u16(b + 16);
}
template <>
__device__ __forceinline__ void load_native<QT_ROCMFP4_FAST>(const uint8_t* row, int u, WUnit<QT_ROCMFP4_FAST>& w) {
    const uint8_t* b = row + (size_t)u * 17;  // byte aligned
#pragma unroll
    for (int k = 0; k < 4; ++k)
        w.q[k] = (uint32_t)b[4 * k] | ((uint32_t)b[4 * k + 1] << 8) | ((uint32_t)b[4 * k + 2] << 16) |
                 ((uint32_t)b[4 * k + 3] << 24);
    w.s[0] = b[16];
}
template <>
__device__ __forceinline__ void load_native<QT_Q4_K>(const uint8_t* row, int u, WUnit<QT_Q4_K>& w) {
    const uint8_t* b = row + (size_t)(u >> 2) * 144;  // 4-byte aligned
    const int c = u & 3;
#pragma unroll
    for (int k = 0; k < 4; ++k) w.s[k] = ld_u32(b + 4 * k);
#pragma unroll
    for (int k = 0; k < 8; ++k) w.q[k] = ld_u32(b + 16 + 32 * c + 4 * k);
}

// ---- split-plane rows: vrow / srow point at the row in the value / scale plane; nu = units per row
template <int TYPE>
__device__ __forceinline__ void load_packed(const uint8_t* vrow, const uint8_t* srow, int u, int nu, WUnit<TYPE>& w,
                                            bool nt = true);

template <>
__device__ __forceinline__ void load_packed<QT_Q8_0>(const uint8_t* vrow, const uint8_t* srow, int u, int nu,
                                                     WUnit<QT_Q8_0>& w, bool nt) {
    const uint4 a = ld_u128(vrow + 16 * u, nt), b = ld_u128(vrow + 16 * (nu + u), nt);
    w.q[0] = a.x, w.q[1] = a.y, w.q[2] = a.z, w.q[3] = a.w;
    w.q[4] = b.x, w.q[5] = b.y, w.q[6] = b.z, w.q[7] = b.w;
    w.s[0] = ld_s16(srow + 2 * u, nt);
}
template <>
__device__ __forceinline__ void load_packed<QT_ROCMFP4>(const uint8_t* vrow, const uint8_t* srow, int u, int nu,
                                                        WUnit<QT_ROCMFP4>& w, bool nt) {
    const uint4 a = ld_u128(vrow + 16 * u, nt);
    w.q[0] = a.x, w.q[1] = a.y, w.q[2] = a.z, w.q[3] = a.w;
    w.s[0] = ld_s16(srow + 2 * u, nt);
}
template <>
__device__ __forceinline__ void load_packed<QT_ROCMFP4_FAST>(const uint8_t* vrow, const uint8_t* srow, int u, int nu,
                                                             WUnit<QT_ROCMFP4_FAST>& w, bool nt) {
    const uint4 a = ld_u128(vrow + 16 * u, nt);
    w.q[0] = a.x, w.q[1] = a.y, w.q[2] = a.z, w.q[3] = a.w;
    w.s[0] = srow[u];
}
template <>
__device__ __forceinline__ void load_packed<QT_Q4_K>(const uint8_t* vrow, const uint8_t* srow, int u, int nu,
                                                     WUnit<QT_Q4_K>& w, bool nt) {
    const uint4 a = ld_u128(vrow + 16 * u, nt), b = ld_u128(vrow + 16 * (nu + u), nt);
    const uint4 h = ld_u128(srow + 16 * (u >> 2), nt);
    w.q[0] = a.x, w.q[1] = a.y, w.q[2] = a.z, w.q[3] = a.w;
    w.q[4] = b.x, w.q[5] = b.y, w.q[6] = b.z, w.q[7] = b.w;
    w.s[0] = h.x, w.s[1] = h.y, w.s[2] = h.z, w.s[3] = h.w;
}

// ---- the activation side of one unit: Q8_0 (32 values, d) or Q8_K (64 values, d, four sums of 16)
template <int TYPE>
struct XUnit {
    int x[Fmt<TYPE>::UV / 4];
    float d;
    int bs[Fmt<TYPE>::Q8K ? 4 : 1];
};

// Activation row pointers: q (int8 values), d (scales), bs (Q8_K sums of 16), all for this input row
template <int TYPE>
__device__ __forceinline__ void load_x(const int8_t* q, const float* d, const int* bs, int u, XUnit<TYPE>& x) {
    constexpr int UV = Fmt<TYPE>::UV;
    const uint4* p = (const uint4*)(q + (size_t)u * UV);
#pragma unroll
    for (int k = 0; k < UV / 16; ++k) {
        const uint4 v = p[k];
        x.x[4 * k] = (int)v.x, x.x[4 * k + 1] = (int)v.y, x.x[4 * k + 2] = (int)v.z, x.x[4 * k + 3] = (int)v.w;
    }
    if constexpr (Fmt<TYPE>::Q8K) {
        x.d = d[u >> 2];
        const int4 s = *(const int4*)(bs + 4 * u);
        x.bs[0] = s.x, x.bs[1] = s.y, x.bs[2] = s.z, x.bs[3] = s.w;
    } else {
        x.d = d[u];
    }
}

// ---- one unit's float term: the integer block dots, then the reference's float combination
// Q8_0: (d_w dx) * sum (src/matvec_q.hip:1530-1536); ROCmFP4: e0 dx s0 + e1 dx s1 (:1287-1289; e dx formed as
// (2 e)(dx / 2), the same bits);
// FAST: e dx (s0 + s1) (:1456-1466); Q4_K: d dx (sc0 slo + sc1 shi) - dmin dx (m0 (bs0 + bs1) + m1 (bs2 + bs3))
// (:1740-1746, summed per 64-value chunk).
template <int TYPE>
__device__ __forceinline__ float unit_term(const WUnit<TYPE>& w, const XUnit<TYPE>& x);

template <>
__device__ __forceinline__ float unit_term<QT_Q8_0>(const WUnit<QT_Q8_0>& w, const XUnit<QT_Q8_0>& x) {
    int s = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) s = dot4((int)w.q[k], x.x[k], s);
    return h2f((uint16_t)w.s[0]) * x.d * (float)s;
}
template <>
__device__ __forceinline__ float unit_term<QT_ROCMFP4>(const WUnit<QT_ROCMFP4>& w, const XUnit<QT_ROCMFP4>& x) {
    int s0 = 0, s1 = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        s0 = dot4((int)fp4x4_to_i8x4(w.q[k]), x.x[k], s0);
        s1 = dot4((int)fp4x4_to_i8x4(w.q[k] >> 4), x.x[4 + k], s1);
    }
    // e0 dx as (2 e0)(dx / 2): the same bits (both factors exact), the scale byte decoded by the converter
    const float dxh = 0.5f * x.d, e0 = ue4m3_x2<0>(w.s[0]), e1 = ue4m3_x2<1>(w.s[0]);
    return e0 * dxh * (float)s0 + e1 * dxh * (float)s1;
}
template <>
__device__ __forceinline__ float unit_term<QT_ROCMFP4_FAST>(const WUnit<QT_ROCMFP4_FAST>& w,
                                                            const XUnit<QT_ROCMFP4_FAST>& x) {
    int s0 = 0, s1 = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        s0 = dot4((int)fp4x4_to_i8x4(w.q[k]), x.x[k], s0);
        s1 = dot4((int)fp4x4_to_i8x4(w.q[k] >> 4), x.x[4 + k], s1);
    }
    return ue4m3_x2<0>(w.s[0]) * (0.5f * x.d) * (float)(s0 + s1);
}
// Q4_K needs the chunk index c = u & 3 for its sub-block scales
__device__ __forceinline__ float unit_term_q4k(const WUnit<QT_Q4_K>& w, const XUnit<QT_Q4_K>& x, int c) {
    int slo = 0, shi = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        slo = dot4((int)(w.q[k] & 0x0f0f0f0fu), x.x[k], slo);
        shi = dot4((int)((w.q[k] >> 4) & 0x0f0f0f0fu), x.x[8 + k], shi);
    }
    const uint32_t sc[3] = {w.s[1], w.s[2], w.s[3]};
    int sc0, m0, sc1, m1;
    q4k_scale_min(2 * c, sc, sc0, m0);
    q4k_scale_min(2 * c + 1, sc, sc1, m1);
    const int isum = sc0 * slo + sc1 * shi;
    const int msum = m0 * (x.bs[0] + x.bs[1]) + m1 * (x.bs[2] + x.bs[3]);
    const float d = h2f((uint16_t)(w.s[0] & 0xffffu)), dmin = h2f((uint16_t)(w.s[0] >> 16));
    return d * x.d * (float)isum - dmin * x.d * (float)msum;
}

template <int TYPE>
__device__ __forceinline__ float term(const WUnit<TYPE>& w, const XUnit<TYPE>& x, int u) {
    if constexpr (TYPE == QT_Q4_K)
        return unit_term_q4k(w, x, u & 3);
    else
        return unit_term<TYPE>(w, x);
}

template <int TYPE, bool PACKED>
__device__ __forceinline__ void load_unit(const uint8_t* vrow, const uint8_t* srow, int u, int nu, WUnit<TYPE>& w,
                                          bool nt = true) {
    if constexpr (PACKED)
        load_packed<TYPE>(vrow, srow, u, nu, w, nt);
    else
        load_native<TYPE>(vrow, u, w);
}

// R rows (row0 + r * stride) of the matrix at (vbase, sbase) against one input row; returns the group sums.
// NUPL > 0: every lane has exactly NUPL units (nu == NUPL * L) and all R * NUPL weight loads (and the NUPL
// activation loads) are issued before any arithmetic; NUPL == 0: a loop over the lane's units.
template <int TYPE, bool PACKED, int L, int R, int NUPL>
__device__ __forceinline__ void rows_dot(const uint8_t* vbase, const uint8_t* sbase, long long vrb, long long srb,
                                         int row0, int stride, int nrows, const int8_t* xq, const float* xd,
                                         const int* xbs, int K, int gl, float acc[R], bool nt = true) {
    const int nu = fmt_units(TYPE, K);
    const uint8_t* vr[R];
    const uint8_t* sr[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = min(row0 + r * stride, nrows - 1);  // rows past the end load a valid row, unused
        vr[r] = vbase + (long long)row * vrb;
        sr[r] = PACKED ? sbase + (long long)row * srb : nullptr;
        acc[r] = 0.0f;
    }
    if constexpr (NUPL > 0) {
        WUnit<TYPE> w[NUPL][R];
        XUnit<TYPE> x[NUPL];
#pragma unroll
        for (int i = 0; i < NUPL; ++i)
#pragma unroll
            for (int r = 0; r < R; ++r) load_unit<TYPE, PACKED>(vr[r], sr[r], gl + i * L, nu, w[i][r], nt);
#pragma unroll
        for (int i = 0; i < NUPL; ++i) load_x<TYPE>(xq, xd, xbs, gl + i * L, x[i]);
#pragma unroll
        for (int i = 0; i < NUPL; ++i)
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] += term<TYPE>(w[i][r], x[i], gl + i * L);
    } else {
        for (int u = gl; u < nu; u += L) {
            XUnit<TYPE> x;
            load_x<TYPE>(xq, xd, xbs, u, x);
            WUnit<TYPE> w[R];
#pragma unroll
            for (int r = 0; r < R; ++r) load_unit<TYPE, PACKED>(vr[r], sr[r], u, nu, w[r], nt);
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] += term<TYPE>(w[r], x, u);
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = group_sum<L>(acc[r]);
}

#endif  // EXPERT_UNITS_H
