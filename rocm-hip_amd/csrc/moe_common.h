// moe_common.h -- device helpers shared by the MoE kernels (gfx950, wave64).
//
// Block formats (ggml type ids): Q8_0 (8) 34-byte blocks of 32 values: FP16 d, int8 qs[32].
// Q4_K (12) 144-byte super-blocks of 256 values: FP16 d, FP16 dmin, 12 bytes of 6-bit scales/mins for eight
// sub-blocks of 32, 128 bytes of nibbles (value 64c + l is the low nibble of byte 32c + l, 64c + 32 + l the
// high one). ROCmFP4 (100) 18-byte blocks: 16 nibble bytes (value j low nibble of byte j, j + 16 high), then
// two UE4M3 half-scales (values 0..15, 16..31). ROCmFP4_FAST (101) 17 bytes: the same with one scale.
// Layouts as the reference's decoders read them (src/quant_types.cpp:182-189, 265-287, 349-381).
#ifndef MOE_COMMON_H
#define MOE_COMMON_H

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#define QT_F32 0
#define QT_Q8_0 8
#define QT_Q4_K 12
#define QT_ROCMFP4 100
#define QT_ROCMFP4_FAST 101

// Activation outputs of the quantizing kernels (the field order of qmatvec_q8_out): Q8_0 values / FP16-rounded
// scales / Q8_1 sums (float bits), Q8_K values / scales / sums of 16. qK == nullptr: no int8 output.
struct Q8Out {
    int8_t* q0;
    float* d0;
    int8_t* qK;
    float* dK;
    int32_t* bsK;
    int32_t* s0;
    uint16_t* xh;
    int xh_bf16;
};

// A 16-byte load of the router rows and the shared expert's gate vector, a nontemporal load when RT_NT is set. Off:
// measured slower (config 1 decode 16.7 -> 17.1 us): with the expert weights streamed by nontemporal loads the
// router matrices stay in the caches from one token to the next, as they should.
#ifndef RT_NT
#define RT_NT 0
#endif
typedef float mc_v4f __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_w4(const float4* p) {
#if RT_NT
    const mc_v4f v = __builtin_nontemporal_load((const mc_v4f*)p);
    return make_float4(v.x, v.y, v.z, v.w);
#else
    return *p;
#endif
}

// p[i] for a run-time i of a kernel-argument array, as a chain of selects over its elements (which arrive with the
// other arguments in scalar registers). Indexing the array itself becomes a vector load from the argument segment:
// one more memory round trip ahead of every load whose address depends on it.
template <int N, typename T>
__device__ __forceinline__ T pick(const T (&p)[N], int i) {
    T r = p[0];
#pragma unroll
    for (int k = 1; k < N; ++k) r = i == k ? p[k] : r;
    return r;
}

// A value every lane of the wave holds, moved to a scalar register: an index into the kernel's plane pointers made
// wave-uniform this way is chosen by scalar selects or a scalar load of the argument, where a per-lane index had
// compiled to a vector load from the kernel-argument segment ahead of every weight load
__device__ __forceinline__ int wave_uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// pick for pointers where the optimizer folds pick's selects back into such a load (it did where i depends on a
// value read from LDS, in the multi-token kernels): every element first passes, unconditionally, through an
// empty asm statement that keeps it in scalar registers. (Not the default: it costs the T = 1 kernels ~0.7 µs.)
template <int N, typename T>
__device__ __forceinline__ T* pick_opaque(T* const (&p)[N], int i) {
    T* q[N];
#pragma unroll
    for (int k = 0; k < N; ++k) {
        uint64_t v = (uint64_t)p[k];
        asm("" : "+s"(v));
        q[k] = (T*)(__attribute__((address_space(1))) T*)v;  // (a global pointer again: global, not flat, loads)
    }
    T* r = q[0];
#pragma unroll
    for (int k = 1; k < N; ++k) r = i == k ? q[k] : r;
    return r;
}

__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }

// UE4M3 scale byte at half scale: (8 + m) 2^(e - 11), subnormals m 2^-10, 0x7f and above 0
// (src/quant_types.cpp:352-357). Built from the exponent bits directly: exact.
__device__ __forceinline__ float ue4m3_half(uint32_t e) {
    const uint32_t ex = (e >> 3) & 15u, m = e & 7u;
    const float normal = __uint_as_float(((ex + 119u) << 23) | (m << 20));  // (1 + m/8) 2^(ex - 8)
    const float sub = (float)m * 0x1p-10f;
    return e >= 0x7fu ? 0.0f : (ex == 0 ? sub : normal);
}

// Signed int8 dot of four bytes, accumulated (v_dot4_i32_i8)
__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// Four FP4 codes (the low nibble of each byte) -> four int8 codebook values (Codebook10: nibbles 0..7 ->
// +{0, 1, 2, 3, 4, 6, 8, 10}, 8..15 their negatives; src/fp4_common.h:29-33) as the XOR of two v_perm_b32 table
// lookups. v_perm_b32 maps a selector byte c < 8 to byte c of its 8-byte table, 8..11 to 0x00 / 0xFF by the sign
// bit of table byte 1 / 3 / 5 / 7, 12 to 0x00 and 13..15 to 0xFF. A = perm(TA, c) and B = perm(TB, c ^ 8) thus give
// table bytes for c < 8 (A) and c >= 8 (B) and a 0x00 / 0xFF byte from the other table's signs; FP4_TA / FP4_TB are
// the one pair of tables (an exhaustive search over the eight sign bits those selectors read) with A ^ B the
// codebook value for all 16 codes. Five operations per four codes, where a magnitude and a negative lookup and a
// third, sign-selecting v_perm_b32 took seven.
#define FP4_TA_HI 0xf5f7f904u  // table bytes 4..7
#define FP4_TA_LO 0x030201ffu  // table bytes 0..3
#define FP4_TB_HI 0x090705fcu
#define FP4_TB_LO 0x0201ff00u
__device__ __forceinline__ uint32_t fp4x4_to_i8x4(uint32_t n) {
    const uint32_t c = n & 0x0f0f0f0fu;
    return __builtin_amdgcn_perm(FP4_TA_HI, FP4_TA_LO, c) ^ __builtin_amdgcn_perm(FP4_TB_HI, FP4_TB_LO, c ^ 0x08080808u);
}

// Twice the UE4M3 half-scale value of byte SEL of s (ue4m3_half's value times 2): the byte read as an OCP FP8 E4M3
// value by gfx950's converter (exact for every byte; (8 + m) 2^(e - 10) normal, m 2^-9 subnormal, as the half
// scale's (8 + m) 2^(e - 11) and m 2^-10 doubled), and 0 for the bytes 0x7f and above, which the converter reads
// as NaN or negative. The kernels fold the 1/2 into the activation scale, an exact factor, so that e dx is formed
// bit for bit as before. Three operations where the bit assembly took about eight.
template <int SEL>
__device__ __forceinline__ float ue4m3_x2(uint32_t s) {
    const float c = __builtin_amdgcn_cvt_f32_fp8((int)s, SEL);
    return c > 0.0f ? c : 0.0f;
}

// Q4_K 6-bit scale / min of sub-block j from the 12 scale bytes held as three dwords s[0..2]
// (src/quant_types.cpp:193-202)
__device__ __forceinline__ uint32_t sbyte(const uint32_t s[3], int i) { return (s[i >> 2] >> (8 * (i & 3))) & 0xffu; }
__device__ __forceinline__ void q4k_scale_min(int j, const uint32_t s[3], int& sc, int& mn) {
    if (j < 4) {
        sc = (int)(sbyte(s, j) & 63u);
        mn = (int)(sbyte(s, j + 4) & 63u);
    } else {
        sc = (int)((sbyte(s, j + 4) & 15u) | ((sbyte(s, j - 4) >> 6) << 4));
        mn = (int)((sbyte(s, j + 4) >> 4) | ((sbyte(s, j) >> 6) << 4));
    }
}

// Cross-lane moves inside a row of 16 lanes (DPP): quad_perm [1,0,3,2] (0xB1), quad_perm [2,3,0,1] (0x4E),
// row_half_mirror (0x141), row_mirror (0x140). After the xor-1 and xor-2 steps every lane of a quad holds the
// quad's value, so the two mirrors combine halves and rows: group sums of 2, 4, 8 and 16 lanes, in every lane.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, false);
}
// Lane l <- lane l ^ 16 within each half-wave (ds_swizzle, bit mode: and 0x1f, xor 0x10)
__device__ __forceinline__ float swz_xor16(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401f));
}

// Sum over groups of G consecutive lanes (G a power of two <= 64); every lane of a group gets the group's sum
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (G >= 2) v += dpp_f<0xb1>(v);
    if constexpr (G >= 4) v += dpp_f<0x4e>(v);
    if constexpr (G >= 8) v += dpp_f<0x141>(v);
    if constexpr (G >= 16) v += dpp_f<0x140>(v);
    if constexpr (G >= 32) v += swz_xor16(v);
    if constexpr (G >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

template <int G>
__device__ __forceinline__ float group_max(float v) {
    if constexpr (G >= 2) v = fmaxf(v, dpp_f<0xb1>(v));
    if constexpr (G >= 4) v = fmaxf(v, dpp_f<0x4e>(v));
    if constexpr (G >= 8) v = fmaxf(v, dpp_f<0x141>(v));
    if constexpr (G >= 16) v = fmaxf(v, dpp_f<0x140>(v));
    if constexpr (G >= 32) v = fmaxf(v, swz_xor16(v));
    if constexpr (G >= 64) v = fmaxf(v, __shfl_xor(v, 32, 64));
    return v;
}

// The value a reduction step of width S (1, 2, 4, 8, 16, 32) pairs this lane with: after the steps below S,
// every lane of an S-lane group holds that group's value, so combining with the partner widens it to 2S.
template <int S>
__device__ __forceinline__ int partner_i(int v) {
    if constexpr (S == 1) return dpp_i<0xb1>(v);
    if constexpr (S == 2) return dpp_i<0x4e>(v);
    if constexpr (S == 4) return dpp_i<0x141>(v);
    if constexpr (S == 8) return dpp_i<0x140>(v);
    if constexpr (S == 16) return __builtin_amdgcn_ds_swizzle(v, 0x401f);
    if constexpr (S == 32) return __shfl_xor(v, 32, 64);
    return v;
}
template <int S>
__device__ __forceinline__ float partner_f(float v) {
    return __int_as_float(partner_i<S>(__float_as_int(v)));
}

template <int G>
__device__ __forceinline__ int group_sum_i(int v) {
    if constexpr (G >= 2) v += partner_i<1>(v);
    if constexpr (G >= 4) v += partner_i<2>(v);
    if constexpr (G >= 8) v += partner_i<4>(v);
    if constexpr (G >= 16) v += partner_i<8>(v);
    if constexpr (G >= 32) v += partner_i<16>(v);
    if constexpr (G >= 64) v += partner_i<32>(v);
    return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }
__device__ __forceinline__ float wave_max(float v) { return group_max<64>(v); }

#endif  // MOE_COMMON_H
