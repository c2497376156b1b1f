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

// Four FP4 codes (the low nibble of each byte) -> four int8 codebook values {0,1,2,3,4,6,8,10} with bit 3 the
// sign. v_perm_b32 picks byte (code & 7) of an 8-byte table of magnitudes and of one of negatives; a per-byte
// mask built from bit 3 selects between them.
__device__ __forceinline__ uint32_t fp4x4_to_i8x4(uint32_t n) {
    const uint32_t sel = n & 0x07070707u;
    const uint32_t pos = __builtin_amdgcn_perm(0x0a080604u, 0x03020100u, sel);
    const uint32_t neg = __builtin_amdgcn_perm(0xf6f8fafcu, 0xfdfeff00u, sel);
    const uint32_t sgn = ((n >> 3) & 0x01010101u) * 0xffu;
    return (pos & ~sgn) | (neg & sgn);
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

// Sum over groups of G consecutive lanes of the wave (G a power of two <= 64)
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

#endif  // MOE_COMMON_H
