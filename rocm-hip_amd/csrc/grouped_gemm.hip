// grouped_gemm.hip -- prefill grouped expert GEMM on int8 MFMA (gfx950), over gpu_moe_group's expert tiles.
//
// Tile k (expert e, up to 64 entries) times a 128-row block of e's weights: four waves, each 32 weight rows x
// 64 entries (two 32 x 32 MFMA tiles). Per 32-value block b (one Q8_0 / FAST block, or each 16-value half of a
// ROCmFP4 block):
//   I = A . B on v_mfma_i32_32x32x32_i8 (32x32x16 for a ROCmFP4 half): the exact integer block dots of every
//       (row, entry) pair; A = the weights' int8 codes (Q8_0 values, or FP4 codes decoded in registers), B =
//       the entries' Q8_0 activation values, both straight from memory into the MFMA operand registers (lane l
//       holds row / entry l % 32 and K half l / 32, which is exactly one 16-byte half of a Q8_0 block);
//   S = the outer product of the weight scales (d, or e0 / e1) and the entries' activation scales, on
//       v_mfma_f32_32x32x8f16 (both scales are FP16 values, so every product is exact in fp32);
//   acc += (float)I * S: two VALU operations per output and block.
// Weights are read from the split-plane copy (qmatvec_pack_weights); the output rows are written to
// y[out_rows[entry]][row]. Semantics per output: the reference's int8 expert kernels (src/matvec_q.hip:
// 2749-2901, the integer block dot times the block's two scales, summed over blocks) in another fp32 order.

#include "expert_units.h"
#include "host_common.h"
#include "qmatvec.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

struct GArgs {
    const uint8_t* v;  // value plane of the stacked experts
    const uint8_t* s;  // scale plane
    long long vrb, srb;
    const int8_t* xq;  // Q8_0 activation values, rows of K
    const float* xd;   // Q8_0 activation scales, rows of K / 32
    float* y;
    int N, K;
    const int* n_tiles;
    const int* tile_e;
    const int* tile_start;
    const int* tile_n;
    const int* in_rows;
    const int* out_rows;
};

#define GG_ROWS 128  // weight rows per workgroup (32 per wave)
#define GG_TILE 64   // entries per tile (two 32-entry MFMA tiles)

// S = dw (x) dx as one MFMA: lanes 0..31 put their row's / entry's scale in k = 0, every other k is 0
__device__ __forceinline__ v16f scale_outer(float dw, float dx, int kh) {
    const v4h a = {kh ? (_Float16)0.0f : (_Float16)dw, (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f};
    const v4h b = {kh ? (_Float16)0.0f : (_Float16)dx, (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f};
    const v16f z = {};
    return __builtin_amdgcn_mfma_f32_32x32x8f16(a, b, z, 0, 0, 0);
}

__device__ __forceinline__ void acc_block(v16f& acc, const v16i& I, const v16f& S) {
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = fmaf((float)I[j], S[j], acc[j]);
}

// The A operand (16 int8 codes, K half kh) of a 32-value block for one weight row, and the block's scale(s)
template <int TYPE>
struct BlockA;

template <>
struct BlockA<QT_Q8_0> {
    v4i a;
    float d;
    __device__ __forceinline__ void load(const uint8_t* vrow, const uint8_t* srow, int b, int nb, int kh) {
        a = *(const v4i*)(vrow + 16 * (kh ? nb + b : b));
        d = h2f(*(const uint16_t*)(srow + 2 * b));
    }
};

template <>
struct BlockA<QT_ROCMFP4_FAST> {
    v4i a;
    float d;
    __device__ __forceinline__ void load(const uint8_t* vrow, const uint8_t* srow, int b, int nb, int kh) {
        const uint4 q = *(const uint4*)(vrow + 16 * b);  // values j: low nibble of byte j, j + 16: high nibble
        const uint32_t sh = kh ? 4 : 0;
        a[0] = (int)fp4x4_to_i8x4(q.x >> sh);
        a[1] = (int)fp4x4_to_i8x4(q.y >> sh);
        a[2] = (int)fp4x4_to_i8x4(q.z >> sh);
        a[3] = (int)fp4x4_to_i8x4(q.w >> sh);
        d = ue4m3_half(srow[b]);
    }
};

// ROCmFP4: two 16-value halves with their own scales; K half kh of half h is values 16 h + 8 kh .. + 7, i.e.
// the low (h = 0) or high (h = 1) nibbles of value bytes 8 kh .. 8 kh + 7
struct BlockA4 {
    long a[2];
    float e[2];
    __device__ __forceinline__ void load(const uint8_t* vrow, const uint8_t* srow, int b, int kh) {
        const uint2 q = *(const uint2*)(vrow + 16 * b + 8 * kh);
        const uint32_t lo0 = fp4x4_to_i8x4(q.x), lo1 = fp4x4_to_i8x4(q.y);
        const uint32_t hi0 = fp4x4_to_i8x4(q.x >> 4), hi1 = fp4x4_to_i8x4(q.y >> 4);
        a[0] = (long)(((unsigned long)lo1 << 32) | lo0);
        a[1] = (long)(((unsigned long)hi1 << 32) | hi0);
        const uint32_t ee = *(const uint16_t*)(srow + 2 * b);
        e[0] = ue4m3_half(ee & 0xffu);
        e[1] = ue4m3_half(ee >> 8);
    }
};

template <int TYPE>
__global__ void __launch_bounds__(256) k_grouped_mfma(GArgs a) {
    const int k = blockIdx.y;
    if (k >= *a.n_tiles) return;
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63, lr = l & 31, kh = l >> 5;
    const int r0 = blockIdx.x * GG_ROWS + w * 32;
    if (r0 >= a.N) return;  // (uniform per wave)
    const int e = a.tile_e[k], st = a.tile_start[k], cnt = a.tile_n[k];
    const bool two = cnt > 32;
    const int row = min(r0 + lr, a.N - 1);
    const long long grow = (long long)e * a.N + row;
    const uint8_t* vrow = a.v + grow * a.vrb;
    const uint8_t* srow = a.s + grow * a.srb;
    const int K = a.K, nb = K / 32;
    const long long in0 = a.in_rows[st + min(lr, cnt - 1)], in1 = a.in_rows[st + min(32 + lr, cnt - 1)];
    const int8_t* x0 = a.xq + in0 * K;
    const int8_t* x1 = a.xq + in1 * K;
    const float* d0 = a.xd + in0 * nb;
    const float* d1 = a.xd + in1 * nb;
    v16f acc0 = {}, acc1 = {};
    const v16i zi = {};
    for (int b = 0; b < nb; ++b) {
        if constexpr (TYPE == QT_ROCMFP4) {
            BlockA4 A;
            A.load(vrow, srow, b, kh);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const long b0 = *(const long*)(x0 + 32 * b + 16 * h + 8 * kh);
                const v16i I0 = __builtin_amdgcn_mfma_i32_32x32x16_i8(A.a[h], b0, zi, 0, 0, 0);
                acc_block(acc0, I0, scale_outer(A.e[h], d0[b], kh));
                if (two) {
                    const long b1 = *(const long*)(x1 + 32 * b + 16 * h + 8 * kh);
                    const v16i I1 = __builtin_amdgcn_mfma_i32_32x32x16_i8(A.a[h], b1, zi, 0, 0, 0);
                    acc_block(acc1, I1, scale_outer(A.e[h], d1[b], kh));
                }
            }
        } else {
            BlockA<TYPE> A;
            A.load(vrow, srow, b, nb, kh);
            const v4i b0 = *(const v4i*)(x0 + 32 * b + 16 * kh);
            const v16i I0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A.a, b0, zi, 0, 0, 0);
            acc_block(acc0, I0, scale_outer(A.d, d0[b], kh));
            if (two) {
                const v4i b1 = *(const v4i*)(x1 + 32 * b + 16 * kh);
                const v16i I1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A.a, b1, zi, 0, 0, 0);
                acc_block(acc1, I1, scale_outer(A.d, d1[b], kh));
            }
        }
    }
    // acc[j] is C[row 8 (j / 4) + 4 kh + j % 4][entry lr] of the wave's 32 x 32 tile
    if (lr < cnt) {
        float* y = a.y + (long long)a.out_rows[st + lr] * a.N;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int ri = r0 + 8 * (j >> 2) + 4 * kh + (j & 3);
            if (ri < a.N) y[ri] = acc0[j];
        }
    }
    if (two && 32 + lr < cnt) {
        float* y = a.y + (long long)a.out_rows[st + 32 + lr] * a.N;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int ri = r0 + 8 * (j >> 2) + 4 * kh + (j & 3);
            if (ri < a.N) y[ri] = acc1[j];
        }
    }
}

// Whether the MFMA kernel takes this matrix: a split-plane type with Q8_0 activations
bool moe_grouped_mfma_type(int type) { return type == QT_Q8_0 || type == QT_ROCMFP4 || type == QT_ROCMFP4_FAST; }

hipError_t moe_launch_grouped_mfma(int type, const uint8_t* v, const uint8_t* s, long long vrb, long long srb,
                                   const qmatvec_q8* q, float* y, int N, int K, int max_tiles, const int32_t* n_tiles,
                                   const int32_t* tile_e, const int32_t* tile_start, const int32_t* tile_n,
                                   const int32_t* in_rows, const int32_t* out_rows, hipStream_t stream) {
    GArgs a = {v, s, vrb, srb, q->q0, q->d0, y, N, K, n_tiles, tile_e, tile_start, tile_n, in_rows, out_rows};
    const dim3 g((N + GG_ROWS - 1) / GG_ROWS, max_tiles), b(256);
    switch (type) {
    case QT_Q8_0: return launch_kernel(k_grouped_mfma<QT_Q8_0>, g, b, 0, stream, a);
    case QT_ROCMFP4: return launch_kernel(k_grouped_mfma<QT_ROCMFP4>, g, b, 0, stream, a);
    case QT_ROCMFP4_FAST: return launch_kernel(k_grouped_mfma<QT_ROCMFP4_FAST>, g, b, 0, stream, a);
    }
    return hipErrorInvalidDeviceFunction;
}
