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
    const int* in_rows;   // nullptr: entry i of a tile is activation row tile_start + i
    const int* out_rows;  // nullptr: entry i writes output row tile_start + i
    long long ldy;        // output row stride
    int T;                // n_tiles == nullptr (dense): T rows of one matrix in tiles of GG_TILE
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

// ---- Pipeline. K runs in stages of GG_KB blocks through one LDS buffer per workgroup (about 25 KB, so several
// workgroups share a CU and hide each other's load latency). All operand bytes move from memory to LDS with
// global_load_lds_dwordx4 (no register staging): lane l of such a load writes its 16 bytes to slot l of a 1 KB
// LDS run, so each load is laid out to be read back as an MFMA operand with one ds_read per lane:
//   weights: per wave and block, lane l loads row (l % 32) of the wave's 32 rows, K half l / 32 (Q8_0), or the
//            block's 16 nibble bytes of that row (FP4 types: the lane decodes its K half from them);
//   activations: per block and 32-entry tile, lane l loads entry (l % 32), K half l / 32;
//   activation scales: one 16-byte load per entry (GG_KB floats).
// The weight rows' scale bytes come through registers.
#define GG_KB 4                          // blocks of 32 values per stage

typedef __attribute__((address_space(3))) void lds_void;

struct GBuf {  // one stage of operands
    uint8_t a[4][GG_KB][1024];  // [wave][block][lane * 16]
    uint8_t b[GG_KB][2][1024];  // [block][entry tile][lane * 16]
    float dx[GG_TILE][GG_KB];   // [entry][block]
};

__device__ __forceinline__ void lds_load16(const void* g, void* lds_run) {
    __builtin_amdgcn_global_load_lds(g, (lds_void*)lds_run, 16, 0, 0);
}

template <int WAITS>
__device__ __forceinline__ void wait_vm() {
    // s_waitcnt vmcnt(WAITS), expcnt and lgkmcnt left at their maxima (gfx9 encoding)
    __builtin_amdgcn_s_waitcnt((WAITS & 0xf) | ((WAITS >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

// Issue one stage's loads into B (see above); the weight scales of the stage go to wsc
template <int TYPE>
__device__ __forceinline__ void g_issue(GBuf& B, int b0, uint4& wsc, const uint8_t* vrow, const uint8_t* srow,
                                        const int8_t* xrow, const float* dxr, int nb, int w, int l, int kh,
                                        int tile_b) {
#pragma unroll
    for (int bb = 0; bb < GG_KB; ++bb) {
        const uint8_t* g = TYPE == QT_Q8_0 ? vrow + 16 * (kh ? nb + b0 + bb : b0 + bb) : vrow + 16 * (b0 + bb);
        lds_load16(g, B.a[w][bb]);
    }
#pragma unroll
    for (int j = 0; j < GG_KB / 2; ++j) {
        const int bb = (w >> 1) + 2 * j;
        lds_load16(xrow + 32 * (b0 + bb), B.b[bb][tile_b]);
    }
    if (l < 16) lds_load16(dxr + b0, &B.dx[16 * w][0]);  // entries 16 w + l (lanes 16.. idle)
    if constexpr (TYPE == QT_ROCMFP4_FAST) {
        wsc = make_uint4(*(const uint32_t*)(srow + b0), 0u, 0u, 0u);
    } else {
        const uint2 v = *(const uint2*)(srow + 2 * b0);
        wsc = make_uint4(v.x, v.y, 0u, 0u);
    }
}

// The MFMAs of one stage from B
template <int TYPE>
__device__ __forceinline__ void g_compute(const GBuf& B, const uint4& wsc, v16f& acc0, v16f& acc1, int w, int l,
                                          int lr, int kh) {
    const v16i zi = {};
#pragma unroll
    for (int bb = 0; bb < GG_KB; ++bb) {
        const float dx0 = B.dx[lr][bb], dx1 = B.dx[32 + lr][bb];
        const uint8_t* arun = B.a[w][bb] + 16 * l;
        if constexpr (TYPE == QT_ROCMFP4) {
            const uint2 q = *(const uint2*)(arun + 8 * kh);  // bytes 8 kh .. 8 kh + 7 of the row's block
            const uint32_t ew = (bb < 2 ? wsc.x : wsc.y) >> (16 * (bb & 1));
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t sh = 4 * h;
                const long A = (long)(((unsigned long)fp4x4_to_i8x4(q.y >> sh) << 32) | fp4x4_to_i8x4(q.x >> sh));
                const float ee = ue4m3_half((ew >> (8 * h)) & 0xffu);
                // B, K half kh of 16-value half h: bytes 16 h + 8 kh of the block = 8 bytes of the slot of the
                // lane that loaded (entry, K half h)
                const long B0 = *(const long*)(B.b[bb][0] + 16 * (lr + 32 * h) + 8 * kh);
                const long B1 = *(const long*)(B.b[bb][1] + 16 * (lr + 32 * h) + 8 * kh);
                acc_block(acc0, __builtin_amdgcn_mfma_i32_32x32x16_i8(A, B0, zi, 0, 0, 0), scale_outer(ee, dx0, kh));
                acc_block(acc1, __builtin_amdgcn_mfma_i32_32x32x16_i8(A, B1, zi, 0, 0, 0), scale_outer(ee, dx1, kh));
            }
        } else {
            const uint4 q = *(const uint4*)arun;
            v4i A;
            float dw;
            if constexpr (TYPE == QT_Q8_0) {
                A = (v4i){(int)q.x, (int)q.y, (int)q.z, (int)q.w};
                dw = h2f((uint16_t)((bb < 2 ? wsc.x : wsc.y) >> (16 * (bb & 1))));
            } else {  // FAST: K half kh = the low (0) or high (1) nibbles of the block's 16 bytes
                const uint32_t sh = kh ? 4 : 0;
                A = (v4i){(int)fp4x4_to_i8x4(q.x >> sh), (int)fp4x4_to_i8x4(q.y >> sh), (int)fp4x4_to_i8x4(q.z >> sh),
                          (int)fp4x4_to_i8x4(q.w >> sh)};
                dw = ue4m3_half((wsc.x >> (8 * bb)) & 0xffu);
            }
            const v4i B0 = *(const v4i*)(B.b[bb][0] + 16 * l);
            const v4i B1 = *(const v4i*)(B.b[bb][1] + 16 * l);
            acc_block(acc0, __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B0, zi, 0, 0, 0), scale_outer(dw, dx0, kh));
            acc_block(acc1, __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B1, zi, 0, 0, 0), scale_outer(dw, dx1, kh));
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

template <int TYPE>
__global__ void __launch_bounds__(256) k_grouped_mfma(GArgs a) {
    __shared__ __attribute__((aligned(1024))) GBuf buf;
    const int k = blockIdx.y;
    int e, st, cnt;
    if (a.n_tiles) {
        if (k >= *a.n_tiles) return;
        e = a.tile_e[k];
        st = a.tile_start[k];
        cnt = __builtin_amdgcn_readfirstlane(a.tile_n[k]);
    } else {  // dense: tile k is rows 64 k .. of the one matrix
        st = k * GG_TILE;
        if (st >= a.T) return;
        e = 0;
        cnt = min(GG_TILE, a.T - st);
    }
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, lr = l & 31, kh = l >> 5;
    auto in_row = [&](int i) { return a.in_rows ? a.in_rows[st + i] : st + i; };
    auto out_row = [&](int i) { return a.out_rows ? a.out_rows[st + i] : st + i; };
    const int K = a.K, nb = K / 32;
    // this lane's weight row (the launcher requires N % 128 == 0 and K % (32 GG_KB) == 0)
    const int r0 = blockIdx.x * GG_ROWS + 32 * w;
    const long long grow = (long long)e * a.N + r0 + lr;
    const uint8_t* vrow = a.v + grow * a.vrb;
    const uint8_t* srow = a.s + grow * a.srb;
    // activation loads: this wave loads blocks (w >> 1) and (w >> 1) + 2 of tile (w & 1), entry 32 (w & 1) + lr
    const int tile_b = w & 1;
    const int8_t* xrow = a.xq + (long long)in_row(min(32 * tile_b + lr, cnt - 1)) * K + 16 * kh;
    // activation scales: this wave's lanes 0..15 load entries 16 w + l
    const float* dxr = a.xd + (long long)in_row(min(16 * w + (l & 15), cnt - 1)) * nb;

    v16f acc0 = {}, acc1 = {};
    const int nst = nb / GG_KB;
    uint4 wsc;
    for (int s = 0; s < nst; ++s) {
        // one stage: its loads, then (with several workgroups per CU hiding the latency of each other's loads)
        // its MFMAs
        g_issue<TYPE>(buf, s * GG_KB, wsc, vrow, srow, xrow, dxr, nb, w, l, kh, tile_b);
        wait_vm<0>();
        __syncthreads();
        g_compute<TYPE>(buf, wsc, acc0, acc1, w, l, lr, kh);
        __syncthreads();
    }
    // acc[j] is C[row 8 (j / 4) + 4 kh + j % 4][entry lr] of the wave's 32 x 32 tile
    if (lr < cnt) {
        float* y = a.y + (long long)out_row(lr) * a.ldy + r0;
#pragma unroll
        for (int j = 0; j < 16; ++j) y[8 * (j >> 2) + 4 * kh + (j & 3)] = acc0[j];
    }
    if (32 + lr < cnt) {
        float* y = a.y + (long long)out_row(32 + lr) * a.ldy + r0;
#pragma unroll
        for (int j = 0; j < 16; ++j) y[8 * (j >> 2) + 4 * kh + (j & 3)] = acc1[j];
    }
}

// ---- Register pipeline (no LDS, no barriers). Every wave loads its own MFMA operands straight from memory
// into the operand registers: lane l holds weight row l % 32 / entry l % 32 and K half l / 32, which is exactly
// one 16-byte half of a Q8_0 block (the split plane keeps the two halves of a row's blocks in two runs), 8 bytes
// of a ROCmFP4 block's nibbles, or a FAST block's 16 bytes. The 4 waves of a workgroup share the activation
// lines through L1. Stage s + 1's loads are issued before stage s's MFMAs, and several waves per SIMD hide the
// rest of the latency.
template <int TYPE, int KB>
struct GStage {
    uint4 a[KB];          // weights: Q8_0 / FAST 16 bytes; ROCmFP4 8 bytes in .x, .y
    uint4 b0[KB], b1[KB];  // entries 0..31 / 32..63: Q8_0 / FAST 16 bytes; ROCmFP4 halves 0 (.x .y), 1 (.z .w)
    float dx0[KB], dx1[KB];
    uint2 ws;             // weight scales of the KB blocks (2 bytes per block; FAST 1 byte per block in .x)
};

template <int TYPE, int KB>
__device__ __forceinline__ void gd_load(GStage<TYPE, KB>& S, int b0, const uint8_t* vrow, const uint8_t* srow,
                                        const int8_t* x0, const int8_t* x1, const float* d0, const float* d1, int nb,
                                        int kh) {
#pragma unroll
    for (int bb = 0; bb < KB; ++bb) {
        const int b = b0 + bb;
        if constexpr (TYPE == QT_Q8_0) {
            S.a[bb] = *(const uint4*)(vrow + 16 * (kh ? nb + b : b));
        } else if constexpr (TYPE == QT_ROCMFP4_FAST) {
            S.a[bb] = *(const uint4*)(vrow + 16 * b);
        } else {
            const uint2 q = *(const uint2*)(vrow + 16 * b + 8 * kh);
            S.a[bb] = make_uint4(q.x, q.y, 0u, 0u);
        }
        if constexpr (TYPE == QT_ROCMFP4) {
            const uint2 p0 = *(const uint2*)(x0 + 32 * b + 8 * kh), q0 = *(const uint2*)(x0 + 32 * b + 16 + 8 * kh);
            const uint2 p1 = *(const uint2*)(x1 + 32 * b + 8 * kh), q1 = *(const uint2*)(x1 + 32 * b + 16 + 8 * kh);
            S.b0[bb] = make_uint4(p0.x, p0.y, q0.x, q0.y);
            S.b1[bb] = make_uint4(p1.x, p1.y, q1.x, q1.y);
        } else {
            S.b0[bb] = *(const uint4*)(x0 + 32 * b + 16 * kh);
            S.b1[bb] = *(const uint4*)(x1 + 32 * b + 16 * kh);
        }
        S.dx0[bb] = d0[b];
        S.dx1[bb] = d1[b];
    }
    if constexpr (TYPE == QT_ROCMFP4_FAST) {
        S.ws = make_uint2(KB == 4 ? *(const uint32_t*)(srow + b0) : (uint32_t) * (const uint16_t*)(srow + b0), 0u);
    } else {
        S.ws = KB == 4 ? *(const uint2*)(srow + 2 * b0) : make_uint2(*(const uint32_t*)(srow + 2 * b0), 0u);
    }
}

template <int TYPE, int KB>
__device__ __forceinline__ void gd_compute(const GStage<TYPE, KB>& S, v16f& acc0, v16f& acc1, int kh) {
    const v16i zi = {};
#pragma unroll
    for (int bb = 0; bb < KB; ++bb) {
        if constexpr (TYPE == QT_ROCMFP4) {
            const uint32_t ew = (bb < 2 ? S.ws.x : S.ws.y) >> (16 * (bb & 1));
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t sh = 4 * h;
                const long A = (long)(((unsigned long)fp4x4_to_i8x4(S.a[bb].y >> sh) << 32) |
                                      fp4x4_to_i8x4(S.a[bb].x >> sh));
                const float ee = ue4m3_half((ew >> (8 * h)) & 0xffu);
                const long B0 = h ? (long)(((unsigned long)S.b0[bb].w << 32) | S.b0[bb].z)
                                  : (long)(((unsigned long)S.b0[bb].y << 32) | S.b0[bb].x);
                const long B1 = h ? (long)(((unsigned long)S.b1[bb].w << 32) | S.b1[bb].z)
                                  : (long)(((unsigned long)S.b1[bb].y << 32) | S.b1[bb].x);
                acc_block(acc0, __builtin_amdgcn_mfma_i32_32x32x16_i8(A, B0, zi, 0, 0, 0),
                          scale_outer(ee, S.dx0[bb], kh));
                acc_block(acc1, __builtin_amdgcn_mfma_i32_32x32x16_i8(A, B1, zi, 0, 0, 0),
                          scale_outer(ee, S.dx1[bb], kh));
            }
        } else {
            const uint4 q = S.a[bb];
            v4i A;
            float dw;
            if constexpr (TYPE == QT_Q8_0) {
                A = (v4i){(int)q.x, (int)q.y, (int)q.z, (int)q.w};
                dw = h2f((uint16_t)((bb < 2 ? S.ws.x : S.ws.y) >> (16 * (bb & 1))));
            } else {
                const uint32_t sh = kh ? 4 : 0;
                A = (v4i){(int)fp4x4_to_i8x4(q.x >> sh), (int)fp4x4_to_i8x4(q.y >> sh), (int)fp4x4_to_i8x4(q.z >> sh),
                          (int)fp4x4_to_i8x4(q.w >> sh)};
                dw = ue4m3_half((S.ws.x >> (8 * bb)) & 0xffu);
            }
            const v4i B0 = {(int)S.b0[bb].x, (int)S.b0[bb].y, (int)S.b0[bb].z, (int)S.b0[bb].w};
            const v4i B1 = {(int)S.b1[bb].x, (int)S.b1[bb].y, (int)S.b1[bb].z, (int)S.b1[bb].w};
            acc_block(acc0, __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B0, zi, 0, 0, 0), scale_outer(dw, S.dx0[bb], kh));
            acc_block(acc1, __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B1, zi, 0, 0, 0), scale_outer(dw, S.dx1[bb], kh));
        }
    }
}

template <int TYPE, int KB>
__global__ void __launch_bounds__(256) k_grouped_direct(GArgs a) {
    const int k = blockIdx.y;
    int e, st, cnt;
    if (a.n_tiles) {
        if (k >= *a.n_tiles) return;
        e = a.tile_e[k];
        st = a.tile_start[k];
        cnt = __builtin_amdgcn_readfirstlane(a.tile_n[k]);
    } else {
        st = k * GG_TILE;
        if (st >= a.T) return;
        e = 0;
        cnt = min(GG_TILE, a.T - st);
    }
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, lr = l & 31, kh = l >> 5;
    auto in_row = [&](int i) { return a.in_rows ? a.in_rows[st + i] : st + i; };
    auto out_row = [&](int i) { return a.out_rows ? a.out_rows[st + i] : st + i; };
    const int K = a.K, nb = K / 32;
    const int r0 = blockIdx.x * GG_ROWS + 32 * w;
    const long long grow = (long long)e * a.N + r0 + lr;
    const uint8_t* vrow = a.v + grow * a.vrb;
    const uint8_t* srow = a.s + grow * a.srb;
    const long long i0 = in_row(min(lr, cnt - 1)), i1 = in_row(min(32 + lr, cnt - 1));
    const int8_t* x0 = a.xq + i0 * K;
    const int8_t* x1 = a.xq + i1 * K;
    const float* d0 = a.xd + i0 * nb;
    const float* d1 = a.xd + i1 * nb;

    v16f acc0 = {}, acc1 = {};
    const int nst = nb / KB;
    GStage<TYPE, KB> cur, nxt;
    gd_load<TYPE, KB>(cur, 0, vrow, srow, x0, x1, d0, d1, nb, kh);
    for (int s = 0; s < nst; ++s) {
        if (s + 1 < nst) gd_load<TYPE, KB>(nxt, (s + 1) * KB, vrow, srow, x0, x1, d0, d1, nb, kh);
        gd_compute<TYPE, KB>(cur, acc0, acc1, kh);
        cur = nxt;
    }
    if (lr < cnt) {
        float* y = a.y + (long long)out_row(lr) * a.ldy + r0;
#pragma unroll
        for (int j = 0; j < 16; ++j) y[8 * (j >> 2) + 4 * kh + (j & 3)] = acc0[j];
    }
    if (32 + lr < cnt) {
        float* y = a.y + (long long)out_row(32 + lr) * a.ldy + r0;
#pragma unroll
        for (int j = 0; j < 16; ++j) y[8 * (j >> 2) + 4 * kh + (j & 3)] = acc1[j];
    }
}

#ifndef GG_DIRECT_KB
#define GG_DIRECT_KB 0  // blocks per register stage of the direct kernel (0: the LDS pipeline)
#endif

template <int TYPE>
static hipError_t launch_grouped_t(const GArgs& a, dim3 g, hipStream_t stream) {
    if constexpr (GG_DIRECT_KB > 0)
        return launch_kernel(k_grouped_direct<TYPE, GG_DIRECT_KB>, g, dim3(256), 0, stream, a);
    else
        return launch_kernel(k_grouped_mfma<TYPE>, g, dim3(256), 0, stream, a);
}

// Whether the MFMA kernel takes this matrix: a split-plane type with Q8_0 activations, whole 128-row blocks and
// whole 4-block K stages
bool moe_grouped_mfma_ok(int type, int N, int K) {
    return (type == QT_Q8_0 || type == QT_ROCMFP4 || type == QT_ROCMFP4_FAST) && N % GG_ROWS == 0 &&
           K % (GG_KB * 32) == 0;
}

hipError_t moe_launch_grouped_mfma(int type, const uint8_t* v, const uint8_t* s, long long vrb, long long srb,
                                   const qmatvec_q8* q, float* y, int N, int K, int max_tiles, const int32_t* n_tiles,
                                   const int32_t* tile_e, const int32_t* tile_start, const int32_t* tile_n,
                                   const int32_t* in_rows, const int32_t* out_rows, hipStream_t stream) {
    GArgs a = {v, s, vrb, srb, q->q0, q->d0, y, N, K, n_tiles, tile_e, tile_start, tile_n, in_rows, out_rows, N, 0};
    const dim3 g((N + GG_ROWS - 1) / GG_ROWS, max_tiles), b(256);
    (void)b;
    switch (type) {
    case QT_Q8_0: return launch_grouped_t<QT_Q8_0>(a, g, stream);
    case QT_ROCMFP4: return launch_grouped_t<QT_ROCMFP4>(a, g, stream);
    case QT_ROCMFP4_FAST: return launch_grouped_t<QT_ROCMFP4_FAST>(a, g, stream);
    }
    return hipErrorInvalidDeviceFunction;
}

// Dense: y[t][0..N) (row stride ldy) = W . x_t for t < T, every token a tile entry of the one matrix
hipError_t moe_launch_dense_mfma(int type, const uint8_t* v, const uint8_t* s, long long vrb, long long srb,
                                 const qmatvec_q8* q, float* y, long long ldy, int N, int K, int T,
                                 hipStream_t stream) {
    GArgs a = {v, s, vrb, srb, q->q0, q->d0, y, N, K, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, ldy, T};
    const dim3 g(N / GG_ROWS, (T + GG_TILE - 1) / GG_TILE), b(256);
    (void)b;
    switch (type) {
    case QT_Q8_0: return launch_grouped_t<QT_Q8_0>(a, g, stream);
    case QT_ROCMFP4: return launch_grouped_t<QT_ROCMFP4>(a, g, stream);
    case QT_ROCMFP4_FAST: return launch_grouped_t<QT_ROCMFP4_FAST>(a, g, stream);
    }
    return hipErrorInvalidDeviceFunction;
}
