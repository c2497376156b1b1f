// grouped_gemm.hip -- prefill grouped expert GEMM on int8 MFMA (gfx950), over gpu_moe_group's expert tiles.
//
// Tile k (expert e, up to GG_TILE entries) times a 128-row block of e's weights: four waves, each 32 weight rows x
// GG_TILE entries (GG_TILE / 32 MFMA tiles of 32 x 32). Per 32-value block b (one Q8_0 / FAST block, or each
// 16-value half of a ROCmFP4 block):
//   I = A . B on v_mfma_i32_32x32x32_i8 (32x32x16 for a ROCmFP4 half): the exact integer block dots of every
//       (row, entry) pair; A = the weights' int8 codes (Q8_0 values, or FP4 codes decoded in registers), B =
//       the entries' Q8_0 activation values (lane l holds row / entry l % 32 and K half l / 32, which is exactly
//       one 16-byte half of a Q8_0 block);
//   S = the outer product of the weight scales (d, or e0 / e1) and the entries' activation scales, on
//       v_mfma_f32_32x32x8f16 (both scales are FP16 values, so every product is exact in fp32);
//   acc += (float)I * S: two VALU operations per output and block.
// Weights are read from the split-plane copy (qmatvec_pack_weights); the output rows are written to
// y[out_rows[entry]][row]. Semantics per output: the reference's int8 expert kernels (src/matvec_q.hip:
// 2749-2901, the integer block dot times the block's two scales, summed over blocks) in another fp32 order.
//
// Measured at config 2 (2,427 tokens, gate: 221 us with 4-block stages, 205 us with 8): each workgroup waits
// ~3x longer for its stage's operands than it computes. Not the fix, each measured: dropping the fp32 epilogue
// (-6%), dropping the scale MFMA (0%), double-buffered stages (0%), an XCD-aware tile order (HBM fetch -40%,
// time +5%), 128-entry tiles (weight traffic halved, +4%), register-direct operands without LDS (+50%).
// 8-block stages read whole 128-byte lines per row and K half.

#include "expert_units.h"
#include "host_common.h"
#include "qmatvec.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

struct GArgs {
    const uint8_t* v;  // value tiles of the stacked experts' first 32-row group (MFMA operand tiles)
    const uint8_t* s;  // scale tiles
    long long vrb, srb;  // bytes of value / scale tiles per 32-row group
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
    const uint8_t* v2;    // the up matrix's tiles (gate / up / SwiGLU kernel)
    const uint8_t* s2;
    int8_t* aq;           // SwiGLU kernel: down's Q8_0 input, rows of N values (out_rows), and scales
    float* ad;
    int xt;               // GX_IN: the input activations are in entry-tile order (below) instead of rows;
                          // GX_OUT: the SwiGLU kernel writes down's input in entry-tile order
};
#define GX_IN 1
#define GX_OUT 2

// Entry-tile order of a Q8_0 activation matrix of K values per entry: tile k's values at xq + k * GG_TILE * K, in
// 1 KB chunks (block b, 32-entry sub-tile t) at ((b * GG_NT + t) * 1024; slot l (16 bytes) of a chunk holds entry
// 32 t + l % 32, values 16 (l / 32) .. + 15 of the block: one contiguous run per 64-lane MFMA operand load. The
// scales are rows: entry i of tile k at xd + (k * GG_TILE + i) * K / 32.

#define GG_ROWS 128  // weight rows per workgroup (32 per wave)
#ifndef GG_TILE
#define GG_TILE 64  // entries per tile (64 or 128: two or four 32-entry MFMA tiles per wave)
#endif
#ifndef GG_KB
#define GG_KB 8  // blocks of 32 values per stage (4 or 8)
#endif
#ifndef GG_KB2
#define GG_KB2 4  // the same for the gate / up / SwiGLU kernel (two matrices per stage)
#endif
#define GG_NT (GG_TILE / 32)

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

// ---- Pipeline. K runs in stages of GG_KB blocks through one LDS buffer per workgroup. All operand bytes move
// from memory to LDS with global_load_lds_dwordx4 (no register staging): lane l of such a load writes its 16
// bytes to slot l of a 1 KB LDS run, so each load is laid out to be read back as an MFMA operand with one ds_read
// per lane:
//   weights: per wave and block, lane l loads row (l % 32) of the wave's 32 rows, K half l / 32 (Q8_0), or the
//            block's 16 nibble bytes of that row (FP4 types: the lane decodes its K half from them);
//   activations: per block and 32-entry tile, lane l loads entry (l % 32), K half l / 32;
//   activation scales: 16-byte loads of 4 blocks per entry.
// The weight rows' scale bytes come through registers.
typedef __attribute__((address_space(3))) void lds_void;

// Weight chunks of 1 KB per stage of KB blocks: one per block (Q8_0), one per block pair (FP4 types)
template <int TYPE, int KB>
struct GChunks {
    static constexpr int PER = TYPE == QT_Q8_0 ? 1 : 2;
    static constexpr int N = KB / PER;
};

template <int TYPE, int NM, int KB>
struct GBuf {  // one stage of operands of NM weight matrices sharing the activations
    uint8_t a[NM][4][GChunks<TYPE, KB>::N][1024];  // [matrix][wave][chunk][lane * 16]
    uint8_t b[KB][GG_NT][1024];     // [block][entry tile][lane * 16]
    float dx[KB / 4][GG_TILE][4];   // [block / 4][entry][block % 4]
};

__device__ __forceinline__ void lds_load16(const void* g, void* lds_run) {
    __builtin_amdgcn_global_load_lds(g, (lds_void*)lds_run, 16, 0, 0);
}

template <int WAITS>
__device__ __forceinline__ void wait_vm() {
    // s_waitcnt vmcnt(WAITS), expcnt and lgkmcnt left at their maxima (gfx9 encoding)
    __builtin_amdgcn_s_waitcnt((WAITS & 0xf) | ((WAITS >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

// Issue one stage's loads into B (see above); the weight scales of the stage go to wsc. Wave w loads the
// activations of entry tile w % GG_NT, blocks w / GG_NT, + 4 / GG_NT, ... (xrow: its lane's entry row), and the
// scales of entries GG_TILE / 4 w .. (dxr: its lane's entry row)
template <int TYPE, int NM, int KB>
__device__ __forceinline__ void g_issue(GBuf<TYPE, NM, KB>& B, int b0, uint4 (&wsc)[NM],
                                        const uint8_t* const (&vt)[NM], const uint8_t* const (&st)[NM],
                                        const int8_t* xrow, int xs, const float* dxr, int w, int l) {
    constexpr int ES = GG_TILE / 4;  // entries whose scales one wave loads
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int c = 0; c < GChunks<TYPE, KB>::N; ++c)  // contiguous 1 KB chunks: one per block, or block pair
            lds_load16(vt[m] + 1024 * (b0 / GChunks<TYPE, KB>::PER + c), B.a[m][w][c]);
#pragma unroll
    for (int j = 0; j < KB * GG_NT / 4; ++j) {
        const int bb = w / GG_NT + (4 / GG_NT) * j;
        lds_load16(xrow + xs * (b0 + bb), B.b[bb][w % GG_NT]);
    }
#pragma unroll
    for (int q = 0; q < KB / 4; ++q)
        if (l < ES) lds_load16(dxr + b0 + 4 * q, &B.dx[q][ES * w][0]);  // (lanes ES.. idle)
#pragma unroll
    for (int m = 0; m < NM; ++m) {  // the lane's row's slot of the stage's 8-block scale group
        if constexpr (TYPE == QT_ROCMFP4_FAST) {  // 1 scale byte per block, 8-byte slots
            const uint8_t* g = st[m] + 256 * (b0 >> 3);
            if constexpr (KB == 4)
                wsc[m] = make_uint4(*(const uint32_t*)(g + 4 * ((b0 >> 2) & 1)), 0u, 0u, 0u);
            else
                wsc[m] = make_uint4(((const uint2*)g)->x, ((const uint2*)g)->y, 0u, 0u);
        } else {  // 2 scale bytes per block, 16-byte slots
            const uint8_t* g = st[m] + 512 * (b0 >> 3);
            if constexpr (KB == 4) {
                const uint2 v = *(const uint2*)(g + 8 * ((b0 >> 2) & 1));
                wsc[m] = make_uint4(v.x, v.y, 0u, 0u);
            } else {
                wsc[m] = *(const uint4*)g;
            }
        }
    }
}

// The MFMAs of one stage from B
template <int TYPE, int NM, int KB>
__device__ __forceinline__ void g_compute(const GBuf<TYPE, NM, KB>& B, const uint4 (&wsc)[NM], v16f (&acc)[NM][GG_NT], int w,
                                          int l, int lr, int kh) {
    const v16i zi = {};
#pragma unroll
    for (int bb = 0; bb < KB; ++bb) {
        float dx[GG_NT];
#pragma unroll
        for (int t = 0; t < GG_NT; ++t) dx[t] = B.dx[bb >> 2][32 * t + lr][bb & 3];
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            const uint32_t w2 = bb < 2 ? wsc[m].x : bb < 4 ? wsc[m].y : bb < 6 ? wsc[m].z : wsc[m].w;  // 2-byte
            const uint32_t w1 = bb < 4 ? wsc[m].x : wsc[m].y;                                        // 1-byte
            // the lane's slot: 16 bytes of block bb (Q8_0), or 8 bytes of block bb in its pair's slot (FP4 types)
            const uint8_t* arun = TYPE == QT_Q8_0 ? B.a[m][w][bb] + 16 * l : B.a[m][w][bb >> 1] + 16 * l + 8 * (bb & 1);
            if constexpr (TYPE == QT_ROCMFP4) {
                const uint2 q = *(const uint2*)arun;  // nibble bytes 8 kh .. 8 kh + 7 of the row's block
                const uint32_t ew = w2 >> (16 * (bb & 1));
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t sh = 4 * h;
                    const long A =
                        (long)(((unsigned long)fp4x4_to_i8x4(q.y >> sh) << 32) | fp4x4_to_i8x4(q.x >> sh));
                    const float ee = ue4m3_half((ew >> (8 * h)) & 0xffu);
                    // B, K half kh of 16-value half h: bytes 16 h + 8 kh of the block = 8 bytes of the slot of the
                    // lane that loaded (entry, K half h)
#pragma unroll
                    for (int t = 0; t < GG_NT; ++t) {
                        const long Bt = *(const long*)(B.b[bb][t] + 16 * (lr + 32 * h) + 8 * kh);
                        acc_block(acc[m][t], __builtin_amdgcn_mfma_i32_32x32x16_i8(A, Bt, zi, 0, 0, 0),
                                  scale_outer(ee, dx[t], kh));
                    }
                }
            } else {
                v4i A;
                float dw;
                if constexpr (TYPE == QT_Q8_0) {
                    const uint4 q = *(const uint4*)arun;
                    A = (v4i){(int)q.x, (int)q.y, (int)q.z, (int)q.w};
                    dw = h2f((uint16_t)(w2 >> (16 * (bb & 1))));
                } else {  // FAST: K half kh's 16 values, value i and i + 8 in byte i's low and high nibble
                    const uint2 q = *(const uint2*)arun;
                    A = (v4i){(int)fp4x4_to_i8x4(q.x), (int)fp4x4_to_i8x4(q.y), (int)fp4x4_to_i8x4(q.x >> 4),
                              (int)fp4x4_to_i8x4(q.y >> 4)};
                    dw = ue4m3_half((w1 >> (8 * (bb & 3))) & 0xffu);
                }
#pragma unroll
                for (int t = 0; t < GG_NT; ++t) {
                    const v4i Bt = *(const v4i*)(B.b[bb][t] + 16 * l);
                    acc_block(acc[m][t], __builtin_amdgcn_mfma_i32_32x32x32_i8(A, Bt, zi, 0, 0, 0),
                              scale_outer(dw, dx[t], kh));
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// NM = 1: y rows (fp32) of one matrix. NM = 2, SwiGLU: gate (a.v) and up (a.v2) rows of the same block, then
// act = SiLU(g) u (the swiglu kernel's expression) and its Q8_0 blocks -- a wave's 32 rows of one entry are one
// block: 16 values in each of lanes l and l + 32 -- into a.aq / a.ad (the quantizer's expressions).
template <int TYPE, int NM, int KB>
__global__ void __launch_bounds__(256) k_grouped(GArgs a) {
    __shared__ __attribute__((aligned(1024))) GBuf<TYPE, NM, KB> buf;
    const int k = blockIdx.y;
    int e, st, cnt;
    if (a.n_tiles) {
        if (k >= *a.n_tiles) return;
        e = a.tile_e[k];
        st = a.tile_start[k];
        cnt = __builtin_amdgcn_readfirstlane(a.tile_n[k]);
    } else {  // dense: tile k is rows GG_TILE k .. of the one matrix
        st = k * GG_TILE;
        if (st >= a.T) return;
        e = 0;
        cnt = min(GG_TILE, a.T - st);
    }
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, lr = l & 31, kh = l >> 5;
    auto in_row = [&](int i) { return a.in_rows ? a.in_rows[st + i] : st + i; };
    auto out_row = [&](int i) { return a.out_rows ? a.out_rows[st + i] : st + i; };
    const int K = a.K, nb = K / 32;
    // the wave's 32-row group of the stacked matrix (the launcher requires N % 128 == 0 and K % 256 == 0) and
    // this lane's slots in its value and scale tiles
    const int r0 = blockIdx.x * GG_ROWS + 32 * w;
    const long long grp = ((long long)e * a.N + r0) / 32;
    constexpr int SB = TYPE == QT_ROCMFP4_FAST ? 8 : 16;
    const uint8_t* vt[NM];
    const uint8_t* sct[NM];
    vt[0] = a.v + grp * a.vrb + 16 * l;
    sct[0] = a.s + grp * a.srb + SB * lr;
    if constexpr (NM == 2) {
        vt[1] = a.v2 + grp * a.vrb + 16 * l;
        sct[1] = a.s2 + grp * a.srb + SB * lr;
    }
    // the entry rows this lane loads: activations of entry 32 (w % GG_NT) + lr, scales of entry GG_TILE / 4 w + l
    const int de = min(GG_TILE / 4 * w + (l & (GG_TILE / 4 - 1)), cnt - 1);  // the entry whose scales this lane loads
    const int8_t* xrow;
    const float* dxr;
    int xs;  // bytes from one block's operand run to the next
    if (a.xt & GX_IN) {
        xrow = a.xq + ((long long)k * nb * GG_NT + w % GG_NT) * 1024 + 16 * l;
        xs = GG_NT * 1024;
        dxr = a.xd + ((long long)k * GG_TILE + de) * nb;
    } else {
        xrow = a.xq + (long long)in_row(min(32 * (w % GG_NT) + lr, cnt - 1)) * K + 16 * kh;
        xs = 32;
        dxr = a.xd + (long long)in_row(de) * nb;
    }

    v16f acc[NM][GG_NT];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int t = 0; t < GG_NT; ++t) acc[m][t] = (v16f){};
    const int nst = nb / KB;
    uint4 wsc[NM];
    for (int s = 0; s < nst; ++s) {
        // one stage: its loads, then (with several workgroups per CU hiding the latency of each other's loads)
        // its MFMAs
        g_issue<TYPE, NM, KB>(buf, s * KB, wsc, vt, sct, xrow, xs, dxr, w, l);
        wait_vm<0>();
        __syncthreads();
        g_compute<TYPE, NM, KB>(buf, wsc, acc, w, l, lr, kh);
        __syncthreads();
    }
    // acc[m][t][j] is C[row 8 (j / 4) + 4 kh + j % 4][entry 32 t + lr] of the wave's 32 x GG_TILE block
    if constexpr (NM == 1) {
#pragma unroll
        for (int t = 0; t < GG_NT; ++t)
            if (32 * t + lr < cnt) {
                float* y = a.y + (long long)out_row(32 * t + lr) * a.ldy + r0;
#pragma unroll
                for (int j = 0; j < 16; ++j) y[8 * (j >> 2) + 4 * kh + (j & 3)] = acc[0][t][j];
            }
    } else {
#pragma unroll
        for (int t = 0; t < GG_NT; ++t) {
            float act[16];
            float am = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const float g = acc[0][t][j];
                act[j] = g / (1.0f + __expf(-g)) * acc[1][t][j];
                am = fmaxf(am, fabsf(act[j]));
            }
            am = fmaxf(am, __shfl_xor(am, 32, 64));  // the block's other 16 rows
            const float id = am != 0.0f ? 127.0f / am : 0.0f;
            if (32 * t + lr < cnt) {
                // entry-tile order: block r0 / 32 of entry 32 t + lr; else the entry's output row
                const bool xo = a.xt & GX_OUT;
                const long long pr = xo ? (long long)k * GG_TILE + 32 * t + lr : out_row(32 * t + lr);
                int8_t* q = xo ? a.aq + (((long long)k * (a.N / 32) + r0 / 32) * GG_NT + t) * 1024 + 16 * lr
                                 : a.aq + pr * a.N + r0;
#pragma unroll
                for (int m4 = 0; m4 < 4; ++m4) {  // rows 8 m4 + 4 kh .. + 3: four consecutive bytes
                    uint32_t pk = 0;
#pragma unroll
                    for (int c = 0; c < 4; ++c) pk |= ((uint32_t)(int)rintf(act[4 * m4 + c] * id) & 0xffu) << (8 * c);
                    const int row = 8 * m4 + 4 * kh;  // of the block: K half row / 16, byte row % 16 of it
                    *(uint32_t*)(q + (xo ? 512 * (row >> 4) + (row & 15) : row)) = pk;
                }
                if (kh == 0) a.ad[pr * (a.N / 32) + r0 / 32] = __half2float(__float2half(am / 127.0f));
            }
        }
    }
}

// Whether the MFMA kernels take this matrix: a split-plane type with Q8_0 activations, whole 128-row blocks and
// whole K stages (of either kernel)
bool moe_grouped_mfma_ok(int type, int N, int K) {
    return (type == QT_Q8_0 || type == QT_ROCMFP4 || type == QT_ROCMFP4_FAST) && N % GG_ROWS == 0 &&
           K % (GG_KB * 32) == 0 && K % (GG_KB2 * 32) == 0;
}

// The entry tile the MFMA kernel takes
int moe_grouped_mfma_tile(void) { return GG_TILE; }

hipError_t moe_launch_grouped_mfma(int type, const uint8_t* v, const uint8_t* s, long long vrb, long long srb,
                                   const qmatvec_q8* q, float* y, int N, int K, int max_tiles, const int32_t* n_tiles,
                                   const int32_t* tile_e, const int32_t* tile_start, const int32_t* tile_n,
                                   const int32_t* in_rows, const int32_t* out_rows, int xt, hipStream_t stream) {
    GArgs a = {v,      s,       vrb,      srb, q->q0, q->d0, y,       N,       K,       n_tiles, tile_e,
               tile_start, tile_n, in_rows, out_rows, N, 0, nullptr, nullptr, nullptr, nullptr, xt};
    const dim3 g(N / GG_ROWS, max_tiles), b(256);
    switch (type) {
    case QT_Q8_0: return launch_kernel(k_grouped<QT_Q8_0, 1, GG_KB>, g, b, 0, stream, a);
    case QT_ROCMFP4: return launch_kernel(k_grouped<QT_ROCMFP4, 1, GG_KB>, g, b, 0, stream, a);
    case QT_ROCMFP4_FAST: return launch_kernel(k_grouped<QT_ROCMFP4_FAST, 1, GG_KB>, g, b, 0, stream, a);
    }
    return hipErrorInvalidDeviceFunction;
}

// Gate and up of the same tiles in one launch, then SwiGLU and down's Q8_0 input (aq rows of N, ad per 32; in
// entry-tile order with xt = GX_OUT) instead of the gate / up outputs. xt: GX_IN / GX_OUT flags (GArgs::xt)
hipError_t moe_launch_grouped_swiglu(int type, const uint8_t* vg, const uint8_t* sg, const uint8_t* vu,
                                     const uint8_t* su, long long vrb, long long srb, const qmatvec_q8* q, int8_t* aq,
                                     float* ad, int N, int K, int max_tiles, const int32_t* n_tiles,
                                     const int32_t* tile_e, const int32_t* tile_start, const int32_t* tile_n,
                                     const int32_t* in_rows, const int32_t* out_rows, int xt, hipStream_t stream) {
    GArgs a = {vg,         sg,     vrb,     srb,      q->q0, q->d0, nullptr, N,  K,  n_tiles, tile_e,
               tile_start, tile_n, in_rows, out_rows, N,     0,     vu,      su, aq, ad, xt};
    const dim3 g(N / GG_ROWS, max_tiles), b(256);
    switch (type) {
    case QT_Q8_0: return launch_kernel(k_grouped<QT_Q8_0, 2, GG_KB2>, g, b, 0, stream, a);
    case QT_ROCMFP4: return launch_kernel(k_grouped<QT_ROCMFP4, 2, GG_KB2>, g, b, 0, stream, a);
    case QT_ROCMFP4_FAST: return launch_kernel(k_grouped<QT_ROCMFP4_FAST, 2, GG_KB2>, g, b, 0, stream, a);
    }
    return hipErrorInvalidDeviceFunction;
}

// Dense: y[t][0..N) (row stride ldy) = W . x_t for t < T, every token a tile entry of the one matrix
hipError_t moe_launch_dense_mfma(int type, const uint8_t* v, const uint8_t* s, long long vrb, long long srb,
                                 const qmatvec_q8* q, float* y, long long ldy, int N, int K, int T,
                                 hipStream_t stream) {
    GArgs a = {v,       s,       vrb,     srb,     q->q0, q->d0, y,       N,       K,       nullptr, nullptr,
               nullptr, nullptr, nullptr, nullptr, ldy,   T,     nullptr, nullptr, nullptr, nullptr, 0};
    const dim3 g(N / GG_ROWS, (T + GG_TILE - 1) / GG_TILE), b(256);
    switch (type) {
    case QT_Q8_0: return launch_kernel(k_grouped<QT_Q8_0, 1, GG_KB>, g, b, 0, stream, a);
    case QT_ROCMFP4: return launch_kernel(k_grouped<QT_ROCMFP4, 1, GG_KB>, g, b, 0, stream, a);
    case QT_ROCMFP4_FAST: return launch_kernel(k_grouped<QT_ROCMFP4_FAST, 1, GG_KB>, g, b, 0, stream, a);
    }
    return hipErrorInvalidDeviceFunction;
}
