// grouped_gemm.hip -- prefill grouped expert GEMM on MFMA (gfx950), over gpu_moe_group's expert tiles.
//
// Tile k (expert e, up to GG_TILE entries) times a 128-row block of e's weights: four waves, each 32 weight rows x
// GG_TILE entries (GG_TILE / 32 MFMA tiles of 32 x 32). Semantics per output: the reference's int8 expert kernels
// (src/matvec_q.hip:2749-2901: per 32-value block, the integer block dot times the block's scales, summed over
// blocks), in another fp32 order. Two kernels by weight type:
//
// Q8_0 weights, on v_mfma_i32_32x32x32_i8. Per block b:
//   I = A . B: the exact integer block dots of every (row, entry) pair; A = the weights' int8 values, B = the
//       entries' Q8_0 activation values (lane l holds row / entry l % 32 and K half l / 32);
//   S = the outer product of the weight and activation scales, on v_mfma_f32_32x32x8f16 (both are FP16 values,
//       so every product is exact in fp32);
//   acc += (float)I * S: two VALU operations per output and block.
//
// ROCmFP4 / FAST weights, on v_mfma_f32_32x32x16_f16 with exact operands. Every codebook value {0, 1, 2, 3, 4, 6,
// 8, 10} (signed) times its UE4M3 (half-)block scale is exact in FP16 (at most 7 significant bits; the operand
// tiles hold the codes as FP6 E2M3 of value / 2, which v_cvt_scalef32_pk32_f16_fp6 decodes 32 at a time with the
// factor 2, and v_pk_mul_f16 applies the scale), and so is every Q8_0 activation value (an integer of at most 127).
// Each product is exact in the fp32 accumulator and each 16-value half's sum of products, a multiple of its scale
// with at most 19 significant bits, is too; the block's two halves are summed by the second MFMA. So per block:
//   P = (e0 . codes0) . q0 + (e1 . codes1) . q1 on two f16 MFMAs, B = the activations converted to FP16 while
//       being staged into LDS (once per workgroup, shared by its four waves);
//   acc += P * dx, dx the entry's activation scale (the lane's own column): one VALU operation per output and
//       block, against four for the int8 form of the same two-scale block (I and S per half).
//
// Weights are read from the MFMA operand tiles of qmatvec_pack_weights (one contiguous 1 KB run per 64-lane
// load); output rows go to y[out_rows[entry]][row]; the SwiGLU variant (two matrices) writes down's Q8_0 input.
//
// Measured at config 2 (Q8_0, 2,427 tokens) before the operand tiles: each workgroup waited ~3x longer for its
// stage's operands than it computed, because each 64-lane load touched 64 rows' cache lines for 16 bytes each.
// Not the fix, each measured then: dropping the fp32 epilogue (-6%), dropping the scale MFMA (0%), double-buffered
// stages (0%), an XCD-aware tile order (HBM fetch -40%, time +5%), 128-entry tiles (+4%), register-direct
// operands (+50%). With the tiles the int8 kernel is VALU-bound: the conversion and FMA of every output and block.
// Also measured with the tiles: the Q8_0 dots on two f16 MFMAs per block (int8 values are exact in FP16 and the
// block sums exact in fp32, so the same bits with one VALU operation per output and block, but the weights'
// conversion to FP16 in every wave): config 2 prefill 0.458 -> 0.53 ms.

#include "expert_units.h"
#include "grouped.h"
#include "host_common.h"
#include "qmatvec.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

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
    // A shared expert as more tiles of the same launch (vs null: none): tiles kr.. hold its sT entries (tokens
    // 0..sT-1, activation rows as they are, output rows sout + token) against the tiles at vs / ss (vs2 / ss2)
    const uint8_t* vs;
    const uint8_t* ss;
    const uint8_t* vs2;
    const uint8_t* ss2;
    int kr, sT;
    long long sout;
    const int* xbs;  // Q4_K: the Q8_K activations' sums of 16 values, rows of K / 16 (xq / xd: Q8_K values / scales)
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
#define GG_KB 4  // blocks of 32 values per stage (4 or 8; 4 keeps the down kernels at 4-5 waves per SIMD)
#endif
#ifndef GG_KB2
#define GG_KB2 4  // the same for the gate / up / SwiGLU kernel (two matrices per stage)
#endif
#define GG_NT (GG_TILE / 32)
#define GG_TRS 36  // floats per entry of the output transpose (32 rows + 4: 16-byte aligned, banks spread)
#ifndef GG_XCD_RANGES
#define GG_XCD_RANGES 1  // each XCD takes a contiguous range of work items (0: round-robin, the dispatch order)
#endif
#define GG_XCDS 8  // XCDs of an MI355X; workgroup i runs on XCD i % 8

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

// ---- Pipeline. Q8_0 and FP4: K runs in stages of KB blocks through one LDS buffer per workgroup. Weight tiles,
// activation scales and (Q8_0 kernel) activations move from memory to LDS with global_load_lds_dwordx4: lane l of
// such a load writes its 16 bytes to slot l of a 1 KB LDS run, so each run is read back as an MFMA operand with one
// ds_read per lane. The FP4 kernel stages its activations through registers instead (converted to FP16 on the
// way). The weight rows' scales come through registers. Q4_K (below) loads everything into registers one stage
// ahead and stages its activations into two LDS buffers in turn.
typedef __attribute__((address_space(3))) void lds_void;
#ifndef GG_WNT
#define GG_WNT 0  // cache policy bits of the FP4 / Q8_0 weight tiles' LDS-direct loads (2, nontemporal, slower:
                  // config 4 layer prefill 0.44 -> 0.48 ms -- the tiles of an expert's row block are re-read by each of
                  // its entry tiles, from L2)
#endif

__device__ __forceinline__ void lds_load16(const void* g, void* lds_run) {
    __builtin_amdgcn_global_load_lds(g, (lds_void*)lds_run, 16, 0, 0);
}
// The weight tiles' 16-byte loads (the cache policy GG_WNT)
__device__ __forceinline__ void lds_load16w(const void* g, void* lds_run) {
    __builtin_amdgcn_global_load_lds(g, (lds_void*)lds_run, 16, 0, GG_WNT);
}

template <int WAITS>
__device__ __forceinline__ void wait_vm() {
    // s_waitcnt vmcnt(WAITS), expcnt and lgkmcnt left at their maxima (gfx9 encoding)
    __builtin_amdgcn_s_waitcnt((WAITS & 0xf) | ((WAITS >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

// One stage of operands of NM weight matrices sharing the activations
template <int TYPE, int NM, int KB>
struct GBuf {  // Q8_0
    uint8_t a[NM][4][KB][1024];   // [matrix][wave][block][lane * 16]
    uint8_t b[KB][GG_NT][1024];   // [block][entry tile][lane * 16]
    float dx[KB / 4][GG_TILE][4];  // [block / 4][entry][block % 4]
};
template <int NM, int KB>
struct HBuf {  // FP4 types
    uint8_t a[NM][4][3 * KB / 4][1024];  // [matrix][wave][chunk][lane * 16]: the stage-major tiles' 16-byte chunks
    uint8_t b[KB][GG_NT][2][1024];   // [block][entry tile][16-value half][lane * 16]: FP16 activations
    float dx[KB / 4][GG_TILE][4];
};
template <int NM, int KB>
struct KBuf {  // Q4_K: one stage = one (KB = 4) or two (KB = 8) 128-value halves of a super-block (weights: registers)
    uint8_t b[KB][GG_NT][2][1024];   // [sub-block][entry tile][16-value half][lane * 16]: FP16 activations
    float bd[GG_TILE][KB];           // [entry][sub-block]: its sum of 32 Q8_K values times the entry's scale
    float dx[GG_TILE];               // [entry]: the Q8_K scale of the stage's super-block
};
template <int TYPE, int NM, int KB>
struct BufOf {
    typedef GBuf<TYPE, NM, KB> type;
};
#ifndef GG_KBQ4
#define GG_KBQ4 4  // Q4_K: 32-value sub-blocks per stage (8, a whole super-block in 68 KB of LDS, measured no faster)
#endif
#define KQ GG_KBQ4
template <int NM, int KB>
struct KBuf2 {  // Q4_K: two stages, one being computed while the next one's loads land
    KBuf<NM, KB> s[2];
};
template <int NM, int KB>
struct BufOf<QT_Q4_K, NM, KB> {
    typedef KBuf2<NM, KQ> type;
};
template <int NM, int KB>
struct BufOf<QT_ROCMFP4, NM, KB> {
    typedef HBuf<NM, KB> type;
};
template <int NM, int KB>
struct BufOf<QT_ROCMFP4_FAST, NM, KB> {
    typedef HBuf<NM, KB> type;
};

#ifndef GG_ROLE
#define GG_ROLE 0  // 1: the Q8_0 / FP4 gate / up launches also with a matrix per pair of waves (Q4_K always; for
                   // Q8_0 / FP4 measured slower, their stage then serving half the rows: config 2 gate / up
                   // 251 -> 265 us, config 4 219 -> 236, at occupancy 4 instead of 3)
#endif
// NM = 2 as roles: a workgroup takes 64 rows of both matrices, waves 0, 1 gate, 2, 3 up (one matrix per wave)
template <int TYPE, int NM>
struct Roles {
    static constexpr bool on = NM == 2 && (TYPE == QT_Q4_K || GG_ROLE);
    static constexpr int per_wave = on ? 1 : NM;  // matrices per wave
};

// ------------------------------------------------------------------ Q8_0: int8 MFMA

// Issue one stage's loads. Wave w loads the activations of entry tile w % GG_NT, blocks w / GG_NT, + 4 / GG_NT, ...
// (xrow: its lane's entry run), and the scales of entries GG_TILE / 4 w .. (dxr: its lane's entry row). The weight
// scales of the stage (8 blocks' FP16 d per 16-byte slot) go to wsc.
template <int NM, int KB>
__device__ __forceinline__ void q_issue(GBuf<QT_Q8_0, NM, KB>& B, int b0, uint4 (&wsc)[NM],
                                        const uint8_t* const (&vt)[NM], const uint8_t* const (&st)[NM],
                                        const int8_t* xrow, int xs, const float* dxr, int w, int l) {
    constexpr int ES = GG_TILE / 4;  // entries whose scales one wave loads
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int c = 0; c < KB; ++c) lds_load16w(vt[m] + 1024 * (b0 + c), B.a[m][w][c]);
#pragma unroll
    for (int j = 0; j < KB * GG_NT / 4; ++j) {
        const int bb = w / GG_NT + (4 / GG_NT) * j;
        lds_load16(xrow + xs * (b0 + bb), B.b[bb][w % GG_NT]);
    }
#pragma unroll
    for (int q = 0; q < KB / 4; ++q)
        if (l < ES) lds_load16(dxr + b0 + 4 * q, &B.dx[q][ES * w][0]);  // (lanes ES.. idle)
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        const uint8_t* g = st[m] + 512 * (b0 >> 3);
        if constexpr (KB == 4) {
            const uint2 v = *(const uint2*)(g + 8 * ((b0 >> 2) & 1));
            wsc[m] = make_uint4(v.x, v.y, 0u, 0u);
        } else {
            wsc[m] = *(const uint4*)g;
        }
    }
}

template <int NM, int KB, int NTU>
__device__ __forceinline__ void q_compute(const GBuf<QT_Q8_0, NM, KB>& B, const uint4 (&wsc)[NM],
                                          v16f (&acc)[NM][NTU], int w, int l, int lr, int kh) {
    const v16i zi = {};
#pragma unroll
    for (int bb = 0; bb < KB; ++bb) {
        float dx[NTU];
#pragma unroll
        for (int t = 0; t < NTU; ++t) dx[t] = B.dx[bb >> 2][32 * t + lr][bb & 3];
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            const uint32_t w2 = bb < 2 ? wsc[m].x : bb < 4 ? wsc[m].y : bb < 6 ? wsc[m].z : wsc[m].w;
            const uint4 q = *(const uint4*)(B.a[m][w][bb] + 16 * l);
            const v4i A = (v4i){(int)q.x, (int)q.y, (int)q.z, (int)q.w};
            const float dw = h2f((uint16_t)(w2 >> (16 * (bb & 1))));
#pragma unroll
            for (int t = 0; t < NTU; ++t) {
                const v4i Bt = *(const v4i*)(B.b[bb][t] + 16 * l);
                acc_block(acc[m][t], __builtin_amdgcn_mfma_i32_32x32x32_i8(A, Bt, zi, 0, 0, 0),
                          scale_outer(dw, dx[t], kh));
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// ------------------------------------------------------------------ FP4 types: exact f16 MFMA

// Eight Q8_0 values (int8, two dwords) as FP16: (x ^ 0x80) in the low byte of FP16 1024 is 1024 + 128 + x, exact
__device__ __forceinline__ uint4 i8x8_to_f16(uint32_t lo, uint32_t hi) {
    const uint32_t tl = lo ^ 0x80808080u, th = hi ^ 0x80808080u;
    const h2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    auto cv = [&](uint32_t t, uint32_t sel) {
        return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, t, sel)) - bias);
    };
    return make_uint4(cv(tl, 0x04010400u), cv(tl, 0x04030402u), cv(th, 0x04010400u), cv(th, 0x04030402u));
}

typedef unsigned v6u __attribute__((ext_vector_type(6)));
typedef _Float16 v32h __attribute__((ext_vector_type(32)));

// Eight decoded values (halves 8 q .. 8 q + 7 of d) times the FP16 scale pair sc: one MFMA operand
__device__ __forceinline__ v8h scaled8(const v32h& d, int q, uint32_t sc) {
    const h2 s = __builtin_bit_cast(h2, sc);
    v8h r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const h2 p = (h2){d[8 * q + 2 * i], d[8 * q + 2 * i + 1]} * s;
        r[2 * i] = p.x;
        r[2 * i + 1] = p.y;
    }
    return r;
}

// Issue one stage: weight tiles and activation scales to LDS, this thread's activation units to registers: unit j
// at xu + xs b0 + xj j (h_unit gives the entry, block and half each one holds).
template <int NM, int KB>
__device__ __forceinline__ void h_issue(HBuf<NM, KB>& B, int b0, uint4 (&wsc)[NM][KB / 4],
                                        const uint8_t* const (&vt)[NM], const uint8_t* const (&st)[NM],
                                        const int8_t* xu, int xs, int xj, uint4 (&xb)[KB / 2], const float* dxr,
                                        int w, int l) {
    constexpr int ES = GG_TILE / 4;
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int c = 0; c < 3 * KB / 4; ++c)  // the stage's 1 KB chunks of the wave's codes
            lds_load16w(vt[m] + 768 * b0 + 1024 * c, B.a[m][w][c]);
#pragma unroll
    for (int q = 0; q < KB / 4; ++q)
        if (l < ES) lds_load16(dxr + b0 + 4 * q, &B.dx[q][ES * w][0]);
#pragma unroll
    for (int j = 0; j < KB / 2; ++j) xb[j] = *(const uint4*)(xu + xs * b0 + xj * j);
#pragma unroll
    for (int m = 0; m < NM; ++m)  // 4 blocks' (e0, e1) FP16 pairs per 16 bytes of the row's 32-byte slot
#pragma unroll
        for (int q = 0; q < KB / 4; ++q) wsc[m][q] = *(const uint4*)(st[m] + 1024 * (b0 >> 3) + 16 * (((b0 >> 2) + q) & 1));
}

// Activation unit j of this thread (16 int8 values: half h of block bb of the stage, for entry e). Entry-tile
// order (rows = false, contiguous 1 KB runs): entry tid % 64, half (tid / 64) % 2, block tid / 128 + 2 j.
// Gathered rows (rows = true): the wave's 16 entries 16 w + l % 16, four lanes each on consecutive 16-byte pieces
// of the entry's run of the stage (unit c = 4 j + l / 16: block c / 2, half c % 2), so that a load touches 16 rows'
// 64-byte pieces instead of 64 rows' 16-byte ones.
__device__ __forceinline__ void h_unit(bool rows, int j, int tid, int& e, int& bb, int& h) {
    const int w = tid >> 6, l = tid & 63, c = 4 * j + (l >> 4);
    e = rows ? 16 * w + (l & 15) : tid & 63;
    bb = rows ? c >> 1 : (tid >> 7) + 2 * j;
    h = rows ? c & 1 : (tid >> 6) & 1;
}

// This thread's activation units, converted, into the FP16 operand runs: values 0..7 of a unit to the slot of
// (entry, K half 0) of its MFMA half, values 8..15 to that of (entry, K half 1)
template <int NM, int KB, typename Buf = HBuf<NM, KB>>
__device__ __forceinline__ void h_stage_b(Buf& B, const uint4 (&xb)[KB / 2], bool rows, int tid) {
#pragma unroll
    for (int j = 0; j < KB / 2; ++j) {
        int e, bb, h;
        h_unit(rows, j, tid, e, bb, h);
        uint8_t* run = B.b[bb][e >> 5][h];
        *(uint4*)(run + 16 * (e & 31)) = i8x8_to_f16(xb[j].x, xb[j].y);
        *(uint4*)(run + 16 * (32 + (e & 31))) = i8x8_to_f16(xb[j].z, xb[j].w);
    }
}

template <int NM, int KB, int NTU>
__device__ __forceinline__ void h_compute(const HBuf<NM, KB>& B, const uint4 (&wsc)[NM][KB / 4],
                                          v16f (&acc)[NM][NTU], int w, int l, int lr) {
    const v16f z = {};
#pragma unroll
    for (int bp = 0; bp < KB; bp += 2) {  // a block pair: 32 FP6 codes a lane, one conversion
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            // blocks bp, bp + 1 of a stage of four: the lane's dwords 3 (bp % 4) .. + 5 of its 12, in chunks
            // 3 (bp / 4) + (bp % 4) / 2 and the next
            const int ch = 3 * (bp >> 2) + ((bp & 3) >> 1);
            const uint4 q0 = *(const uint4*)(B.a[m][w][ch] + 16 * l), q1 = *(const uint4*)(B.a[m][w][ch + 1] + 16 * l);
            const v6u c6 = (bp & 2) ? (v6u){q0.z, q0.w, q1.x, q1.y, q1.z, q1.w} : (v6u){q0.x, q0.y, q0.z, q0.w, q1.x, q1.y};
            const v32h d = __builtin_amdgcn_cvt_scalef32_pk32_f16_fp6(c6, 2.0f);
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int bb = bp + k;
                const uint4 ws = wsc[m][bb >> 2];
                const uint32_t sc = (bb & 3) == 0 ? ws.x : (bb & 3) == 1 ? ws.y : (bb & 3) == 2 ? ws.z : ws.w;
                const v8h A0 = scaled8(d, 2 * k, __builtin_amdgcn_perm(sc, sc, 0x01000100u));      // (e0, e0)
                const v8h A1 = scaled8(d, 2 * k + 1, __builtin_amdgcn_perm(sc, sc, 0x03020302u));  // (e1, e1)
#pragma unroll
                for (int t = 0; t < NTU; ++t) {
                    const float dx = B.dx[bb >> 2][32 * t + lr][bb & 3];
                    const v8h B0 = *(const v8h*)(B.b[bb][t][0] + 16 * l);
                    const v8h B1 = *(const v8h*)(B.b[bb][t][1] + 16 * l);
                    const v16f P = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                        A1, B1, __builtin_amdgcn_mfma_f32_32x32x16_f16(A0, B0, z, 0, 0, 0), 0, 0, 0);
#pragma unroll
                    for (int j = 0; j < 16; ++j) acc[m][t][j] = fmaf(P[j], dx, acc[m][t][j]);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// ------------------------------------------------------------------ Q4_K: exact f16 MFMA, integer sums per 128 values
//
// Per 128-value half c of a super-block (one stage of four 32-value sub-blocks j), for each (row, entry):
//   isum = sum_j sc_j . sum_{i in j} q_i qx_i   on eight f16 MFMAs with A = sc_j q (the FP6 codes decoded with the
//          factor 2, times the FP16 sub-block scale: integers <= 945, exact), B = qx (Q8_K values, exact): every
//          partial sum an integer below 945 x 127 x 128 < 2^24, so exact in fp32 in any order;
//   acc += (d dx) isum                         S = d (x) dx, the row's FP16 d times the entry's Q8_K scale, from an
//                                              outer-product f32 MFMA (one rounding), then one VALU FMA per output;
//   acc -= sum_j (dmin m_j) (bsum_j dx)        two f32 MFMAs accumulating into acc: A = -dmin m_j (exact in fp32),
//                                              B = bsum_j dx, bsum_j the sub-block's sum of 32 Q8_K values.
// The reference's K-quant WMMA kernel forms the same integer sums per 128-value chunk (src/matvec_q.hip:2952-3008)
// and the same float step (d isum - dmin msum) dx, in another fp32 order.
template <int KB>
struct KSc {  // a lane's row scales for each 128-value half of a stage: its tile record (sc_j and m_j as bytes, d, dmin)
    uint4 h[KB / 4];
};

// Issue one stage's loads, all into registers: the wave's weight codes (the stage-major tiles: three 16-byte chunks
// a lane, each load one contiguous 1 KB run) and its rows' scale records; and the activations of the wave's 16 entries 16 w + l % 16,
// lanes l / 16 reading consecutive 16-byte units of each entry's run of the stage, so that one load touches 16
// entries' 64-byte pieces (a lane per entry, as the other kernels stage them, makes every load touch 64 rows):
// unit c = 4 j + l / 16 of the stage (sub-block c / 2, 16-value half c % 2), the sums of 16 of sub-blocks
// l / 16 + 4 q (a pair each) and the entry's scale. xu, bsr, dxr: the lane's entry row's values (+ 16 (l / 16)),
// sums of 16 (+ 2 (l / 16)) and scales.
template <int KB>
__device__ __forceinline__ void k_issue(int b0, uint4 (&wv)[3 * KB / 4], KSc<KB>& ks, const uint8_t* vt,
                                        const uint8_t* sct, const int8_t* xu, uint4 (&xb)[KB / 2],
                                        int2 (&bsv)[KB / 4], float& dxv, const int* bsr, const float* dxr) {
    static_assert(KB == 4 || KB == 8, "a Q4_K stage is one or two 128-value halves of a super-block");
#pragma unroll
    for (int c = 0; c < 3 * KB / 4; ++c) wv[c] = *(const uint4*)(vt + 768 * b0 + 1024 * c);
#pragma unroll
    for (int j = 0; j < KB / 2; ++j) xb[j] = *(const uint4*)(xu + 32 * b0 + 64 * j);
#pragma unroll
    for (int q = 0; q < KB / 4; ++q) bsv[q] = *(const int2*)(bsr + 2 * b0 + 8 * q);
    dxv = dxr[b0 >> 3];
    const uint8_t* slot = sct + Q4K_TILE_SLOT * 32 * (b0 >> 3) + 16 * ((b0 >> 2) & 1);
#pragma unroll
    for (int h = 0; h < KB / 4; ++h) ks.h[h] = *(const uint4*)(slot + 16 * h);
}

// (v_fence: the value is taken as changed here, so that the compiler neither hoists the conversions that use it
// above this point, next to the loads issued a stage earlier, nor waits for those loads before it)
__device__ __forceinline__ void v_fence(float& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void v_fence(int2& v) { asm volatile("" : "+v"(v.x), "+v"(v.y)); }
__device__ __forceinline__ void v_fence(uint4& v) { asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w)); }

// The stage's activations into the FP16 operand runs (values 0..7 of a unit to the slot of (entry, K half 0) of its
// sub-block's run for its 16-value half, values 8..15 to that of (entry, K half 1): the 16 lanes of one unit write
// 16 consecutive slots), each sub-block's sum of 32 values times the entry's scale, and the scale
template <int NM, int KB>
__device__ __forceinline__ void k_stage(KBuf<NM, KB>& B, uint4 (&xb)[KB / 2], int2 (&bsv)[KB / 4], float& dxv,
                                        int w, int l) {
#pragma unroll
    for (int j = 0; j < KB / 2; ++j) v_fence(xb[j]);
#pragma unroll
    for (int q = 0; q < KB / 4; ++q) v_fence(bsv[q]);
    v_fence(dxv);
    const int e = 16 * w + (l & 15), u = l >> 4;
#pragma unroll
    for (int j = 0; j < KB / 2; ++j) {
        const int c = 4 * j + u;
        uint8_t* run = B.b[c >> 1][e >> 5][c & 1];
        *(uint4*)(run + 16 * (e & 31)) = i8x8_to_f16(xb[j].x, xb[j].y);
        *(uint4*)(run + 16 * (32 + (e & 31))) = i8x8_to_f16(xb[j].z, xb[j].w);
    }
#pragma unroll
    for (int q = 0; q < KB / 4; ++q) B.bd[e][u + 4 * q] = (float)(bsv[q].x + bsv[q].y) * dxv;  // (the sum: exact)
    if (u == 0) B.dx[e] = dxv;
}

// (sc, sc) as an FP16 pair for sub-block j's scale byte in w: the byte under FP16 1024's exponent is 1024 + sc
__device__ __forceinline__ uint32_t sc_pair(uint32_t w, int j) {
    const h2 v = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, w, 0x04000400u | (0x00010001u * j)));
    return __builtin_bit_cast(uint32_t, v - (h2){(_Float16)1024.0f, (_Float16)1024.0f});
}

template <int NM, int KB, int NTU>
__device__ __forceinline__ void k_compute(const KBuf<NM, KB>& B, const uint4 (&wv)[3 * KB / 4], const KSc<KB>& ks,
                                          v16f (&acc)[NTU], int l, int lr, int kh) {
    const v16f z = {};
    uint32_t wd[3 * KB];  // the lane's codes: 3 dwords (16 FP6 codes) per sub-block
#pragma unroll
    for (int c = 0; c < 3 * KB / 4; ++c) {
        wd[4 * c] = wv[c].x;
        wd[4 * c + 1] = wv[c].y;
        wd[4 * c + 2] = wv[c].z;
        wd[4 * c + 3] = wv[c].w;
    }
#pragma unroll
    for (int hc = 0; hc < KB / 4; ++hc) {  // each 128-value half: its integer sums, then the float steps
        const uint4 r = ks.h[hc];
        const h2 dd = __builtin_bit_cast(h2, r.z);
        const float aD = kh ? 0.0f : (float)dd.x;  // S's A: the lane's row's d in k = 0
        const float ndm = -(float)dd.y;
        // A of the half's four sub-blocks: codes decoded two sub-blocks at a time, times the sub-block's scale
        v8h A0[4], A1[4];
#pragma unroll
        for (int bp = 0; bp < 4; bp += 2) {
            const uint32_t* c = wd + 12 * hc + 3 * bp;
            const v32h d = __builtin_amdgcn_cvt_scalef32_pk32_f16_fp6((v6u){c[0], c[1], c[2], c[3], c[4], c[5]}, 2.0f);
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const int jj = bp + kk;
                const uint32_t sc = sc_pair(r.x, jj);
                A0[jj] = scaled8(d, 2 * kk, sc);
                A1[jj] = scaled8(d, 2 * kk + 1, sc);
            }
        }
        // the mins' A: k = kh of the first MFMA is sub-block kh, of the second sub-block 2 + kh (exact products)
        const float am0 = ndm * (float)((r.y >> (8 * kh)) & 0xffu);
        const float am1 = ndm * (float)((r.y >> (16 + 8 * kh)) & 0xffu);
#pragma unroll
        for (int t = 0; t < NTU; ++t) {
            v16f P = z;
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                const v8h B0 = *(const v8h*)(B.b[4 * hc + jj][t][0] + 16 * l);
                const v8h B1 = *(const v8h*)(B.b[4 * hc + jj][t][1] + 16 * l);
                P = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                    A1[jj], B1, __builtin_amdgcn_mfma_f32_32x32x16_f16(A0[jj], B0, P, 0, 0, 0), 0, 0, 0);
            }
            const float* bd = B.bd[32 * t + lr];
            const float bdx = kh ? 0.0f : B.dx[32 * t + lr];
            const v16f S = __builtin_amdgcn_mfma_f32_32x32x2f32(aD, bdx, z, 0, 0, 0);
#pragma unroll
            for (int j = 0; j < 16; ++j) acc[t][j] = fmaf(P[j], S[j], acc[t][j]);
            acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(am0, bd[4 * hc + kh], acc[t], 0, 0, 0);
            acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(am1, bd[4 * hc + 2 + kh], acc[t], 0, 0, 0);
        }
    }
}

// ------------------------------------------------------------------ the kernel

template <int TYPE, int NM, int KB, int NTU>
__device__ __forceinline__ void grouped_tile(const GArgs& a,
                                             typename BufOf<TYPE, Roles<TYPE, NM>::per_wave, KB>::type& buf, int k,
                                             int rb, int e, int st, int cnt, bool shk);

// NM = 1: y rows (fp32) of one matrix. NM = 2, SwiGLU: gate (a.v) and up (a.v2) rows of the same block, then
// act = SiLU(g) u (the swiglu kernel's expression) and its Q8_0 blocks -- a wave's 32 rows of one entry are one
// block: 16 values in each of lanes l and l + 32 -- into a.aq / a.ad (the quantizer's expressions).
template <int TYPE, int NM, int KB>
#ifndef GG_WPE
#define GG_WPE 3  // waves per SIMD asked of the compiler (0: its choice; 3 measured 3-8% faster than its 2)
#endif
#ifndef GG_WPE_Q4K
#define GG_WPE_Q4K 2  // the Q4_K kernel: its stage loads in flight during the previous stage's compute take registers
#endif
#ifndef GG_WPE_D8
#define GG_WPE_D8 5  // the same for the one-matrix Q8_0 kernel (96 VGPRs: five workgroups per CU; 6 spilled, config 2 +13%)
#endif
__global__ void __launch_bounds__(256)
#if GG_WPE
__attribute__((amdgpu_waves_per_eu(TYPE == QT_Q8_0 && NM == 1 ? GG_WPE_D8 : TYPE == QT_Q4_K ? GG_WPE_Q4K : GG_WPE)))
#endif
k_grouped(GArgs a) {
    __shared__ __attribute__((aligned(1024))) typename BufOf<TYPE, Roles<TYPE, NM>::per_wave, KB>::type buf;
    // Work items (tile, 128-row block), tile-major, over the tiles that exist: the routed tiles 0 .. n_tiles - 1
    // (or the dense rows' tiles), then the shared expert's. Each XCD takes one contiguous range of items (the
    // hardware deals workgroup i to XCD i % 8), so the consecutive tiles of one expert, which read the same
    // weight rows, run together on one XCD and share its L2 instead of fetching those rows once per XCD.
    // (NM = 2 as roles: 64 rows of both matrices a workgroup, a matrix per pair of waves)
    const int nrb = a.N / (Roles<TYPE, NM>::on ? GG_ROWS / 2 : GG_ROWS);
    const int nrt = a.n_tiles ? *a.n_tiles : (a.T + GG_TILE - 1) / GG_TILE;  // routed / dense tiles
    const int nsh = a.vs ? (a.sT + GG_TILE - 1) / GG_TILE : 0;
    const int items = (nrt + nsh) * nrb;
#if GG_XCD_RANGES
    const int per = (items + GG_XCDS - 1) / GG_XCDS, slot = blockIdx.x / GG_XCDS;
    const int item = (blockIdx.x % GG_XCDS) * per + slot;
    if (slot >= per || item >= items) return;
#else
    const int item = blockIdx.x;
    if (item >= items) return;
#endif
    const int kv = item / nrb, rb = item - kv * nrb;
    const bool shk = kv >= nrt;  // a shared-expert tile
    const int k = shk ? a.kr + (kv - nrt) : kv;
    int e, st, cnt;
    if (shk) {
        st = (kv - nrt) * GG_TILE;
        e = 0;
        cnt = min(GG_TILE, a.sT - st);
    } else if (a.n_tiles) {
        e = a.tile_e[k];
        st = a.tile_start[k];
        cnt = __builtin_amdgcn_readfirstlane(a.tile_n[k]);
    } else {  // dense: tile k is rows GG_TILE k .. of the one matrix
        st = k * GG_TILE;
        e = 0;
        cnt = min(GG_TILE, a.T - st);
    }
    // a tile of at most 32 entries leaves its second 32-entry MFMA tile empty: the loop without it
    if (cnt > 32)
        grouped_tile<TYPE, NM, KB, GG_NT>(a, buf, k, rb, e, st, cnt, shk);
    else
        grouped_tile<TYPE, NM, KB, 1>(a, buf, k, rb, e, st, cnt, shk);
}

// One workgroup's tile k (expert e, entries st .. st + cnt - 1) and row block rb, with NTU of its GG_NT 32-entry
// MFMA tiles in use
template <int TYPE, int NM, int KB, int NTU>
__device__ __forceinline__ void grouped_tile(const GArgs& a,
                                             typename BufOf<TYPE, Roles<TYPE, NM>::per_wave, KB>::type& buf, int k,
                                             int rb, int e, int st, int cnt, bool shk) {
    constexpr bool F16 = TYPE != QT_Q8_0;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, lr = l & 31, kh = l >> 5;
    auto in_row = [&](int i) { return !shk && a.in_rows ? a.in_rows[st + i] : st + i; };
    auto out_row = [&](int i) { return shk ? a.sout + st + i : a.out_rows ? a.out_rows[st + i] : st + i; };
    const int K = a.K, nb = K / 32;
    // the wave's 32-row group of the stacked matrix (the launcher requires N % 128 == 0 and K % 256 == 0) and
    // this lane's slots in its value and scale tiles (scale slots: 16 bytes per 8 blocks for Q8_0, 32 for FP4)
    constexpr bool Q4K = TYPE == QT_Q4_K;
    // NM = 2 as roles: waves 0, 1 take 32 gate rows each, waves 2, 3 the same rows of up
    constexpr bool ROLE = Roles<TYPE, NM>::on;
    constexpr int NMW = Roles<TYPE, NM>::per_wave;
    const int r0 = ROLE ? rb * (GG_ROWS / 2) + 32 * (w & 1) : rb * GG_ROWS + 32 * w;
    const long long grp = ((long long)e * a.N + r0) / 32;
    constexpr int SB = Q4K ? Q4K_TILE_SLOT : F16 ? 32 : 16;
    constexpr int VS = 16;  // value slot bytes (FP4, Q4_K: a lane's 16-byte chunk of its stage)
    const uint8_t* vt[NMW];
    const uint8_t* sct[NMW];
    const bool up_role = ROLE && w >= 2;
    vt[0] = (shk ? (up_role ? a.vs2 : a.vs) : up_role ? a.v2 : a.v) + grp * a.vrb + VS * l;
    sct[0] = (shk ? (up_role ? a.ss2 : a.ss) : up_role ? a.s2 : a.s) + grp * a.srb + SB * lr;
    if constexpr (NM == 2 && !ROLE) {
        vt[1] = (shk ? a.vs2 : a.v2) + grp * a.vrb + VS * l;
        sct[1] = (shk ? a.ss2 : a.s2) + grp * a.srb + SB * lr;
    }
    const int de = min(GG_TILE / 4 * w + (l & (GG_TILE / 4 - 1)), cnt - 1);  // the entry whose scales this lane loads
    const float* dxr = a.xd + ((a.xt & GX_IN) ? (long long)k * GG_TILE + de : (long long)in_row(de)) * nb;

    v16f acc[NMW][NTU];
#pragma unroll
    for (int m = 0; m < NMW; ++m)
#pragma unroll
        for (int t = 0; t < NTU; ++t) acc[m][t] = (v16f){};
    const int nst = nb / KB;
    if constexpr (Q4K) {
        // this lane's entry 16 w + l % 16 (the last one for lanes past the tile's entries) and unit l / 16
        const long long br = in_row(min(16 * w + (l & 15), cnt - 1));
        const int8_t* xu = a.xq + br * K + 16 * (l >> 4);
        const int* bsr = a.xbs + br * (K / 16) + 2 * (l >> 4);
        const float* kdr = a.xd + br * (K / 256);
        // Software-pipelined over the two stage buffers: stage s + 1's loads are issued after the barrier that
        // publishes stage s and land while stage s is computed; one barrier per stage (a wave past it has finished
        // computing stage s - 1, whose buffer the loads then reuse). The stage count nb / KQ is even (K % 256 == 0).
        KSc<KQ> ksn;
        uint4 wvn[3 * KQ / 4];
        uint4 xb[KQ / 2];
        int2 bsv[KQ / 4];
        float dxv;
        const int ns = nb / KQ;
        k_issue<KQ>(0, wvn, ksn, vt[0], sct[0], xu, xb, bsv, dxv, bsr, kdr);
        auto step = [&](KBuf<NMW, KQ>& cur, int s) {
            k_stage<NMW, KQ>(cur, xb, bsv, dxv, w, l);
            KSc<KQ> ks = ksn;
            uint4 wv[3 * KQ / 4];
#pragma unroll
            for (int c = 0; c < 3 * KQ / 4; ++c) {
                wv[c] = wvn[c];
                v_fence(wv[c]);
            }
#pragma unroll
            for (int h = 0; h < KQ / 4; ++h) v_fence(ks.h[h]);
            __syncthreads();
            // (the last stage loads itself again, from L2: an unconditional issue keeps every stage's registers
            // in one place, where a skipped one would make the compiler copy them and wait for the loads)
            k_issue<KQ>(min(s + 1, ns - 1) * KQ, wvn, ksn, vt[0], sct[0], xu, xb, bsv, dxv, bsr, kdr);
            k_compute<NMW, KQ, NTU>(cur, wv, ks, acc[0], l, lr, kh);
            __builtin_amdgcn_sched_barrier(0);  // (the next stage's staging stays after this compute)
        };
        for (int s = 0; s < ns; s += 2) {
            step(buf.s[0], s);
            step(buf.s[1], s + 1);
        }
        __syncthreads();  // (the output transpose below reuses the buffers)
    } else if constexpr (!F16) {
        // this lane's activation run: entry 32 (w % GG_NT) + lr, K half kh
        const int8_t* xrow;
        int xs;  // bytes from one block's run to the next
        if (a.xt & GX_IN) {
            xrow = a.xq + ((long long)k * nb * GG_NT + w % GG_NT) * 1024 + 16 * l;
            xs = GG_NT * 1024;
        } else {
            xrow = a.xq + (long long)in_row(min(32 * (w % GG_NT) + lr, cnt - 1)) * K + 16 * kh;
            xs = 32;
        }
        uint4 wsc[NMW];
        for (int s = 0; s < nst; ++s) {
            q_issue<NMW, KB>(buf, s * KB, wsc, vt, sct, xrow, xs, dxr, w, l);
            wait_vm<0>();
            __syncthreads();
            q_compute<NMW, KB, NTU>(buf, wsc, acc, w, l, lr, kh);
            __syncthreads();
        }
    } else {
        // this thread's activation units (h_unit)
        const bool rows = !(a.xt & GX_IN);
        int ue, ub, uh;
        h_unit(rows, 0, tid, ue, ub, uh);
        const int8_t* xu;
        int xs, xj;
        if (!rows) {  // unit j: block ub + 2 j
            xu = a.xq + ((long long)k * nb * GG_NT + (ue >> 5)) * 1024 + 16 * (32 * uh + (ue & 31)) +
                 (long long)GG_NT * 1024 * ub;
            xs = GG_NT * 1024;
            xj = 2 * GG_NT * 1024;
        } else {  // unit j: byte 64 j + 16 (l / 16) of the entry's 128-byte run of the stage
            xu = a.xq + (long long)in_row(min(ue, cnt - 1)) * K + 16 * (l >> 4);
            xs = 32;
            xj = 64;
        }
        uint4 wsc[NMW][KB / 4];
        uint4 xb[KB / 2];
        for (int s = 0; s < nst; ++s) {
            h_issue<NMW, KB>(buf, s * KB, wsc, vt, sct, xu, xs, xj, xb, dxr, w, l);
            wait_vm<0>();
            h_stage_b<NMW, KB>(buf, xb, rows, tid);
            __syncthreads();
            h_compute<NMW, KB, NTU>(buf, wsc, acc, w, l, lr);
            __syncthreads();
        }
    }
    // acc[m][t][j] is C[row 8 (j / 4) + 4 kh + j % 4][entry 32 t + lr] of the wave's 32 x GG_TILE block
    // ROLE: the gate waves hand g over through LDS (Q4_K: past the up waves' transpose areas) and leave
    constexpr int GX0 = Q4K ? 4 * 32 * GG_TRS : 0;
    static_assert(!ROLE || sizeof(buf) >= (GX0 + 2 * GG_NT * 16 * 64) * sizeof(float), "g fits the buffer");
    float* gx = (float*)&buf + GX0 + (w & 1) * (GG_NT * 16 * 64);
    if constexpr (ROLE) {
        if (w < 2)
#pragma unroll
            for (int t = 0; t < NTU; ++t)
#pragma unroll
                for (int j = 0; j < 16; ++j) gx[(t * 16 + j) * 64 + l] = acc[0][t][j];
        __syncthreads();
        if (w < 2) return;
    }
    // gate and up of output j of tile t (the two matrices of a wave, or g from LDS and the wave's up)
    auto gate_of = [&](int t, int j) { return ROLE ? gx[(t * 16 + j) * 64 + l] : acc[0][t][j]; };
    auto up_of = [&](int t, int j) { return acc[NMW - 1][t][j]; };
    if constexpr (ROLE && Q4K) {  // SwiGLU (the swiglu kernel's expression), stored as fp32 rows below
#pragma unroll
        for (int t = 0; t < NTU; ++t)
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const float g = gate_of(t, j);
                acc[0][t][j] = g / (1.0f + __expf(-g)) * up_of(t, j);
            }
    }
    if constexpr (NM == 1 || (ROLE && Q4K)) {
        if (((uintptr_t)a.y | (uintptr_t)(a.ldy * 4)) & 15) {  // (uniform) rows not 16-byte aligned: 4-byte stores
#pragma unroll
            for (int t = 0; t < NTU; ++t)
                if (32 * t + lr < cnt) {
                    float* y = a.y + (long long)out_row(32 * t + lr) * a.ldy + r0;
#pragma unroll
                    for (int j = 0; j < 16; ++j) y[8 * (j >> 2) + 4 * kh + (j & 3)] = acc[0][t][j];
                }
        } else {
            // each 32 x 32 block turned through this wave's part of the (now idle) stage buffer, so that a store
            // writes 16 bytes a lane and whole 128-byte rows of 32 outputs (8 per store), not 8 bytes of 32 rows
            static_assert(sizeof(buf) >= 4 * 32 * GG_TRS * sizeof(float), "four waves' 32 x 32 blocks fit the buffer");
            float* tr = (float*)&buf + w * 32 * GG_TRS;
#pragma unroll
            for (int t = 0; t < NTU; ++t) {
                const int orow = 32 * t + lr < cnt ? out_row(32 * t + lr) : 0;  // lane lr: entry 32 t + lr's row
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    *(float4*)&tr[lr * GG_TRS + 8 * q + 4 * kh] =
                        make_float4(acc[0][t][4 * q], acc[0][t][4 * q + 1], acc[0][t][4 * q + 2], acc[0][t][4 * q + 3]);
                __atomic_signal_fence(__ATOMIC_SEQ_CST);  // (a wave's LDS operations complete in order)
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const int e = (l >> 3) + 8 * p;  // entry of the tile; this lane's rows 4 (l % 8) .. + 3
                    const float4 v = *(const float4*)&tr[e * GG_TRS + 4 * (l & 7)];
                    const int oe = __shfl(orow, e, 64);
                    if (32 * t + e < cnt) *(float4*)(a.y + (long long)oe * a.ldy + r0 + 4 * (l & 7)) = v;
                }
                __atomic_signal_fence(__ATOMIC_SEQ_CST);
            }
        }
    } else {
#pragma unroll
        for (int t = 0; t < NTU; ++t) {
            float act[16];
            float am = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const float g = gate_of(t, j);
                act[j] = g / (1.0f + __expf(-g)) * up_of(t, j);
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
    return (type == QT_Q8_0 || type == QT_ROCMFP4 || type == QT_ROCMFP4_FAST || type == QT_Q4_K) && N % GG_ROWS == 0 &&
           K % (GG_KB * 32) == 0 && K % (GG_KB2 * 32) == 0 && (type != QT_Q4_K || K % 256 == 0);
}

// The entry tile the MFMA kernel takes
int moe_grouped_mfma_tile(void) { return GG_TILE; }

// The shared-expert tiles of a launch (GArgs::vs ..); sh null: none
static void bind_shared(GArgs& a, const GShared* sh, int max_tiles, int& tiles) {
    if (!sh) return;
    a.vs = sh->v;
    a.ss = sh->s;
    a.vs2 = sh->v2;
    a.ss2 = sh->s2;
    a.kr = max_tiles;
    a.sT = sh->T;
    a.sout = sh->out0;
    tiles += (sh->T + GG_TILE - 1) / GG_TILE;
}

// Q4_K reads the Q8_K part of the activation bundle: values, scales per 256, sums per 16
static void bind_q8k(GArgs& a, const qmatvec_q8* q) {
    a.xq = q->qK;
    a.xd = q->dK;
    a.xbs = q->bsK;
}

// A 1-D grid with a workgroup for every (tile, row block) item that can exist, rounded up to whole XCD rounds
static dim3 grid_of(int N, int tiles) {
    const long long n = (long long)(N / GG_ROWS) * tiles;
    return dim3((unsigned)((n + GG_XCDS - 1) / GG_XCDS * GG_XCDS));
}

hipError_t moe_launch_grouped_mfma(int type, const uint8_t* v, const uint8_t* s, long long vrb, long long srb,
                                   const qmatvec_q8* q, float* y, int N, int K, int max_tiles, const int32_t* n_tiles,
                                   const int32_t* tile_e, const int32_t* tile_start, const int32_t* tile_n,
                                   const int32_t* in_rows, const int32_t* out_rows, int xt, const GShared* sh,
                                   hipStream_t stream) {
    GArgs a = {v,      s,       vrb,      srb, q->q0, q->d0, y,       N,       K,       n_tiles, tile_e,
               tile_start, tile_n, in_rows, out_rows, N, 0, nullptr, nullptr, nullptr, nullptr, xt};
    int tiles = max_tiles;
    bind_shared(a, sh, max_tiles, tiles);
    const dim3 g = grid_of(N, tiles), b(256);
    if (type == QT_Q4_K) {  // Q8_K activations, rows as they are
        if (xt || sh) return hipErrorInvalidValue;
        bind_q8k(a, q);
        return launch_kernel(k_grouped<QT_Q4_K, 1, GG_KB>, g, b, 0, stream, a);
    }
    switch (type) {
    case QT_Q8_0: return launch_kernel(k_grouped<QT_Q8_0, 1, GG_KB>, g, b, 0, stream, a);
    case QT_ROCMFP4: return launch_kernel(k_grouped<QT_ROCMFP4, 1, GG_KB>, g, b, 0, stream, a);
    case QT_ROCMFP4_FAST: return launch_kernel(k_grouped<QT_ROCMFP4_FAST, 1, GG_KB>, g, b, 0, stream, a);
    }
    return hipErrorInvalidDeviceFunction;
}

// Gate and up of the same tiles in one launch, then SwiGLU and down's Q8_0 input (aq rows of N, ad per 32; in
// entry-tile order with xt = GX_OUT) instead of the gate / up outputs. xt: GX_IN / GX_OUT flags (GArgs::xt); sh: a
// shared expert's tiles after the max_tiles routed ones (its entries' rows in entry-tile order continue there)
hipError_t moe_launch_grouped_swiglu(int type, const uint8_t* vg, const uint8_t* sg, const uint8_t* vu,
                                     const uint8_t* su, long long vrb, long long srb, const qmatvec_q8* q, int8_t* aq,
                                     float* ad, int N, int K, int max_tiles, const int32_t* n_tiles,
                                     const int32_t* tile_e, const int32_t* tile_start, const int32_t* tile_n,
                                     const int32_t* in_rows, const int32_t* out_rows, int xt, const GShared* sh,
                                     hipStream_t stream) {
    GArgs a = {vg,         sg,     vrb,     srb,      q->q0, q->d0, nullptr, N,  K,  n_tiles, tile_e,
               tile_start, tile_n, in_rows, out_rows, N,     0,     vu,      su, aq, ad, xt};
    int tiles = max_tiles;
    bind_shared(a, sh, max_tiles, tiles);
    const dim3 g = grid_of(GG_ROLE ? 2 * N : N, tiles), b(256);  // (roles: 64-row blocks)
    switch (type) {
    case QT_Q8_0: return launch_kernel(k_grouped<QT_Q8_0, 2, GG_KB2>, g, b, 0, stream, a);
    case QT_ROCMFP4: return launch_kernel(k_grouped<QT_ROCMFP4, 2, GG_KB2>, g, b, 0, stream, a);
    case QT_ROCMFP4_FAST: return launch_kernel(k_grouped<QT_ROCMFP4_FAST, 2, GG_KB2>, g, b, 0, stream, a);
    }
    return hipErrorInvalidDeviceFunction;
}

// Q4_K gate and up of the same tiles in one launch (64 rows of each matrix a workgroup: its gate waves hand g to its
// up waves), then SwiGLU: y rows of N fp32 values (out_rows) of SiLU(g) u, the same bits as the two one-matrix
// launches and the swiglu kernel; the caller quantizes them to down's Q8_K input (one scale per 256 values, which a
// workgroup's rows cannot form)
hipError_t moe_launch_grouped_gate_up(int type, const uint8_t* vg, const uint8_t* sg, const uint8_t* vu,
                                      const uint8_t* su, long long vrb, long long srb, const qmatvec_q8* q, float* y,
                                      int N, int K, int max_tiles, const int32_t* n_tiles, const int32_t* tile_e,
                                      const int32_t* tile_start, const int32_t* tile_n, const int32_t* in_rows,
                                      const int32_t* out_rows, hipStream_t stream) {
    if (type != QT_Q4_K) return hipErrorInvalidValue;
    GArgs a = {vg,         sg,     vrb,     srb,      q->q0, q->d0, y,  N,       K,       n_tiles, tile_e,
               tile_start, tile_n, in_rows, out_rows, N,     0,     vu, su, nullptr, nullptr, 0};
    bind_q8k(a, q);
    return launch_kernel(k_grouped<QT_Q4_K, 2, GG_KB>, grid_of(2 * N, max_tiles), dim3(256), 0, stream, a);
}

// Dense: y[t][0..N) (row stride ldy) = W . x_t for t < T, every token a tile entry of the one matrix
hipError_t moe_launch_dense_mfma(int type, const uint8_t* v, const uint8_t* s, long long vrb, long long srb,
                                 const qmatvec_q8* q, float* y, long long ldy, int N, int K, int T,
                                 hipStream_t stream) {
    GArgs a = {v,       s,       vrb,     srb,     q->q0, q->d0, y,       N,       K,       nullptr, nullptr,
               nullptr, nullptr, nullptr, nullptr, ldy,   T,     nullptr, nullptr, nullptr, nullptr, 0};
    const dim3 g = grid_of(N, (T + GG_TILE - 1) / GG_TILE), b(256);
    if (type == QT_Q4_K) bind_q8k(a, q);
    switch (type) {
    case QT_Q4_K: return launch_kernel(k_grouped<QT_Q4_K, 1, GG_KB>, g, b, 0, stream, a);
    case QT_Q8_0: return launch_kernel(k_grouped<QT_Q8_0, 1, GG_KB>, g, b, 0, stream, a);
    case QT_ROCMFP4: return launch_kernel(k_grouped<QT_ROCMFP4, 1, GG_KB>, g, b, 0, stream, a);
    case QT_ROCMFP4_FAST: return launch_kernel(k_grouped<QT_ROCMFP4_FAST, 1, GG_KB>, g, b, 0, stream, a);
    }
    return hipErrorInvalidDeviceFunction;
}
