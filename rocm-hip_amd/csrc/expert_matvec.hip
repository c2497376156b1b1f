// expert_matvec.hip -- decode expert matvecs (and the dense / per-entry variants) on gfx950, wave64, plus the
// split-plane weight registry and the C-ABI launchers of the int8 path.
//
// Kernel shape: a workgroup of four waves; in a wave, groups of L lanes (L in {8, 16, 32, 64}) each own one
// weight row at a time and R rows in flight (the R rows' loads are issued together). Lane gl of a group takes
// the row's units gl, gl + L, ...; the group then sums its lanes. Each unit's integer dot is exact; the float
// terms are added per lane and then by an xor tree over the group.
//
// Expert indirection (src/matvec_q.hip:1905-1933): slot j of token t uses expert e = ids[t * n_used + j] (rows
// e * N .. of W), input row t (x_per_slot 0) or t * n_used + j (1), output row t * n_used + j; grid.y >=
// n_used selects the second matrix (W2 -> y2); e = -1 selects the extra matrix Wx / W2x.

#include <atomic>
#include <map>
#include <mutex>

#include "expert_units.h"
#include "grouped.h"
#include "host_common.h"
#include "qmatvec.h"

struct MvArgs {
    const uint8_t* v[4];  // W, W2, Wx, W2x: native rows, or the value planes of their split-plane copies
    const uint8_t* s[4];  // scale planes (split-plane only)
    long long vrb, srb;   // bytes per row in the value / scale plane (native: row_bytes, 0)
    const int* ids;       // nullptr: dense (no expert choice)
    int n_used, x_per_slot;
    const int8_t* xq;  // activations: int8 values, scales, Q8_K sums
    const float* xd;
    const int* xbs;
    float* y;
    float* y2;
    long long ldy;  // output row stride (id mode: N)
    int N, N2, K;
};

template <int TYPE>
__device__ __forceinline__ void act_row(const MvArgs& a, long long in_row, const int8_t*& xq, const float*& xd,
                                        const int*& xbs) {
    xq = a.xq + in_row * a.K;
    xd = a.xd + in_row * (a.K / (Fmt<TYPE>::Q8K ? 256 : 32));
    xbs = Fmt<TYPE>::Q8K ? a.xbs + in_row * (a.K / 16) : nullptr;
}

// grid (row blocks, n_used * (1 or 2) slots, T tokens) in id mode; (row blocks, 1 or 2 matrices, T) dense
// NT: the weights as nontemporal loads (each row read once per launch: decode, one token or the id launches); the
// dense batches of several tokens re-read the matrix per token from L2 and take ordinary loads
template <int TYPE, bool PACKED, int L, int R, int NUPL, bool NT>
__global__ void __launch_bounds__(256) k_expert_mv(MvArgs a) {
    constexpr int G = 64 / L;  // row groups per wave
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int gl = lane & (L - 1), grp = lane / L;
    const int row0 = (blockIdx.x * 4 + wv) * (R * G) + grp;
    const int t = blockIdx.z;
    int slot, mi, e;
    long long out_row;
    if (a.ids) {
        const bool m2 = (int)blockIdx.y >= a.n_used;
        slot = blockIdx.y - (m2 ? a.n_used : 0);
        e = wave_uniform(a.ids[(long long)t * a.n_used + slot]);
        mi = (e >= 0 ? 0 : 2) + (m2 ? 1 : 0);
        out_row = (long long)t * a.n_used + slot;
    } else {
        slot = 0;
        e = 0;
        mi = blockIdx.y;
        out_row = t;
    }
    const int nrows = mi & 1 ? a.N2 : a.N;
    if (row0 - grp >= nrows) return;  // the whole wave is past the end (uniform per wave)
    const long long rbase = e >= 0 ? (long long)e * nrows : 0;
    const uint8_t* vbase = pick(a.v, mi) + rbase * a.vrb;
    const uint8_t* sbase = PACKED ? pick(a.s, mi) + rbase * a.srb : nullptr;
    const long long in_row = a.ids && a.x_per_slot ? (long long)t * a.n_used + slot : t;
    const int8_t* xq;
    const float* xd;
    const int* xbs;
    act_row<TYPE>(a, in_row, xq, xd, xbs);
    float acc[R];
    rows_dot<TYPE, PACKED, L, R, NUPL>(vbase, sbase, a.vrb, a.srb, row0, G, nrows, xq, xd, xbs, a.K, gl, acc, NT);
    if (gl == 0) {
        float* y = (mi & 1 ? a.y2 : a.y) + out_row * a.ldy;
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (row0 + r * G < nrows) y[row0 + r * G] = acc[r];
    }
}

// Prefill per-entry kernel on gpu_moe_group's tiles: grid (row blocks, max_tiles). Each entry of the tile gets
// the sum the decode kernel would give it (the weights are re-read per entry from L2).
template <int TYPE, bool PACKED, int L, int R>
__global__ void __launch_bounds__(256) k_expert_entries(MvArgs a, const int* n_tiles, const int* tile_e,
                                                        const int* tile_start, const int* tile_n, const int* in_rows,
                                                        const int* out_rows) {
    constexpr int G = 64 / L;
    const int k = blockIdx.y;
    if (k >= *n_tiles) return;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int gl = lane & (L - 1), grp = lane / L;
    const int row0 = (blockIdx.x * 4 + wv) * (R * G) + grp;
    if (row0 - grp >= a.N) return;
    const long long rbase = (long long)tile_e[k] * a.N;
    const uint8_t* vbase = a.v[0] + rbase * a.vrb;
    const uint8_t* sbase = PACKED ? a.s[0] + rbase * a.srb : nullptr;
    const int st = tile_start[k], cnt = tile_n[k];
    for (int i = 0; i < cnt; ++i) {
        const int8_t* xq;
        const float* xd;
        const int* xbs;
        act_row<TYPE>(a, in_rows[st + i], xq, xd, xbs);
        float acc[R];
        rows_dot<TYPE, PACKED, L, R, 0>(vbase, sbase, a.vrb, a.srb, row0, G, a.N, xq, xd, xbs, a.K, gl, acc,
                                        false);  // (the rows are re-read per entry: ordinary loads keep them in L2)
        if (gl == 0) {
            float* y = a.y + (long long)out_rows[st + i] * a.N;
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (row0 + r * G < a.N) y[row0 + r * G] = acc[r];
        }
    }
}

// ------------------------------------------------------------------ split-plane copies

// One thread per native block (32 values; 256 for Q4_K). UNPACK = false: native rows W -> planes V / S; true: the
// inverse (planes -> native rows, for unregistering a matrix packed in place)
template <int TYPE, bool UNPACK = false>
__global__ void __launch_bounds__(256) k_pack(const uint8_t* W, long long row_bytes, long long rows, int K, uint8_t* V,
                                              uint8_t* S) {
    constexpr int BV = TYPE == QT_Q4_K ? 256 : 32, BB = Fmt<TYPE>::BLOCK_BYTES;
    const int nb = K / BV;
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * nb) return;
    const long long r = i / nb;
    const int b = (int)(i - r * nb);
    uint8_t* src = (uint8_t*)W + r * row_bytes + (long long)b * BB;
    uint8_t* vr = V + r * fmt_value_row(TYPE, K);
    uint8_t* sr = S + r * fmt_scale_row(TYPE, K);
    // moves one byte between its native place n and its plane place p, in the direction of UNPACK
    auto mv = [](uint8_t& n, uint8_t& p) {
        if constexpr (UNPACK)
            n = p;
        else
            p = n;
    };
    if constexpr (TYPE == QT_Q8_0) {
        mv(src[0], sr[2 * b]);
        mv(src[1], sr[2 * b + 1]);
        for (int j = 0; j < 16; ++j) {
            mv(src[2 + j], vr[16 * b + j]);
            mv(src[18 + j], vr[16 * (nb + b) + j]);
        }
    } else if constexpr (TYPE == QT_ROCMFP4) {
        for (int j = 0; j < 16; ++j) mv(src[j], vr[16 * b + j]);
        mv(src[16], sr[2 * b]);
        mv(src[17], sr[2 * b + 1]);
    } else if constexpr (TYPE == QT_ROCMFP4_FAST) {
        for (int j = 0; j < 16; ++j) mv(src[j], vr[16 * b + j]);
        mv(src[16], sr[b]);
    } else {  // Q4_K: head -> scale plane, chunk c (32 value bytes) -> unit 4b + c in the two half planes
        const int nu = K / 64;
        for (int j = 0; j < 16; ++j) mv(src[j], sr[16 * b + j]);
        for (int c = 0; c < 4; ++c) {
            const int u = 4 * b + c;
            for (int j = 0; j < 16; ++j) {
                mv(src[16 + 32 * c + j], vr[16 * u + j]);
                mv(src[16 + 32 * c + 16 + j], vr[16 * (nu + u) + j]);
            }
        }
    }
}

// ------------------------------------------------------------------ MFMA operand tiles (prefill kernels)
//
// A second copy of a Q8_0 / ROCmFP4 / FAST matrix in the order the grouped MFMA kernels' lanes read it, so that
// each 64-lane load of it is one contiguous run instead of 64 pieces of 64 rows. Per group of 32 rows g and block
// b, one run of 64 lane slots, slot l for row 32 g + l % 32 and K half h = l / 32:
//   Q8_0:      16-byte slots: the block's int8 values 16 h .. 16 h + 15 (the int8 MFMA's A);
//   FP4 types: 12-byte slots: the block's values 8 h .. 8 h + 7, then 16 + 8 h .. + 7 (the f16 MFMAs' A of each
//              16-value half), each as the FP6 E2M3 code of codebook value / 2, 6 bits per value from bit 0 up;
//   Q4_K:      the same 12-byte slots per 32-value sub-block, each code the FP6 E2M3 of quant / 2 (quant 0..15);
//              both stage-major: the four slots of a lane for blocks 4 s .. 4 s + 3 as 48 contiguous bytes, split
//              in three 16-byte chunks, chunk i at 1024 i + 16 l of the stage's 3 KB (three coalesced loads a stage).
// Scale tiles, per group g and 8-block group q (Q4_K: super-block), 32 row slots: Q8_0 16 bytes (8 blocks' FP16 d);
// FP4 types 32 bytes (per block the FP16 pair (e0, e1) of its UE4M3 half-scales, FAST (e, e)); Q4_K 32 bytes, 16
// per 128-value half c: the sub-block scales sc_4c..sc_4c+3 and mins m_4c..m_4c+3 as bytes, the FP16 d and dmin,
// 4 zero bytes.
__device__ __forceinline__ uint32_t fp4_code(const uint8_t* qs, int v) {  // code of value v (0..31) of a block
    return v < 16 ? (qs[v] & 0x0fu) : (qs[v - 16] >> 4);
}
// The E2M3 code of codebook value / 2 for a 4-bit code (sign bit 3): magnitudes {0, 1, 2, 3, 4, 6, 8, 10} / 2 are
// E2M3 0, 0.5 (subnormal 4/8), 1, 1.5, 2, 3, 4, 5 (1.25 x 4)
__device__ __forceinline__ uint32_t fp4_to_e2m3(uint32_t c) {
    const uint8_t tab[8] = {0x00, 0x04, 0x08, 0x0c, 0x10, 0x14, 0x18, 0x1a};
    return tab[c & 7] | ((c & 8) << 2);  // E2M3 sign is bit 5
}
// The E2M3 code of q / 2 for a Q4_K quant q (0..15): 0, 0.5 (subnormal 4/8), then (1 + m / 8) 2^(e - 1):
// 1, 1.5 (e 1), 2, 2.5, 3, 3.5 (e 2), 4, 4.5, .., 7.5 (e 3)
__device__ __forceinline__ uint32_t q4_to_e2m3(uint32_t q) {
    const uint8_t tab[16] = {0, 4, 8, 12, 16, 18, 20, 22, 24, 25, 26, 27, 28, 29, 30, 31};
    return tab[q & 15];
}
// Value v (0..255) of a Q4_K super-block: the low nibble of byte 32 c + l of the quants for v = 64 c + l (l < 32),
// the high nibble for v = 64 c + 32 + l
__device__ __forceinline__ uint32_t q4k_quant(const uint8_t* blk, int v) {
    const uint8_t b = blk[16 + 32 * (v >> 6) + (v & 31)];
    return (v & 32) ? (b >> 4) : (b & 15u);
}

template <int TYPE>
__global__ void __launch_bounds__(256) k_pack_tiles(const uint8_t* W, long long row_bytes, long long rows, int K,
                                                    uint8_t* V, uint8_t* S) {
    constexpr int BB = Fmt<TYPE>::BLOCK_BYTES;
    constexpr int SS = TYPE == QT_Q8_0 ? 16 : 12;  // value slot bytes
    const int nb = K / 32;
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    const long long nslots = rows / 32 * nb * 64;
    if (i < nslots) {  // value slot (g, block b, lane l)
        const int l = (int)(i & 63), h = l >> 5;
        const long long gb = i >> 6, g = gb / nb;
        const int b = (int)(gb - g * nb);
        // the native block holding block b (Q4_K: super-block b / 8, of which b is sub-block b % 8)
        const uint8_t* blk = W + (32 * g + (l & 31)) * row_bytes + (long long)(TYPE == QT_Q4_K ? b >> 3 : b) * BB;
        uint8_t* dst = V + SS * i;
        if constexpr (TYPE != QT_Q8_0)  // stage-major: byte p of the lane's 48 for the stage (4 blocks)
            dst = V + (long long)g * nb * 768 + 3072 * (b >> 2) + 16 * l;
        if constexpr (TYPE == QT_Q8_0) {
            for (int j = 0; j < 16; ++j) dst[j] = blk[2 + 16 * h + j];
        } else {
            uint32_t w[3] = {0u, 0u, 0u};
            for (int n = 0; n < 16; ++n) {
                const int v = (n < 8 ? 8 * h : 16 + 8 * h) + (n & 7);
                uint32_t f;
                if constexpr (TYPE == QT_Q4_K)
                    f = q4_to_e2m3(q4k_quant(blk, 32 * (b & 7) + v));
                else
                    f = fp4_to_e2m3(fp4_code(blk, v));
                const int bit = 6 * n;
                w[bit >> 5] |= f << (bit & 31);
                if ((bit & 31) > 26) w[(bit >> 5) + 1] |= f >> (32 - (bit & 31));
            }
            for (int j = 0; j < 12; ++j) {
                const int p = 12 * (b & 3) + j;
                dst[1024 * (p >> 4) + (p & 15)] = (uint8_t)(w[j >> 2] >> (8 * (j & 3)));
            }
        }
        return;
    }
    const long long k = i - nslots;  // scale slot (row r, 8-block group q)
    const int nq = nb / 8;
    if (k >= rows * nq) return;
    const long long r = k / nq;
    const int q = (int)(k - r * nq);
    const uint8_t* row = W + r * row_bytes;
    constexpr int SB = TYPE == QT_Q8_0 ? 16 : TYPE == QT_Q4_K ? Q4K_TILE_SLOT : 32;  // slot bytes
    uint8_t* dst = S + ((r / 32) * nq + q) * (32 * SB) + (r & 31) * SB;
    if constexpr (TYPE == QT_Q4_K) {  // super-block q, per half c: sc_4c..+3, m_4c..+3 (bytes), d, dmin, zeros
        const uint8_t* blk = row + (long long)q * BB;
        uint32_t sw[3];
        for (int j = 0; j < 3; ++j)
            sw[j] = (uint32_t)blk[4 + 4 * j] | (uint32_t)blk[5 + 4 * j] << 8 | (uint32_t)blk[6 + 4 * j] << 16 |
                    (uint32_t)blk[7 + 4 * j] << 24;
        for (int j = 0; j < 8; ++j) {
            int sc, mn;
            q4k_scale_min(j, sw, sc, mn);
            dst[16 * (j >> 2) + (j & 3)] = (uint8_t)sc;
            dst[16 * (j >> 2) + 4 + (j & 3)] = (uint8_t)mn;
        }
        for (int c = 0; c < 2; ++c) {
            for (int j = 0; j < 4; ++j) dst[16 * c + 8 + j] = blk[j];  // d, dmin (FP16)
            for (int j = 12; j < 16; ++j) dst[16 * c + j] = 0;
        }
        return;
    }
    for (int b = 0; b < 8; ++b) {
        const uint8_t* blk = row + (long long)(8 * q + b) * BB;
        if constexpr (TYPE == QT_Q8_0) {
            dst[2 * b] = blk[0];
            dst[2 * b + 1] = blk[1];
        } else {
            const uint16_t e0 = __half_as_ushort(__float2half(ue4m3_half(blk[16])));
            const uint16_t e1 = TYPE == QT_ROCMFP4 ? __half_as_ushort(__float2half(ue4m3_half(blk[17]))) : e0;
            *(uint32_t*)(dst + 4 * b) = (uint32_t)e0 | (uint32_t)e1 << 16;
        }
    }
}

namespace {

struct Packed {
    uintptr_t end;
    int type, K;
    size_t row_bytes;
    long long rows;
    uint8_t* mem;    // value plane, then scale plane (packed in place: the native buffer W itself)
    uint8_t* tiles;  // MFMA operand tiles (value tiles, then scale tiles), or nullptr
    bool inplace;    // the planes replaced the native rows in W
    uint8_t* alloc;  // the device memory the registration allocated (planes and / or tiles), or nullptr
    bool broken;     // an in-place rewrite is under way or failed part-way: W holds neither layout whole, so no
                     // launch may read it (find_* miss it, packed_in_place names it)
};

// Whether a registered matrix also gets MFMA operand tiles: a type of the MFMA kernels, whole 32-row groups and
// whole 8-block scale groups
bool tiles_ok(int type, long long rows, int K) {
    return (type == QT_Q8_0 || type == QT_ROCMFP4 || type == QT_ROCMFP4_FAST || type == QT_Q4_K) && rows % 32 == 0 &&
           K % 256 == 0;
}

std::mutex g_pack_mu;
std::map<uintptr_t, Packed> g_packed;  // keyed by the native W's start address

size_t native_row(int type, int K) {
    switch (type) {
    case QT_Q8_0: return K % 32 ? 0 : (size_t)K / 32 * 34;
    case QT_ROCMFP4: return K % 32 ? 0 : (size_t)K / 32 * 18;
    case QT_ROCMFP4_FAST: return K % 32 ? 0 : (size_t)K / 32 * 17;
    case QT_Q4_K: return K % 256 ? 0 : (size_t)K / 256 * 144;
    default: return 0;
    }
}

// The split-plane copy covering the native row pointer W (value and scale rows), or false
bool find_packed(const void* W, int type, int K, size_t row_bytes, const uint8_t** v, const uint8_t** s) {
    if (!W) return false;
    std::lock_guard<std::mutex> lk(g_pack_mu);
    auto it = g_packed.upper_bound((uintptr_t)W);
    if (it == g_packed.begin()) return false;
    --it;
    const Packed& p = it->second;
    const uintptr_t off = (uintptr_t)W - it->first;
    if ((uintptr_t)W >= p.end || p.broken || p.type != type || p.K != K || p.row_bytes != row_bytes ||
        off % row_bytes)
        return false;
    const long long row = (long long)(off / row_bytes);
    *v = p.mem + row * fmt_value_row(type, K);
    *s = p.mem + (size_t)p.rows * fmt_value_row(type, K) + row * fmt_scale_row(type, K);
    return true;
}

// The MFMA operand tiles of the registered matrix whose native rows start at W (at a 32-row group boundary): the
// value tiles and scale tiles of W's first row group and their bytes per 32-row group (and, when rows_from_w is
// given, the registered rows from W on), or false
bool find_tiles(const void* W, int type, int K, size_t row_bytes, const uint8_t** vt, const uint8_t** st,
                long long* vgs, long long* sgs, long long* rows_from_w = nullptr) {
    if (!W) return false;
    std::lock_guard<std::mutex> lk(g_pack_mu);
    auto it = g_packed.upper_bound((uintptr_t)W);
    if (it == g_packed.begin()) return false;
    --it;
    const Packed& p = it->second;
    const uintptr_t off = (uintptr_t)W - it->first;
    if ((uintptr_t)W >= p.end || p.broken || !p.tiles || p.type != type || p.K != K || p.row_bytes != row_bytes ||
        off % (32 * row_bytes))
        return false;
    const long long g = (long long)(off / (32 * row_bytes));
    *vt = p.tiles + g * 32 * tile_value_row(type, K);
    *st = p.tiles + (size_t)p.rows * tile_value_row(type, K) + g * 32 * tile_scale_row(type, K);
    *vgs = 32ll * tile_value_row(type, K);
    *sgs = 32ll * tile_scale_row(type, K);
    if (rows_from_w) *rows_from_w = p.rows - 32 * g;
    return true;
}

// Lanes per row L and units per lane NUPL: the largest L in {64, 32, 16, 8} that splits the row's units evenly
// into at most 4 per lane (then every load is issued up front); else the largest L not above the unit count,
// with a loop over units (NUPL 0)
struct MvShape {
    int L, nupl;
};
MvShape mv_shape(int type, int K) {
    const int nu = fmt_units(type, K);
    for (int L = 64; L >= 8; L /= 2)
        if (nu % L == 0 && nu / L <= 4) return {L, nu / L};
    int L = 64;
    while (L > 8 && L > nu) L /= 2;
    return {L, 0};
}
int lanes_for(int type, int K) { return mv_shape(type, K).L; }

// Rows in flight per lane group: about four loads of weights per lane
constexpr int rows_in_flight(int L, int nupl) { return nupl >= 4 ? 1 : nupl >= 2 ? 2 : nupl == 1 ? 4 : (L == 64 ? 4 : 2); }
int rows_per_block(int L, int nupl) { return 4 * rows_in_flight(L, nupl) * (64 / L); }

template <int TYPE, bool PACKED, int L, int NUPL>
hipError_t launch_mv_l(const MvArgs& a, dim3 yz, int nrows, hipStream_t st) {
    constexpr int R = rows_in_flight(L, NUPL);
    const int rpb = 4 * R * (64 / L);
    const dim3 g((nrows + rpb - 1) / rpb, yz.y, yz.z), b(256);
    if (a.ids || yz.z == 1) return launch_kernel(k_expert_mv<TYPE, PACKED, L, R, NUPL, true>, g, b, 0, st, a);
    return launch_kernel(k_expert_mv<TYPE, PACKED, L, R, NUPL, false>, g, b, 0, st, a);
}

template <int TYPE, bool PACKED, int L>
hipError_t launch_mv_n(const MvArgs& a, dim3 yz, int nupl, int nrows, hipStream_t st) {
    if constexpr (PACKED) {
        switch (nupl) {
        case 1: return launch_mv_l<TYPE, PACKED, L, 1>(a, yz, nrows, st);
        case 2: return launch_mv_l<TYPE, PACKED, L, 2>(a, yz, nrows, st);
        case 3: return launch_mv_l<TYPE, PACKED, L, 3>(a, yz, nrows, st);
        case 4: return launch_mv_l<TYPE, PACKED, L, 4>(a, yz, nrows, st);
        }
    }
    return launch_mv_l<TYPE, PACKED, L, 0>(a, yz, nrows, st);
}

template <int TYPE, bool PACKED>
hipError_t launch_mv_t(const MvArgs& a, dim3 yz, MvShape sh, int nrows, hipStream_t st) {
    switch (sh.L) {
    case 64: return launch_mv_n<TYPE, PACKED, 64>(a, yz, sh.nupl, nrows, st);
    case 32: return launch_mv_n<TYPE, PACKED, 32>(a, yz, sh.nupl, nrows, st);
    case 16: return launch_mv_n<TYPE, PACKED, 16>(a, yz, sh.nupl, nrows, st);
    default: return launch_mv_n<TYPE, PACKED, 8>(a, yz, sh.nupl, nrows, st);
    }
}

template <int TYPE, bool PACKED>
hipError_t launch_entries_t(const MvArgs& a, int max_tiles, int L, const int32_t* n_tiles, const int32_t* tile_e,
                            const int32_t* tile_start, const int32_t* tile_n, const int32_t* in_rows,
                            const int32_t* out_rows, hipStream_t st) {
    const dim3 g((a.N + rows_per_block(L, 0) - 1) / rows_per_block(L, 0), max_tiles), b(256);
#define ENTRIES_CASE(LL)                                                                                             \
    return launch_kernel(k_expert_entries<TYPE, PACKED, LL, rows_in_flight(LL, 0)>, g, b, 0, st, a, n_tiles, tile_e, \
                         tile_start, tile_n, in_rows, out_rows)
    switch (L) {
    case 64: ENTRIES_CASE(64);
    case 32: ENTRIES_CASE(32);
    case 16: ENTRIES_CASE(16);
    default: ENTRIES_CASE(8);
    }
#undef ENTRIES_CASE
}

hipError_t launch_mv(int type, bool packed, const MvArgs& a, dim3 yz, int nrows, hipStream_t st) {
    const MvShape sh = mv_shape(type, a.K);
    switch (type) {
    case QT_Q8_0: return packed ? launch_mv_t<QT_Q8_0, true>(a, yz, sh, nrows, st) : launch_mv_t<QT_Q8_0, false>(a, yz, sh, nrows, st);
    case QT_ROCMFP4: return packed ? launch_mv_t<QT_ROCMFP4, true>(a, yz, sh, nrows, st) : launch_mv_t<QT_ROCMFP4, false>(a, yz, sh, nrows, st);
    case QT_ROCMFP4_FAST: return packed ? launch_mv_t<QT_ROCMFP4_FAST, true>(a, yz, sh, nrows, st) : launch_mv_t<QT_ROCMFP4_FAST, false>(a, yz, sh, nrows, st);
    case QT_Q4_K: return packed ? launch_mv_t<QT_Q4_K, true>(a, yz, sh, nrows, st) : launch_mv_t<QT_Q4_K, false>(a, yz, sh, nrows, st);
    }
    return hipErrorInvalidDeviceFunction;
}

// Whether the registered matrix covering W (if any) was packed in place: its native rows are gone
bool packed_in_place(const void* W) {
    std::lock_guard<std::mutex> lk(g_pack_mu);
    auto it = g_packed.upper_bound((uintptr_t)W);
    if (it == g_packed.begin()) return false;
    --it;
    return (uintptr_t)W < it->second.end && it->second.inplace;
}

// Fill the weight side of a: every non-null matrix from its split-plane copy if all of them have one, else all
// native. Returns 1 when the copies are used, 0 for native rows, -1 when the matrices cannot be read together (one
// packed in place, which has no native rows left, with one that is not registered for this shape).
int bind_weights(MvArgs& a, int type, int K, size_t row_bytes, const void* const W[4]) {
    const uint8_t* v[4] = {nullptr, nullptr, nullptr, nullptr};
    const uint8_t* s[4] = {nullptr, nullptr, nullptr, nullptr};
    bool all = true;
    for (int i = 0; i < 4; ++i)
        if (W[i] && !find_packed(W[i], type, K, row_bytes, &v[i], &s[i])) all = false;
    if (!all)
        for (int i = 0; i < 4; ++i)
            if (W[i] && packed_in_place(W[i])) return -1;
    for (int i = 0; i < 4; ++i) {
        a.v[i] = all ? v[i] : (const uint8_t*)W[i];
        a.s[i] = all ? s[i] : nullptr;
    }
    a.vrb = all ? fmt_value_row(type, K) : (long long)row_bytes;
    a.srb = all ? fmt_scale_row(type, K) : 0;
    return all ? 1 : 0;
}

void bind_acts(MvArgs& a, int type, const qmatvec_q8* q) {
    const bool kq = type == QT_Q4_K;
    a.xq = kq ? q->qK : q->q0;
    a.xd = kq ? q->dK : q->d0;
    a.xbs = kq ? q->bsK : nullptr;
}

}  // namespace

// ------------------------------------------------------------------ C ABI

extern "C" int qmatvec_q8_supported(int type, int K) {
    if (K <= 0) return 0;
    switch (type) {
    case QT_Q8_0:
    case QT_ROCMFP4:
    case QT_ROCMFP4_FAST: return K % 32 == 0;
    case QT_Q4_K: return K % 256 == 0;
    default: return 0;
    }
}

extern "C" size_t qmatvec_packed_bytes(int type, long long rows, int K) {
    const size_t rb = native_row(type, K);
    return rows > 0 ? rb * (size_t)rows : 0;
}

// Bytes of the split-plane copy (value plane + scale plane)
static size_t packed_planes_bytes(int type, long long rows, int K) {
    return (size_t)rows * (size_t)(fmt_value_row(type, K) + fmt_scale_row(type, K));
}

template <int TYPE>
static hipError_t launch_tiles(const void* W, size_t rb, long long rows, int K, uint8_t* tiles, hipStream_t st) {
    const long long nt = rows / 32 * (K / 32) * 64 + rows * (K / 256);
    return launch_kernel(k_pack_tiles<TYPE>, dim3((unsigned)((nt + 255) / 256)), dim3(256), 0, st, (const uint8_t*)W,
                         (long long)rb, rows, K, tiles, tiles + (size_t)rows * tile_value_row(TYPE, K));
}

// Native rows W (rows of rb bytes) -> value rows at V and scale rows at S
template <int TYPE>
static hipError_t launch_pack(const void* W, size_t rb, long long rows, int K, uint8_t* V, uint8_t* S,
                              hipStream_t st) {
    constexpr int BV = TYPE == QT_Q4_K ? 256 : 32;
    const long long n = rows * (K / BV);
    return launch_kernel(k_pack<TYPE, false>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, (const uint8_t*)W,
                         (long long)rb, rows, K, V, S);
}

// Value rows V and scale rows S -> native rows W (unregistering a matrix packed in place)
template <int TYPE>
static hipError_t launch_unpack(uint8_t* W, size_t rb, long long rows, int K, const uint8_t* V, const uint8_t* S,
                                hipStream_t st) {
    constexpr int BV = TYPE == QT_Q4_K ? 256 : 32;
    const long long n = rows * (K / BV);
    return launch_kernel(k_pack<TYPE, true>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, (const uint8_t*)W,
                         (long long)rb, rows, K, (uint8_t*)V, (uint8_t*)S);
}

static hipError_t tiles_type(int type, const void* W, size_t rb, long long rows, int K, uint8_t* tiles,
                             hipStream_t st) {
#define CALL_(T) launch_tiles<T>(W, rb, rows, K, tiles, st)
    switch (type) {
    case QT_Q8_0: return CALL_(QT_Q8_0);
    case QT_ROCMFP4: return CALL_(QT_ROCMFP4);
    case QT_ROCMFP4_FAST: return CALL_(QT_ROCMFP4_FAST);
    default: return CALL_(QT_Q4_K);
    }
#undef CALL_
}

static hipError_t pack_type(int type, const void* W, size_t rb, long long rows, int K, uint8_t* V, uint8_t* S,
                            hipStream_t st) {
#define CALL_(T) launch_pack<T>(W, rb, rows, K, V, S, st)
    switch (type) {
    case QT_Q8_0: return CALL_(QT_Q8_0);
    case QT_ROCMFP4: return CALL_(QT_ROCMFP4);
    case QT_ROCMFP4_FAST: return CALL_(QT_ROCMFP4_FAST);
    default: return CALL_(QT_Q4_K);
    }
#undef CALL_
}

static hipError_t unpack_type(int type, uint8_t* W, size_t rb, long long rows, int K, const uint8_t* V,
                              const uint8_t* S, hipStream_t st) {
#define CALL_(T) launch_unpack<T>(W, rb, rows, K, V, S, st)
    switch (type) {
    case QT_Q8_0: return CALL_(QT_Q8_0);
    case QT_ROCMFP4: return CALL_(QT_ROCMFP4);
    case QT_ROCMFP4_FAST: return CALL_(QT_ROCMFP4_FAST);
    default: return CALL_(QT_Q4_K);
    }
#undef CALL_
}

// ---- in-place rewrites through bounded staging: the whole scale plane (1/17 of a Q8_0 or FAST matrix, 1/9 of a
// ROCmFP4 or Q4_K one) plus one chunk of rows, never a copy of the matrix
//
// Pack, rows ascending in chunks [a, b): the chunk's native rows are copied out, then its value rows written to
// [a vrow, b vrow). Those bytes held native rows below b only (vrow < rb), all consumed by now or in the chunk;
// the native rows at and past b (from b rb on) are untouched. The scale rows collect in the staging and land
// after the value plane at the end, over native bytes every chunk has already consumed.
// Unpack, the reverse, rows descending: the scale plane is copied out first; chunk [a, b)'s value rows are copied
// out and its native rows written to [a rb, b rb), which holds only value rows at and past a (a vrow <= a rb) --
// the chunk's own, already copied, and those of chunks done before it -- and the scale plane.

static std::atomic<int> g_fail_allocs{0};         // test hook: fail this many of the next staging allocations
static std::atomic<long long> g_chunk_bytes{16ll << 20};  // staging chunk (native bytes of whole rows)

static hipError_t staging_alloc(void** p, size_t n) {
    int f = g_fail_allocs.load();
    while (f > 0)
        if (g_fail_allocs.compare_exchange_weak(f, f - 1)) return hipErrorOutOfMemory;
    return hipMalloc(p, n);
}

static long long chunk_rows(size_t rb, long long rows) {
    const long long c = g_chunk_bytes.load() / (long long)rb;
    return c < 1 ? 1 : c > rows ? rows : c;
}

// *started: whether W has been written (a failure after that leaves W in neither layout)
static hipError_t pack_in_place(int type, uint8_t* W, size_t rb, long long rows, int K, hipStream_t st,
                                bool* started) {
    const size_t vrow = fmt_value_row(type, K), srow = fmt_scale_row(type, K);
    const long long C = chunk_rows(rb, rows);
    void* m = nullptr;
    hipError_t e = staging_alloc(&m, (size_t)rows * srow + (size_t)C * rb);
    if (e != hipSuccess) return e;
    uint8_t* sst = (uint8_t*)m;
    uint8_t* chunk = sst + (size_t)rows * srow;
    for (long long a = 0; a < rows && e == hipSuccess; a += C) {
        const long long n = rows - a < C ? rows - a : C;
        e = hipMemcpyAsync(chunk, W + (size_t)a * rb, (size_t)n * rb, hipMemcpyDeviceToDevice, st);
        *started = true;
        if (e == hipSuccess) e = pack_type(type, chunk, rb, n, K, W + (size_t)a * vrow, sst + (size_t)a * srow, st);
    }
    if (e == hipSuccess)
        e = hipMemcpyAsync(W + (size_t)rows * vrow, sst, (size_t)rows * srow, hipMemcpyDeviceToDevice, st);
    const hipError_t es = hipStreamSynchronize(st);  // the staging is freed next
    (void)hipFree(m);
    return e != hipSuccess ? e : es;
}

static hipError_t unpack_in_place(int type, uint8_t* W, size_t rb, long long rows, int K, bool* started) {
    const size_t vrow = fmt_value_row(type, K), srow = fmt_scale_row(type, K);
    const long long C = chunk_rows(rb, rows);
    void* m = nullptr;
    hipError_t e = staging_alloc(&m, (size_t)rows * srow + (size_t)C * vrow);
    if (e != hipSuccess) return e;
    uint8_t* sst = (uint8_t*)m;
    uint8_t* chunk = sst + (size_t)rows * srow;
    hipStream_t st = nullptr;  // the null stream, after a device synchronization
    e = hipMemcpyAsync(sst, W + (size_t)rows * vrow, (size_t)rows * srow, hipMemcpyDeviceToDevice, st);
    for (long long b = rows; b > 0 && e == hipSuccess; b -= C) {
        const long long a = b > C ? b - C : 0, n = b - a;
        e = hipMemcpyAsync(chunk, W + (size_t)a * vrow, (size_t)n * vrow, hipMemcpyDeviceToDevice, st);
        *started = true;
        if (e == hipSuccess) e = unpack_type(type, W + (size_t)a * rb, rb, n, K, chunk, sst + (size_t)a * srow, st);
    }
    const hipError_t es = hipStreamSynchronize(st);
    (void)hipFree(m);
    return e != hipSuccess ? e : es;
}

extern "C" void qmatvec_test_registry(int fail_allocs, long long chunk_bytes) {
    g_fail_allocs.store(fail_allocs > 0 ? fail_allocs : 0);
    g_chunk_bytes.store(chunk_bytes > 0 ? chunk_bytes : 16ll << 20);
}

static size_t tile_bytes_of(int type, long long rows, int K, int flags) {
    if ((flags & QMATVEC_PACK_NO_TILES) || !tiles_ok(type, rows, K)) return 0;
    return (size_t)rows * (size_t)(tile_value_row(type, K) + tile_scale_row(type, K));
}

extern "C" size_t qmatvec_registered_bytes(int type, long long rows, int K, int flags) {
    if (!qmatvec_q8_supported(type, K) || rows <= 0 || (flags & ~3)) return 0;
    return ((flags & QMATVEC_PACK_INPLACE) ? 0 : packed_planes_bytes(type, rows, K)) +
           tile_bytes_of(type, rows, K, flags);
}

extern "C" hipError_t qmatvec_pack_weights_ex(int type, void* W, size_t row_bytes, long long rows, int K, int flags,
                                              hipStream_t stream) {
    if (!moe_lib_ready()) return hipErrorNotInitialized;
    if (!qmatvec_q8_supported(type, K)) return hipErrorInvalidDeviceFunction;
    if (!W || rows <= 0 || row_bytes != native_row(type, K) || (flags & ~3)) return hipErrorInvalidValue;
    const size_t bytes = row_bytes * (size_t)rows;
    {
        std::lock_guard<std::mutex> lk(g_pack_mu);
        auto it = g_packed.lower_bound((uintptr_t)W);
        if (it != g_packed.end() && it->first < (uintptr_t)W + bytes) return hipErrorInvalidValue;  // overlap
        if (it != g_packed.begin() && std::prev(it)->second.end > (uintptr_t)W) return hipErrorInvalidValue;
    }
    const bool inplace = flags & QMATVEC_PACK_INPLACE;
    const size_t planes = packed_planes_bytes(type, rows, K);  // (== bytes: the planes hold the native bytes)
    const size_t tile_bytes = tile_bytes_of(type, rows, K, flags);
    const size_t keep = (inplace ? 0 : planes) + tile_bytes;  // what the registration holds
    uint8_t* alloc = nullptr;
    if (keep) {
        void* m = nullptr;
        const hipError_t e = hipMalloc(&m, keep);
        if (e != hipSuccess) return e;
        alloc = (uint8_t*)m;
    }
    uint8_t* tiles = tile_bytes ? alloc + (inplace ? 0 : planes) : nullptr;
    hipError_t e = hipSuccess;
    if (tiles) e = tiles_type(type, W, row_bytes, rows, K, tiles, stream);  // from the native rows, first
    bool started = false;  // (in place) whether W has been written
    if (e == hipSuccess) {
        if (!inplace)
            e = pack_type(type, W, row_bytes, rows, K, alloc, alloc + (size_t)rows * fmt_value_row(type, K), stream);
        else
            e = pack_in_place(type, (uint8_t*)W, row_bytes, rows, K, stream, &started);
    }
    if (e != hipSuccess && !started) {
        if (alloc) {
            (void)hipStreamSynchronize(stream);
            (void)hipFree(alloc);
        }
        return e;
    }
    // registered on success; after a failure part-way through an in-place rewrite, registered as broken, so that
    // no launch reads W as either layout (unregistering then drops it without a restore)
    std::lock_guard<std::mutex> lk(g_pack_mu);
    g_packed[(uintptr_t)W] = Packed{(uintptr_t)W + bytes, type, K, row_bytes, rows,
                                    inplace ? (uint8_t*)W : alloc, tiles, inplace, alloc, e != hipSuccess};
    return e;
}

extern "C" hipError_t qmatvec_pack_weights(int type, const void* W, size_t row_bytes, long long rows, int K,
                                           hipStream_t stream) {
    return qmatvec_pack_weights_ex(type, (void*)W, row_bytes, rows, K, 0, stream);
}

extern "C" hipError_t qmatvec_unpack_weights(const void* W) {
    Packed p;
    {
        std::lock_guard<std::mutex> lk(g_pack_mu);
        auto it = g_packed.find((uintptr_t)W);
        if (it == g_packed.end()) return hipSuccess;
        p = it->second;
        if (!p.inplace || p.broken) {
            g_packed.erase(it);
        } else {
            it->second.broken = true;  // no new launch reads it while the native rows come back
        }
    }
    // launches already queued on any stream may still read the copy (or, packed in place, W's planes)
    hipError_t e = hipDeviceSynchronize();
    if (p.inplace && !p.broken) {
        bool started = false;
        if (e == hipSuccess) e = unpack_in_place(p.type, (uint8_t*)W, p.row_bytes, p.rows, p.K, &started);
        std::lock_guard<std::mutex> lk(g_pack_mu);
        auto it = g_packed.find((uintptr_t)W);
        if (e != hipSuccess) {  // still registered: usable again if W was not touched, else broken
            if (it != g_packed.end()) it->second.broken = started;
            return e;
        }
        if (it != g_packed.end()) g_packed.erase(it);
    }
    if (p.alloc) (void)hipFree(p.alloc);
    return e;
}

// The per-operation kernels' lane shape for a row of K values (the fused layer kernel copies it)
void moe_mv_shape(int type, int K, int* lanes, int* units_per_lane) {
    const MvShape sh = mv_shape(type, K);
    *lanes = sh.L;
    *units_per_lane = sh.nupl;
}

// The split-plane rows of the registered matrix at W (for the fused layer kernel)
bool moe_packed_planes(const void* W, int type, int K, size_t row_bytes, const uint8_t** v, const uint8_t** s) {
    return find_packed(W, type, K, row_bytes, v, s);
}

// The MFMA operand tiles of the registered matrix at W (for the layer's grouped launches)
bool moe_packed_tiles(const void* W, int type, int K, size_t row_bytes, const uint8_t** vt, const uint8_t** st,
                      long long* vgs, long long* sgs) {
    return find_tiles(W, type, K, row_bytes, vt, st, vgs, sgs);
}

// Drop every registration (library teardown). Matrices packed in place keep their planes: W may already be gone
// here, so teardown writes nothing into it
void moe_unpack_all(void) {
    std::map<uintptr_t, Packed> all;
    {
        std::lock_guard<std::mutex> lk(g_pack_mu);
        all.swap(g_packed);
    }
    if (all.empty()) return;
    (void)hipDeviceSynchronize();
    for (auto& kv : all)
        if (kv.second.alloc) (void)hipFree(kv.second.alloc);
}

static hipError_t check_common(int type, const void* W, size_t row_bytes, const qmatvec_q8* q, int K,
                               long long in_rows) {
    if (!moe_lib_ready()) return hipErrorNotInitialized;
    if (!qmatvec_q8_supported(type, K)) return hipErrorInvalidDeviceFunction;
    if (!W || !q || row_bytes != native_row(type, K) || (row_bytes & 3) || !aligned(W, 4) ||
        in_rows * K > (long long)q->max_k)
        return hipErrorInvalidValue;
    return hipSuccess;
}

extern "C" hipError_t qmatvec_launch_q8_id_x(int type, const void* W, const void* W2, const void* Wx, const void* W2x,
                                             size_t row_bytes, const int32_t* ids, int n_used, int x_per_slot,
                                             const qmatvec_q8* q, float* y, float* y2, int N, int K, int T,
                                             hipStream_t stream) {
    // the reference's order (src/qmatvec.cpp:550-554): an unsupported type / K first, then shapes and capacity
    if (!moe_lib_ready()) return hipErrorNotInitialized;
    if (!qmatvec_q8_supported(type, K)) return hipErrorInvalidDeviceFunction;
    if (T <= 0 || n_used <= 0 || N <= 0 || !ids || !y || (W2 && !y2)) return hipErrorInvalidValue;
    const hipError_t c = check_common(type, W, row_bytes, q, K, (long long)T * (x_per_slot ? n_used : 1));
    if (c != hipSuccess) return c;
    if (!aligned(W2, 4) || !aligned(Wx, 4) || !aligned(W2x, 4)) return hipErrorInvalidValue;
    MvArgs a = {};
    const void* Ws[4] = {W, W2, Wx, W2 ? W2x : nullptr};
    const int bw = bind_weights(a, type, K, row_bytes, Ws);
    if (bw < 0) return hipErrorInvalidValue;
    const bool packed = bw > 0;
    bind_acts(a, type, q);
    a.ids = ids;
    a.n_used = n_used;
    a.x_per_slot = x_per_slot ? 1 : 0;
    a.y = y;
    a.y2 = y2;
    a.ldy = N;
    a.N = a.N2 = N;
    a.K = K;
    return launch_mv(type, packed, a, dim3(1, n_used * (W2 ? 2 : 1), T), N, stream);
}

extern "C" hipError_t qmatvec_launch_q8_id(int type, const void* W, size_t row_bytes, const int32_t* ids, int n_used,
                                           int x_per_slot, const qmatvec_q8* q, float* y, int N, int K, int T,
                                           hipStream_t stream) {
    return qmatvec_launch_q8_id_x(type, W, nullptr, nullptr, nullptr, row_bytes, ids, n_used, x_per_slot, q, y,
                                  nullptr, N, K, T, stream);
}

extern "C" hipError_t qmatvec_launch_q8_id_pair(int type, const void* W, const void* W2, size_t row_bytes,
                                                const int32_t* ids, int n_used, int x_per_slot, const qmatvec_q8* q,
                                                float* y, float* y2, int N, int K, int T, hipStream_t stream) {
    if (!W2) return hipErrorInvalidValue;
    return qmatvec_launch_q8_id_x(type, W, W2, nullptr, nullptr, row_bytes, ids, n_used, x_per_slot, q, y, y2, N, K,
                                  T, stream);
}

static hipError_t dense(int type, const void* W, int N, float* y, const void* W2, int N2, float* y2,
                        size_t row_bytes, const qmatvec_q8* q, int K, int T, long long ldy, hipStream_t stream) {
    if (N <= 0 || T <= 0 || !y || (W2 && (N2 <= 0 || !y2)) || ldy < N) return hipErrorInvalidValue;
    const hipError_t c = check_common(type, W, row_bytes, q, K, T);
    if (c != hipSuccess) return c;
    if (!aligned(W2, 4)) return hipErrorInvalidValue;
    MvArgs a = {};
    const void* Ws[4] = {W, W2, nullptr, nullptr};
    const int bw = bind_weights(a, type, K, row_bytes, Ws);
    if (bw < 0) return hipErrorInvalidValue;
    const bool packed = bw > 0;
    bind_acts(a, type, q);
    a.ids = nullptr;
    a.n_used = 1;
    a.y = y;
    a.y2 = y2;
    a.ldy = ldy;
    a.N = N;
    a.N2 = W2 ? N2 : 0;
    a.K = K;
    return launch_mv(type, packed, a, dim3(1, W2 ? 2 : 1, T), W2 && N2 > N ? N2 : N, stream);
}

extern "C" hipError_t qmatvec_launch_q8_pair(int type, const void* W, int N, float* y, const void* W2, int N2,
                                             float* y2, size_t row_bytes, const qmatvec_q8* q, int K,
                                             hipStream_t stream) {
    if (W2 && N2 > 0) {
        if (N2 != N) return hipErrorInvalidValue;  // one output stride for both (the two row counts match)
        return dense(type, W, N, y, W2, N2, y2, row_bytes, q, K, 1, N, stream);
    }
    return dense(type, W, N, y, nullptr, 0, nullptr, row_bytes, q, K, 1, N, stream);
}

extern "C" hipError_t qmatvec_launch_q8(int type, const void* W, size_t row_bytes, const qmatvec_q8* q, float* y,
                                        int N, int K, hipStream_t stream) {
    return dense(type, W, N, y, nullptr, 0, nullptr, row_bytes, q, K, 1, N, stream);
}

// A registered matrix runs T tokens on the MFMA kernel when that is estimated faster than the matvec kernel. The
// MFMA launch is a chain of K / 128 stages of ~1.8 us each whatever T, over (N / 128) ceil(T / 64) workgroups
// (about 768 resident at once); the matvec kernel reads the matrix once per token from L2, at ~18 TB/s for Q8_0 rows,
// ~9.5 for Q4_K and ~6 for the FP4 types (their decode). Measured (N 768, K 2048; Q4_K N 1024, K 3072), us per
// launch, matvec / MFMA: Q8_0 T 64 8.2 / 28.8, T 256 22.8 / 28.9, T 512 43.2 / 29.1; ROCmFP4 T 128 21.4 / 26.5,
// T 256 39.4 / 26.7; Q4_K T 128 25.9 / 41.5, T 256 47.5 / 41.9, T 2,427 387 / 55.6.
static bool dense_mfma_faster(int type, size_t row_bytes, int N, int K, int T) {
    const double items = (double)(N / 128) * ((T + 63) / 64), rounds = items <= 768 ? 1.0 : items / 768.0;
    const double t_mfma = K / 128 * 1.8 * rounds;
    const double bw = type == QT_Q8_0 ? 18e6 : type == QT_Q4_K ? 9.5e6 : 6e6;  // bytes per us
    const double t_mv = (double)T * N * (double)row_bytes / bw;
    return t_mfma < t_mv;
}

static std::atomic<int> g_dense_mode{0};
extern "C" void qmatvec_dense_mfma_mode(int mode) { g_dense_mode.store(mode, std::memory_order_relaxed); }

extern "C" hipError_t qmatvec_launch_q8_batch(int type, const void* W, size_t row_bytes, const qmatvec_q8* q, float* y,
                                              long long ldy, int N, int K, int T, hipStream_t stream) {
    const uint8_t *v = nullptr, *s = nullptr;
    long long vgs = 0, sgs = 0;
    const int mode = g_dense_mode.load(std::memory_order_relaxed);
    if (T >= 8 && mode != 2 && N > 0 && ldy >= N && y && check_common(type, W, row_bytes, q, K, T) == hipSuccess &&
        moe_grouped_mfma_ok(type, N, K) && (mode == 1 || dense_mfma_faster(type, row_bytes, N, K, T)) &&
        find_tiles(W, type, K, row_bytes, &v, &s, &vgs, &sgs))
        return moe_launch_dense_mfma(type, v, s, vgs, sgs, q, y, ldy, N, K, T, stream);
    return dense(type, W, N, y, nullptr, 0, nullptr, row_bytes, q, K, T, ldy, stream);
}

// Entry tiles of the grouped kernels (the MFMA kernel's 64; the per-entry fallback takes any)
#define ENTRY_TILE 64

static hipError_t moe_launch_entries(int type, const void* W, size_t row_bytes, const qmatvec_q8* q, float* y, int N,
                                     int K, int max_tiles, const int32_t* n_tiles, const int32_t* tile_e,
                                     const int32_t* tile_start, const int32_t* tile_n, const int32_t* in_rows,
                                     const int32_t* out_rows, hipStream_t stream) {
    MvArgs a = {};
    const void* Ws[4] = {W, nullptr, nullptr, nullptr};
    const int bw = bind_weights(a, type, K, row_bytes, Ws);
    if (bw < 0) return hipErrorInvalidValue;
    const bool packed = bw > 0;
    bind_acts(a, type, q);
    a.N = a.N2 = N;
    a.ldy = N;
    a.K = K;
    a.y = y;
    const int L = lanes_for(type, K);
#define ENT(TT)                                                                                                       \
    return packed ? launch_entries_t<TT, true>(a, max_tiles, L, n_tiles, tile_e, tile_start, tile_n, in_rows,        \
                                               out_rows, stream)                                                      \
                  : launch_entries_t<TT, false>(a, max_tiles, L, n_tiles, tile_e, tile_start, tile_n, in_rows,       \
                                                out_rows, stream)
    switch (type) {
    case QT_Q8_0: ENT(QT_Q8_0);
    case QT_ROCMFP4: ENT(QT_ROCMFP4);
    case QT_ROCMFP4_FAST: ENT(QT_ROCMFP4_FAST);
    case QT_Q4_K: ENT(QT_Q4_K);
    }
#undef ENT
    return hipErrorInvalidDeviceFunction;
}


// The MFMA kernel's tile where it can take the matrix (once registered), else the per-entry kernel's (any tile;
// 64 keeps its grids filled)
extern "C" int qmatvec_id_batch_tile(int type, int N, int K) {
    if (!qmatvec_q8_supported(type, K)) return 16;
    return moe_grouped_mfma_ok(type, N, K) ? moe_grouped_mfma_tile() : ENTRY_TILE;
}

extern "C" int qmatvec_q8_id_batch_supported(int type, int K) { return qmatvec_q8_supported(type, K); }

extern "C" hipError_t qmatvec_launch_q8_id_batch(int type, const void* W, size_t row_bytes, const qmatvec_q8* q,
                                                 float* y, int N, int K, int max_tiles, int tile,
                                                 const int32_t* n_tiles, const int32_t* tile_e,
                                                 const int32_t* tile_start, const int32_t* tile_n,
                                                 const int32_t* in_rows, const int32_t* out_rows, hipStream_t stream) {
    // the reference's order (src/qmatvec.cpp:601-604): an unsupported type / K first, then the rest
    if (!moe_lib_ready()) return hipErrorNotInitialized;
    if (!qmatvec_q8_supported(type, K)) return hipErrorInvalidDeviceFunction;
    if (N <= 0 || max_tiles <= 0 || tile <= 0 || tile > qmatvec_id_batch_tile(type, N, K) || !y || !n_tiles ||
        !tile_e || !tile_start || !tile_n || !in_rows || !out_rows)
        return hipErrorInvalidValue;
    if (!W || !q || row_bytes != native_row(type, K) || !aligned(W, 4)) return hipErrorInvalidValue;
    const uint8_t *v = nullptr, *s = nullptr;
    long long vgs = 0, sgs = 0, rows = 0;
    // Q4_K with fewer entries than 3/4 of the experts (max_tiles = gpu_moe_max_tiles(T, n_used, n_expert, tile) is
    // then T n_used, and the registration holds n_expert N rows from W): the per-entry kernel, whose rows go through
    // the sub-block decode once per entry, beats 64-entry MFMA tiles left mostly empty (config 3's layer shape,
    // gate + up + SwiGLU + down + routing: T 8 103 against 160 us, T 16 165 against 187, even at T 24 = 0.75 x 256 / 8)
    if (moe_grouped_mfma_ok(type, N, K) && find_tiles(W, type, K, row_bytes, &v, &s, &vgs, &sgs, &rows) &&
        (type != QT_Q4_K || 4ll * max_tiles >= 3 * (rows / N)))
        return moe_launch_grouped_mfma(type, v, s, vgs, sgs, q, y, N, K,
                                       max_tiles, n_tiles, tile_e, tile_start, tile_n, in_rows, out_rows, 0, nullptr,
                                       stream);
    return moe_launch_entries(type, W, row_bytes, q, y, N, K, max_tiles, n_tiles, tile_e, tile_start, tile_n, in_rows,
                              out_rows, stream);
}
