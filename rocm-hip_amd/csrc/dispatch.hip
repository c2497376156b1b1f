// dispatch.hip -- device-side token -> expert dispatch for the grouped prefill GEMM (gfx950, wave64).
//
// Semantics of the reference's moe_group (src/gpu_ops.hip:266-320): a histogram of the (token, slot) entries
// per expert, exclusive scans of the entry counts and of the tile counts ceil(count / tile), the tile table in
// expert order, and the entries grouped by expert (tok_rows = token, pair_rows = token * n_used + slot). The
// reference orders entries inside an expert's run by atomic slot (nondeterministic); here they are in ascending
// entry order, so the permutation is a pure function of ids.
//
// One workgroup of 8 waves; tokens in chunks of 512, one token per lane. Every entry of a token's row carries its
// occurrence index: how many earlier entries of the row hold the same expert id (0 for every entry of a row without
// repeats). The chunk is processed in levels k = 0 .. (largest occurrence index): at level k each wave ORs its lanes
// into a 64-bit mask per expert in LDS (bit l: lane l's row holds at least k + 1 entries of that expert); one
// thread per expert then turns the masks into the wave prefixes and the chunk's count. Summed over the levels, a
// wave prefix plus the popcount of the wave's mask below a lane is the number of that expert's entries in the
// chunk's earlier tokens. Pass 1 sums the counts over the chunks (then the scans and the tile table); pass 2
// places each entry at its expert's first entry + the entries of earlier chunks + that sum + its occurrence index,
// which is ascending entry order within every expert's run. A row without repeats takes one level: one mask per
// expert, as a plain histogram would. Ids outside [0, n_expert) are skipped.

#include <atomic>

#include "gpu_ops.h"
#include "host_common.h"
#include "moe_common.h"

#define GROUP_WAVES 8

// A token's row in registers: pk[j] = id | occurrence index << 16 for a valid entry, -1 otherwise (and for
// entries past nu, and for a token past T). NM = 8, 16 or 64: the smallest that holds n_used (<= 64).
// Returns the row's number of levels (largest occurrence index + 1; 0 for no valid entry). The loads are
// unconditional within a live row: under a per-id branch each one had waited for the previous.
// (row: a valid row even for a token past T -- the caller clamps it -- so that every load is unconditional: loads
// under the live condition had compiled to branches that waited for each pair before issuing the next)
template <int NM>
__device__ __forceinline__ void group_row_load(const int* row, int nu, bool live, int (&r)[NM]) {
#pragma unroll
    for (int j = 0; j < NM; ++j) {
        const int v = row[min(j, nu - 1)];
        r[j] = live ? v : -1;
    }
}
template <int NM>
__device__ __forceinline__ int group_row_keys(const int (&r)[NM], int nu, int ne, int (&pk)[NM]) {
    int lv = 0;
#pragma unroll
    for (int j = 0; j < NM; ++j) {
        const bool ok = j < nu && r[j] >= 0 && r[j] < ne;
        int occ = 0;
#pragma unroll
        for (int k = 0; k < j; ++k) occ += r[k] == r[j] ? 1 : 0;
        pk[j] = ok ? (r[j] | occ << 16) : -1;
        lv = ok ? max(lv, occ + 1) : lv;
    }
    return lv;
}
template <int NM>
__device__ __forceinline__ int group_row(const int* row, int nu, int ne, bool live, int (&pk)[NM]) {
    int r[NM];
    group_row_load<NM>(row, nu, live, r);
    return group_row_keys<NM>(r, nu, ne, pk);
}

// The largest of the workgroup's lv (LDS word *slot, which the caller set to 0 before a barrier)
__device__ __forceinline__ int group_levels(int lv, int* slot) {
    if (lv > 1) atomicMax(slot, lv);
    __syncthreads();
    const int l = max(*slot, 1);
    return l;
}

// One level of the masks: clears this wave's masks, ORs the lanes whose row has an entry of occurrence index k,
// then (one thread per expert) the wave prefixes pre[w][e] and the level's count of each expert, added to
// cnt_add[e] when cnt_add is not null. Ends with a barrier.
template <int WAVES, int NM>
__device__ __forceinline__ void group_level(const int (&pk)[NM], int k, int ne, unsigned long long* masks,
                                            uint16_t* pre, int* cnt_add) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    unsigned long long* my = masks + (size_t)w * ne;
    for (int e = lane; e < ne; e += 64) my[e] = 0ull;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NM; ++j)
        if (pk[j] >= 0 && (pk[j] >> 16) == k) atomicOr(&my[pk[j] & 0xffff], 1ull << lane);
    __syncthreads();
    for (int e = tid; e < ne; e += 64 * WAVES) {
        int s = 0;
#pragma unroll
        for (int q = 0; q < WAVES; ++q) {
            pre[(size_t)q * ne + e] = (uint16_t)s;
            s += __popcll(masks[(size_t)q * ne + e]);
        }
        if (cnt_add) cnt_add[e] += s;
    }
    __syncthreads();
}

// acc[j] += the entries of entry j's expert in the lower lanes' and waves' rows at this level (after group_level)
template <int NM>
__device__ __forceinline__ void group_accumulate(const int (&pk)[NM], int ne, const unsigned long long* masks,
                                                 const uint16_t* pre, int (&acc)[NM]) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const unsigned long long below = (1ull << lane) - 1ull;
#pragma unroll
    for (int j = 0; j < NM; ++j)
        if (pk[j] >= 0) {
            const int e = pk[j] & 0xffff;
            acc[j] += pre[(size_t)w * ne + e] + __popcll(masks[(size_t)w * ne + e] & below);
        }
}

template <int NM>
__global__ void __launch_bounds__(64 * GROUP_WAVES) k_moe_group(const int* ids, int T, int nu, int ne, int tile,
                                                                int* tok_rows, int* pair_rows, int* n_tiles,
                                                                int* tile_e, int* tile_start, int* tile_n) {
    extern __shared__ unsigned long long g_smem[];
    constexpr int NT = 64 * GROUP_WAVES;
    unsigned long long* masks = g_smem;                            // [GROUP_WAVES][ne]
    uint16_t* pre = (uint16_t*)(masks + (size_t)GROUP_WAVES * ne);  // [GROUP_WAVES][ne] wave prefixes
    int* cnt = (int*)(pre + (size_t)GROUP_WAVES * ne);             // [ne] entry counts (16 ne bytes in)
    int* eoff = cnt + ne;                                          // [ne] first entry of each expert
    int* run = eoff + ne;                                          // [ne] entries of earlier chunks
    int* ctot = run + ne;                                          // [ne] entries of the current chunk
    __shared__ int wpart[2][GROUP_WAVES];
    __shared__ int lvmax;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;

    for (int e = tid; e < ne; e += NT) cnt[e] = run[e] = ctot[e] = 0;
    // pass 0: counts; pass 1: placement
    for (int pass = 0; pass < 2; ++pass) {
        for (int t0 = 0; t0 < T; t0 += NT) {
            if (tid == 0) lvmax = 0;
            __syncthreads();
            const int t = t0 + tid;
            int pk[NM], acc[NM];
            const int levels = group_levels(group_row<NM>(ids + (size_t)min(t, T - 1) * nu, nu, ne, t < T, pk), &lvmax);
#pragma unroll
            for (int j = 0; j < NM; ++j) acc[j] = 0;
            for (int k = 0; k < levels; ++k) {
                group_level<GROUP_WAVES, NM>(pk, k, ne, masks, pre, pass == 0 ? cnt : ctot);
                if (pass == 1) group_accumulate<NM>(pk, ne, masks, pre, acc);
            }
            if (pass == 1) {
#pragma unroll
                for (int j = 0; j < NM; ++j)
                    if (pk[j] >= 0) {
                        const int e = pk[j] & 0xffff;
                        const int p = eoff[e] + run[e] + acc[j] + (pk[j] >> 16);
                        tok_rows[p] = t;
                        pair_rows[p] = t * nu + j;
                    }
                __syncthreads();
                for (int e = tid; e < ne; e += NT) {
                    run[e] += ctot[e];
                    ctot[e] = 0;
                }
            }
            __syncthreads();
        }
        if (pass == 1) break;
        // exclusive scans over the experts (entries and tiles), one expert per thread and round
        int ca = 0, cb = 0;  // carries of earlier rounds
        for (int e0 = 0; e0 < ne; e0 += NT) {
            const int e = e0 + tid;
            const int c = e < ne ? cnt[e] : 0, nt = (c + tile - 1) / tile;
            int a = c, b = nt;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const int ua = __shfl_up(a, d, 64), ub = __shfl_up(b, d, 64);
                if (lane >= d) {
                    a += ua;
                    b += ub;
                }
            }
            if (lane == 63) {
                wpart[0][w] = a;
                wpart[1][w] = b;
            }
            __syncthreads();
            int ba = ca, bb = cb;
            for (int k = 0; k < w; ++k) {
                ba += wpart[0][k];
                bb += wpart[1][k];
            }
            const int eo = ba + a - c, to = bb + b - nt;
            if (e < ne) {
                eoff[e] = eo;
                for (int k = 0; k < nt; ++k) {
                    tile_e[to + k] = e;
                    tile_start[to + k] = eo + k * tile;
                    tile_n[to + k] = min(tile, c - k * tile);
                }
                if (e == ne - 1) *n_tiles = to + nt;
            }
            for (int k = 0; k < GROUP_WAVES; ++k) {
                ca += wpart[0][k];
                cb += wpart[1][k];
            }
            __syncthreads();
        }
    }
}

// ---- Several workgroups, with a workspace (gpu_moe_group_ws): the same outputs. Tokens in blocks of 256 (4
// waves, one token per lane).
//   k_group_count: per block, the 64-bit expert masks of its 4 waves level by level, then per expert the block's
//                  entry count into ws[block][expert];
//   k_group_place: per block, from the counts: each expert's total and this block's offset within the expert's
//                  run (the blocks before it), the exclusive scan over the experts (their first entries; block
//                  0 also scans the tile counts and writes the tile table, k_moe_group's rules); then the masks
//                  again, level by level, and each entry's position: the expert's first entry + the block's
//                  offset + the summed wave prefixes and popcounts below its lane + its occurrence index. (Every block redoes
//                  the scans over at most 1,024 experts: cheaper than a launch between the two kernels.)
#define GB_WAVES 4

template <int NM>
__global__ void __launch_bounds__(64 * GB_WAVES) k_group_count(const int* ids, int T, int nu, int ne, int* ws) {
    extern __shared__ unsigned long long g_smem[];
    unsigned long long* masks = g_smem;
    uint16_t* pre = (uint16_t*)(masks + (size_t)GB_WAVES * ne);  // [GB_WAVES][ne]
    int* bc = (int*)(pre + (size_t)GB_WAVES * ne);                // [ne] the block's counts
    __shared__ int lvmax;
    const int tid = threadIdx.x, t = blockIdx.x * 64 * GB_WAVES + tid;
    for (int e = tid; e < ne; e += 64 * GB_WAVES) bc[e] = 0;
    if (tid == 0) lvmax = 0;
    __syncthreads();
    int pk[NM];
    const int levels = group_levels(group_row<NM>(ids + (size_t)min(t, T - 1) * nu, nu, ne, t < T, pk), &lvmax);
    for (int k = 0; k < levels; ++k) group_level<GB_WAVES, NM>(pk, k, ne, masks, pre, bc);
    for (int e = tid; e < ne; e += 64 * GB_WAVES) ws[(size_t)blockIdx.x * ne + e] = bc[e];
}

// Exclusive scan of v[0..n) in place by the 256-thread workgroup (4 consecutive values a thread), n <= 1024;
// returns the total. part: 4 ints of LDS.
__device__ int block256_exscan(int* v, int n, int* part) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    int x[4], s = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        x[k] = 4 * tid + k < n ? v[4 * tid + k] : 0;
        s += x[k];
    }
    int inc = s;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int u = __shfl_up(inc, d, 64);
        if (lane >= d) inc += u;
    }
    if (lane == 63) part[w] = inc;
    __syncthreads();
    int run = inc - s;
    for (int k = 0; k < w; ++k) run += part[k];
    const int total = (part[0] + part[1]) + (part[2] + part[3]);
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (4 * tid + k < n) {
            v[4 * tid + k] = run;
            run += x[k];
        }
    __syncthreads();
    return total;
}

template <int NM>
__global__ void __launch_bounds__(64 * GB_WAVES) k_group_place(const int* ids, int T, int nu, int ne, int tile,
                                                               const int* ws, int nblk, int* tok_rows, int* pair_rows,
                                                               int* n_tiles, int* tile_e, int* tile_start,
                                                               int* tile_n) {
    extern __shared__ unsigned long long g_smem[];
    unsigned long long* masks = g_smem;
    uint16_t* pre = (uint16_t*)(masks + (size_t)GB_WAVES * ne);  // [GB_WAVES][ne]
    int* eoff = (int*)(pre + (size_t)GB_WAVES * ne);              // [ne] the experts' first entries
    int* boff = eoff + ne;                                        // [ne] this block's offset in each run
    int* tot = boff + ne;                                         // [ne] block 0: the experts' totals
    int* tsc = tot + ne;                                          // [ne] block 0: tile counts, then first tiles
    __shared__ int part[4];
    __shared__ int lvmax;
    const int tid = threadIdx.x, t = blockIdx.x * 64 * GB_WAVES + tid;
    // this thread's row of ids loaded first: those loads fly with the count table's
    int r[NM];
    group_row_load<NM>(ids + (size_t)min(t, T - 1) * nu, nu, t < T, r);
    if (tid == 0) lvmax = 0;  // (visible after the barrier below)
    for (int e = tid; e < ne; e += 64 * GB_WAVES) {
        int off = 0, all = 0;
        for (int b0 = 0; b0 < nblk; b0 += 8) {  // eight blocks' counts loaded at once (clamped: unconditional loads)
            int c[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) c[q] = ws[(size_t)min(b0 + q, nblk - 1) * ne + e];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int b = b0 + q, v = b < nblk ? c[q] : 0;
                off += b < (int)blockIdx.x ? v : 0;
                all += v;
            }
        }
        boff[e] = off;
        eoff[e] = all;
        if (blockIdx.x == 0) {
            tot[e] = all;
            tsc[e] = (all + tile - 1) / tile;
        }
    }
    __syncthreads();
    block256_exscan(eoff, ne, part);
    if (blockIdx.x == 0) {  // the tile table (uniform branch)
        const int nt = block256_exscan(tsc, ne, part);
        for (int e = tid; e < ne; e += 64 * GB_WAVES) {
            const int c = tot[e], k0 = tsc[e];
            for (int k = 0; k * tile < c; ++k) {
                tile_e[k0 + k] = e;
                tile_start[k0 + k] = eoff[e] + k * tile;
                tile_n[k0 + k] = min(tile, c - k * tile);
            }
        }
        if (tid == 0) *n_tiles = nt;
    }
    int pk[NM], acc[NM];
    const int levels = group_levels(group_row_keys<NM>(r, nu, ne, pk), &lvmax);
#pragma unroll
    for (int j = 0; j < NM; ++j) acc[j] = 0;
    for (int k = 0; k < levels; ++k) {
        group_level<GB_WAVES, NM>(pk, k, ne, masks, pre, nullptr);
        group_accumulate<NM>(pk, ne, masks, pre, acc);
    }
#pragma unroll
    for (int j = 0; j < NM; ++j)
        if (pk[j] >= 0) {
            const int e = pk[j] & 0xffff;
            const int p = eoff[e] + boff[e] + acc[j] + (pk[j] >> 16);
            tok_rows[p] = t;
            pair_rows[p] = t * nu + j;
        }
}

extern "C" size_t gpu_moe_group_ws_bytes(int T, int n_expert) {
    if (T <= 0 || n_expert <= 0) return 0;
    const size_t nblk = ((size_t)T + 64 * GB_WAVES - 1) / (64 * GB_WAVES);
    return nblk * (size_t)n_expert * 4;
}

extern "C" hipError_t gpu_moe_group_ws(const int* ids, int T, int n_used, int n_expert, int tile, int* tok_rows,
                                       int* pair_rows, int* n_tiles, int* tile_e, int* tile_start, int* tile_n,
                                       void* ws, size_t ws_bytes, hipStream_t stream) {
    if (!moe_lib_ready()) return hipErrorNotInitialized;
    if (T <= 0 || n_used <= 0 || n_used > 64 || n_expert <= 0 || n_expert > 1024 || tile <= 0 ||
        (long long)T * n_used > 0x7fffffffLL || !ws || ws_bytes < gpu_moe_group_ws_bytes(T, n_expert) ||
        ((uintptr_t)ws & 3))
        return hipErrorInvalidValue;
    const int nblk = (T + 64 * GB_WAVES - 1) / (64 * GB_WAVES);
    int* cnt = (int*)ws;
    const size_t shm_m = (size_t)GB_WAVES * n_expert * (8 + 2), shm_c = shm_m + (size_t)n_expert * 4,
                 shm_p = shm_m + 4 * (size_t)n_expert * 4;
    hipError_t e = launch_kernel(n_used > 16 ? k_group_count<64> : n_used > 8 ? k_group_count<16> : k_group_count<8>,
                                 dim3(nblk), dim3(64 * GB_WAVES), shm_c, stream, ids, T, n_used, n_expert, cnt);
    if (e == hipSuccess)
        e = launch_kernel(n_used > 16 ? k_group_place<64> : n_used > 8 ? k_group_place<16> : k_group_place<8>,
                          dim3(nblk), dim3(64 * GB_WAVES), shm_p,
                          stream, ids, T, n_used, n_expert, tile, (const int*)cnt, nblk, tok_rows, pair_rows, n_tiles,
                          tile_e, tile_start, tile_n);
    return e;
}

static size_t group_smem(int ne) {
    return (size_t)GROUP_WAVES * ne * 8 + (size_t)GROUP_WAVES * ne * 2 + 4 * (size_t)ne * 4;
}

extern "C" hipError_t gpu_moe_group(const int* ids, int T, int n_used, int n_expert, int tile, int* tok_rows,
                                    int* pair_rows, int* n_tiles, int* tile_e, int* tile_start, int* tile_n,
                                    hipStream_t stream) {
    if (!moe_lib_ready()) return hipErrorNotInitialized;
    if (T <= 0 || n_used <= 0 || n_used > 64 || n_expert <= 0 || n_expert > 1024 || tile <= 0 ||
        (long long)T * n_used > 0x7fffffffLL)
        return hipErrorInvalidValue;
    const size_t shm = group_smem(n_expert);
    static std::atomic<bool> attr_set{false};  // (setting it twice from racing threads is harmless)
    if (!attr_set.load(std::memory_order_acquire)) {
        for (const void* f : {(const void*)k_moe_group<8>, (const void*)k_moe_group<16>, (const void*)k_moe_group<64>}) {
            const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)group_smem(1024));
            if (e != hipSuccess) return e;
        }
        attr_set.store(true, std::memory_order_release);
    }
    return launch_kernel(n_used > 16 ? k_moe_group<64> : n_used > 8 ? k_moe_group<16> : k_moe_group<8>, dim3(1), dim3(64 * GROUP_WAVES), shm, stream,
                         ids, T, n_used, n_expert, tile, tok_rows, pair_rows, n_tiles, tile_e, tile_start, tile_n);
}
