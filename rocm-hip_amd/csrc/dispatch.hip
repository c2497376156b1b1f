// dispatch.hip -- device-side token -> expert dispatch for the grouped prefill GEMM (gfx950, wave64).
//
// Semantics of the reference's moe_group (src/gpu_ops.hip:266-320): a histogram of the (token, slot) entries
// per expert, exclusive scans of the entry counts and of the tile counts ceil(count / tile), the tile table in
// expert order, and the entries grouped by expert (tok_rows = token, pair_rows = token * n_used + slot). The
// reference orders entries inside an expert's run by atomic slot (nondeterministic); here they are in ascending
// entry order, so the permutation is a pure function of ids.
//
// One workgroup of 16 waves. The permutation runs over chunks of 1024 tokens, one token per lane: each wave ORs
// its lanes into a 64-bit mask per expert in LDS (bit l = lane l's token chose that expert); an entry's rank in
// its expert's run is the running count from earlier chunks, plus the popcounts of the lower waves' masks, plus
// the popcount of its own wave's mask below its lane. A token's repeated id (a malformed row) and ids outside
// [0, n_expert) are skipped everywhere, so the counts, ranks and positions stay consistent.

#include "gpu_ops.h"
#include "host_common.h"
#include "moe_common.h"

#define GROUP_WAVES 16

// Whether entry j of the token's row is the first occurrence of a valid expert id
__device__ __forceinline__ bool group_valid(const int* row, int j, int ne) {
    const int e = row[j];
    if (e < 0 || e >= ne) return false;
    for (int k = 0; k < j; ++k)
        if (row[k] == e) return false;
    return true;
}

__global__ void __launch_bounds__(1024) k_moe_group(const int* ids, int T, int nu, int ne, int tile, int* tok_rows,
                                                    int* pair_rows, int* n_tiles, int* tile_e, int* tile_start,
                                                    int* tile_n) {
    extern __shared__ unsigned long long g_smem[];
    unsigned long long* masks = g_smem;                     // [GROUP_WAVES][ne]
    int* cnt = (int*)(masks + (size_t)GROUP_WAVES * ne);    // [ne] entry counts
    int* eoff = cnt + ne;                                   // [ne] first entry of each expert
    int* run = eoff + ne;                                   // [ne] entries placed by earlier chunks
    __shared__ int wpart[2][GROUP_WAVES];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;

    for (int e = tid; e < ne; e += 1024) cnt[e] = run[e] = 0;
    __syncthreads();
    const int n = T * nu;
    for (int i = tid; i < n; i += 1024) {
        const int t = i / nu, j = i - t * nu;
        if (group_valid(ids + (size_t)t * nu, j, ne)) atomicAdd(&cnt[ids[i]], 1);
    }
    __syncthreads();

    // exclusive scans over the experts, one expert per thread (ne <= 1024)
    const int c = tid < ne ? cnt[tid] : 0, nt = (c + tile - 1) / tile;
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
    int ba = 0, bb = 0;
    for (int k = 0; k < w; ++k) {
        ba += wpart[0][k];
        bb += wpart[1][k];
    }
    const int eo = ba + a - c, to = bb + b - nt;
    if (tid < ne) {
        eoff[tid] = eo;
        for (int k = 0; k < nt; ++k) {
            tile_e[to + k] = tid;
            tile_start[to + k] = eo + k * tile;
            tile_n[to + k] = min(tile, c - k * tile);
        }
        if (tid == ne - 1) *n_tiles = to + nt;
    }
    __syncthreads();

    unsigned long long* my = masks + (size_t)w * ne;
    const unsigned long long below = (1ull << lane) - 1ull;
    for (int t0 = 0; t0 < T; t0 += 1024) {
        for (int e = lane; e < ne; e += 64) my[e] = 0ull;
        __syncthreads();
        const int t = t0 + tid;
        const int* row = ids + (size_t)t * nu;
        if (t < T)
            for (int j = 0; j < nu; ++j)
                if (group_valid(row, j, ne)) atomicOr(&my[row[j]], 1ull << lane);
        __syncthreads();
        if (t < T)
            for (int j = 0; j < nu; ++j) {
                if (!group_valid(row, j, ne)) continue;
                const int e = row[j];
                int r = run[e] + __popcll(my[e] & below);
                for (int k = 0; k < w; ++k) r += __popcll(masks[(size_t)k * ne + e]);
                const int p = eoff[e] + r;
                tok_rows[p] = t;
                pair_rows[p] = t * nu + j;
            }
        __syncthreads();
        for (int e = tid; e < ne; e += 1024) {
            int s = 0;
            for (int k = 0; k < GROUP_WAVES; ++k) s += __popcll(masks[(size_t)k * ne + e]);
            run[e] += s;
        }
        __syncthreads();
    }
}

static size_t group_smem(int ne) { return (size_t)GROUP_WAVES * ne * 8 + 3 * (size_t)ne * 4; }

extern "C" hipError_t gpu_moe_group(const int* ids, int T, int n_used, int n_expert, int tile, int* tok_rows,
                                    int* pair_rows, int* n_tiles, int* tile_e, int* tile_start, int* tile_n,
                                    hipStream_t stream) {
    if (!moe_lib_ready()) return hipErrorNotInitialized;
    if (T <= 0 || n_used <= 0 || n_used > 64 || n_expert <= 0 || n_expert > 1024 || tile <= 0 ||
        (long long)T * n_used > 0x7fffffffLL)
        return hipErrorInvalidValue;
    const size_t shm = group_smem(n_expert);
    static bool attr_set = false;
    if (!attr_set) {
        const hipError_t e = hipFuncSetAttribute((const void*)k_moe_group, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)group_smem(1024));
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    return launch_kernel(k_moe_group, dim3(1), dim3(1024), shm, stream, ids, T, n_used, n_expert, tile, tok_rows,
                         pair_rows, n_tiles, tile_e, tile_start, tile_n);
}
