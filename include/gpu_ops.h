// gpu_ops.h -- MI355X (gfx950) router, dispatch, SwiGLU and combine behind the reference's gpu_ops C ABI.
//
// Drop-in for the mixture-of-experts subset of CowboyTim/rocm-hip's src/gpu_ops.h: same names, argument
// meaning and hipError_t conventions. Pointers are device memory; launches are asynchronous on `stream`.

#ifndef GPU_OPS_H
#define GPU_OPS_H

#include <hip/hip_runtime.h>

#include "qmatvec.h"

#ifdef __cplusplus
extern "C" {
#endif

// Replaces src/gpu_ops.h:17-18 (kernels are linked in; co_path is not read). 0 on a gfx950 device, else -1.
int gpu_ops_init(const char* co_path);
void gpu_ops_free(void);

// Replaces src/gpu_ops.h:24-25: for each of T rows of n values, x_out = x_in + add, then y = RMSNorm(x_out) * w
// (w NULL: no gamma); add NULL: y = RMSNorm(x_in) * w and x_out unwritten. q8 set: the T rows of y are quantized
// into it as one flattened [T * n] vector (n % 256 == 0, T * n <= q8->max_k).
hipError_t gpu_add_rmsnorm(const float* x_in, const float* add, float* x_out, const float* w, float* y, int n, int T,
                           float eps, const qmatvec_q8* q8, hipStream_t stream);

// Replaces src/gpu_ops.h:29: out = SiLU(g) * u, quantized into q8 when set (n % 32 == 0).
hipError_t gpu_swiglu(const float* g, const float* u, float* out, int n, const qmatvec_q8* q8, hipStream_t stream);

// Replaces src/gpu_ops.h:36-37: per token, softmax over n_expert logits, the n_used largest in descending order
// (ties to the lower index), their weights renormalised by max(sum, 6.103515625e-5), and sg = sigmoid(x . w_shexp)
// when w_shexp is set. n_expert <= 1024, n_used <= 64. ids_stride (0: n_used) > n_used: the entry after the
// selection is set to -1 (the shared expert as one more slot).
hipError_t gpu_moe_router(const float* logits, const float* x, const float* w_shexp, int* ids, float* wts, float* sg,
                          int n_expert, int n_used, int n, int T, hipStream_t stream, int ids_stride);

// Replaces src/gpu_ops.h:40-41: out [T][n] = sum_j wts[t][j] * down[t][j] (slot order) + sg[t] * shared[t].
hipError_t gpu_moe_combine(const float* down, const float* wts, const float* shared, const float* sg, float* out,
                           int n_used, int n, int T, hipStream_t stream);
// Replaces src/gpu_ops.h:44-46: each expert's output scaled by exp_scale[ids[t][j]] first (NULL: none); shared
// NULL: no shared expert.
hipError_t gpu_moe_combine_scaled(const float* down, const float* wts, const float* shared, const float* sg,
                                  const int* ids, const float* exp_scale, float* out, int n_used, int n, int T,
                                  hipStream_t stream);

// Replaces src/gpu_ops.h:72-77. Group T tokens' selected experts (ids [T][n_used]) by expert: entries sorted by
// expert, and within an expert by entry index t * n_used + j (deterministic); tok_rows[i] = token,
// pair_rows[i] = t * n_used + j. Each expert's run is cut into tiles of up to `tile` entries (tile_e,
// tile_start, tile_n; *n_tiles of them, in expert order), which need gpu_moe_max_tiles entries. Ids outside
// [0, n_expert) and repeats of an expert within one token's row are skipped.
static inline int gpu_moe_max_tiles(int T, int n_used, int n_expert, int tile) {
    const int n = T * n_used, bound = n_expert + n / tile;
    return n < bound ? n : bound;
}
hipError_t gpu_moe_group(const int* ids, int T, int n_used, int n_expert, int tile, int* tok_rows, int* pair_rows,
                         int* n_tiles, int* tile_e, int* tile_start, int* tile_n, hipStream_t stream);

// No counterpart in the reference (additive). gpu_moe_group with a caller workspace of gpu_moe_group_ws_bytes(T,
// n_expert) bytes (4-byte aligned): the same outputs bit for bit, from several workgroups (per-block counts, one
// scan, per-block placement) instead of one.
size_t gpu_moe_group_ws_bytes(int T, int n_expert);
hipError_t gpu_moe_group_ws(const int* ids, int T, int n_used, int n_expert, int tile, int* tok_rows,
                            int* pair_rows, int* n_tiles, int* tile_e, int* tile_start, int* tile_n, void* ws,
                            size_t ws_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif  // GPU_OPS_H
