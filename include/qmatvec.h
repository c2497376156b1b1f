// qmatvec.h -- MI355X (gfx950) expert matvecs and grouped expert GEMMs behind the reference's qmatvec C ABI.
//
// Drop-in for the mixture-of-experts subset of CowboyTim/rocm-hip's src/qmatvec.h: same names, argument
// meaning, hipError_t conventions and asynchronous launches on the caller's stream. Types: Q8_0 (8), Q4_K (12),
// ROCmFP4 (100), ROCmFP4_FAST (101) on the int8 path; F32 (0) on the float path (the router logits).
// Pointers are device memory (hipMalloc). Weight matrices W are native GGUF rows (row_bytes =
// qt_row_size(type, K)); a matrix registered with qmatvec_pack_weights is read from its split-plane copy.
//
// Errors: hipErrorInvalidDeviceFunction for a type / K without a kernel, hipErrorInvalidValue for bad shapes,
// alignment or capacity, hipErrorNotInitialized before qmatvec_init.

#ifndef QMATVEC_H
#define QMATVEC_H

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// Replaces src/qmatvec.h:18-19. The kernels are linked into this library, so co_path is not read (NULL is
// fine); returns 0 when the current device is a gfx950, else -1.
int qmatvec_init(const char *co_path);
void qmatvec_free(void);

// Replaces src/qmatvec.h:25-26 (NVFP4's global scale). None of this library's types carries one: accepted and
// ignored, returns 0.
int qmatvec_set_out_scale(const void *owner, const void *W, size_t bytes, const float *s, int n);
void qmatvec_drop_out_scales(const void *owner);

// Replaces src/qmatvec.h:29: 1 if a float-path kernel exists for the type (F32 only).
int qmatvec_supported(int type);

// Replaces src/qmatvec.h:33-34: y[N] = W[N x K] x[K], F32 weights (the router logits).
hipError_t qmatvec_launch(int type, const void *W, size_t row_bytes, const float *x, float *y, int N, int K,
                          hipStream_t stream);

// Replaces src/qmatvec.h:39-40: the same for T rows of x [T][K] -> y [T][N] (prefill router logits).
hipError_t qmatvec_launch_batch(int type, const void *W, size_t row_bytes, const float *x, float *y, int N, int K,
                                int T, hipStream_t stream);

// ---------------------------------------------------------------- int8 path

// Replaces src/qmatvec.h:70-81 (same layout).
typedef struct qmatvec_q8 {
    int8_t *q0;    // Q8_0 values [K]
    float *d0;     // Q8_0 scales [K / 32] (FP16-rounded)
    int8_t *qK;    // Q8_K values [K]
    float *dK;     // Q8_K scales [K / 256]
    int32_t *bsK;  // Q8_K sums of every 16 values [K / 16]
    int32_t *s0;   // per 32 values: ggml's Q8_1 s, F16(d * sum of the block's q), as float bits
    int max_k;
    uint16_t *xh;  // optional (NULL: none): the values rounded to BF16 (xh_bf16) or F16 [K]
    int xh_bf16;
} qmatvec_q8;

// Replaces src/qmatvec.h:85-109: the output pointers as the quantizing kernels take them.
typedef struct qmatvec_q8_out {
    int8_t *q0;
    float *d0;
    int8_t *qK;
    float *dK;
    int32_t *bsK;
    int32_t *s0;
    uint16_t *xh;
    int xh_bf16;
} qmatvec_q8_out;

static inline qmatvec_q8_out qmatvec_q8_outputs(const qmatvec_q8 *q) {
    qmatvec_q8_out o = {0, 0, 0, 0, 0, 0, 0, 0};
    if (q) {
        o.q0 = q->q0;
        o.d0 = q->d0;
        o.qK = q->qK;
        o.dK = q->dK;
        o.bsK = q->bsK;
        o.s0 = q->s0;
        o.xh = q->xh;
        o.xh_bf16 = q->xh_bf16;
    }
    return o;
}

// Replaces src/qmatvec.h:113-114: device bytes a qmatvec_q8 for up to max_k values needs (max_k % 256 == 0),
// and binding it to such memory (16-byte aligned).
size_t qmatvec_q8_bytes(int max_k);
void qmatvec_q8_bind(qmatvec_q8 *q, void *mem, int max_k);

// Replaces src/qmatvec.h:118: 1 if an int8 kernel handles the type at this K (Q8_0 / ROCmFP4 / FAST: K % 32,
// Q4_K: K % 256).
int qmatvec_q8_supported(int type, int K);

// Replaces src/qmatvec.h:122: quantize x[K] into q (both formats). K % 32 == 0, K <= q->max_k.
hipError_t qmatvec_quantize(const float *x, int K, const qmatvec_q8 *q, hipStream_t stream);

// Replaces src/qmatvec.h:125-126: y = W x with x given by its quantized form q.
hipError_t qmatvec_launch_q8(int type, const void *W, size_t row_bytes, const qmatvec_q8 *q, float *y, int N, int K,
                             hipStream_t stream);

// Replaces src/qmatvec.h:129-130: y = W x (N rows), y2 = W2 x (N2 rows) in one launch.
hipError_t qmatvec_launch_q8_pair(int type, const void *W, int N, float *y, const void *W2, int N2, float *y2,
                                  size_t row_bytes, const qmatvec_q8 *q, int K, hipStream_t stream);

// Replaces src/qmatvec.h:148-149: Y[t] = W X[t] for T tokens, q holding the T inputs as one flattened [T * K]
// vector; row t of the result at y + t * ldy.
hipError_t qmatvec_launch_q8_batch(int type, const void *W, size_t row_bytes, const qmatvec_q8 *q, float *y,
                                   long long ldy, int N, int K, int T, hipStream_t stream);

// No counterpart in the reference (a test hook). Which kernel qmatvec_launch_q8_batch gives a registered matrix
// from T = 8 tokens: 0 (the default) the one estimated faster, the MFMA kernel (a chain of K / 128 stages, its
// weights read once per 64 tokens) or the matvec kernel (the weights once per token); 1 always the MFMA kernel;
// 2 always the matvec kernel. Process-wide; the outputs agree within fp32 reordering either way.
void qmatvec_dense_mfma_mode(int mode);

// Replaces src/qmatvec.h:156-157. Mixture-of-experts matvecs with the expert choice read from device memory:
// W stacks every expert's N rows; for token t and slot j < n_used, expert e = ids[t * n_used + j] multiplies
// input row t (x_per_slot = 0) or t * n_used + j (x_per_slot = 1) of q into row t * n_used + j of y.
// T = 2..4 reads each distinct expert's weights once for all the tokens that chose it.
hipError_t qmatvec_launch_q8_id(int type, const void *W, size_t row_bytes, const int32_t *ids, int n_used,
                                int x_per_slot, const qmatvec_q8 *q, float *y, int N, int K, int T, hipStream_t stream);
// Replaces src/qmatvec.h:159-161: two stacked matrices of one shape and type on the same input (W -> y, W2 -> y2).
hipError_t qmatvec_launch_q8_id_pair(int type, const void *W, const void *W2, size_t row_bytes, const int32_t *ids,
                                     int n_used, int x_per_slot, const qmatvec_q8 *q, float *y, float *y2, int N, int K,
                                     int T, hipStream_t stream);
// Replaces src/qmatvec.h:164-166: an id of -1 selects one more N-row matrix Wx (W2x for the second), e.g. the
// shared expert as one more slot.
hipError_t qmatvec_launch_q8_id_x(int type, const void *W, const void *W2, const void *Wx, const void *W2x,
                                  size_t row_bytes, const int32_t *ids, int n_used, int x_per_slot,
                                  const qmatvec_q8 *q, float *y, float *y2, int N, int K, int T, hipStream_t stream);

// Replaces src/qmatvec.h:175-180. MoE prefill on the tiles of gpu_moe_group: tile k < *n_tiles covers
// tile_n[k] <= tile entries of expert tile_e[k], entries tile_start[k] .. of in_rows (rows of q) and out_rows
// (rows of y, N values each). qmatvec_id_batch_tile: the largest tile the kernel for this matrix takes.
int qmatvec_id_batch_tile(int type, int N, int K);
int qmatvec_q8_id_batch_supported(int type, int K);
hipError_t qmatvec_launch_q8_id_batch(int type, const void *W, size_t row_bytes, const qmatvec_q8 *q, float *y, int N,
                                      int K, int max_tiles, int tile, const int32_t *n_tiles, const int32_t *tile_e,
                                      const int32_t *tile_start, const int32_t *tile_n, const int32_t *in_rows,
                                      const int32_t *out_rows, hipStream_t stream);

// ---------------------------------------------------------------- split-plane weights (additive)
// No counterpart in the reference (its UMA engine reads GGUF blocks in place). Registers the matrix at W
// (rows native rows of row_size(type, K) bytes, device memory) and builds its split-plane copy on the stream:
// per row, the value bytes of every block in one plane and the scale bytes in another, so that each lane
// streams 16-byte loads. The launchers above then read the copy for any W inside the registered range. The
// caller keeps W unchanged while registered; qmatvec_unpack_weights(W) frees the copy. Q8_0 / ROCmFP4 / FAST / Q4_K
// matrices of whole 32-row groups (K % 256 == 0) also get the prefill MFMA kernels' operand tiles (Q8_0: the
// native size; the FP4 types: ~1.56 times it; Q4_K ~1.67 times). Device memory per registered matrix: native +
// planes + tiles.
hipError_t qmatvec_pack_weights(int type, const void *W, size_t row_bytes, long long rows, int K, hipStream_t stream);
// The same with flags (0: as qmatvec_pack_weights):
//   QMATVEC_PACK_INPLACE: the split planes replace the native rows in W itself (no copy: every launcher reads the
//     planes, and a launch that would need W's native rows -- together with a matrix that is not registered --
//     returns hipErrorInvalidValue). The call waits for the rewrite, done in row chunks through a transient buffer of
//     the matrix's scale bytes plus 16 MiB (never a full copy); qmatvec_unpack_weights(W) writes the native rows
//     back the same way before it returns. If the transient buffer cannot be had, W is left untouched: the pack
//     returns the error unregistered, the unpack returns it with the registration still in force. A failure after
//     W has been partly rewritten leaves the matrix registered as unreadable (every launch that would touch it
//     returns hipErrorInvalidValue) and returns the error; unregistering it then frees it without a restore.
//   QMATVEC_PACK_NO_TILES: no operand tiles (prefill then runs the per-entry kernels on the planes).
// Device memory held per matrix, W included: default 3x native for Q8_0 (3.56x FP4, 3.67x Q4_K); INPLACE 2x
// (2.56x, 2.67x); INPLACE | NO_TILES 1x.
#define QMATVEC_PACK_INPLACE 1
#define QMATVEC_PACK_NO_TILES 2
hipError_t qmatvec_pack_weights_ex(int type, void *W, size_t row_bytes, long long rows, int K, int flags,
                                   hipStream_t stream);
// Unregisters W (see above); hipSuccess also for a W that is not registered.
hipError_t qmatvec_unpack_weights(const void *W);
// No counterpart in the reference (a test hook). The next fail_allocs transient buffers of in-place registration
// and unregistration fail as out of memory; chunk_bytes sets the rewrite's row chunk (0: 16 MiB). Process-wide.
void qmatvec_test_registry(int fail_allocs, long long chunk_bytes);
// Device bytes the split-plane copy of such a matrix takes (the same as the native rows).
size_t qmatvec_packed_bytes(int type, long long rows, int K);
// Device bytes a registration with these flags allocates besides W (the copy and / or the tiles); 0 for a bad
// type, shape or flag
size_t qmatvec_registered_bytes(int type, long long rows, int K, int flags);

#ifdef __cplusplus
}
#endif

#endif  // QMATVEC_H
