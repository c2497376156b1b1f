// moe_layer.h -- one mixture-of-experts FFN layer driven through the qmatvec / gpu_ops C ABI.
//
// The caller side of the path: the launch sequence of the reference's QwenModel::moe_core and moe_core_one
// (src/qwen_model.cpp:864-937), as a C entry point so that a harness (or the engine's forward pass) can run a
// whole layer with one call. Router logits (F32 matvec, or given), moe_router, then:
//   T == 1: the experts' gate/up in one launch (the shared expert as one more slot, id -1, when it has the
//           experts' width and type), SwiGLU quantized for down, down, moe_combine;
//   T 2..7: the same per token (each token's experts read once per token);
//   T >= 8: gpu_moe_group, the grouped gate / up / down on the expert tiles, the shared expert dense, combine.
// T <= 7 with every expert matrix registered (qmatvec_pack_weights) runs as three fused kernels with the same
// results bit for bit (T >= 2: each distinct expert's rows read once for all the tokens that chose it). All
// buffers are device memory; scratch is caller-owned (moe_layer_scratch_bytes). Asynchronous on `stream`.

#ifndef MOE_LAYER_H
#define MOE_LAYER_H

#include <hip/hip_runtime.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct moe_layer_desc {
    int type;          // expert weight type (gate, up and down share it): 8, 12, 100 or 101
    int n_embd;        // E
    int n_expert;      // NE
    int n_used;        // NU
    int n_ff;          // FE (the shared expert, when present, has the same width)
    const float* w_router;   // [NE][E] F32
    const void* w_gate;      // [NE * FE] native rows of qt_row_size(type, E)
    const void* w_up;
    const void* w_down;      // [NE * E] native rows of qt_row_size(type, FE)
    const void* s_gate;      // shared expert [FE] rows, or NULL
    const void* s_up;
    const void* s_down;      // [E] rows
    const float* w_shexp;    // [E] sigmoid gate of the shared expert, or NULL (gate 1)
} moe_layer_desc;

// Device bytes of scratch a call with up to max_t tokens needs
size_t moe_layer_scratch_bytes(const moe_layer_desc* d, int max_t);

// out [T][E] = MoE(x [T][E]); logits [T][NE] (NULL: W_router x). ids_out [T][NU] / wts_out [T][NU] (optional,
// NULL) receive the routing. scratch: moe_layer_scratch_bytes(d, >= T) bytes, 256-byte aligned.
hipError_t moe_layer_forward(const moe_layer_desc* d, const float* x, const float* logits, int T, float* out,
                             int* ids_out, float* wts_out, void* scratch, size_t scratch_bytes, hipStream_t stream);

// No counterpart in the reference as one call (its engine issues gpu_add_rmsnorm, then the layer): the RMSNorm
// producer fused in front of the layer. y = RMSNorm(x_in + add) * w_norm (add NULL: of x_in; w_norm NULL: no gamma;
// eps as gpu_add_rmsnorm), x_out = x_in + add (add set: x_out required), then out = MoE(y) as moe_layer_forward.
// The same bits as gpu_add_rmsnorm followed by moe_layer_forward; at T == 1 on the fused kernels the normalization
// happens inside their first kernel (one launch less per layer). Same scratch as moe_layer_forward.
hipError_t moe_layer_forward_norm(const moe_layer_desc* d, const float* x_in, const float* add, float* x_out,
                                  const float* w_norm, float eps, const float* logits, int T, float* out,
                                  int* ids_out, float* wts_out, void* scratch, size_t scratch_bytes,
                                  hipStream_t stream);

// No counterpart in the reference: for callers that cannot allocate (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc). moe_layer_forward with its scratch in a library-owned device array of
// MOE_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends) instead of a caller buffer; allocates nothing.
// Returns hipErrorInvalidValue when moe_layer_scratch_bytes(d, T) exceeds the array (decode T <= 7 of every
// benchmark configuration fits, and prefill batches up to ~64 tokens). Calls that overlap on one GPU share the
// array and race: serialize them (one stream, or events between streams).
#define MOE_NOALLOC_SCRATCH_BYTES (64u << 20)
hipError_t moe_layer_forward_noalloc(const moe_layer_desc* d, const float* x, const float* logits, int T,
                                     float* out, int* ids_out, float* wts_out, hipStream_t stream);

// No counterpart in the reference. Whether T == 1 calls may use the fused kernels (1, the default) or always take
// the per-operation launches (0); process-wide. Profiling only: 0x100 | mask launches just the fused kernels in
// mask (bit 0: logits / quantize, bit 1: routing + gate / up, bit 2: down + combine), which then read what earlier
// calls left in scratch; a layer's results are undefined in that mode. 0x200 | mask (profiling, T >= 8) launches
// only the prefill stages in mask (bit 0: router logits, quantize, router, dispatch; bit 1: the grouped gate / up /
// SwiGLU launch; bit 2: the grouped down launch; bit 3: the combine), reading what earlier calls left in scratch;
// T <= 7 then runs as with 1. Other values select 1.
void moe_layer_set_fused(int mode);

// No counterpart in the reference (its QWEN_PROFILE times sections on the host). Profiling: every later fused
// layer writes wall-clock stamps (100 MHz) per workgroup to stamps: [workgroup][8], kernel 1 in columns 0, 1
// (start, done), kernel 2 in 2..4 (start, routed, done) and 7 (row dots done), kernel 3 in 5, 6; rows for the largest grid
// (max(NE + 2, NS * FE / 32, E) always suffices); NULL stops. Launches capture the pointer current at the call.
void moe_layer_fused_stamps(void* stamps);

// No counterpart in the reference. Whether Q4_K layers at T = 2..7 use the multi-token union kernels (on != 0)
// or (0, the default: faster for Q4_K's shapes) four launches per batch up to T = 4 and the per-operation
// launches beyond; process-wide. All give the same bits.
void moe_layer_fused_multi_q4k(int on);

#ifdef __cplusplus
}
#endif

#endif  // MOE_LAYER_H
