// moe_ffn_engine.h -- an engine-side caller of the MoE boundary: the MoE FFN sublayer of a qwen3moe / qwen35moe
// forward pass issued through the launchers of qmatvec.h / gpu_ops.h only, in the order the reference's engine
// issues them (QwenModel::moe_ffn / moe_core / moe_core_one, src/qwen_model.cpp:839-937). It is built against the
// reference's own src/qmatvec.h and src/gpu_ops.h when that tree is present (else against this repository's
// identical declarations) and linked against librocm_hip_moe.so: the binding a maintainer of the reference would
// keep when swapping in this library. C entry points for tests and harnesses.
#ifndef MOE_FFN_ENGINE_H
#define MOE_FFN_ENGINE_H

#include <hip/hip_runtime.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

// One weight matrix as the engine holds it (the reference's QuantWeight): type, device data, bytes per row,
// N rows (per expert for the stacked expert tensors) of K values
typedef struct moe_engine_weight {
    int type;
    const void* data;
    size_t row_bytes;
    int N, K;
} moe_engine_weight;

typedef struct moe_engine_layer {
    int n_embd, n_expert, n_used, n_ff_exp, n_ff_shexp;
    moe_engine_weight router;                        // F32 [n_expert][n_embd]
    moe_engine_weight exp_gate, exp_up, exp_down;    // stacked experts
    moe_engine_weight sh_gate, sh_up, sh_down;       // the shared expert (data NULL: none)
    const float* shexp_gate;                         // [n_embd] sigmoid gate of the shared expert, or NULL
} moe_engine_layer;

typedef struct moe_engine moe_engine;

// The engine's device buffers for batches of up to max_t tokens of layers shaped like L (hipMalloc'd once);
// NULL on failure
moe_engine* moe_engine_create(const moe_engine_layer* L, int max_t);
void moe_engine_destroy(moe_engine* e);

// The MoE FFN sublayer for T tokens, as the engine's moe_ffn: x_mid = x + proj, xn = RMSNorm(x_mid) * ffn_norm
// (quantized for the int8 launchers), out = MoE(xn) (moe_core: the shared expert as one more slot of the expert
// launches at T = 1 when it fits, the grouped expert launches from T = 8), then x_next = x_mid + out and
// xn_next = RMSNorm(x_next) * next_norm. All [T][n_embd] device rows; asynchronous on stream.
hipError_t moe_engine_ffn(moe_engine* e, const moe_engine_layer* L, const float* x, const float* proj,
                          const float* ffn_norm, const float* next_norm, float eps, int T, float* x_mid, float* out,
                          float* x_next, float* xn_next, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif  // MOE_FFN_ENGINE_H
