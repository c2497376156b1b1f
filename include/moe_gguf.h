// moe_gguf.h -- bind one MoE FFN layer's tensors from a GGUF file and upload them to HBM.
//
// The expert-binding step of CowboyTim/rocm-hip's model load (src/inference.cpp:234-262 bind_weight, :298-302
// check_shape and :519-545, the MoE branch of the layer binding), producing a moe_layer_desc for moe_layer_forward. Tensors of
// layer i, with their GGUF shapes (ne[0] first) and the hparams "<arch>.expert_count" (NE),
// "<arch>.expert_used_count" (NU), "<arch>.expert_feed_forward_length" (FE),
// "<arch>.expert_shared_feed_forward_length" (FS) and "<arch>.embedding_length" (E):
//   blk.i.ffn_gate_inp.weight        F32 {E, NE}          router
//   blk.i.ffn_{gate,up}_exps.weight  {E, FE, NE}          expert e's rows are [e * FE, (e + 1) * FE) of one
//   blk.i.ffn_down_exps.weight       {FE, E, NE}          stacked matrix (down: [e * E, (e + 1) * E))
//   blk.i.ffn_{gate,up}_shexp.weight {E, FS}              shared expert, present iff ffn_gate_shexp is
//   blk.i.ffn_down_shexp.weight      {FS, E}
//   blk.i.ffn_gate_inp_shexp.weight  F32 {E}              its sigmoid gate
// Checks follow the reference: a missing tensor, hparams out of range (NE, NU, FE > 0, NU <= NE, FS > 0 exactly
// when the shared expert is present), a shape other than the above, or a byte size other than rows x row bytes
// fail with a message. On top of those, the layer path needs gate, up, down (and the shared expert) in one of its
// types (Q8_0 8, Q4_K 12, ROCmFP4 100, FAST 101), FS == FE, and the dimensions moe_layer_forward accepts.

#ifndef MOE_GGUF_H
#define MOE_GGUF_H

#include <hip/hip_runtime.h>
#include <stddef.h>

#include "gguf_mmap.h"
#include "moe_layer.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct moe_gguf_layer {
    moe_layer_desc desc;  // device pointers into dev
    void* dev;            // one device allocation holding every tensor of the layer, each 256-byte aligned
    size_t dev_bytes;
    int packed;           // the expert matrices are registered with qmatvec_pack_weights
} moe_gguf_layer;

// Check layer `layer` and fill desc with pointers into the file mapping (host memory: for inspection and tests,
// not for moe_layer_forward). 0, or -1 with the reason in moe_gguf_error().
int moe_gguf_layer_bind(const gguf_model_t* model, int layer, moe_layer_desc* desc);

// Bind, then copy the layer's tensors into one device allocation (through pinned staging buffers, on stream) and,
// with pack set, register gate, up, down and the shared expert with qmatvec_pack_weights_ex (flags pack - 1:
// 1 the default copy and tiles, 2 in place, 3 a copy without tiles, 4 in place without tiles) so that
// moe_layer_forward takes its fused and MFMA paths. Synchronous: returns once the copies are done. On failure
// nothing stays allocated: hipErrorInvalidValue for a binding error (moe_gguf_error()), else the HIP error.
hipError_t moe_gguf_layer_upload(const gguf_model_t* model, int layer, int pack, moe_gguf_layer* out,
                                 hipStream_t stream);

// Unregister the packed copies and free the device allocation; the struct is zeroed. NULL or zeroed: no-op.
void moe_gguf_layer_release(moe_gguf_layer* layer);

// Why the last moe_gguf_layer_bind / moe_gguf_layer_upload on this thread failed ("" after a success).
const char* moe_gguf_error(void);

#ifdef __cplusplus
}
#endif

#endif  // MOE_GGUF_H
