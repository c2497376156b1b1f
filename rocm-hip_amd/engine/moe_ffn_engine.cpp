// moe_ffn_engine.cpp -- the MoE FFN sublayer of the reference's engine (QwenModel::moe_ffn / moe_core /
// moe_core_one, src/qwen_model.cpp:839-937) as a caller of the boundary launchers only. Compiled against whichever
// qmatvec.h / gpu_ops.h the include path names first (the reference's src/, or this repository's include/) and
// linked against librocm_hip_moe.so. See include/moe_ffn_engine.h.
#include "moe_ffn_engine.h"

#include <algorithm>
#include <new>

#include "gpu_ops.h"
#include "qmatvec.h"

struct moe_engine {
    int max_t = 0, E = 0, NE = 0, NU = 0, FE = 0, FS = 0;
    // routing
    float* logits = nullptr;
    int* ids = nullptr;  // [max_t][NU + 1] (one more slot at T = 1 for the shared expert)
    float* wts = nullptr;
    float* sg = nullptr;
    // expert activations: gate, up, SwiGLU, down (NU + 1 slots per token)
    float *g = nullptr, *u = nullptr, *act = nullptr, *down = nullptr;
    // the shared expert's
    float *sg_g = nullptr, *sg_u = nullptr, *sact = nullptr, *sout = nullptr;
    // normalized input
    float* xn = nullptr;
    // grouping of a prefill batch
    int *tok = nullptr, *pair = nullptr, *ntiles = nullptr, *tile_e = nullptr, *tile_start = nullptr,
        *tile_n = nullptr;
    int max_tiles_cap = 0;
    // one int8 activation bundle, reused by each producer in stream order
    void* q8_mem = nullptr;
    qmatvec_q8 q8{};
    int q8_max_k = 0;
};

namespace {

template <typename T>
bool dev_alloc(T*& p, size_t n) {
    void* m = nullptr;
    if (hipMalloc(&m, n * sizeof(T) + 16) != hipSuccess) return false;
    p = (T*)m;
    return true;
}

#define TRY(x)                          \
    do {                                \
        const hipError_t e_ = (x);      \
        if (e_ != hipSuccess) return e_; \
    } while (0)

// W[T rows] . x on the int8 path (x quantized in q): one launch per call as the engine's matvec does
hipError_t matvec_q8(const moe_engine_weight& W, const qmatvec_q8* q, float* y, int T, hipStream_t st) {
    if (T == 1) return qmatvec_launch_q8(W.type, W.data, W.row_bytes, q, y, W.N, W.K, st);
    return qmatvec_launch_q8_batch(W.type, W.data, W.row_bytes, q, y, W.N, W.N, W.K, T, st);
}

// The shared expert can ride along as slot NU of the expert launches: one token, the experts' width, type and
// row sizes (the engine's shared_as_slot)
bool shared_as_slot(const moe_engine_layer& L, int T) {
    return T == 1 && L.sh_gate.data && L.n_ff_shexp == L.n_ff_exp && L.sh_gate.type == L.exp_gate.type &&
           L.sh_up.type == L.exp_up.type && L.exp_gate.type == L.exp_up.type && L.sh_down.type == L.exp_down.type &&
           L.sh_gate.row_bytes == L.exp_gate.row_bytes && L.sh_down.row_bytes == L.exp_down.row_bytes &&
           qmatvec_q8_supported(L.exp_gate.type, L.n_embd) && qmatvec_q8_supported(L.exp_down.type, L.n_ff_exp);
}

// moe_core_one: router logits, the router with the shared expert as slot NU (id -1), gate / up of NU + 1 slots in
// one launch, SwiGLU quantized for down, down of NU + 1 slots, combine with the shared output last
hipError_t core_one(moe_engine& e, const moe_engine_layer& L, float* out, hipStream_t st) {
    const int E = e.E, NE = e.NE, NU = e.NU, FE = e.FE, NS = NU + 1;
    TRY(qmatvec_launch_batch(L.router.type, L.router.data, L.router.row_bytes, e.xn, e.logits, NE, E, 1, st));
    TRY(gpu_moe_router(e.logits, e.xn, L.shexp_gate, e.ids, e.wts, e.sg, NE, NU, E, 1, st, NS));
    TRY(qmatvec_launch_q8_id_x(L.exp_gate.type, L.exp_gate.data, L.exp_up.data, L.sh_gate.data, L.sh_up.data,
                               L.exp_gate.row_bytes, e.ids, NS, 0, &e.q8, e.g, e.u, FE, E, 1, st));
    TRY(gpu_swiglu(e.g, e.u, e.act, NS * FE, &e.q8, st));
    TRY(qmatvec_launch_q8_id_x(L.exp_down.type, L.exp_down.data, nullptr, L.sh_down.data, nullptr,
                               L.exp_down.row_bytes, e.ids, NS, 1, &e.q8, e.down, nullptr, E, FE, 1, st));
    // (qwen_model.cpp:933 passes s.sg whether or not there is a gate vector; with none its router leaves sg
    // unwritten, so NULL here -- a weight of 1 for the shared row -- is the same result without reading it)
    return gpu_moe_combine(e.down, e.wts, e.down + (size_t)NU * E, L.shexp_gate ? e.sg : nullptr, out, NU, E, 1, st);
}

// moe_core for T tokens: per-token expert launches below 8 tokens, the grouped (expert-tiled) launches from 8; the
// shared expert as a dense FFN on all tokens; combine
hipError_t core(moe_engine& e, const moe_engine_layer& L, int T, float* out, hipStream_t st) {
    if (shared_as_slot(L, T)) return core_one(e, L, out, st);
    const int E = e.E, NE = e.NE, NU = e.NU, FE = e.FE, FS = e.FS;
    const bool grouped = T >= 8;
    int tile = 0, max_tiles = 0;
    if (grouped) {  // the largest tile the kernels of all three expert matrices take
        tile = std::min({qmatvec_id_batch_tile(L.exp_gate.type, FE, E), qmatvec_id_batch_tile(L.exp_up.type, FE, E),
                         qmatvec_id_batch_tile(L.exp_down.type, E, FE)});
        max_tiles = gpu_moe_max_tiles(T, NU, NE, tile);
        if (max_tiles > e.max_tiles_cap) return hipErrorInvalidValue;
    }
    TRY(qmatvec_launch_batch(L.router.type, L.router.data, L.router.row_bytes, e.xn, e.logits, NE, E, T, st));
    TRY(gpu_moe_router(e.logits, e.xn, L.shexp_gate, e.ids, e.wts, e.sg, NE, NU, E, T, st, 0));
    if (grouped) {
        TRY(gpu_moe_group(e.ids, T, NU, NE, tile, e.tok, e.pair, e.ntiles, e.tile_e, e.tile_start, e.tile_n, st));
        TRY(qmatvec_launch_q8_id_batch(L.exp_gate.type, L.exp_gate.data, L.exp_gate.row_bytes, &e.q8, e.g, FE, E,
                                       max_tiles, tile, e.ntiles, e.tile_e, e.tile_start, e.tile_n, e.tok, e.pair,
                                       st));
        TRY(qmatvec_launch_q8_id_batch(L.exp_up.type, L.exp_up.data, L.exp_up.row_bytes, &e.q8, e.u, FE, E, max_tiles,
                                       tile, e.ntiles, e.tile_e, e.tile_start, e.tile_n, e.tok, e.pair, st));
    } else {
        TRY(qmatvec_launch_q8_id_pair(L.exp_gate.type, L.exp_gate.data, L.exp_up.data, L.exp_gate.row_bytes, e.ids,
                                      NU, 0, &e.q8, e.g, e.u, FE, E, T, st));
    }
    if (L.sh_gate.data) {  // the shared expert's gate and up on the same quantized input
        if (T == 1)
            TRY(qmatvec_launch_q8_pair(L.sh_gate.type, L.sh_gate.data, FS, e.sg_g, L.sh_up.data, FS, e.sg_u,
                                       L.sh_gate.row_bytes, &e.q8, E, st));
        else {
            TRY(matvec_q8(L.sh_gate, &e.q8, e.sg_g, T, st));
            TRY(matvec_q8(L.sh_up, &e.q8, e.sg_u, T, st));
        }
    }
    TRY(gpu_swiglu(e.g, e.u, e.act, T * NU * FE, &e.q8, st));
    if (grouped)
        TRY(qmatvec_launch_q8_id_batch(L.exp_down.type, L.exp_down.data, L.exp_down.row_bytes, &e.q8, e.down, E, FE,
                                       max_tiles, tile, e.ntiles, e.tile_e, e.tile_start, e.tile_n, e.pair, e.pair,
                                       st));
    else
        TRY(qmatvec_launch_q8_id(L.exp_down.type, L.exp_down.data, L.exp_down.row_bytes, e.ids, NU, 1, &e.q8, e.down,
                                 E, FE, T, st));
    if (!L.sh_gate.data) return gpu_moe_combine(e.down, e.wts, nullptr, nullptr, out, NU, E, T, st);
    TRY(gpu_swiglu(e.sg_g, e.sg_u, e.sact, T * FS, &e.q8, st));
    TRY(matvec_q8(L.sh_down, &e.q8, e.sout, T, st));
    // (NULL without a gate vector, as above)
    return gpu_moe_combine(e.down, e.wts, e.sout, L.shexp_gate ? e.sg : nullptr, out, NU, E, T, st);
}

}  // namespace

extern "C" moe_engine* moe_engine_create(const moe_engine_layer* L, int max_t) {
    if (!L || max_t <= 0) return nullptr;
    moe_engine* e = new (std::nothrow) moe_engine;
    if (!e) return nullptr;
    e->max_t = max_t;
    e->E = L->n_embd;
    e->NE = L->n_expert;
    e->NU = L->n_used;
    e->FE = L->n_ff_exp;
    e->FS = L->sh_gate.data ? L->n_ff_shexp : 0;
    const size_t T = (size_t)max_t, NS = (size_t)e->NU + 1;
    e->max_tiles_cap = gpu_moe_max_tiles(max_t, e->NU, e->NE, 1);  // covers every tile size
    const long long lt = max_t;
    const long long qk = std::max({lt * e->E, lt * (e->NU + 1) * e->FE, lt * e->FS});
    e->q8_max_k = (int)((qk + 255) / 256 * 256);
    bool ok = dev_alloc(e->logits, T * e->NE) && dev_alloc(e->ids, T * NS) && dev_alloc(e->wts, T * NS) &&
              dev_alloc(e->sg, T) && dev_alloc(e->g, T * NS * e->FE) && dev_alloc(e->u, T * NS * e->FE) &&
              dev_alloc(e->act, T * NS * e->FE) && dev_alloc(e->down, T * NS * e->E) && dev_alloc(e->xn, T * e->E) &&
              dev_alloc(e->tok, T * e->NU) && dev_alloc(e->pair, T * e->NU) && dev_alloc(e->ntiles, 1) &&
              dev_alloc(e->tile_e, (size_t)e->max_tiles_cap) && dev_alloc(e->tile_start, (size_t)e->max_tiles_cap) &&
              dev_alloc(e->tile_n, (size_t)e->max_tiles_cap);
    if (ok && e->FS)
        ok = dev_alloc(e->sg_g, T * e->FS) && dev_alloc(e->sg_u, T * e->FS) && dev_alloc(e->sact, T * e->FS) &&
             dev_alloc(e->sout, T * e->E);
    if (ok) ok = hipMalloc(&e->q8_mem, qmatvec_q8_bytes(e->q8_max_k)) == hipSuccess;
    if (!ok) {
        moe_engine_destroy(e);
        return nullptr;
    }
    qmatvec_q8_bind(&e->q8, e->q8_mem, e->q8_max_k);
    return e;
}

extern "C" void moe_engine_destroy(moe_engine* e) {
    if (!e) return;
    (void)hipDeviceSynchronize();
    void* bufs[] = {e->logits, e->ids, e->wts,  e->sg,    e->g,     e->u,      e->act,        e->down,
                    e->xn,     e->tok, e->pair, e->ntiles, e->tile_e, e->tile_start, e->tile_n, e->sg_g,
                    e->sg_u,   e->sact, e->sout, e->q8_mem};
    for (void* p : bufs)
        if (p) (void)hipFree(p);
    delete e;
}

extern "C" hipError_t moe_engine_ffn(moe_engine* e, const moe_engine_layer* L, const float* x, const float* proj,
                                     const float* ffn_norm, const float* next_norm, float eps, int T, float* x_mid,
                                     float* out, float* x_next, float* xn_next, hipStream_t st) {
    if (!e || !L || T <= 0 || T > e->max_t || L->n_embd != e->E || L->n_expert != e->NE || L->n_used != e->NU ||
        L->n_ff_exp != e->FE || (L->sh_gate.data ? L->n_ff_shexp : 0) != e->FS)
        return hipErrorInvalidValue;
    const int E = e->E;
    // x_mid = x + proj; xn = RMSNorm(x_mid) * ffn_norm, quantized for the expert launches
    TRY(gpu_add_rmsnorm(x, proj, x_mid, ffn_norm, e->xn, E, T, eps, &e->q8, st));
    TRY(core(*e, *L, T, out, st));
    // the residual add of the MoE output fused with the next RMSNorm
    return gpu_add_rmsnorm(x_mid, out, x_next, next_norm, xn_next, E, T, eps, nullptr, st);
}
