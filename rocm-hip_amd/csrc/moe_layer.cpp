// moe_layer.cpp -- moe_layer_forward: one MoE FFN layer as the reference's QwenModel::moe_core issues it
// (src/qwen_model.cpp:864-937), through this library's C ABI only. See include/moe_layer.h.

#include "moe_layer.h"

#include <stdint.h>

#include <algorithm>
#include <atomic>

#include "fused_common.h"
#include "gpu_ops.h"
#include "grouped.h"
#include "host_common.h"
#include "qmatvec.h"

struct FArgs;
size_t moe_fused_scratch_bytes(const moe_layer_desc* d, int T);

// The fused decode kernel's arguments are built in fused_decode.hip; this file only sees these entry points
bool moe_fused_try(const moe_layer_desc* d, const float* x, const float* logits, float* out, int* ids_out,
                   float* wts_out, void* scratch, int kernels, hipStream_t st, hipError_t* err, const FNorm* norm);
bool moe_fused_multi_try(const moe_layer_desc* d, const float* x, const float* logits, int T, float* out,
                         int* ids_out, float* wts_out, void* scratch, int kernels, hipStream_t st, hipError_t* err);


hipError_t moe_quantize_q8_0(const float* x, int n, const qmatvec_q8* q, hipStream_t stream);
hipError_t moe_quantize_q8k(const float* x, int n, const qmatvec_q8* q, hipStream_t stream);

static std::atomic<int> g_fused{1};

#define FUSED_MAX_T 7  // the fused kernels take 1..7 tokens

namespace {

size_t a256(size_t v) { return (v + 255) & ~(size_t)255; }
int r256(long long k) { return (int)((k + 255) / 256 * 256); }


size_t row_size(int type, int k) {
    switch (type) {
    case 8: return (size_t)k / 32 * 34;
    case 100: return (size_t)k / 32 * 18;
    case 101: return (size_t)k / 32 * 17;
    case 12: return (size_t)k / 256 * 144;
    }
    return 0;
}

// Scratch carve-up; every piece 256-byte aligned
struct Plan {
    size_t fused, logits, ids, wts, sg, qx, g, u, qa, down, sg_, su, qs, sout, tok, pair, ntile, te, ts, tn,
        gws, ynorm, total;
    int NS, qx_k, qa_k, qs_k, max_tiles, tile;
};

Plan plan(const moe_layer_desc* d, int T) {
    Plan p = {};
    const int E = d->n_embd, NE = d->n_expert, NU = d->n_used, FE = d->n_ff;
    const bool sh = d->s_gate != nullptr;
    p.NS = NU + (sh ? 1 : 0);
    const int t_in = qmatvec_id_batch_tile(d->type, FE, E), t_out = qmatvec_id_batch_tile(d->type, E, FE);
    p.tile = t_in < t_out ? t_in : t_out;  // one grouping serves gate / up and down
    p.fused = moe_fused_scratch_bytes(d, T < FUSED_MAX_T ? T : FUSED_MAX_T);
    p.max_tiles = gpu_moe_max_tiles(T, NU, NE, p.tile);
    p.qx_k = r256((long long)T * E);
    // down's input: pair rows, or (the fused prefill) entry tiles of p.tile rows each, the shared expert's after
    // the routed ones
    const long long sh_tiles = sh ? (T + p.tile - 1) / p.tile : 0;
    p.qa_k = r256(std::max((long long)T * p.NS, ((long long)p.max_tiles + sh_tiles) * p.tile) * FE);
    p.qs_k = r256((long long)T * FE);
    size_t o = a256(p.fused);  // the fused kernels' region first
    auto take = [&](size_t bytes) {
        const size_t at = o;
        o += a256(bytes);
        return at;
    };
    p.logits = take((size_t)T * NE * 4);
    p.ids = take((size_t)T * p.NS * 4);
    p.wts = take((size_t)T * NU * 4);
    p.sg = take((size_t)T * 4);
    p.qx = take(qmatvec_q8_bytes(p.qx_k));
    p.g = take((size_t)T * p.NS * FE * 4);
    p.u = take((size_t)T * p.NS * FE * 4);
    p.qa = take(qmatvec_q8_bytes(p.qa_k));
    p.down = take((size_t)T * p.NS * E * 4);
    p.sg_ = take(sh ? (size_t)T * FE * 4 : 0);
    p.su = take(sh ? (size_t)T * FE * 4 : 0);
    p.qs = take(sh ? qmatvec_q8_bytes(p.qs_k) : 0);
    p.sout = take(sh ? (size_t)T * E * 4 : 0);
    p.tok = take((size_t)T * NU * 4);
    p.pair = take((size_t)T * NU * 4);
    p.ntile = take(4);
    p.te = take((size_t)p.max_tiles * 4);
    p.ts = take((size_t)p.max_tiles * 4);
    p.tn = take((size_t)p.max_tiles * 4);
    p.gws = take(gpu_moe_group_ws_bytes(T, NE));
    p.ynorm = take((size_t)T * E * 4);  // moe_layer_forward_norm's normalized input (unfused paths)
    p.total = o;
    return p;
}

#define CHECK(x)                           \
    do {                                   \
        const hipError_t e_ = (x);         \
        if (e_ != hipSuccess) return e_;   \
    } while (0)

}  // namespace

extern "C" void moe_layer_set_fused(int mode) {
    g_fused.store(mode == 0 || mode == 1 || (mode >= 0x100 && mode <= 0x107) || (mode >= 0x200 && mode <= 0x20f)
                      ? mode
                      : 1);
}

extern "C" size_t moe_layer_scratch_bytes(const moe_layer_desc* d, int max_t) {
    if (!d || max_t <= 0) return 0;
    return plan(d, max_t).total;
}

// xq: x's quantized bundle is already in the plan's qx (the producer wrote it; T >= 8 only)
static hipError_t layer_forward(const moe_layer_desc* d, const float* x, const float* logits_in, int T, float* out,
                                int* ids_out, float* wts_out, void* scratch, size_t scratch_bytes, hipStream_t st,
                                bool xq) {
    if (!d || !x || !out || T <= 0 || !scratch || ((uintptr_t)scratch & 255)) return hipErrorInvalidValue;
    const Plan p = plan(d, T);
    if (scratch_bytes < p.total) return hipErrorInvalidValue;
    const int E = d->n_embd, NE = d->n_expert, NU = d->n_used, FE = d->n_ff, type = d->type;
    const bool sh = d->s_gate != nullptr;
    const int mode = g_fused.load(std::memory_order_relaxed);
    // profiling subsets: 0x100 | mask, the fused decode kernels in mask; 0x200 | mask, the prefill stages in mask
    // (bit 0: logits, quantize, router, dispatch; 1: grouped gate / up; 2: grouped down; 3: combine)
    const int pm = (mode & 0x200) ? mode & 0xf : 0xf;
    if (T <= FUSED_MAX_T && mode) {
        hipError_t e = hipSuccess;
        const int kernels = (mode & 0x100) ? mode & 7 : 7;
        if (T == 1 ? moe_fused_try(d, x, logits_in, out, ids_out, wts_out, scratch, kernels, st, &e, nullptr)
                   : moe_fused_multi_try(d, x, logits_in, T, out, ids_out, wts_out, scratch, kernels, st, &e))
            return e;
    }
    const size_t rb_in = row_size(type, E), rb_out = row_size(type, FE);
    char* s = (char*)scratch;
    float* lg = (float*)(s + p.logits);
    int* ids = (int*)(s + p.ids);
    float* wts = (float*)(s + p.wts);
    float* sg = (float*)(s + p.sg);
    float* g = (float*)(s + p.g);
    float* u = (float*)(s + p.u);
    float* down = (float*)(s + p.down);
    qmatvec_q8 qx, qa, qs;
    qmatvec_q8_bind(&qx, s + p.qx, p.qx_k);
    qmatvec_q8_bind(&qa, s + p.qa, p.qa_k);

    const bool front = T < 8 || (pm & 1);  // the prefill profiling subsets may leave the front out
    // router logits and routing
    if (logits_in)
        lg = (float*)logits_in;
    else if (front)
        CHECK(qmatvec_launch_batch(0, d->w_router, (size_t)E * 4, x, lg, NE, E, T, st));
    // the prefill's router launch quantizes x as well (saving the quantizer's launch), unless the producer did
    const bool fuse_q = T >= 8 && (pm & 1) && !xq && E % 256 == 0 && aligned(x, 16) && aligned(qx.q0, 4) &&
                        aligned(qx.qK, 4);
    if (!front || xq || fuse_q) {
    } else if (type == 12) {  // Q4_K reads Q8_K activations; the others read Q8_0 values and scales only
        CHECK(moe_quantize_q8k(x, T * E, &qx, st));
    } else {
        CHECK(moe_quantize_q8_0(x, T * E, &qx, st));
    }

    const bool slot = T == 1 && sh;  // moe_core_one: the shared expert as slot NU
    bool shared_done = false;  // the prefill path ran the shared expert and the combine with the routed experts
    if (T < 8) {
        const int ns = slot ? NU + 1 : NU;
        CHECK(gpu_moe_router(lg, x, d->w_shexp, ids, wts, sg, NE, NU, E, T, st, ns));
        if (slot)
            CHECK(qmatvec_launch_q8_id_x(type, d->w_gate, d->w_up, d->s_gate, d->s_up, rb_in, ids, ns, 0, &qx, g, u,
                                         FE, E, T, st));
        else
            CHECK(qmatvec_launch_q8_id_pair(type, d->w_gate, d->w_up, rb_in, ids, ns, 0, &qx, g, u, FE, E, T, st));
        CHECK(moe_swiglu_q8(g, u, nullptr, T * ns * FE, &qa, st, type == 12 ? 2 : 1));
        if (slot)
            CHECK(qmatvec_launch_q8_id_x(type, d->w_down, nullptr, d->s_down, nullptr, rb_out, ids, ns, 1, &qa, down,
                                         nullptr, E, FE, T, st));
        else
            CHECK(qmatvec_launch_q8_id(type, d->w_down, rb_out, ids, ns, 1, &qa, down, E, FE, T, st));
        if (slot) {
            CHECK(gpu_moe_combine(down, wts, down + (size_t)NU * E, d->w_shexp ? sg : nullptr, out, NU, E, 1, st));
        } else if (!sh) {
            CHECK(gpu_moe_combine(down, wts, nullptr, nullptr, out, NU, E, T, st));
        }
    } else {
        if (fuse_q)
            CHECK(moe_router_quantize(lg, x, d->w_shexp, ids, wts, sg, NE, NU, E, T, NU, &qx, type == 12 ? 2 : 1, st));
        else if (pm & 1)
            CHECK(gpu_moe_router(lg, x, d->w_shexp, ids, wts, sg, NE, NU, E, T, st, NU));
        int* tok = (int*)(s + p.tok);
        int* pair = (int*)(s + p.pair);
        int* ntile = (int*)(s + p.ntile);
        int* te = (int*)(s + p.te);
        int* ts = (int*)(s + p.ts);
        int* tn = (int*)(s + p.tn);
        if (pm & 1)
            CHECK(gpu_moe_group_ws(ids, T, NU, NE, p.tile, tok, pair, ntile, te, ts, tn, s + p.gws,
                                   gpu_moe_group_ws_bytes(T, NE), st));
        const uint8_t *vg = nullptr, *sgp = nullptr, *vu = nullptr, *sup = nullptr, *vd = nullptr, *sdp = nullptr;
        long long gvs = 0, gss = 0, dvs = 0, dss = 0;  // tile bytes per 32-row group (gate and up alike, down)
        // (Q4_K: down's input is Q8_K, one scale per 256 values, which a workgroup's 32-row blocks cannot form: its
        // gate, up, SwiGLU and down run as the separate launches below, each on the MFMA kernel when registered)
        if (mode && type != 12 && moe_grouped_mfma_ok(type, FE, E) && moe_grouped_mfma_ok(type, E, FE) &&
            moe_packed_tiles(d->w_gate, type, E, rb_in, &vg, &sgp, &gvs, &gss) &&
            moe_packed_tiles(d->w_up, type, E, rb_in, &vu, &sup, &gvs, &gss) &&
            moe_packed_tiles(d->w_down, type, FE, rb_out, &vd, &sdp, &dvs, &dss)) {
            // The shared expert (when its matrices have tiles too) as more tiles of the same two launches: its
            // outputs are rows T NU .. of down
            GShared shg = {}, shd = {};
            long long v0, s0;
            const bool merged = sh && moe_packed_tiles(d->s_gate, type, E, rb_in, &shg.v, &shg.s, &v0, &s0) &&
                                moe_packed_tiles(d->s_up, type, E, rb_in, &shg.v2, &shg.s2, &v0, &s0) &&
                                moe_packed_tiles(d->s_down, type, FE, rb_out, &shd.v, &shd.s, &v0, &s0);
            shg.T = shd.T = T;
            shg.out0 = shd.out0 = (long long)T * NU;
            // gate, up, SwiGLU and down's Q8_0 input in one launch (the same bits as the three launches below); the
            // input handed to down in entry-tile order
            if (pm & 2)
                CHECK(moe_launch_grouped_swiglu(type, vg, sgp, vu, sup, gvs, gss, &qx, qa.q0, qa.d0, FE, E,
                                                p.max_tiles, ntile, te, ts, tn, tok, pair,
                                                2 /* down's input in entry-tile order */, merged ? &shg : nullptr,
                                                st));
            if (pm & 4)
                CHECK(moe_launch_grouped_mfma(type, vd, sdp, dvs, dss, &qa, down, E, FE, p.max_tiles, ntile, te, ts,
                                              tn, nullptr, pair, 1 /* input in entry-tile order */,
                                              merged ? &shd : nullptr, st));
            if (!(pm & 8)) return hipSuccess;
            if (merged) {
                CHECK(gpu_moe_combine(down, wts, down + (size_t)T * NU * E, d->w_shexp ? sg : nullptr, out, NU, E, T,
                                      st));
                shared_done = true;
            }
        } else {
            // Q4_K: gate, up and SwiGLU in one MFMA launch when both matrices have tiles and the tiles are mostly
            // full (the per-entry kernel's condition in qmatvec_launch_q8_id_batch), then down's Q8_K input
            const bool q4k_fused = (pm & 2) && mode && type == 12 && p.tile == moe_grouped_mfma_tile() &&
                                   moe_grouped_mfma_ok(type, FE, E) && 4ll * p.max_tiles >= 3ll * NE &&
                                   moe_packed_tiles(d->w_gate, type, E, rb_in, &vg, &sgp, &gvs, &gss) &&
                                   moe_packed_tiles(d->w_up, type, E, rb_in, &vu, &sup, &gvs, &gss);
            if (q4k_fused) {
                CHECK(moe_launch_grouped_gate_up(type, vg, sgp, vu, sup, gvs, gss, &qx, g, FE, E, p.max_tiles, ntile,
                                                 te, ts, tn, tok, pair, st));
                CHECK(moe_quantize_q8k(g, T * NU * FE, &qa, st));
            } else if (pm & 2) {
                CHECK(qmatvec_launch_q8_id_batch(type, d->w_gate, rb_in, &qx, g, FE, E, p.max_tiles, p.tile, ntile,
                                                 te, ts, tn, tok, pair, st));
                CHECK(qmatvec_launch_q8_id_batch(type, d->w_up, rb_in, &qx, u, FE, E, p.max_tiles, p.tile, ntile, te,
                                                 ts, tn, tok, pair, st));
                CHECK(moe_swiglu_q8(g, u, nullptr, T * NU * FE, &qa, st, type == 12 ? 2 : 1));
            }
            if (pm & 4)
                CHECK(qmatvec_launch_q8_id_batch(type, d->w_down, rb_out, &qa, down, E, FE, p.max_tiles, p.tile,
                                                 ntile, te, ts, tn, pair, pair, st));
        }
        if (!sh && (pm & 8)) CHECK(gpu_moe_combine(down, wts, nullptr, nullptr, out, NU, E, T, st));
    }
    if (sh && !slot && !shared_done) {  // the shared expert as a dense FFN on all T tokens, then the combine
        float* sgt = (float*)(s + p.sg_);
        float* sut = (float*)(s + p.su);
        float* sout = (float*)(s + p.sout);
        qmatvec_q8_bind(&qs, s + p.qs, p.qs_k);
        if (pm & 2) {  // (the prefill profiling subsets: its gate / up with the routed ones', its down with down)
            CHECK(qmatvec_launch_q8_batch(type, d->s_gate, rb_in, &qx, sgt, FE, FE, E, T, st));
            CHECK(qmatvec_launch_q8_batch(type, d->s_up, rb_in, &qx, sut, FE, FE, E, T, st));
            CHECK(moe_swiglu_q8(sgt, sut, nullptr, T * FE, &qs, st, type == 12 ? 2 : 1));
        }
        if (pm & 4) CHECK(qmatvec_launch_q8_batch(type, d->s_down, rb_out, &qs, sout, E, E, FE, T, st));
        if (pm & 8) CHECK(gpu_moe_combine(down, wts, sout, d->w_shexp ? sg : nullptr, out, NU, E, T, st));
    }
    if (!(pm & 8)) return hipSuccess;  // (a profiling subset: the results are not complete)
    const int ns_used = slot ? NU + 1 : NU;
    if (ids_out)
        CHECK(hipMemcpy2DAsync(ids_out, (size_t)NU * 4, ids, (size_t)ns_used * 4, (size_t)NU * 4, T,
                               hipMemcpyDeviceToDevice, st));
    if (wts_out) CHECK(hipMemcpyAsync(wts_out, wts, (size_t)T * NU * 4, hipMemcpyDeviceToDevice, st));
    return hipSuccess;
}

extern "C" hipError_t moe_layer_forward(const moe_layer_desc* d, const float* x, const float* logits_in, int T,
                                        float* out, int* ids_out, float* wts_out, void* scratch, size_t scratch_bytes,
                                        hipStream_t st) {
    return layer_forward(d, x, logits_in, T, out, ids_out, wts_out, scratch, scratch_bytes, st, false);
}

// The producer fused in: y = RMSNorm(x_in + add) * w_norm, x_out = x_in + add, then the layer on y. T == 1 with the
// fused decode kernels forms y inside their first kernel; every other case runs gpu_add_rmsnorm into scratch first.
// Either way the results equal gpu_add_rmsnorm followed by moe_layer_forward bit for bit.
extern "C" hipError_t moe_layer_forward_norm(const moe_layer_desc* d, const float* x_in, const float* add,
                                             float* x_out, const float* w_norm, float eps, const float* logits, int T,
                                             float* out, int* ids_out, float* wts_out, void* scratch,
                                             size_t scratch_bytes, hipStream_t st) {
    if (!d || !x_in || !out || T <= 0 || !scratch || ((uintptr_t)scratch & 255) || (add && !x_out))
        return hipErrorInvalidValue;
    const Plan p = plan(d, T);
    if (scratch_bytes < p.total) return hipErrorInvalidValue;
    const int mode = g_fused.load(std::memory_order_relaxed);
    if (T == 1 && mode == 1 && d->n_embd <= 4096) {
        const FNorm nm = {add, w_norm, x_out, eps};
        hipError_t e = hipSuccess;
        if (moe_fused_try(d, x_in, logits, out, ids_out, wts_out, scratch, 7, st, &e, &nm)) return e;
    }
    float* y = (float*)((char*)scratch + p.ynorm);
    if (T >= 8) {  // the prefill: the norm writes y's quantized bundle too, where its wave path applies
        qmatvec_q8 qx;
        qmatvec_q8_bind(&qx, (char*)scratch + p.qx, p.qx_k);
        const hipError_t e =
            moe_add_rmsnorm_q8(x_in, add, x_out, w_norm, y, d->n_embd, T, eps, &qx, d->type == 12 ? 2 : 1, st);
        if (e == hipSuccess)
            return layer_forward(d, y, logits, T, out, ids_out, wts_out, scratch, scratch_bytes, st, true);
        if (e != hipErrorInvalidValue) return e;  // (invalid value: its wave path does not take this row length)
    }
    CHECK(gpu_add_rmsnorm(x_in, add, x_out, w_norm, y, d->n_embd, T, eps, nullptr, st));
    return layer_forward(d, y, logits, T, out, ids_out, wts_out, scratch, scratch_bytes, st, false);
}
