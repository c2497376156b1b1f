"""The engine-side caller (libmoe_ffn_engine.so, built against the reference's own qmatvec.h / gpu_ops.h): the MoE
FFN sublayer issued launcher by launcher as the reference's QwenModel::moe_ffn / moe_core / moe_core_one do
(src/qwen_model.cpp:839-937), on this library. Per T (1: the shared expert as a slot; 3: per-token launches; 40:
the grouped launches): the residual x + proj bit-exact; the MoE output equal bit for bit to moe_layer_forward_norm
on the same inputs (the layer entry point's fused kernels give the per-operation bits; the shared expert's dense
launches held to the MFMA kernel, and within 1e-6 of those bits on the default kernel choice) and within the decode /
prefill tolerance of the oracle; the next residual and norm consistent."""
import ctypes

import numpy as np
import pytest
import torch

import moe_hip
import synth
from gpu_util import announce, cvoid, dev, host, rel_l2, zeros

pytestmark = pytest.mark.gpu
Q8_0, FP4, FAST, Q4_K = 8, 100, 101, 12
EPS = 1e-6
S = moe_hip.stream_handle


def _weight(t, qtype, N, K):
    return moe_hip.EngineWeight(qtype, t.data_ptr() if t is not None else None,
                                moe_hip.row_size(qtype, K) if qtype else K * 4, N, K)


@pytest.mark.parametrize("spec", [synth.LayerSpec(FP4, 512, 16, 4, 256, True),
                                  synth.LayerSpec(Q8_0, 1024, 32, 8, 512, False),
                                  synth.LayerSpec(Q4_K, 768, 32, 8, 512, False),
                                  synth.CONFIGS[1]], ids=lambda s: f"{s.qtype}-{s.E}")
@pytest.mark.parametrize("packed", [True, False])
def test_engine_moe_ffn(moe, oracle, spec, packed):
    announce("engine", spec.qtype, spec.E, spec.NE, packed)
    eng = moe_hip.load_engine()
    L = synth.make_layer(spec, seed=120 + spec.qtype)
    d = {k: dev(v) for k, v in L.items()}
    mats = {"w_gate": (spec.NE * spec.FE, spec.E), "w_up": (spec.NE * spec.FE, spec.E),
            "w_down": (spec.NE * spec.E, spec.FE), "s_gate": (spec.FE, spec.E), "s_up": (spec.FE, spec.E),
            "s_down": (spec.E, spec.FE)}
    if packed:
        for k, (rows, K) in mats.items():
            if k in d:
                moe.qmatvec_pack_weights(spec.qtype, cvoid(d[k]), moe_hip.row_size(spec.qtype, K), rows, K, S())
    sh = spec.shared
    el = moe_hip.EngineLayer(spec.E, spec.NE, spec.NU, spec.FE, spec.FE if sh else 0,
                             _weight(d["w_router"], 0, spec.NE, spec.E),
                             _weight(d["w_gate"], spec.qtype, spec.FE, spec.E),
                             _weight(d["w_up"], spec.qtype, spec.FE, spec.E),
                             _weight(d["w_down"], spec.qtype, spec.E, spec.FE),
                             _weight(d.get("s_gate"), spec.qtype, spec.FE, spec.E),
                             _weight(d.get("s_up"), spec.qtype, spec.FE, spec.E),
                             _weight(d.get("s_down"), spec.qtype, spec.E, spec.FE),
                             d["w_shexp"].data_ptr() if sh else None)
    desc = moe_hip.LayerDesc(spec.qtype, spec.E, spec.NE, spec.NU, spec.FE, cvoid(d["w_router"]), cvoid(d["w_gate"]),
                             cvoid(d["w_up"]), cvoid(d["w_down"]), cvoid(d.get("s_gate")), cvoid(d.get("s_up")),
                             cvoid(d.get("s_down")), cvoid(d.get("w_shexp")))
    e = eng.moe_engine_create(ctypes.byref(el), 40)
    assert e
    rng = np.random.default_rng(121)
    w1 = (1.0 + 0.1 * rng.standard_normal(spec.E)).astype(np.float32)
    w2 = (1.0 + 0.1 * rng.standard_normal(spec.E)).astype(np.float32)
    try:
        for T in (1, 3, 40):
            x = rng.standard_normal((T, spec.E)).astype(np.float32)
            proj = rng.standard_normal((T, spec.E)).astype(np.float32)
            xd, pd, w1d, w2d = dev(x), dev(proj), dev(w1), dev(w2)
            x_mid, out, x_next, xn_next = (zeros((T, spec.E), torch.float32) for _ in range(4))
            # (the shared expert's dense launches on the MFMA kernel, as the layer entry point's merged tiles: the
            # same bits; the default choice, checked below, may take the matvec kernel at small T)
            moe.lib.qmatvec_dense_mfma_mode(1)
            try:
                assert eng.moe_engine_ffn(e, ctypes.byref(el), cvoid(xd), cvoid(pd), cvoid(w1d), cvoid(w2d), EPS, T,
                                          cvoid(x_mid), cvoid(out), cvoid(x_next), cvoid(xn_next), S()) == 0
            finally:
                moe.lib.qmatvec_dense_mfma_mode(0)
            g_mid, g_out, g_next, g_xn = (host(t) for t in (x_mid, out, x_next, xn_next))
            # the layer entry point on the same sublayer input
            nb = moe.lib.moe_layer_scratch_bytes(ctypes.byref(desc), T)
            sc = zeros(nb + 256, torch.uint8)
            ref_mid, ref_out = zeros((T, spec.E), torch.float32), zeros((T, spec.E), torch.float32)
            moe.moe_layer_forward_norm(ctypes.byref(desc), cvoid(xd), cvoid(pd), cvoid(ref_mid), cvoid(w1d), EPS,
                                       None, T, cvoid(ref_out), None, None,
                                       ctypes.c_void_p((sc.data_ptr() + 255) // 256 * 256), nb, S())
            r_mid, r_out = host(ref_mid), host(ref_out)
            assert np.array_equal(g_mid.view(np.uint32), (x + proj).view(np.uint32)), T
            assert np.array_equal(g_mid.view(np.uint32), r_mid.view(np.uint32)), T
            assert np.array_equal(g_out.view(np.uint32), r_out.view(np.uint32)), T
            assert np.array_equal(g_next.view(np.uint32), (g_mid + g_out).view(np.uint32)), T
            if T >= 8:  # the default kernel choice for the dense launches: within fp32 reordering of those bits
                out0 = zeros((T, spec.E), torch.float32)
                assert eng.moe_engine_ffn(e, ctypes.byref(el), cvoid(xd), cvoid(pd), cvoid(w1d), cvoid(w2d), EPS, T,
                                          cvoid(x_mid), cvoid(out0), cvoid(x_next), cvoid(xn_next), S()) == 0
                assert rel_l2(host(out0), r_out) < 1e-6, T
            # the oracle on a few rows: RMSNorm, router logits, layer
            rows = np.arange(T) if T < 8 else rng.choice(T, 6, replace=False)
            y = np.stack([oracle.rmsnorm(g_mid[r], w1, EPS) for r in rows])
            lg = np.stack([oracle.matvec_f32(L["w_router"], y[k]) for k in range(len(rows))])
            want, _, _ = oracle.moe_forward(spec, L, y, logits=lg)
            assert rel_l2(g_out[rows], want) < (1e-5 if T < 8 else 1e-3), (T, rel_l2(g_out[rows], want))
            xn_want = np.stack([oracle.rmsnorm(g_next[r], w2, EPS) for r in rows])
            assert rel_l2(g_xn[rows], xn_want) < 1e-6
    finally:
        eng.moe_engine_destroy(e)
        if packed:
            torch.cuda.synchronize()
            for k in mats:
                if k in d:
                    moe.qmatvec_unpack_weights(cvoid(d[k]))
