"""A seeded sweep of whole MoE layers over shapes, types, token counts and registration, each against the oracle's
layer (orc_moe_forward) with the oracle's router logits: ids exact, weights to 2e-6; for decode (T < 8: the fused
single- and multi-token kernels or the per-operation launches) every token within 1e-5 relative L2, except a token
one of whose SwiGLU outputs lies within 1e-5 of a rounding boundary of the quantizer that feeds down (there the
GPU's fp32 gate / up sums, ~1e-7 from the oracle's double ones, may give the neighbouring code), which must then
be within 1e-3; for the grouped prefill (T >= 8: dispatch, the MFMA or per-entry expert kernels, the shared expert
as tiles or dense) 1e-3. The shapes are drawn from the ranges the launchers take (E and FE multiples of 256, up to
128 experts, top-1 to top-8, with and without a shared expert), so the paths' selection rules meet shapes no fixed
test has. Decode outputs also equal the per-operation launches' bit for bit.
"""
import numpy as np
import pytest

import synth
from gpu_util import announce, rel_l2
from test_gpu_parity import _run_layer
from test_gpu_parity import test_layer_forward_norm_equals_add_rmsnorm_then_layer as _norm_case

pytestmark = pytest.mark.gpu
Q8_0, FP4, FAST, Q4_K = 8, 100, 101, 12


def _case(i):
    rng = np.random.default_rng(7000 + i)
    qtype = [Q8_0, FP4, FAST, Q4_K][i % 4]
    E = int(rng.choice([256, 512, 768, 1024] if qtype == Q4_K else [256, 512, 768, 1024, 2048]))
    FE = int(rng.choice([256, 512, 768]))
    NE = int(rng.choice([4, 8, 12, 16, 24, 32, 60, 64, 128]))
    NU = int(rng.integers(1, min(NE, 8) + 1))
    shared = bool(rng.integers(0, 2))
    T = int(rng.choice([1, 2, 3, 4, 5, 7, 8, 13, 33, 64, 100]))
    packed = bool(rng.integers(0, 4))  # (registered three times in four)
    return qtype, E, FE, NE, NU, shared, T, packed


CASES = [_case(i) for i in range(64)]


def _quant_near_tie(oracle, spec, L, x, ids, window=1e-5):
    """Whether a down input of this token (SiLU(g) u of a chosen expert or the shared one, on the oracle's gate / up
    sums) lies within window of a rounding boundary of the layer's quantizer (Q8_0 per 32, Q8_K per 256): there the
    GPU's fp32 gate / up sums, ~1e-7 from the oracle's double ones, may round it to the neighbouring integer -- the
    quantization counterpart of a router near-tie."""
    FE, E = spec.FE, spec.E
    mats = [(L["w_gate"][e * FE:(e + 1) * FE], L["w_up"][e * FE:(e + 1) * FE]) for e in ids]
    if spec.shared:
        mats.append((L["s_gate"], L["s_up"]))
    for wg, wu in mats:
        a = oracle.swiglu(oracle.matvec(spec.qtype, wg, x, FE, E), oracle.matvec(spec.qtype, wu, x, FE, E))
        n = 256 if spec.qtype == Q4_K else 32
        for blk in a.reshape(-1, n):
            if spec.qtype == Q4_K:
                mx = blk[np.argmax(np.abs(blk))]
                v = np.float32(-127.0) / mx * blk if mx != 0 else blk * 0
            else:
                am = np.abs(blk).max()
                v = blk * (np.float32(127.0) / am) if am != 0 else blk * 0
            if np.any(np.abs(np.abs(v) % 1.0 - 0.5) < window):
                return True
    return False


@pytest.mark.parametrize("qtype,E,FE,NE,NU,shared,T,packed", CASES)
def test_layer_sweep(moe, oracle, qtype, E, FE, NE, NU, shared, T, packed):
    announce("sweep", qtype, E, FE, NE, NU, shared, T, packed)
    spec = synth.LayerSpec(qtype, E, NE, NU, FE, shared)
    L = synth.make_layer(spec, seed=E + FE + NE + NU + T + qtype)
    rng = np.random.default_rng(E * 3 + T)
    x = rng.standard_normal((T, E)).astype(np.float32)
    logits = np.stack([oracle.matvec_f32(L["w_router"], x[t]) for t in range(T)])
    got, ids, wts = _run_layer(moe, spec, L, x, logits=logits, packed=packed)
    rows = np.arange(T) if T <= 16 else np.sort(rng.choice(T, 16, replace=False))
    want, wids, wwts = oracle.moe_forward(spec, L, x[rows], logits=logits[rows])
    assert np.array_equal(ids[rows], wids)
    np.testing.assert_allclose(wts[rows], wwts, rtol=2e-6)
    assert np.isfinite(got).all()
    if T >= 8:
        err = rel_l2(got[rows], want)
        assert err < 1e-3, err
        return
    for k, t in enumerate(rows):  # decode: 1e-5 per token, unless a down input sits at a quantizer rounding boundary
        err = rel_l2(got[t], want[k])
        if err >= 1e-5:
            assert err < 1e-3 and _quant_near_tie(oracle, spec, L, x[t], wids[k]), (t, err)
    # the per-operation launches give the same bits as whatever decode path ran (fused or not)
    moe.lib.moe_layer_set_fused(0)
    try:
        ref, rids, rwts = _run_layer(moe, spec, L, x, logits=logits, packed=packed)
    finally:
        moe.lib.moe_layer_set_fused(1)
    assert np.array_equal(ids, rids) and np.array_equal(wts, rwts)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


NORM_SWEEP = [(synth.LayerSpec(c[0], c[1], c[3], c[4], c[2], c[5]), c[6], bool(i % 2), bool(i % 3))
              for i, c in enumerate(CASES[:24])]


@pytest.mark.parametrize("spec,T,with_add,with_w", NORM_SWEEP, ids=lambda v: str(getattr(v, "qtype", v)))
def test_norm_layer_sweep(moe, spec, T, with_add, with_w):
    """The sweep's first 24 shapes through moe_layer_forward_norm (the RMSNorm producer fused into the layer's first
    kernel where the fused path takes the layer): the bits of gpu_add_rmsnorm followed by moe_layer_forward."""
    _norm_case(moe, spec, T, with_add, with_w)
