"""The committed golden fixtures (tests/golden/gen_golden.py): the oracle still reproduces them, on the CPU; the
decoders' fixtures hold the reference's own qt_to_float outputs."""
import os

import numpy as np
import pytest

import synth

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(G, name), allow_pickle=False)


@pytest.mark.parametrize("qtype", [8, 12, 100, 101])
def test_oracle_decoders_match_reference_vectors(oracle, qtype):
    f = _load("dequant_ref.npz")
    raw, want = f[f"raw_{qtype}"], f[f"deq_{qtype}"]
    got = oracle.dequant(qtype, raw, want.size)
    ok = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert ok.all()


def test_oracle_quantizers_match_fixture(oracle):
    f = _load("quant.npz")
    q0, d0, s0 = oracle.quantize_q8_0(f["x"])
    qK, dK, bsK = oracle.quantize_q8_K(f["x"])
    for a, b in ((q0, f["q0"]), (d0, f["d0"]), (s0, f["s0"]), (qK, f["qK"]), (dK, f["dK"]), (bsK, f["bsK"])):
        assert np.array_equal(a, b)


def layer_fixture(f, qtype):
    t, E, NE, NU, FE, sh = (int(v) for v in f[f"{qtype}_spec"])
    spec = synth.LayerSpec(t, E, NE, NU, FE, bool(sh))
    keys = ["w_router", "w_gate", "w_up", "w_down"] + (["s_gate", "s_up", "s_down", "w_shexp"] if sh else [])
    L = {k: f[f"{qtype}_{k}"] for k in keys}
    return spec, L, f[f"{qtype}_x"], f[f"{qtype}_logits"], f[f"{qtype}_out"], f[f"{qtype}_ids"], f[f"{qtype}_wts"]


@pytest.mark.parametrize("qtype", [8, 12, 100, 101])
def test_oracle_layer_matches_fixture(oracle, qtype):
    spec, L, x, logits, out, ids, wts = layer_fixture(_load("layer_small.npz"), qtype)
    o, i, w = oracle.moe_forward(spec, L, x, logits=logits)
    assert np.array_equal(i, ids) and np.array_equal(w, wts) and np.array_equal(o, out)
