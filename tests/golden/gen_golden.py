"""Writes the golden fixtures under tests/golden/ (run from the repo root: python tests/golden/gen_golden.py).

dequant_ref.npz  random blocks of each type and their decoding by the reference's own qt_to_float, compiled from
                 src/quant_types.cpp into oracle/_ref (the reference's code, not a restatement)
quant.npz        activation vectors (with the quantizer's special cases) and their Q8_0 / Q8_K encodings
layer_small.npz  one small MoE layer per type: weights, inputs, router logits and the oracle's outputs
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "tests"), os.path.join(ROOT, "rocm-hip_amd")]
import oracle_lib  # noqa: E402
import synth  # noqa: E402

TYPES = [8, 12, 100, 101]


def main():
    orc, ref = oracle_lib.Oracle(), oracle_lib.RefCPU()
    rng = np.random.default_rng(20240601)
    out = {}
    for t in TYPES:
        bv, bb = synth.BLOCK[t]
        raw = rng.integers(0, 256, size=(64 if bv == 32 else 16, bb), dtype=np.uint8)
        out[f"raw_{t}"] = raw
        out[f"deq_{t}"] = ref.to_float(t, raw, raw.shape[0] * bv)
    np.savez_compressed(os.path.join(HERE, "dequant_ref.npz"), **out)

    x = (rng.standard_normal(2048) * 10.0 ** rng.integers(-3, 3, 2048)).astype(np.float32)
    x[:32] = 0.0
    x[32:40] = [127.0, 2.5, 3.5, -2.5, -3.5, 0.5, 1.5, -0.5]
    x[256:512] = 0.0
    x[512 + 5], x[512 + 9] = -50.0, 50.0
    q0, d0, s0 = orc.quantize_q8_0(x)
    qK, dK, bsK = orc.quantize_q8_K(x)
    np.savez_compressed(os.path.join(HERE, "quant.npz"), x=x, q0=q0, d0=d0, s0=s0, qK=qK, dK=dK, bsK=bsK)

    lay = {}
    for t in TYPES:
        E, FE = (256, 256) if t == 12 else (256, 128)
        spec = synth.LayerSpec(t, E, 3, 2, FE, shared=(t != 12))
        L = synth.make_layer(spec, seed=100 + t)
        xx = np.random.default_rng(200 + t).standard_normal((3, E)).astype(np.float32)
        logits = np.stack([orc.matvec_f32(L["w_router"], xx[i]) for i in range(3)])
        o, ids, wts = orc.moe_forward(spec, L, xx, logits=logits)
        for k, v in L.items():
            lay[f"{t}_{k}"] = v
        lay[f"{t}_x"], lay[f"{t}_logits"], lay[f"{t}_out"], lay[f"{t}_ids"], lay[f"{t}_wts"] = xx, logits, o, ids, wts
        lay[f"{t}_spec"] = np.array([t, E, 3, 2, FE, int(spec.shared)], np.int32)
    np.savez_compressed(os.path.join(HERE, "layer_small.npz"), **lay)


if __name__ == "__main__":
    main()
