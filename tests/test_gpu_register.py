"""Weight registration modes (qmatvec_pack_weights_ex): in place (the split planes replace the native rows) and
without the MFMA operand tiles. Each gives the default registration's bits where both run the same kernels
(decode: the planes; prefill with tiles: the tiles), stays within the oracle's tolerance, restores the native bytes
at unregistration, and refuses a launch that would read an in-place matrix as native rows."""
import ctypes

import numpy as np
import pytest
import torch

import moe_hip
import synth
from gpu_util import announce, cvoid, dev, host, rel_l2, zeros

pytestmark = pytest.mark.gpu
Q8_0, Q4_K, FP4, FAST = 8, 12, 100, 101
INPLACE, NO_TILES = 1, 2
INVALID_VALUE = 1
S = moe_hip.stream_handle
MATS = ("w_gate", "w_up", "w_down", "s_gate", "s_up", "s_down")


def _shapes(spec):
    return {"w_gate": (spec.NE * spec.FE, spec.E), "w_up": (spec.NE * spec.FE, spec.E),
            "w_down": (spec.NE * spec.E, spec.FE), "s_gate": (spec.FE, spec.E), "s_up": (spec.FE, spec.E),
            "s_down": (spec.E, spec.FE)}


def _register(moe, spec, d, flags):
    for k, (rows, K) in _shapes(spec).items():
        if k in d:
            assert moe.lib.qmatvec_pack_weights_ex(spec.qtype, cvoid(d[k]), moe_hip.row_size(spec.qtype, K), rows, K,
                                                   flags, S()) == 0, k


def _unregister(moe, d):
    torch.cuda.synchronize()
    for k in MATS:
        if k in d:
            moe.qmatvec_unpack_weights(cvoid(d[k]))


def _layer_run(moe, spec, d, x, logits):
    T = x.shape[0]
    desc = moe_hip.LayerDesc(spec.qtype, spec.E, spec.NE, spec.NU, spec.FE, cvoid(d["w_router"]), cvoid(d["w_gate"]),
                             cvoid(d["w_up"]), cvoid(d["w_down"]), cvoid(d.get("s_gate")), cvoid(d.get("s_up")),
                             cvoid(d.get("s_down")), cvoid(d.get("w_shexp")))
    nb = moe.lib.moe_layer_scratch_bytes(ctypes.byref(desc), T)
    sc = zeros(nb + 256, torch.uint8)
    out, ids = zeros((T, spec.E), torch.float32), zeros((T, spec.NU), torch.int32)
    moe.moe_layer_forward(ctypes.byref(desc), cvoid(dev(x)), cvoid(dev(logits)), T, cvoid(out), cvoid(ids), None,
                          ctypes.c_void_p((sc.data_ptr() + 255) // 256 * 256), nb, S())
    return host(out), host(ids)


SPECS = [synth.LayerSpec(FP4, 512, 16, 4, 256, True), synth.LayerSpec(Q8_0, 768, 16, 4, 256, False),
         synth.LayerSpec(Q4_K, 512, 8, 2, 512, False), synth.LayerSpec(FAST, 512, 8, 8, 256, True)]


@pytest.mark.parametrize("spec", SPECS, ids=lambda s: str(s.qtype))
@pytest.mark.parametrize("flags", [INPLACE, NO_TILES, INPLACE | NO_TILES])
def test_registration_modes(moe, oracle, spec, flags):
    announce("registration", spec.qtype, flags)
    L = synth.make_layer(spec, seed=90 + spec.qtype)
    rng = np.random.default_rng(91)
    base = {}
    d = {k: dev(v) for k, v in L.items()}
    cases = []
    for T in (1, 3, 24):
        x = rng.standard_normal((T, spec.E)).astype(np.float32)
        logits = np.stack([oracle.matvec_f32(L["w_router"], x[t]) for t in range(T)])
        cases.append((x, logits))
    # the runs it must equal: the default copy registration for decode and (with tiles) prefill; a copy without
    # tiles for prefill without tiles
    ref_flags = flags & NO_TILES
    _register(moe, spec, d, ref_flags)
    for i, (x, lg) in enumerate(cases):
        base[i] = _layer_run(moe, spec, d, x, lg)
    _unregister(moe, d)
    d = {k: dev(v) for k, v in L.items()}
    _register(moe, spec, d, flags)
    try:
        if flags & INPLACE:  # the native rows are gone from W
            k = "w_gate"
            assert not np.array_equal(host(d[k]), L[k])
        for i, (x, lg) in enumerate(cases):
            got, ids = _layer_run(moe, spec, d, x, lg)
            want, wids, _ = oracle.moe_forward(spec, L, x, logits=lg)
            assert np.array_equal(ids, wids) and np.array_equal(ids, base[i][1])
            assert np.array_equal(got.view(np.uint32), base[i][0].view(np.uint32)), x.shape[0]
            assert rel_l2(got, want) < (1e-5 if x.shape[0] < 8 else 1e-3)
    finally:
        _unregister(moe, d)
    for k in MATS:  # unregistering restores the native rows
        if k in d:
            assert np.array_equal(host(d[k]), L[k]), k


def test_inplace_matrix_is_not_read_as_native_rows(moe, oracle):
    """An id launch over an in-place matrix and an unregistered shared-expert matrix is refused (its native rows
    are gone); with both registered it runs and matches the oracle."""
    announce("inplace mixed")
    spec = synth.LayerSpec(Q8_0, 512, 8, 2, 256, True)
    L = synth.make_layer(spec, seed=95)
    d = {k: dev(v) for k, v in L.items()}
    rb = moe_hip.row_size(spec.qtype, spec.E)
    assert moe.lib.qmatvec_pack_weights_ex(spec.qtype, cvoid(d["w_gate"]), rb, spec.NE * spec.FE, spec.E, INPLACE,
                                           S()) == 0
    try:
        q = moe_hip.Q8Buffer(moe, spec.E)
        x = np.random.default_rng(96).standard_normal(spec.E).astype(np.float32)
        moe.qmatvec_quantize(cvoid(dev(x)), spec.E, q.ref(), S())
        ids = dev(np.array([3, -1], np.int32))
        y = zeros((2, spec.FE), torch.float32)
        e = moe.lib.qmatvec_launch_q8_id_x(spec.qtype, cvoid(d["w_gate"]), None, cvoid(d["s_gate"]), None, rb,
                                           cvoid(ids), 2, 0, q.ref(), cvoid(y), None, spec.FE, spec.E, 1, S())
        assert e == INVALID_VALUE
        assert moe.lib.qmatvec_pack_weights_ex(spec.qtype, cvoid(d["s_gate"]), rb, spec.FE, spec.E, INPLACE,
                                               S()) == 0
        e = moe.lib.qmatvec_launch_q8_id_x(spec.qtype, cvoid(d["w_gate"]), None, cvoid(d["s_gate"]), None, rb,
                                           cvoid(ids), 2, 0, q.ref(), cvoid(y), None, spec.FE, spec.E, 1, S())
        assert e == 0
        got = host(y)
        want = np.stack([oracle.matvec(spec.qtype, L["w_gate"][3 * spec.FE:4 * spec.FE], x, spec.FE, spec.E),
                         oracle.matvec(spec.qtype, L["s_gate"], x, spec.FE, spec.E)])
        assert rel_l2(got, want) < 1e-5
    finally:
        torch.cuda.synchronize()
        moe.qmatvec_unpack_weights(cvoid(d["w_gate"]))
        moe.qmatvec_unpack_weights(cvoid(d["s_gate"]))


OUT_OF_MEMORY = 2


@pytest.mark.parametrize("qtype,flags", [(Q8_0, INPLACE), (FP4, INPLACE | NO_TILES), (Q4_K, INPLACE), (FAST, INPLACE)])
def test_inplace_rewrite_failures_and_chunks(moe, oracle, qtype, flags):
    """In-place registration runs in row chunks through a bounded transient buffer (here 3 rows' worth, so every
    chunk boundary case occurs) and restores W bit for bit. When the transient buffer cannot be had, pack leaves
    W untouched and unregistered, and unpack leaves the registration in force and usable."""
    announce("inplace chunks / failures", qtype, flags)
    spec = synth.LayerSpec(qtype, 512, 8, 2, 256, False)
    L = synth.make_layer(spec, seed=97 + qtype)
    rows, K = spec.NE * spec.FE, spec.E
    rb = moe_hip.row_size(qtype, K)
    d = {k: dev(v) for k, v in L.items()}
    W = d["w_gate"]
    q = moe_hip.Q8Buffer(moe, K)
    x = np.random.default_rng(98).standard_normal(K).astype(np.float32)
    moe.qmatvec_quantize(cvoid(dev(x)), K, q.ref(), S())
    ids = dev(np.array([5, 1], np.int32))
    want = np.stack([oracle.matvec(qtype, L["w_gate"][e * spec.FE:(e + 1) * spec.FE], x, spec.FE, K) for e in (5, 1)])

    def run():
        y = zeros((2, spec.FE), torch.float32)
        e = moe.lib.qmatvec_launch_q8_id(qtype, cvoid(W), rb, cvoid(ids), 2, 0, q.ref(), cvoid(y), spec.FE, K, 1, S())
        return e, (host(y) if e == 0 else None)
    try:
        moe.lib.qmatvec_test_registry(1, 3 * rb)  # the pack's transient buffer fails
        assert moe.lib.qmatvec_pack_weights_ex(qtype, cvoid(W), rb, rows, K, flags, S()) == OUT_OF_MEMORY
        assert np.array_equal(host(W), L["w_gate"])  # untouched, and read as native rows
        e, y = run()
        assert e == 0 and rel_l2(y, want) < 1e-5
        assert moe.lib.qmatvec_pack_weights_ex(qtype, cvoid(W), rb, rows, K, flags, S()) == 0
        assert not np.array_equal(host(W), L["w_gate"])
        e, y_packed = run()
        assert e == 0 and rel_l2(y_packed, want) < 1e-5
        moe.lib.qmatvec_test_registry(1, 3 * rb)  # the unpack's transient buffer fails: still registered
        assert moe.lib.qmatvec_unpack_weights(cvoid(W)) == OUT_OF_MEMORY
        e, y = run()
        assert e == 0 and np.array_equal(y, y_packed)
        assert moe.lib.qmatvec_unpack_weights(cvoid(W)) == 0
        assert np.array_equal(host(W), L["w_gate"])  # the native rows back, bit for bit
        e, y = run()
        assert e == 0 and rel_l2(y, want) < 1e-5
    finally:
        moe.lib.qmatvec_test_registry(0, 0)
        torch.cuda.synchronize()
        moe.lib.qmatvec_unpack_weights(cvoid(W))
