"""Pins the CPU oracle (oracle/moe_oracle.c) before anything is compared against it.

Each check is chosen so that a plausible mistake in the oracle fails it: the decoders are compared bit for bit
with the reference's own qt_to_float (built from src/quant_types.cpp into oracle/_ref) and with hand-built
known-answer blocks; the integer block dots with int64 dots over codes the reference's decoder yields at unit
scale; the quantizers with their special cases and error bounds; the router with brute force; the dispatch with
its invariants; the layer with an independent float64 route through the reference's decoder.
"""
import os

import numpy as np
import pytest

import synth
from oracle_lib import REF, RefCPU

Q8_0, Q4_K, FP4, FAST = 8, 12, 100, 101
TYPES = [Q8_0, Q4_K, FP4, FAST]
HAS_REF = os.path.exists(REF)
needs_ref = pytest.mark.skipif(not HAS_REF, reason="oracle/_ref not built (needs the reference tree)")


@pytest.fixture(scope="module")
def ref():
    return RefCPU()


# ------------------------------------------------------------------ scalars

def test_fp16_to_f32_all_halves(oracle):
    h = np.arange(65536, dtype=np.uint32)
    got = np.array([oracle.lib.orc_fp16_to_f32(int(v)) for v in h], np.float32)
    want = h.astype(np.uint16).view(np.float16).astype(np.float32)
    assert np.array_equal(got.view(np.uint32)[~np.isnan(want)], want.view(np.uint32)[~np.isnan(want)])
    assert np.isnan(got[np.isnan(want)]).all()


def test_f32_to_fp16_rne(oracle):
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 6, 20000),
                        np.array([65504, 65519.99, 65520, 1e-8, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 2.0 ** -24,
                                  3 * 2.0 ** -26, -0.0, 0.0, np.inf, -np.inf])]).astype(np.float32)
    got = np.array([oracle.lib.orc_f32_to_fp16(float(v)) for v in x], np.uint16)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_ue4m3_known_answers(oracle):
    # 0x38 -> 0.5 and 0x40 -> 1.0 (the engine's half scale), 0x7f and above -> 0, subnormals m 2^-10
    assert oracle.lib.orc_ue4m3_half(0x38) == 0.5
    assert oracle.lib.orc_ue4m3_half(0x40) == 1.0
    assert oracle.lib.orc_ue4m3_half(0x7F) == 0.0
    assert oracle.lib.orc_ue4m3_half(0xFF) == 0.0
    assert oracle.lib.orc_ue4m3_half(0x03) == 3 * 2.0 ** -10
    assert oracle.lib.orc_ue4m3_half(0x7E) == 14 * 16.0
    table = synth.ue4m3_half_table()
    assert all(oracle.lib.orc_ue4m3_half(e) == table[e] for e in range(256))


# ------------------------------------------------------------------ decoders

def _random_blocks(qtype, n, rng):
    bv, bb = synth.BLOCK[qtype]
    return rng.integers(0, 256, size=(n, bb), dtype=np.uint8)


@needs_ref
@pytest.mark.parametrize("qtype", TYPES)
def test_dequant_matches_reference_build(oracle, ref, qtype):
    """Fully random bytes (every scale and code pattern) decode to the same bits as the reference's decoder."""
    rng = np.random.default_rng(qtype)
    bv, _ = synth.BLOCK[qtype]
    raw = _random_blocks(qtype, 4096, rng)
    n = raw.shape[0] * bv
    a, b = oracle.dequant(qtype, raw, n), ref.to_float(qtype, raw, n)
    ok = (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))
    assert ok.all()


def test_dequant_known_answer_fp4(oracle):
    # all 16 codes in the low nibbles, reversed in the high nibbles, e0 = 0x38 (0.5), e1 = 0x40 (1.0)
    cb = np.array([0, 1, 2, 3, 4, 6, 8, 10, 0, -1, -2, -3, -4, -6, -8, -10], np.float32)
    blk = np.zeros(18, np.uint8)
    blk[:16] = np.arange(16) | ((15 - np.arange(16)) << 4)
    blk[16], blk[17] = 0x38, 0x40
    y = oracle.dequant(FP4, blk, 32)
    assert np.array_equal(y[:16], 0.5 * cb) and np.array_equal(y[16:], cb[::-1])
    blk[16] = 0x7F  # a scale byte of 0x7f decodes to 0
    assert np.all(oracle.dequant(FP4, blk, 32)[:16] == 0)
    fast = np.concatenate([blk[:16], [0x40]]).astype(np.uint8)
    y = oracle.dequant(FAST, fast, 32)
    assert np.array_equal(y[:16], cb) and np.array_equal(y[16:], cb[::-1])


def test_dequant_known_answer_q8_0(oracle):
    blk = np.zeros(34, np.uint8)
    blk[0:2] = np.array([2.0], np.float16).view(np.uint8)
    q = np.arange(-16, 16, dtype=np.int8)
    blk[2:] = q.view(np.uint8)
    assert np.array_equal(oracle.dequant(Q8_0, blk, 32), 2.0 * q.astype(np.float32))


def _q4k_pack_scales(sc, mn):
    """ggml's documented Q4_K 6-bit packing of eight (scale, min) pairs into 12 bytes."""
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    return s


def test_dequant_known_answer_q4k(oracle):
    rng = np.random.default_rng(7)
    sc, mn = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
    q = rng.integers(0, 16, 256)
    blk = np.zeros(144, np.uint8)
    blk[0:4] = np.array([0.25, 0.125], np.float16).view(np.uint8)
    blk[4:16] = _q4k_pack_scales(sc, mn)
    for c in range(4):  # value 64c + l: low nibble of byte 32c + l; 64c + 32 + l: high nibble
        blk[16 + 32 * c:16 + 32 * c + 32] = q[64 * c:64 * c + 32] | (q[64 * c + 32:64 * c + 64] << 4)
    want = np.array([0.25 * sc[i // 32] * q[i] - 0.125 * mn[i // 32] for i in range(256)], np.float32)
    assert np.array_equal(oracle.dequant(Q4_K, blk, 256), want)


def _unit_scale_blocks(qtype, n, rng):
    """Blocks whose scales decode to exactly 1 (Q4_K: d 1, dmin 0, all sub-scales 1): decoded = integer codes."""
    raw = _random_blocks(qtype, n, rng)
    if qtype == Q8_0:
        raw[:, 0:2] = np.array([1.0], np.float16).view(np.uint8)
    elif qtype == FP4:
        raw[:, 16] = raw[:, 17] = 0x40
    elif qtype == FAST:
        raw[:, 16] = 0x40
    else:
        raw[:, 0:4] = np.array([1.0, 0.0], np.float16).view(np.uint8)
        raw[:, 4:16] = _q4k_pack_scales(np.ones(8, int), np.zeros(8, int))
    return raw


@needs_ref
@pytest.mark.parametrize("qtype", TYPES)
def test_block_dots_against_reference_codes(oracle, ref, qtype):
    """Integer block dots equal int64 dots of the codes the reference's decoder yields at unit scale."""
    rng = np.random.default_rng(100 + qtype)
    K = 512
    bv, bb = synth.BLOCK[qtype]
    wrow = _unit_scale_blocks(qtype, K // bv, rng).ravel()
    codes = ref.to_float(qtype, wrow, K).astype(np.int64)
    xq = rng.integers(-127, 128, K).astype(np.int8)
    got = oracle.block_dots(qtype, wrow, xq, K)
    unit = 16 if qtype == FP4 else 32
    want = (codes * xq.astype(np.int64)).reshape(-1, unit).sum(axis=1)
    assert np.array_equal(got.astype(np.int64), want)


@pytest.mark.parametrize("qtype", TYPES)
def test_row_dot_int_equals_dequant_route(oracle, qtype):
    """The integer-dot route and the decode-then-dot route give the same number (two independent routes)."""
    rng = np.random.default_rng(200 + qtype)
    K = 1024
    W = synth.matrix(qtype, 16, K, rng)
    x = rng.standard_normal(K).astype(np.float32)
    xr = oracle.roundtrip(qtype, x)
    if qtype == Q4_K:
        xq, xd, xbs = oracle.quantize_q8_K(x)
    else:
        xq, xd, _ = oracle.quantize_q8_0(x)
        xbs = None
    for r in range(16):
        a = oracle.row_dot_int(qtype, W[r], xq, xd, xbs, K)
        b = oracle.row_dot_deq(qtype, W[r], xr, K)
        assert abs(a - b) <= 1e-6 * (abs(b) + 1e-3), (r, a, b)


# ------------------------------------------------------------------ activation quantizers

def test_q8_0_special_cases(oracle):
    x = np.zeros(64, np.float32)
    x[32:] = [127.0, 2.5, 3.5, -2.5, -3.5, 0.5, 1.5, -0.5] + [0.0] * 24
    q, d, s = oracle.quantize_q8_0(x)
    assert np.all(q[:32] == 0) and d[0] == 0 and s[0] == 0  # all-zero block
    assert d[1] == 1.0  # amax 127 -> id 1 exactly: round half to even below
    assert list(q[32:40]) == [127, 2, 4, -2, -4, 0, 2, 0]
    assert s[1] == np.float32(127 + 2 + 4 - 2 - 4 + 0 + 2 + 0).view(np.int32)


def test_q8_0_bounds(oracle):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(32 * 512) * 10.0 ** rng.integers(-3, 3, 32 * 512)).astype(np.float32)
    q, d, s = oracle.quantize_q8_0(x)
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    assert np.array_equal(d, (amax / np.float32(127)).astype(np.float16).astype(np.float32))
    assert np.array_equal(np.abs(q.reshape(-1, 32)).max(axis=1), np.full(512, 127))  # the max maps to +-127
    err = np.abs(q.reshape(-1, 32) * (amax / 127)[:, None] - xb)
    assert np.all(err <= (amax / 127)[:, None] * 0.5 * (1 + 1e-6))
    sums = q.reshape(-1, 32).astype(np.int64).sum(axis=1)
    want_s = ((amax / np.float32(127)).astype(np.float32) * sums.astype(np.float32)).astype(np.float16)
    assert np.array_equal(s.view(np.float32), want_s.astype(np.float32))


def test_q8_K_special_cases(oracle):
    x = np.zeros(512, np.float32)
    x[256 + 3], x[256 + 7], x[256 + 9] = -2.0, 2.0, 1.0  # equal |max|: the first (negative) one wins
    q, d, bs = oracle.quantize_q8_K(x)
    assert np.all(q[:256] == 0) and d[0] == 0 and np.all(bs[:16] == 0)
    iscale = np.float32(-127) / np.float32(-2.0)
    assert d[1] == np.float32(1) / iscale
    assert q[256 + 3] == -127 and q[256 + 7] == 127  # the first max maps to -127, its opposite to +127
    assert q[256 + 9] == int(np.rint(iscale * np.float32(1.0)))
    assert np.array_equal(bs[16:], q[256:].reshape(16, 16).astype(np.int64).sum(axis=1))


def test_q8_K_bounds(oracle):
    rng = np.random.default_rng(4)
    x = rng.standard_normal(256 * 64).astype(np.float32)
    q, d, bs = oracle.quantize_q8_K(x)
    err = np.abs(q.reshape(-1, 256) * d[:, None] - x.reshape(-1, 256))
    assert np.all(err <= np.abs(d)[:, None] * 0.5 * (1 + 1e-5))
    assert np.array_equal(bs, q.reshape(-1, 16).astype(np.int64).sum(axis=1))
    assert q.min() >= -127


# ------------------------------------------------------------------ router

def test_router_brute_force(oracle):
    rng = np.random.default_rng(5)
    for ne, nu in [(8, 2), (16, 4), (128, 8), (256, 8), (1024, 64)]:
        t = 5
        lg = rng.standard_normal((t, ne)).astype(np.float32)
        lg[0, : min(ne, 12)] = 0.5  # a block of ties: lower indices first
        ids, wts, _ = oracle.router(lg, ne, nu)
        p = np.exp(lg.astype(np.float64) - lg.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        want = np.argsort(-p, axis=1, kind="stable")[:, :nu]
        assert np.array_equal(ids, want)
        sel = np.take_along_axis(p, want, axis=1)
        np.testing.assert_allclose(wts, sel / sel.sum(axis=1, keepdims=True), rtol=1e-6)


def test_router_all_equal_and_shared_slot(oracle):
    ids, wts, _ = oracle.router(np.zeros((2, 16), np.float32), 16, 4, ids_stride=5)
    assert np.array_equal(ids, [[0, 1, 2, 3, -1]] * 2)
    assert np.all(wts == np.float32(0.25))
    x = np.ones(8, np.float32)
    w = np.full(8, 0.25, np.float32)
    _, _, sg = oracle.router(np.zeros((1, 16), np.float32), 16, 4, x=x, w_shexp=w)
    assert abs(sg[0] - 1 / (1 + np.exp(-2.0))) < 1e-7


# ------------------------------------------------------------------ dispatch

def test_group_invariants(oracle):
    rng = np.random.default_rng(6)
    for t, nu, ne, tile in [(37, 8, 128, 16), (300, 4, 64, 64), (5, 2, 1024, 1)]:
        ids = np.stack([rng.permutation(ne)[:nu] for _ in range(t)]).astype(np.int32)
        g = oracle.group(ids, t, nu, ne, tile)
        flat = ids.ravel()
        assert np.array_equal(g["counts"], np.bincount(flat, minlength=ne))
        assert np.array_equal(g["offsets"], np.concatenate([[0], np.cumsum(g["counts"])[:-1]]))
        for e in range(ne):
            run = g["pair_rows"][g["offsets"][e]:g["offsets"][e] + g["counts"][e]]
            assert np.array_equal(run, np.flatnonzero(flat == e))  # ascending entry order
        assert np.array_equal(g["tok_rows"], g["pair_rows"] // nu)
        assert g["n_tiles"] == sum((c + tile - 1) // tile for c in g["counts"])
        assert g["n_tiles"] <= oracle.lib.orc_max_tiles(t, nu, ne, tile)
        for k in range(g["n_tiles"]):
            e = g["tile_e"][k]
            assert g["offsets"][e] <= g["tile_start"][k] < g["offsets"][e] + g["counts"][e]
            assert 1 <= g["tile_n"][k] <= tile
        assert g["tile_n"].sum() == t * nu


def _group_brute(ids, nu, ne, tile):
    """moe_group's outputs by brute force (src/gpu_ops.hip:273-320): every entry with an id in [0, ne), repeats
    within a row included, stably sorted by expert; tiles of each expert's run in expert order."""
    flat = ids.ravel()
    ok = (flat >= 0) & (flat < ne)
    entries = np.flatnonzero(ok)
    order = entries[np.argsort(flat[entries], kind="stable")]
    counts = np.bincount(flat[entries], minlength=ne)
    offs = np.concatenate([[0], np.cumsum(counts)[:-1]])
    te, ts, tn = [], [], []
    for e in range(ne):
        for k in range(0, counts[e], tile):
            te.append(e), ts.append(offs[e] + k), tn.append(min(tile, counts[e] - k))
    return dict(counts=counts, pair_rows=order, tok_rows=order // nu, tile_e=te, tile_start=ts, tile_n=tn)


def test_group_counts_repeats_and_skips_invalid(oracle):
    """A repeated id within a token's row is counted and placed twice, as the reference's histogram and atomic
    placement do (src/gpu_ops.hip:281, 316-320); ids outside [0, ne) are skipped."""
    ids = np.array([[1, 1, 3], [0, 9, -1]], np.int32)  # a repeat, an id past n_expert, a negative id
    g = oracle.group(ids, 2, 3, 4, 2)
    assert list(g["counts"]) == [1, 2, 0, 1]
    assert list(g["pair_rows"][:4]) == [3, 0, 1, 2]
    assert list(g["tok_rows"][:4]) == [1, 0, 0, 0]
    assert g["n_tiles"] == 3 and list(g["tile_n"][:3]) == [1, 2, 1]


@pytest.mark.parametrize("t,nu,ne,tile", [(50, 8, 16, 4), (9, 20, 6, 3), (300, 3, 2, 64), (1, 64, 3, 1)])
def test_group_repeats_brute_force(oracle, t, nu, ne, tile):
    rng = np.random.default_rng(t * nu + ne)
    ids = rng.integers(-1, ne + 1, size=(t, nu)).astype(np.int32)  # many repeats, some invalid ids
    g = oracle.group(ids, t, nu, ne, tile)
    b = _group_brute(ids, nu, ne, tile)
    n = len(b["pair_rows"])
    assert np.array_equal(g["counts"], b["counts"])
    assert np.array_equal(g["pair_rows"][:n], b["pair_rows"]) and np.array_equal(g["tok_rows"][:n], b["tok_rows"])
    assert g["n_tiles"] == len(b["tile_e"])
    for k in ("tile_e", "tile_start", "tile_n"):
        assert np.array_equal(g[k][:g["n_tiles"]], b[k]), k


# ------------------------------------------------------------------ SwiGLU and RMSNorm

def _special_floats(rng, n):
    """Random floats across magnitudes plus the special values: +-0, denormals, +-1e+-30, +-88/89 (expf's
    overflow edge), +-inf."""
    v = (rng.standard_normal(n) * np.exp(rng.uniform(-20, 20, n))).astype(np.float32)
    sp = np.array([0.0, -0.0, 1e-40, -1e-40, 1e-30, -1e-30, 1e30, -1e30, 88.0, -88.0, 89.0, -89.0, 100.0, -100.0,
                   np.inf, -np.inf, 1.0, -1.0, 0.5, -0.5], np.float32)
    return np.concatenate([v, sp])


@needs_ref
def test_swiglu_matches_reference_silu(oracle, ref):
    """orc_swiglu == the reference's qwen_silu(g) * u (src/qwen_ops.h:47) bit for bit, special values included."""
    rng = np.random.default_rng(31)
    g = _special_floats(rng, 50000)
    u = np.concatenate([rng.standard_normal(50000).astype(np.float32),
                        np.array([1, -1, 2, 0, 3, 1e-30, 1e30, -1, 1, 2, -2, 1, -1, 1, 1, 1, 7, -7, 1, 1], np.float32)])
    a, b = oracle.swiglu(g, u), ref.swiglu(g, u)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    gg = rng.standard_normal(4096).astype(np.float32)
    assert np.array_equal(oracle.swiglu(gg, np.ones_like(gg)), np.array([ref.lib.ref_silu(float(v)) for v in gg],
                                                                          np.float32))


def test_swiglu_closed_forms(oracle):
    """SiLU's fixed points: silu(0) = 0; silu(x) = x where e^-x is below half an ulp of 1; g / (1 + e^-g) is NaN at
    g = -inf (-inf / inf, as in the reference's expression); the float64 value within 3 ulp elsewhere."""
    one = np.ones(1, np.float32)
    assert oracle.swiglu(np.zeros(1, np.float32), one)[0] == 0.0
    big = np.array([30.0, 50.0, 1e6], np.float32)
    assert np.array_equal(oracle.swiglu(big, np.ones(3, np.float32)), big)
    assert np.isnan(oracle.swiglu(np.array([-np.inf], np.float32), one)[0])
    rng = np.random.default_rng(32)
    g = rng.uniform(-20, 20, 20000).astype(np.float32)
    u = rng.standard_normal(20000).astype(np.float32)
    exact = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    got = oracle.swiglu(g, u)
    assert np.all(np.abs(got - exact) <= 3 * np.spacing(np.abs(exact).astype(np.float32)) + 1e-37)


@needs_ref
@pytest.mark.parametrize("n", [1, 7, 2048, 3072, 4096])
@pytest.mark.parametrize("with_w", [True, False])
def test_rmsnorm_matches_reference(oracle, ref, n, with_w):
    """orc_rmsnorm == the reference's qwen_rmsnorm (src/qwen_ops.cpp:8-13) bit for bit: random rows, rows of
    zeros, rows at 1e+-30 magnitudes, denormal rows, with and without a weight (w = NULL)."""
    rng = np.random.default_rng(n)
    w = rng.standard_normal(n).astype(np.float32) if with_w else None
    rows = [rng.standard_normal(n).astype(np.float32), np.zeros(n, np.float32),
            (rng.standard_normal(n) * 1e30).astype(np.float32), (rng.standard_normal(n) * 1e-30).astype(np.float32),
            np.full(n, 1e-40, np.float32), (rng.standard_normal(n) * 100).astype(np.float32)]
    for eps in (1e-6, 1e-5, 0.0):
        for x in rows:
            a, b = oracle.rmsnorm(x, w, eps), ref.rmsnorm(x, w, eps)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (eps, x[:3])


def test_rmsnorm_closed_forms(oracle):
    """A constant row c maps to c / sqrt(c^2 + eps) (times w); a row of zeros with eps > 0 stays zero; scaling x
    by a power of two leaves the output unchanged where eps is negligible; float64 agreement within 2 ulp."""
    n = 2048
    for c in (1.0, -3.0, 0.25):
        y = oracle.rmsnorm(np.full(n, c, np.float32), None, 1e-6)
        assert np.allclose(y, c / np.sqrt(c * c + 1e-6), rtol=2e-7, atol=0)
    assert not np.any(oracle.rmsnorm(np.zeros(n, np.float32), None, 1e-6))
    rng = np.random.default_rng(33)
    x, w = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    a = oracle.rmsnorm(x, w, 0.0)
    assert np.array_equal(a, oracle.rmsnorm(x * np.float32(64), w, 0.0))
    x64 = x.astype(np.float64)
    exact = x64 / np.sqrt(np.mean(x64 * x64) + 1e-5) * w
    got = oracle.rmsnorm(x, w, 1e-5)
    assert np.all(np.abs(got - exact) <= 3 * np.spacing(np.abs(exact).astype(np.float32)))


# ------------------------------------------------------------------ combine and the layer

def test_combine_order_and_one_hot(oracle):
    rng = np.random.default_rng(8)
    t, nu, n = 3, 4, 64
    down = rng.standard_normal((t, nu, n)).astype(np.float32)
    wts = np.zeros((t, nu), np.float32)
    wts[:, 2] = 1.0
    out = oracle.combine(down, wts, None, None, nu, n, t)
    assert np.array_equal(out, down[:, 2, :])
    wts = rng.random((t, nu)).astype(np.float32)
    sh = rng.standard_normal((t, n)).astype(np.float32)
    sg = rng.random(t).astype(np.float32)
    out = oracle.combine(down, wts, sh, sg, nu, n, t)
    acc = wts[:, 0:1] * down[:, 0]
    for j in range(1, nu):
        acc = acc + wts[:, j:j + 1] * down[:, j]
    assert np.array_equal(out, acc + sh * sg[:, None])


@needs_ref
@pytest.mark.parametrize("qtype", TYPES)
def test_layer_against_reference_decoder(oracle, ref, qtype):
    """The oracle's layer equals a float64 route through the reference's own decoder and the round trips."""
    E, FE = (256, 256) if qtype == Q4_K else (256, 64)
    spec = synth.LayerSpec(qtype, E, 8, 2, FE, shared=True)
    L = synth.make_layer(spec, seed=11)
    rng = np.random.default_rng(12)
    x = rng.standard_normal((3, E)).astype(np.float32)
    out, ids, wts = oracle.moe_forward(spec, L, x)
    dec = {k: ref.to_float(qtype, L[k], L[k].size // synth.BLOCK[qtype][1] * synth.BLOCK[qtype][0])
           for k in ("w_gate", "w_up", "w_down", "s_gate", "s_up", "s_down")}
    g_all = dec["w_gate"].reshape(8, FE, E)
    u_all = dec["w_up"].reshape(8, FE, E)
    d_all = dec["w_down"].reshape(8, E, FE)

    def ffn(g, u, d, xr):
        gg = (g.astype(np.float64) @ xr).astype(np.float32)
        uu = (u.astype(np.float64) @ xr).astype(np.float32)
        a = oracle.swiglu(gg, uu)
        return (d.astype(np.float64) @ oracle.roundtrip(qtype, a)).astype(np.float32)

    for t in range(3):
        logits = (L["w_router"].astype(np.float64) @ x[t]).astype(np.float32)
        p = np.exp(logits.astype(np.float64) - logits.max())
        p /= p.sum()
        sel = np.argsort(-p, kind="stable")[:2]
        assert np.array_equal(ids[t], sel)
        xr = oracle.roundtrip(qtype, x[t])
        want = sum(np.float64(wts[t, j]) * ffn(g_all[e], u_all[e], d_all[e], xr) for j, e in enumerate(sel))
        sg = 1 / (1 + np.exp(-np.dot(x[t].astype(np.float64), L["w_shexp"])))
        want = want + sg * ffn(dec["s_gate"].reshape(FE, E), dec["s_up"].reshape(FE, E),
                               dec["s_down"].reshape(E, FE), xr)
        np.testing.assert_allclose(out[t], want, rtol=1e-5, atol=1e-6 * np.abs(want).max())
