"""A CPU model of the decode kernels' fp32 arithmetic: the same terms, in the same order, rounded the same way.

TEST INFRASTRUCTURE ONLY (it uses the oracle's integer block dots and quantizers as building blocks). It exists to
explain, term by term, where a GPU decode layer departs from the oracle's double route, and to bound that
departure with the reference's own criterion.

What the HIP kernels compute for one output row (rows_dot in rocm-hip_amd/csrc/expert_units.h, which the fused
decode kernels share):
  * per unit (32 values; Q4_K 64) an exact integer dot, then one fp32 term in the kernel's expression:
      Q8_0   (d_w * d_x) * s
      FP4    fma(e0 * d_x, s0, (e1 * d_x) * s1)           (the compiler's contraction, read in the gfx950 code)
      FAST   (e * d_x) * (float)(s0 + s1)
      Q4_K   fma(d_x * d, isum, (d_x * dmin) * -msum)
  * lane l of a group of L lanes sums its units l, l + L, l + 2L, ... in that order from 0.0f;
  * the group's L partial sums meet in a pairwise tree over adjacent lanes (DPP xor-1, xor-2, half-row and row
    mirrors, swizzle xor-16, xor-32: fp32 addition is commutative, so every lane holds the same bits).
  L and the units per lane come from the kernel shape rule (mv_shape in expert_matvec.hip).
The layer: gate / up row dots on x's quantized bundle, SwiGLU, the quantizer, down row dots, then the combine
acc = w0 d0; acc = fma(w_j, d_j, acc); acc = acc + (shared sg) (k_combine in vector_ops.hip: the shared term is
an operand of a conditional expression, so the compiler does not contract it).

The one part not modelled bit for bit is SwiGLU's exponential: the kernels use __expf, the model the host's expf
(the oracle's SwiGLU, the reference's qwen_silu); they can differ in the last bit.

The reference's acceptance rule for a row (tests/matvec_verify.cpp:8, 137-142 of the reference tree):
|gpu - ref| <= 1e-5 * sum_k |w_k x_k|, ref the decoded row times the round-tripped x in double. For a layer output
the same rule is applied through the combine: bound_n = 1e-5 * (sum_s |wt_s| sum_k |Wdown_s[n, k] a_s[k]|
+ |sg| sum_k |Sdown[n, k] a_sh[k]|), a_s the round-tripped down input.
"""
import numpy as np

import synth

Q8_0, Q4_K, FP4, FAST = 8, 12, 100, 101
_UE = synth.ue4m3_half_table()
f32 = np.float32


def fma32(a, b, c):
    """fp32 fused multiply-add: the product is exact in 80-bit extended precision (24 + 24 bits), one rounding of
    the sum there and one to fp32 (a double rounding that can differ from a single one only at a 2^-40 chance)."""
    ld = np.longdouble
    return (np.asarray(a, f32).astype(ld) * np.asarray(b, f32).astype(ld) + np.asarray(c, f32).astype(ld)).astype(f32)


def mv_shape(qtype, K):
    """Lanes per row L and units per lane (0: a loop) -- the kernels' shape rule (expert_matvec.hip mv_shape)."""
    nu = K // 64 if qtype == Q4_K else K // 32
    for L in (64, 32, 16, 8):
        if nu % L == 0 and nu // L <= 4:
            return L, nu // L
    L = 64
    while L > 8 and L > nu:
        L //= 2
    return L, 0


def _f16(W, off):
    return W[:, off:off + 2].copy().view(np.float16).astype(f32).reshape(-1)


def _q4k_scale_min(h, j):
    """Sub-block j's 6-bit scale and min from the 12 packed bytes h [rows, 12] (ggml's get_scale_min_k4)."""
    h = h.astype(np.int64)
    if j < 4:
        return h[:, j] & 63, h[:, j + 4] & 63
    return (h[:, j + 4] & 15) | ((h[:, j - 4] >> 6) << 4), (h[:, j + 4] >> 4) | ((h[:, j] >> 6) << 4)


def quantize(oracle, qtype, x):
    """x's activation bundle for the type: (q, d, bs) -- Q8_0 (d per 32) or Q8_K (d per 256, bs per 16)."""
    if qtype == Q4_K:
        return oracle.quantize_q8_K(x)
    return oracle.quantize_q8_0(x)


def unit_terms(oracle, qtype, W, act, K):
    """fp32 unit terms [rows, units] of rows W (uint8 [rows, row bytes]) against the bundle act = (q, d, bs)."""
    q, d, bs = act
    W = np.ascontiguousarray(W)
    dots = np.stack([oracle.block_dots(qtype, W[r], q, K) for r in range(W.shape[0])]).astype(np.int64)
    rows = W.shape[0]
    if qtype == Q8_0:
        nb = K // 32
        dw = np.stack([_f16(W, 34 * b) for b in range(nb)], 1)
        return ((dw * d[None, :nb].astype(f32)).astype(f32) * dots.astype(f32)).astype(f32)
    if qtype == FP4:
        nb = K // 32
        e0 = _UE[W[:, 18 * np.arange(nb) + 16]]
        e1 = _UE[W[:, 18 * np.arange(nb) + 17]]
        dx = d[None, :nb].astype(f32)
        s0, s1 = dots[:, 0::2].astype(f32), dots[:, 1::2].astype(f32)
        return fma32((e0 * dx).astype(f32), s0, ((e1 * dx).astype(f32) * s1).astype(f32))
    if qtype == FAST:
        nb = K // 32
        e = _UE[W[:, 17 * np.arange(nb) + 16]]
        return ((e * d[None, :nb].astype(f32)).astype(f32) * dots.astype(f32)).astype(f32)
    # Q4_K: unit u = chunk c = u % 4 of super-block u // 4: sub-blocks 2c (low nibbles) and 2c + 1 (high)
    nsb = K // 256
    out = np.empty((rows, 4 * nsb), f32)
    for sb in range(nsb):
        base = 144 * sb
        dd, dm = _f16(W, base), _f16(W, base + 2)
        h = W[:, base + 4:base + 16]
        dx = f32(d[sb])
        for c in range(4):
            u = 4 * sb + c
            sc0, m0 = _q4k_scale_min(h, 2 * c)
            sc1, m1 = _q4k_scale_min(h, 2 * c + 1)
            isum = sc0 * dots[:, 2 * u] + sc1 * dots[:, 2 * u + 1]
            msum = m0 * (int(bs[4 * u]) + int(bs[4 * u + 1])) + m1 * (int(bs[4 * u + 2]) + int(bs[4 * u + 3]))
            neg = ((dx * dm).astype(f32) * (-msum).astype(f32)).astype(f32)
            out[:, u] = fma32((dx * dd).astype(f32), isum.astype(f32), neg)
    return out


def row_dots(oracle, qtype, W, act, K):
    """The kernels' fp32 result of every row of W against act: lane sums, then the pairwise lane tree."""
    return reduce_lanes(unit_terms(oracle, qtype, W, act, K), mv_shape(qtype, K)[0])


def reduce_lanes(t, L):
    """fp32 unit terms [rows, units] -> the group sum of L lanes: lane l adds its units l, l + L, ... in order from
    0.0f, then the pairwise tree over adjacent lanes."""
    nu = t.shape[1]
    lanes = np.zeros((t.shape[0], L), f32)
    for u in range(nu):  # lane u % L takes its units in ascending order
        lanes[:, u % L] = (lanes[:, u % L] + t[:, u]).astype(f32)
    while lanes.shape[1] > 1:
        lanes = (lanes[:, 0::2] + lanes[:, 1::2]).astype(f32)
    return lanes[:, 0]


def dequant_rows(oracle, qtype, W, K):
    W = np.ascontiguousarray(W)
    return oracle.dequant(qtype, W, W.shape[0] * K).reshape(W.shape[0], K).astype(np.float64)


def roundtrip(qtype, act, K):
    """The bundle's values as the reference's CPU harness sees them: code * (its block's FP16-rounded scale)."""
    q, d, _ = act
    per = 256 if qtype == Q4_K else 32
    return q[:K].astype(np.float64) * np.repeat(d[:K // per].astype(np.float64), per)


def expert_slots(spec, L, ids_row):
    """(gate, up, down) rows of each slot of a token: the chosen experts, then the shared expert."""
    FE, E = spec.FE, spec.E
    out = [(L["w_gate"][e * FE:(e + 1) * FE], L["w_up"][e * FE:(e + 1) * FE], L["w_down"][e * E:(e + 1) * E])
           for e in ids_row]
    if spec.shared:
        out.append((L["s_gate"], L["s_up"], L["s_down"]))
    return out


def combine32(down, wts, shared=None, sg=None):
    """k_combine's fp32 order over the slot rows down [NU, E]."""
    acc = (f32(wts[0]) * down[0]).astype(f32)
    for j in range(1, len(wts)):
        acc = fma32(np.full_like(acc, wts[j]), down[j], acc)
    if shared is not None:
        acc = (acc + (shared if sg is None else (shared * f32(sg)).astype(f32))).astype(f32)
    return acc


def token_model(oracle, spec, L, x, ids_row, wts_row, sg=None):
    """One decode token through the model of the kernels. Returns a dict: per slot g, u (fp32), the down input
    a (SwiGLU, host expf), its bundle, the down rows (fp32), and out (the combine)."""
    E, FE, qt = spec.E, spec.FE, spec.qtype
    ax = quantize(oracle, qt, x)
    slots = []
    for wg, wu, wd in expert_slots(spec, L, ids_row):
        g = row_dots(oracle, qt, wg, ax, E)
        u = row_dots(oracle, qt, wu, ax, E)
        a = oracle.swiglu(g, u)
        aq = quantize(oracle, qt, a)
        slots.append(dict(g=g, u=u, a=a, aq=aq, down=row_dots(oracle, qt, wd, aq, FE)))
    nu = spec.NU
    down = np.stack([s["down"] for s in slots[:nu]])
    shared = slots[nu]["down"] if spec.shared else None
    out = combine32(down, wts_row, shared, None if (sg is None or not spec.shared) else f32(sg))
    return dict(slots=slots, out=out, x_act=ax)


def double_route(oracle, spec, L, ids_row, wts_row, bundles, sg=None):
    """The layer output in double from given down-input bundles (one per slot), and the reference's per-element
    bound 1e-5 * sum |w a| carried through the combine. Returns (out, bound)."""
    E, FE, qt = spec.E, spec.FE, spec.qtype
    out = np.zeros(E)
    mag = np.zeros(E)
    for j, ((_, _, wd), b) in enumerate(zip(expert_slots(spec, L, ids_row), bundles)):
        Wd = dequant_rows(oracle, qt, wd, FE)
        a = roundtrip(qt, b, FE)
        w = float(wts_row[j]) if j < spec.NU else (1.0 if sg is None else float(sg))
        out += w * (Wd @ a)
        mag += abs(w) * (np.abs(Wd) @ np.abs(a))
    return out, 1e-5 * mag


def gate_up_double(oracle, spec, L, x, ids_row):
    """Per slot the gate and up rows in double on x's round trip, and the reference's row bounds 1e-5 sum |w x|."""
    E, qt = spec.E, spec.qtype
    xr = roundtrip(qt, quantize(oracle, qt, x), E)
    res = []
    for wg, wu, _ in expert_slots(spec, L, ids_row):
        Wg, Wu = dequant_rows(oracle, qt, wg, E), dequant_rows(oracle, qt, wu, E)
        res.append((Wg @ xr, 1e-5 * (np.abs(Wg) @ np.abs(xr)), Wu @ xr, 1e-5 * (np.abs(Wu) @ np.abs(xr))))
    return res
