"""ctypes binding of the CPU oracle (oracle/liboracle.so) and of the reference's own CPU code built from its
sources (oracle/_ref/libref_cpu.so). Test infrastructure: the checker, never the product path."""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE = os.path.join(ROOT, "oracle", "liboracle.so")
REF = os.path.join(ROOT, "oracle", "_ref", "libref_cpu.so")

_P, _I, _L, _Z, _F, _D = (ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_float,
                          ctypes.c_double)


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


class Layer(ctypes.Structure):
    _fields_ = [("type", _I), ("n_embd", _I), ("n_expert", _I), ("n_used", _I), ("n_ff", _I),
                ("w_router", _P), ("w_gate", _P), ("w_up", _P), ("w_down", _P),
                ("s_gate", _P), ("s_up", _P), ("s_down", _P), ("w_shexp", _P)]


class Oracle:
    def __init__(self, path=ORACLE):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = self.lib = ctypes.CDLL(path)
        sig = {
            "orc_fp16_to_f32": (_F, [ctypes.c_uint16]), "orc_f32_to_fp16": (ctypes.c_uint16, [_F]),
            "orc_ue4m3_half": (_F, [ctypes.c_uint8]), "orc_row_size": (_Z, [_I, _L]),
            "orc_dequant": (_I, [_I, _P, _P, _L]), "orc_quantize_q8_0": (None, [_P, _L, _P, _P, _P]),
            "orc_quantize_q8_K": (None, [_P, _L, _P, _P, _P]), "orc_q8_roundtrip": (None, [_I, _P, _P, _L]),
            "orc_block_dots": (_I, [_I, _P, _P, _I, _P]), "orc_row_dot_int": (_D, [_I, _P, _P, _P, _P, _I]),
            "orc_row_dot_deq": (_D, [_I, _P, _P, _I]), "orc_matvec": (None, [_I, _P, _Z, _P, _P, _I, _I]),
            "orc_matvec_f32": (None, [_P, _P, _P, _I, _I]),
            "orc_router": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I]),
            "orc_group": (_I, [_P, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _I]),
            "orc_max_tiles": (_I, [_I, _I, _I, _I]), "orc_swiglu": (None, [_P, _P, _P, _L]),
            "orc_combine": (None, [_P, _P, _P, _P, _P, _I, _I, _I]), "orc_rmsnorm": (None, [_P, _P, _P, _I, _F]),
            "orc_moe_forward": (_I, [ctypes.POINTER(Layer), _P, _P, _I, _P, _P, _P]),
            "orc_set_threads": (_I, [_I]),
        }
        for k, (r, a) in sig.items():
            f = getattr(L, k)
            f.restype, f.argtypes = r, a

    # ---- numpy-level wrappers
    def dequant(self, qtype, raw, n):
        out = np.empty(n, np.float32)
        assert self.lib.orc_dequant(qtype, _p(np.ascontiguousarray(raw)), _p(out), n) == 0
        return out

    def quantize_q8_0(self, x):
        x = np.ascontiguousarray(x, np.float32)
        n = x.size
        q, d, s = np.empty(n, np.int8), np.empty(n // 32, np.float32), np.empty(n // 32, np.int32)
        self.lib.orc_quantize_q8_0(_p(x), n, _p(q), _p(d), _p(s))
        return q, d, s

    def quantize_q8_K(self, x):
        x = np.ascontiguousarray(x, np.float32)
        n = x.size
        q, d, bs = np.empty(n, np.int8), np.empty(n // 256, np.float32), np.empty(n // 16, np.int32)
        self.lib.orc_quantize_q8_K(_p(x), n, _p(q), _p(d), _p(bs))
        return q, d, bs

    def roundtrip(self, qtype, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        self.lib.orc_q8_roundtrip(qtype, _p(x), _p(out), x.size)
        return out

    def block_dots(self, qtype, wrow, xq, k):
        out = np.empty(k // 16 + 8, np.int32)
        n = self.lib.orc_block_dots(qtype, _p(np.ascontiguousarray(wrow)), _p(np.ascontiguousarray(xq)), k, _p(out))
        return out[:n]

    def row_dot_int(self, qtype, wrow, xq, xd, xbs, k):
        return self.lib.orc_row_dot_int(qtype, _p(np.ascontiguousarray(wrow)), _p(xq), _p(xd), _p(xbs), k)

    def row_dot_deq(self, qtype, wrow, x_rt, k):
        return self.lib.orc_row_dot_deq(qtype, _p(np.ascontiguousarray(wrow)), _p(np.ascontiguousarray(x_rt, np.float32)), k)

    def matvec(self, qtype, W, x, n, k):
        W = np.ascontiguousarray(W)
        y = np.empty(n, np.float32)
        self.lib.orc_matvec(qtype, _p(W), W.shape[-1] if W.ndim == 2 else W.size // n, _p(np.ascontiguousarray(x, np.float32)), _p(y), n, k)
        return y

    def matvec_f32(self, W, x):
        W = np.ascontiguousarray(W, np.float32)
        y = np.empty(W.shape[0], np.float32)
        self.lib.orc_matvec_f32(_p(W), _p(np.ascontiguousarray(x, np.float32)), _p(y), W.shape[0], W.shape[1])
        return y

    def router(self, logits, ne, nu, x=None, w_shexp=None, ids_stride=0):
        logits = np.ascontiguousarray(logits, np.float32)
        t = logits.size // ne
        stride = ids_stride or nu
        ids = np.empty(t * stride, np.int32)
        wts = np.empty(t * nu, np.float32)
        sg = np.empty(t, np.float32)
        n = 0 if x is None else x.size // t
        assert self.lib.orc_router(_p(logits), _p(None if x is None else np.ascontiguousarray(x, np.float32)),
                                   _p(w_shexp), _p(ids), _p(wts), _p(sg), ne, nu, n, t, stride) == 0
        return ids.reshape(t, stride), wts.reshape(t, nu), sg

    def group(self, ids, t, nu, ne, tile):
        ids = np.ascontiguousarray(ids, np.int32)
        mt = self.lib.orc_max_tiles(t, nu, ne, tile)
        counts, offsets = np.empty(ne, np.int32), np.empty(ne, np.int32)
        tok, pair = np.full(t * nu, -1, np.int32), np.full(t * nu, -1, np.int32)
        nt = np.zeros(1, np.int32)
        te, ts, tn = np.empty(mt, np.int32), np.empty(mt, np.int32), np.empty(mt, np.int32)
        assert self.lib.orc_group(_p(ids), t, nu, ne, tile, _p(counts), _p(offsets), _p(tok), _p(pair), _p(nt),
                                  _p(te), _p(ts), _p(tn), mt) == 0
        n = int(nt[0])
        return dict(counts=counts, offsets=offsets, tok_rows=tok, pair_rows=pair, n_tiles=n, tile_e=te[:n],
                    tile_start=ts[:n], tile_n=tn[:n])

    def swiglu(self, g, u):
        g, u = np.ascontiguousarray(g, np.float32), np.ascontiguousarray(u, np.float32)
        out = np.empty_like(g)
        self.lib.orc_swiglu(_p(g), _p(u), _p(out), g.size)
        return out

    def rmsnorm(self, x, w, eps):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        self.lib.orc_rmsnorm(_p(x), _p(None if w is None else np.ascontiguousarray(w, np.float32)), _p(y), x.size, eps)
        return y

    def combine(self, down, wts, shared, sg, nu, n, t):
        out = np.empty(t * n, np.float32)
        self.lib.orc_combine(_p(np.ascontiguousarray(down, np.float32)), _p(np.ascontiguousarray(wts, np.float32)),
                             _p(shared), _p(sg), _p(out), nu, n, t)
        return out.reshape(t, n)

    def moe_forward(self, spec, layer, x, logits=None):
        keep = {k: np.ascontiguousarray(v) for k, v in layer.items()}
        L = Layer(spec.qtype, spec.E, spec.NE, spec.NU, spec.FE, _p(keep["w_router"]), _p(keep["w_gate"]),
                  _p(keep["w_up"]), _p(keep["w_down"]), _p(keep.get("s_gate")), _p(keep.get("s_up")),
                  _p(keep.get("s_down")), _p(keep.get("w_shexp")))
        x = np.ascontiguousarray(x, np.float32)
        t = x.size // spec.E
        out = np.empty((t, spec.E), np.float32)
        ids = np.empty((t, spec.NU), np.int32)
        wts = np.empty((t, spec.NU), np.float32)
        lg = None if logits is None else np.ascontiguousarray(logits, np.float32)
        assert self.lib.orc_moe_forward(ctypes.byref(L), _p(x), _p(lg), t, _p(out), _p(ids), _p(wts)) == 0
        return out, ids, wts


class RefCPU:
    """The reference's own src/quant_types.cpp + src/qwen_ops.cpp, compiled from its sources (oracle/Makefile)."""

    def __init__(self, path=REF):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        L = self.lib = ctypes.CDLL(path)
        L.qt_to_float.restype, L.qt_to_float.argtypes = _I, [_I, _P, _P, _L]
        L.qt_row_size.restype, L.qt_row_size.argtypes = _Z, [_I, _L]
        L.ref_rmsnorm.restype, L.ref_rmsnorm.argtypes = None, [_P, _P, _P, _I, _F]
        L.ref_silu.restype, L.ref_silu.argtypes = _F, [_F]
        L.ref_swiglu.restype, L.ref_swiglu.argtypes = None, [_P, _P, _P, _L]

    def swiglu(self, g, u):
        g, u = np.ascontiguousarray(g, np.float32), np.ascontiguousarray(u, np.float32)
        out = np.empty_like(g)
        self.lib.ref_swiglu(_p(g), _p(u), _p(out), g.size)
        return out

    def rmsnorm(self, x, w, eps):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        self.lib.ref_rmsnorm(_p(x), _p(None if w is None else np.ascontiguousarray(w, np.float32)), _p(y), x.size, eps)
        return y

    def to_float(self, qtype, raw, n):
        out = np.empty(n, np.float32)
        assert self.lib.qt_to_float(qtype, _p(np.ascontiguousarray(raw)), _p(out), n) == 0
        return out
