"""ctypes binding of librocm_hip_moe.so, the MI355X MoE FFN path's C ABI (include/qmatvec.h, include/gpu_ops.h).

This is how Python callers (the tests, bench.py) reach the HIP kernels: every call goes through the exported C
symbols with plain pointers. Device memory comes from torch tensors (``tensor.data_ptr()``); torch is only the
allocator and stream provider here. There is no CPU fallback: a missing library or a non-gfx950 device raises.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("ROCM_HIP_MOE_LIB") or os.path.join(HERE, "librocm_hip_moe.so")  # (the variable: a build of the library elsewhere)

QT_F32, QT_Q8_0, QT_Q4_K, QT_ROCMFP4, QT_ROCMFP4_FAST = 0, 8, 12, 100, 101
TYPE_NAMES = {QT_Q8_0: "q8_0", QT_Q4_K: "q4_K", QT_ROCMFP4: "q4_0_rocmfp4", QT_ROCMFP4_FAST: "q4_0_rocmfp4_fast"}

# values per block, bytes per block (src/quant_types.cpp:591-615)
BLOCK = {QT_F32: (1, 4), QT_Q8_0: (32, 34), QT_Q4_K: (256, 144), QT_ROCMFP4: (32, 18), QT_ROCMFP4_FAST: (32, 17)}


def row_size(qtype, k):
    bv, bb = BLOCK[qtype]
    assert k % bv == 0, (qtype, k)
    return k // bv * bb


def reads_q8k(qtype):
    return qtype == QT_Q4_K


class Q8(ctypes.Structure):
    """struct qmatvec_q8 (include/qmatvec.h)."""
    _fields_ = [("q0", ctypes.c_void_p), ("d0", ctypes.c_void_p), ("qK", ctypes.c_void_p), ("dK", ctypes.c_void_p),
                ("bsK", ctypes.c_void_p), ("s0", ctypes.c_void_p), ("max_k", ctypes.c_int),
                ("xh", ctypes.c_void_p), ("xh_bf16", ctypes.c_int)]


_P, _I, _L, _Z, _F = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_size_t, ctypes.c_float
_Q8P = ctypes.POINTER(Q8)

# name -> (restype, argtypes); the exported C ABI
SIGNATURES = {
    "qmatvec_init": (_I, [ctypes.c_char_p]),
    "qmatvec_free": (None, []),
    "gpu_ops_init": (_I, [ctypes.c_char_p]),
    "gpu_ops_free": (None, []),
    "qmatvec_set_out_scale": (_I, [_P, _P, _Z, _P, _I]),
    "qmatvec_drop_out_scales": (None, [_P]),
    "qmatvec_supported": (_I, [_I]),
    "qmatvec_launch": (_I, [_I, _P, _Z, _P, _P, _I, _I, _P]),
    "qmatvec_launch_batch": (_I, [_I, _P, _Z, _P, _P, _I, _I, _I, _P]),
    "qmatvec_q8_bytes": (_Z, [_I]),
    "qmatvec_q8_bind": (None, [_Q8P, _P, _I]),
    "qmatvec_q8_supported": (_I, [_I, _I]),
    "qmatvec_quantize": (_I, [_P, _I, _Q8P, _P]),
    "qmatvec_launch_q8": (_I, [_I, _P, _Z, _Q8P, _P, _I, _I, _P]),
    "qmatvec_launch_q8_pair": (_I, [_I, _P, _I, _P, _P, _I, _P, _Z, _Q8P, _I, _P]),
    "qmatvec_launch_q8_batch": (_I, [_I, _P, _Z, _Q8P, _P, _L, _I, _I, _I, _P]),
    "qmatvec_launch_q8_id": (_I, [_I, _P, _Z, _P, _I, _I, _Q8P, _P, _I, _I, _I, _P]),
    "qmatvec_launch_q8_id_pair": (_I, [_I, _P, _P, _Z, _P, _I, _I, _Q8P, _P, _P, _I, _I, _I, _P]),
    "qmatvec_launch_q8_id_x": (_I, [_I, _P, _P, _P, _P, _Z, _P, _I, _I, _Q8P, _P, _P, _I, _I, _I, _P]),
    "qmatvec_id_batch_tile": (_I, [_I, _I, _I]),
    "qmatvec_q8_id_batch_supported": (_I, [_I, _I]),
    "qmatvec_launch_q8_id_batch": (_I, [_I, _P, _Z, _Q8P, _P, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P]),
    "qmatvec_pack_weights": (_I, [_I, _P, _Z, _L, _I, _P]),
    "qmatvec_unpack_weights": (_I, [_P]),
    "qmatvec_test_registry": (None, [_I, _L]),
    "qmatvec_pack_weights_ex": (_I, [_I, _P, _Z, _L, _I, _I, _P]),
    "qmatvec_registered_bytes": (_Z, [_I, _L, _I, _I]),
    "qmatvec_packed_bytes": (_Z, [_I, _L, _I]),
    "gpu_add_rmsnorm": (_I, [_P, _P, _P, _P, _P, _I, _I, _F, _Q8P, _P]),
    "gpu_swiglu": (_I, [_P, _P, _P, _I, _Q8P, _P]),
    "gpu_moe_router": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _I]),
    "gpu_moe_combine": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _P]),
    "gpu_moe_combine_scaled": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P]),
    "gpu_moe_group": (_I, [_P, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P]),
    "gpu_moe_group_ws_bytes": (_Z, [_I, _I]),
    "gpu_moe_group_ws": (_I, [_P, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _Z, _P]),
    "moe_layer_scratch_bytes": (_Z, [ctypes.c_void_p, _I]),
    "moe_layer_forward": (_I, [ctypes.c_void_p, _P, _P, _I, _P, _P, _P, _P, _Z, _P]),
    "moe_layer_forward_norm": (_I, [ctypes.c_void_p, _P, _P, _P, _P, _F, _P, _I, _P, _P, _P, _P, _Z, _P]),
    "moe_layer_forward_noalloc": (_I, [ctypes.c_void_p, _P, _P, _I, _P, _P, _P, _P]),
    "moe_layer_set_fused": (None, [_I]),
    "qmatvec_dense_mfma_mode": (None, [_I]),
    "moe_layer_fused_stamps": (None, [_P]),
    "moe_layer_fused_multi_q4k": (None, [_I]),
    # include/gguf_mmap.h (host only: the file mapping)
    "gguf_mmap_open": (_P, [ctypes.c_char_p]),
    "gguf_mmap_close": (None, [_P]),
    "gguf_mmap_get_tensor": (_P, [_P, ctypes.c_char_p, ctypes.POINTER(_Z)]),
    "gguf_get_tensor_ptr": (_P, [_P, ctypes.c_char_p, ctypes.POINTER(_Z)]),
    "gguf_n_tensors": (_L, [_P]),
    "gguf_tensor_name": (ctypes.c_char_p, [_P, _L]),
    "gguf_tensor_type": (_I, [_P, _L]),
    "gguf_tensor_ne": (ctypes.POINTER(ctypes.c_int64), [_P, _L]),
    "gguf_tensor_dims": (ctypes.c_uint8, [_P, _L]),
    "gguf_tensor_block_size": (_Z, [_P, _L]),
    "gguf_tensor_type_size": (_Z, [_P, _L]),
    "gguf_tensor_offset": (ctypes.c_uint64, [_P, _L]),
    "gguf_tensor_nbytes": (_Z, [_P, _L]),
    "gguf_n_kv": (_L, [_P]),
    "gguf_kv_key": (ctypes.c_char_p, [_P, _L]),
    "gguf_kv_type": (_I, [_P, _L]),
    "gguf_kv_get_u8": (ctypes.c_int32, [_P, _L, ctypes.POINTER(ctypes.c_uint8)]),
    "gguf_kv_get_i8": (ctypes.c_int32, [_P, _L, ctypes.POINTER(ctypes.c_int8)]),
    "gguf_kv_get_u16": (ctypes.c_int32, [_P, _L, ctypes.POINTER(ctypes.c_uint16)]),
    "gguf_kv_get_i16": (ctypes.c_int32, [_P, _L, ctypes.POINTER(ctypes.c_int16)]),
    "gguf_kv_get_u32": (ctypes.c_int32, [_P, _L, ctypes.POINTER(ctypes.c_uint32)]),
    "gguf_kv_get_i32": (ctypes.c_int32, [_P, _L, ctypes.POINTER(ctypes.c_int32)]),
    "gguf_kv_get_f32": (ctypes.c_int32, [_P, _L, ctypes.POINTER(ctypes.c_float)]),
    "gguf_kv_get_u64": (ctypes.c_int32, [_P, _L, ctypes.POINTER(ctypes.c_uint64)]),
    "gguf_kv_get_i64": (ctypes.c_int32, [_P, _L, ctypes.POINTER(ctypes.c_int64)]),
    "gguf_kv_get_f64": (ctypes.c_int32, [_P, _L, ctypes.POINTER(ctypes.c_double)]),
    "gguf_alignment": (_Z, [_P]),
    "gguf_data_offset": (_Z, [_P]),
    "gguf_version": (ctypes.c_uint32, [_P]),
    "gguf_arch": (ctypes.c_char_p, [_P]),
    "gguf_block_count": (_L, [_P]),
    "gguf_arch_int": (_L, [_P, ctypes.c_char_p, _L]),
    "gguf_arch_float": (_F, [_P, ctypes.c_char_p, _F]),
    "gguf_kv_str_val": (ctypes.c_char_p, [_P, _L]),
    "gguf_find_kv": (_L, [_P, ctypes.c_char_p]),
    "gguf_kv_get_array": (ctypes.c_int32, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int32),
                                           ctypes.POINTER(_P), ctypes.POINTER(_Z)]),
    "gguf_n_maps": (_I, [_P]),
    "gguf_map_at": (_P, [_P, _I, ctypes.POINTER(_Z)]),
    "gguf_last_error": (ctypes.c_char_p, []),
    # include/moe_gguf.h
    "moe_gguf_layer_bind": (_I, [_P, _I, _P]),
    "moe_gguf_layer_upload": (_I, [_P, _I, _I, _P, _P]),
    "moe_gguf_layer_release": (None, [_P]),
    "moe_gguf_error": (ctypes.c_char_p, []),
}


class LayerDesc(ctypes.Structure):
    """struct moe_layer_desc (include/moe_layer.h)."""
    _fields_ = [("type", _I), ("n_embd", _I), ("n_expert", _I), ("n_used", _I), ("n_ff", _I),
                ("w_router", _P), ("w_gate", _P), ("w_up", _P), ("w_down", _P),
                ("s_gate", _P), ("s_up", _P), ("s_down", _P), ("w_shexp", _P)]


class GgufLayer(ctypes.Structure):
    """struct moe_gguf_layer (include/moe_gguf.h)."""
    _fields_ = [("desc", LayerDesc), ("dev", _P), ("dev_bytes", _Z), ("packed", _I)]


class HipError(RuntimeError):
    pass


def load_library(path=LIB_PATH):
    """Load the shared library and declare every exported function's signature (no GPU call)."""
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built: run `make -C rocm-hip_amd` (or __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


ENGINE_PATH = os.path.join(HERE, "libmoe_ffn_engine.so")


class EngineWeight(ctypes.Structure):
    """struct moe_engine_weight (include/moe_ffn_engine.h)."""
    _fields_ = [("type", _I), ("data", _P), ("row_bytes", _Z), ("N", _I), ("K", _I)]


class EngineLayer(ctypes.Structure):
    """struct moe_engine_layer (include/moe_ffn_engine.h)."""
    _fields_ = [("n_embd", _I), ("n_expert", _I), ("n_used", _I), ("n_ff_exp", _I), ("n_ff_shexp", _I),
                ("router", EngineWeight), ("exp_gate", EngineWeight), ("exp_up", EngineWeight),
                ("exp_down", EngineWeight), ("sh_gate", EngineWeight), ("sh_up", EngineWeight),
                ("sh_down", EngineWeight), ("shexp_gate", _P)]


ENGINE_SIGNATURES = {
    "moe_engine_create": (_P, [_P, _I]),
    "moe_engine_destroy": (None, [_P]),
    "moe_engine_ffn": (_I, [_P, _P, _P, _P, _P, _P, _F, _I, _P, _P, _P, _P, _P]),
}


def load_engine(path=ENGINE_PATH):
    """The engine-side caller library (built with the library by `make -C rocm-hip_amd`); no GPU call."""
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built: run `make -C rocm-hip_amd` (or __graft_entry__.build())")
    load_library()  # its dependency, with signatures declared
    lib = ctypes.CDLL(path)
    for name, (res, args) in ENGINE_SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def gpu_moe_max_tiles(T, n_used, n_expert, tile):
    """include/gpu_ops.h's inline gpu_moe_max_tiles."""
    n = T * n_used
    return min(n, n_expert + n // tile)


class MoeLib:
    """The library, initialised on the current GPU. Methods raise HipError on a non-zero hipError_t."""

    def __init__(self, path=LIB_PATH):
        self.lib = load_library(path)
        if self.lib.qmatvec_init(None) != 0 or self.lib.gpu_ops_init(None) != 0:
            raise HipError("qmatvec_init: the current device is not a gfx950 (MI355X)")

    def __getattr__(self, name):
        fn = getattr(self.lib, name)

        def call(*args):
            r = fn(*args)
            if fn.restype is _I and name not in ("qmatvec_supported", "qmatvec_q8_supported", "qmatvec_id_batch_tile",
                                                 "qmatvec_q8_id_batch_supported", "qmatvec_set_out_scale") \
                    and not name.startswith("gguf_") and r != 0:
                why = f": {self.lib.moe_gguf_error().decode()}" if name.startswith("moe_gguf_") else ""
                raise HipError(f"{name} returned {r}{why}")
            return r
        return call


def ptr(t):
    """Device pointer of a torch tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


class Q8Buffer:
    """A qmatvec_q8 bound to a torch uint8 device tensor of qmatvec_q8_bytes(max_k)."""

    def __init__(self, moe, max_k, device="cuda"):
        import torch
        assert max_k % 256 == 0
        self.mem = torch.zeros(moe.lib.qmatvec_q8_bytes(max_k), dtype=torch.uint8, device=device)
        self.q = Q8()
        moe.lib.qmatvec_q8_bind(ctypes.byref(self.q), ctypes.c_void_p(self.mem.data_ptr()), max_k)
        self.max_k = max_k

    def ref(self):
        return ctypes.byref(self.q)

    def views(self, k):
        """Host copies of the first k values: (q0, d0, s0, qK, dK, bsK) as numpy arrays."""
        import numpy as np
        m = self.mem.cpu().numpy()
        base = self.mem.data_ptr()

        def arr(p, n, dt):
            off = p - base
            return m[off:off + n * np.dtype(dt).itemsize].view(dt).copy()
        return (arr(self.q.q0, k, np.int8), arr(self.q.d0, k // 32, np.float32), arr(self.q.s0, k // 32, np.int32),
                arr(self.q.qK, k, np.int8), arr(self.q.dK, k // 256, np.float32), arr(self.q.bsK, k // 16, np.int32))


def stream_handle(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)
