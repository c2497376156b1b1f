"""The C-ABI library loads and exports every function include/*.h declares (no GPU call is made here)."""
import ctypes
import glob
import os
import re
import subprocess

import pytest

import moe_hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = open(h).read()
        src = re.sub(r"//[^\n]*", "", src)
        src = re.sub(r"static inline[^{]*\{.*?\n\}", "", src, flags=re.S)  # header-only helpers
        for m in re.finditer(r"^(?:const\s+)?(?:hipError_t|int|void|size_t|int32_t|int64_t|uint8_t|uint32_t|uint64_t|float|char|"
                             r"gguf_model_t)\s*\**\s*(\w+)\s*\(", src, flags=re.M):
            names.add(m.group(1))
    return names


def test_headers_declare_the_boundary():
    names = declared_functions()
    for must in ("qmatvec_launch_q8_id", "qmatvec_launch_q8_id_x", "qmatvec_launch_q8_id_batch", "gpu_moe_router",
                 "gpu_moe_group", "gpu_moe_combine", "gpu_swiglu", "qmatvec_quantize", "moe_layer_forward"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(moe_hip.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_every_declared_symbol():
    assert declared_functions() <= set(moe_hip.SIGNATURES), declared_functions() - set(moe_hip.SIGNATURES)
    moe_hip.load_library()  # declares every signature without touching the GPU


def test_exports_are_c_linkage():
    out = subprocess.run(["nm", "-D", "--defined-only", moe_hip.LIB_PATH], capture_output=True, text=True).stdout
    syms = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert declared_functions() <= syms


def test_host_side_queries_need_no_gpu():
    lib = moe_hip.load_library()
    assert lib.qmatvec_q8_supported(8, 2048) == 1 and lib.qmatvec_q8_supported(12, 3072) == 1
    assert lib.qmatvec_q8_supported(12, 640) == 0 and lib.qmatvec_q8_supported(2, 2048) == 0
    assert lib.qmatvec_supported(0) == 1 and lib.qmatvec_supported(8) == 0
    assert lib.qmatvec_q8_bytes(2048) >= 2048 * 2 + 2048 // 32 * 8
    assert lib.qmatvec_packed_bytes(100, 10, 2048) == 10 * 1152


def test_launch_before_init_fails_loudly():
    lib = moe_hip.load_library()
    # without a device (or before init) the library refuses to launch rather than fall back
    assert lib.qmatvec_quantize(None, 256, None, None) != 0


def test_no_unresolved_library_symbols():
    """Every symbol the library needs is defined in it or versioned by a system library (a missing internal
    definition would only fail at load time on the GPU box)."""
    out = subprocess.run(["nm", "-D", "--undefined-only", moe_hip.LIB_PATH], capture_output=True, text=True).stdout
    missing = [line.split()[-1] for line in out.splitlines() if " U " in line and "@" not in line]
    assert not missing, missing
