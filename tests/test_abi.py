"""The C-ABI library loads and exports every function include/*.h declares (no GPU call is made here)."""
import ctypes
import glob
import os
import re
import subprocess

import pytest

import moe_hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


ENGINE_HEADER = "moe_ffn_engine.h"  # declares the engine-side caller's library (libmoe_ffn_engine.so)


def declared_functions(engine=False):
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        if (os.path.basename(h) == ENGINE_HEADER) != engine:
            continue
        src = open(h).read()
        src = re.sub(r"//[^\n]*", "", src)
        src = re.sub(r"static inline[^{]*\{.*?\n\}", "", src, flags=re.S)  # header-only helpers
        for m in re.finditer(r"^(?:const\s+)?(?:hipError_t|int|void|size_t|int32_t|int64_t|uint8_t|uint32_t|uint64_t|float|char|"
                             r"gguf_model_t|moe_engine)\s*\**\s*(\w+)\s*\(", src, flags=re.M):
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


def test_engine_library_exports_its_header():
    """libmoe_ffn_engine.so exports (C linkage) every function include/moe_ffn_engine.h declares, and the binding
    declares them; it needs only the library's symbols and the HIP runtime's."""
    names = declared_functions(engine=True)
    assert names == set(moe_hip.ENGINE_SIGNATURES), names ^ set(moe_hip.ENGINE_SIGNATURES)
    out = subprocess.run(["nm", "-D", "--defined-only", moe_hip.ENGINE_PATH], capture_output=True, text=True).stdout
    assert names <= {line.split()[-1] for line in out.splitlines() if " T " in line}
    moe_hip.load_engine()
    und = subprocess.run(["nm", "-D", "--undefined-only", moe_hip.ENGINE_PATH], capture_output=True, text=True).stdout
    lib = ctypes.CDLL(moe_hip.LIB_PATH)
    missing = [ln.split()[-1] for ln in und.splitlines()
               if " U " in ln and "@" not in ln and not hasattr(lib, ln.split()[-1])]
    assert not missing, missing


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


# ------------------------------------------------------------------ the boundary against the reference's headers

REF_SRC = "/root/reference/src"
# The section-8(b) boundary: every function a caller of the reference's MoE path binds
BOUNDARY = ["qmatvec_init", "qmatvec_free", "qmatvec_set_out_scale", "qmatvec_drop_out_scales", "qmatvec_supported",
            "qmatvec_launch", "qmatvec_launch_batch", "qmatvec_q8_bytes", "qmatvec_q8_bind", "qmatvec_q8_supported",
            "qmatvec_quantize", "qmatvec_launch_q8", "qmatvec_launch_q8_pair", "qmatvec_launch_q8_batch",
            "qmatvec_launch_q8_id", "qmatvec_launch_q8_id_pair", "qmatvec_launch_q8_id_x", "qmatvec_id_batch_tile",
            "qmatvec_q8_id_batch_supported", "qmatvec_launch_q8_id_batch", "gpu_ops_init", "gpu_ops_free",
            "gpu_add_rmsnorm", "gpu_swiglu", "gpu_moe_router", "gpu_moe_combine", "gpu_moe_combine_scaled",
            "gpu_moe_max_tiles", "gpu_moe_group"]
needs_ref_headers = pytest.mark.skipif(not os.path.exists(os.path.join(REF_SRC, "qmatvec.h")),
                                       reason="the reference tree (its src/qmatvec.h, src/gpu_ops.h) is not present")
CLANG = "/opt/rocm/llvm/bin/clang++"
CXXFLAGS = ["-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include"]


def _signatures(incdir, tmp_path):
    """name -> the function type clang gives each boundary declaration in that include directory's headers."""
    import json
    src = tmp_path / f"decl_{os.path.basename(incdir)}.cpp"
    src.write_text('#include "qmatvec.h"\n#include "gpu_ops.h"\n')
    out = subprocess.run([CLANG, *CXXFLAGS, "-I", incdir, "-fsyntax-only", "-Xclang", "-ast-dump=json", str(src)],
                         capture_output=True, text=True, check=True).stdout
    sigs = {}

    def walk(n):
        if isinstance(n, dict):
            if n.get("kind") == "FunctionDecl" and n.get("name") in BOUNDARY:
                sigs[n["name"]] = n["type"]["qualType"]
            for v in n.get("inner", []):
                walk(v)
    walk(json.loads(out))
    return sigs


@needs_ref_headers
def test_boundary_signatures_match_the_reference_headers(tmp_path):
    """Every boundary function has the same C type in include/ as in the reference's src/qmatvec.h / gpu_ops.h."""
    ref = _signatures(REF_SRC, tmp_path)
    ours = _signatures(os.path.join(ROOT, "include"), tmp_path)
    assert set(ref) == set(BOUNDARY), set(BOUNDARY) - set(ref)
    diff = {n: (ref[n], ours.get(n)) for n in BOUNDARY if ref[n] != ours.get(n)}
    assert not diff, diff


@needs_ref_headers
def test_caller_built_on_the_reference_headers_links_and_runs(tmp_path):
    """A caller compiled against the reference's headers links against librocm_hip_moe.so and calls every boundary
    function (no GPU: init fails and every launcher refuses); the same caller compiled against include/ prints the
    same lines (the qmatvec_q8 layout, the host-side answers, the return codes)."""
    outs = []
    for inc in (REF_SRC, os.path.join(ROOT, "include")):
        exe = tmp_path / f"caller_{len(outs)}"
        subprocess.run([CLANG, *CXXFLAGS, "-I", inc, os.path.join(ROOT, "tests", "abi_ref", "boundary_caller.cpp"),
                        "-o", str(exe), "-L", os.path.dirname(moe_hip.LIB_PATH), "-lrocm_hip_moe",
                        "-Wl,-rpath," + os.path.dirname(moe_hip.LIB_PATH), "-L/opt/rocm/lib", "-lamdhip64"],
                       check=True, capture_output=True, text=True)
        r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stderr
        outs.append(r.stdout)
    assert outs[0] == outs[1]
    assert all(line.endswith("= 1") for line in outs[0].splitlines() if "!= " in line or ">= " in line), outs[0]


def test_registered_bytes_per_mode():
    """Device bytes a registration allocates besides W: the copy (native size) unless in place, the tiles (Q8_0: the
    native size; FP4: 0.75 K + K / 8 bytes per row; Q4_K: 0.75 K + 32 bytes per super-block) unless left out."""
    lib = moe_hip.load_library()
    rows, K = 128 * 768, 2048
    for t, rb, tile_row in ((8, 2176, 2048 + 128), (100, 1152, 1536 + 256), (12, 1152, 1536 + 8 * 32)):
        native = rows * rb
        assert lib.qmatvec_registered_bytes(t, rows, K, 0) == native + rows * tile_row
        assert lib.qmatvec_registered_bytes(t, rows, K, 1) == rows * tile_row
        assert lib.qmatvec_registered_bytes(t, rows, K, 2) == native
        assert lib.qmatvec_registered_bytes(t, rows, K, 3) == 0
    assert lib.qmatvec_registered_bytes(8, rows, K, 4) == 0 and lib.qmatvec_registered_bytes(2, rows, K, 0) == 0


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus above 1 exits at once with a message that says so (no GPU needed)."""
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)
