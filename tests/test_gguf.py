"""The GGUF mapping (include/gguf_mmap.h) and the MoE layer binding (include/moe_gguf.h), host side only.

The parser is pinned by a file assembled byte by byte from the GGUF v3 layout in this test (independent of the
writer), then exercised through the writer: every key/value type, alignment, split models, truncation and
corruption. The binding is checked against the reference's rules (src/inference.cpp:234-262, 298-302, 519-545):
tensors found by name, 3-D expert stacks bound as one matrix, shapes and sizes checked, errors named.
"""
import ctypes
import struct

import numpy as np
import pytest

import gguf_file as gf
import moe_hip
import synth


@pytest.fixture(scope="module")
def lib():
    return moe_hip.load_library()


class Model:
    def __init__(self, lib, path):
        self.lib = lib
        self.h = lib.gguf_mmap_open(str(path).encode())

    def __enter__(self):
        return self

    def __exit__(self, *a):
        if self.h:
            self.lib.gguf_mmap_close(self.h)

    def tensor(self, name):
        n = ctypes.c_size_t(0)
        p = self.lib.gguf_get_tensor_ptr(self.h, name.encode(), ctypes.byref(n))
        return None if not p else ctypes.string_at(p, n.value)


def _s(b):
    return struct.pack("<Q", len(b)) + b


def test_known_answer_file(lib, tmp_path):
    """A file written from the format's definition, not by the writer: two key/values, two tensors."""
    head = b"GGUF" + struct.pack("<IQQ", 3, 2, 2)
    head += _s(b"general.architecture") + struct.pack("<I", 8) + _s(b"toy")
    head += _s(b"toy.expert_count") + struct.pack("<II", 4, 7)
    head += _s(b"a") + struct.pack("<I", 2) + struct.pack("<QQ", 3, 2) + struct.pack("<IQ", 0, 0)
    head += _s(b"b") + struct.pack("<I", 1) + struct.pack("<Q", 32) + struct.pack("<IQ", 8, 32)
    pad = (-len(head)) % 32
    a = np.arange(6, dtype=np.float32).tobytes()
    b = bytes(range(34))
    blob = head + b"\0" * pad + a + b"\0" * (32 - len(a)) + b
    p = tmp_path / "k.gguf"
    p.write_bytes(blob)
    with Model(lib, p) as m:
        assert m.h, lib.gguf_last_error()
        assert lib.gguf_version(m.h) == 3 and lib.gguf_n_kv(m.h) == 2 and lib.gguf_n_tensors(m.h) == 2
        assert lib.gguf_data_offset(m.h) == len(head) + pad and lib.gguf_alignment(m.h) == 32
        assert lib.gguf_arch(m.h) == b"toy" and lib.gguf_arch_int(m.h, b"expert_count", -1) == 7
        assert lib.gguf_arch_int(m.h, b"absent", -5) == -5
        assert lib.gguf_tensor_name(m.h, 1) == b"b" and lib.gguf_tensor_type(m.h, 1) == 8
        assert lib.gguf_tensor_dims(m.h, 0) == 2 and list(lib.gguf_tensor_ne(m.h, 0)[:4]) == [3, 2, 1, 1]
        assert lib.gguf_tensor_offset(m.h, 1) == 32 and lib.gguf_tensor_nbytes(m.h, 1) == 34
        assert lib.gguf_tensor_block_size(m.h, 1) == 32 and lib.gguf_tensor_type_size(m.h, 1) == 34
        assert m.tensor("a") == a and m.tensor("b") == b and m.tensor("c") is None
        n = ctypes.c_size_t(0)
        assert lib.gguf_mmap_get_tensor(m.h, b"b", ctypes.byref(n)) and n.value == 34
        assert not lib.gguf_get_tensor_ptr(m.h, b"b", None)  # no out_bytes: NULL, as the reference


def test_writer_matches_known_answer(tmp_path):
    """The writer produces the same bytes for the same content."""
    kvs = [("general.architecture", gf.STRING, "toy"), ("toy.expert_count", gf.U32, 7)]
    ts = [gf.Tensor("a", 0, [3, 2], np.arange(6, dtype=np.float32)), gf.Tensor("b", 8, [32], np.arange(34, dtype=np.uint8))]
    head = b"GGUF" + struct.pack("<IQQ", 3, 2, 2)
    head += _s(b"general.architecture") + struct.pack("<I", 8) + _s(b"toy")
    head += _s(b"toy.expert_count") + struct.pack("<II", 4, 7)
    head += _s(b"a") + struct.pack("<I", 2) + struct.pack("<QQ", 3, 2) + struct.pack("<IQ", 0, 0)
    head += _s(b"b") + struct.pack("<I", 1) + struct.pack("<Q", 32) + struct.pack("<IQ", 8, 32)
    want = head + b"\0" * ((-len(head)) % 32) + np.arange(6, dtype=np.float32).tobytes() + b"\0" * 8
    want += bytes(range(34)) + b"\0" * 30
    assert gf.file_bytes(kvs, ts) == want


def test_every_kv_type(lib, tmp_path):
    kvs = [("u8", gf.U8, 200), ("i8", gf.I8, -100), ("u16", gf.U16, 60000), ("i16", gf.I16, -30000),
           ("u32", gf.U32, 4000000000), ("i32", gf.I32, -2000000000), ("f32", gf.F32, 1.5), ("b", gf.BOOL, True),
           ("s", gf.STRING, "hello"), ("u64", gf.U64, 2 ** 40 + 3), ("i64", gf.I64, -(2 ** 40)), ("f64", gf.F64, 2.25),
           ("arr", gf.ARRAY, (gf.I32, [5, -6, 7])), ("sarr", gf.ARRAY, (gf.STRING, ["x", "yz"])),
           ("general.architecture", gf.STRING, "m"), ("m.n", gf.U16, 12), ("m.f", gf.F64, 0.5)]
    p = tmp_path / "kv.gguf"
    gf.write(p, kvs, [])
    getters = {gf.U8: ("u8", ctypes.c_uint8), gf.I8: ("i8", ctypes.c_int8), gf.U16: ("u16", ctypes.c_uint16),
               gf.I16: ("i16", ctypes.c_int16), gf.U32: ("u32", ctypes.c_uint32), gf.I32: ("i32", ctypes.c_int32),
               gf.F32: ("f32", ctypes.c_float), gf.U64: ("u64", ctypes.c_uint64), gf.I64: ("i64", ctypes.c_int64),
               gf.F64: ("f64", ctypes.c_double)}
    with Model(lib, p) as m:
        assert m.h, lib.gguf_last_error()
        for key, vt, v in kvs:
            i = lib.gguf_find_kv(m.h, key.encode())
            assert i >= 0 and lib.gguf_kv_key(m.h, i) == key.encode() and lib.gguf_kv_type(m.h, i) == vt
            if vt in getters:
                suffix, ct = getters[vt]
                out = ct()
                assert getattr(lib, "gguf_kv_get_" + suffix)(m.h, i, ctypes.byref(out)) == 0
                assert out.value == v
                wrong = "u8" if suffix != "u8" else "i8"
                other = ctypes.c_uint8() if wrong == "u8" else ctypes.c_int8()
                assert getattr(lib, "gguf_kv_get_" + wrong)(m.h, i, ctypes.byref(other)) == -1
        assert lib.gguf_kv_str_val(m.h, lib.gguf_find_kv(m.h, b"s")) == b"hello"
        assert lib.gguf_kv_str_val(m.h, lib.gguf_find_kv(m.h, b"u8")) is None
        et, data, cnt = ctypes.c_int32(), ctypes.c_void_p(), ctypes.c_size_t()
        assert lib.gguf_kv_get_array(m.h, b"arr", ctypes.byref(et), ctypes.byref(data), ctypes.byref(cnt)) == 0
        assert et.value == gf.I32 and cnt.value == 3
        assert list(np.frombuffer(ctypes.string_at(data, 12), np.int32)) == [5, -6, 7]
        assert lib.gguf_kv_get_array(m.h, b"sarr", ctypes.byref(et), ctypes.byref(data), ctypes.byref(cnt)) == -1
        assert lib.gguf_find_kv(m.h, b"nope") == -1
        assert lib.gguf_arch_int(m.h, b"n", 0) == 12 and lib.gguf_arch_float(m.h, b"f", 0.0) == 0.5
        assert lib.gguf_arch_float(m.h, b"n", 0.0) == 12.0 and lib.gguf_arch_float(m.h, b"x", 3.0) == 3.0


@pytest.mark.parametrize("align", [32, 64, 4096])
def test_alignment_and_many_tensors(lib, tmp_path, align):
    rng = np.random.default_rng(align)
    ts = []
    for i in range(40):
        qt = [0, 8, 12, 100, 101][i % 5]
        bv, bb = {0: (1, 4), 8: (32, 34), 12: (256, 144), 100: (32, 18), 101: (32, 17)}[qt]
        k, rows = bv * int(rng.integers(1, 4)) * (8 if bv == 1 else 1), int(rng.integers(1, 5))
        data = rng.integers(0, 256, size=rows * (k // bv) * bb, dtype=np.uint8)
        ts.append(gf.Tensor(f"t{i}", qt, [k, rows], data))
    p = tmp_path / "a.gguf"
    gf.write(p, [("general.architecture", "x")], ts, alignment=align)
    with Model(lib, p) as m:
        assert lib.gguf_alignment(m.h) == align and lib.gguf_data_offset(m.h) % align == 0
        for i, t in enumerate(ts):
            assert lib.gguf_tensor_offset(m.h, i) % align == 0
            assert m.tensor(t.name) == t.data
            assert lib.gguf_tensor_nbytes(m.h, i) == len(t.data)


def test_bad_files_fail_cleanly(lib, tmp_path):
    kvs = [("general.architecture", "x"), ("x.v", gf.ARRAY, (gf.STRING, ["a", "b"]))]
    ts = [gf.Tensor("w", 8, [64, 2], np.zeros(136, np.uint8))]
    good = gf.file_bytes(kvs, ts)
    hdr = len(gf.file_bytes(kvs, ts, alignment=1)) - 136  # the header without its padding
    cases = {"magic": b"GGUX" + good[4:], "v2": good[:4] + struct.pack("<I", 2) + good[8:], "empty": b"",
             "huge_count": good[:8] + struct.pack("<Q", 2 ** 60) + good[16:]}
    for name, blob in cases.items():
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(blob)
        assert not lib.gguf_mmap_open(str(p).encode()), name
        assert lib.gguf_last_error(), name
    assert not lib.gguf_mmap_open(str(tmp_path / "missing.gguf").encode())
    assert b"cannot open" in lib.gguf_last_error()
    # Every truncation inside the header fails; one inside the data section opens, without that tensor's data
    for cut in range(0, hdr, 3):
        p = tmp_path / "cut.gguf"
        p.write_bytes(good[:cut])
        h = lib.gguf_mmap_open(str(p).encode())
        if h:
            lib.gguf_mmap_close(h)
        assert not h, cut
    p.write_bytes(good[:-40])
    with Model(lib, p) as m:
        assert m.h and m.tensor("w") is None and lib.gguf_tensor_nbytes(m.h, 0) == 136


def test_bad_alignment_rejected(lib, tmp_path):
    p = tmp_path / "al.gguf"
    p.write_bytes(gf.file_bytes([("general.alignment", gf.U32, 48)], []))
    assert not lib.gguf_mmap_open(str(p).encode()) and b"alignment" in lib.gguf_last_error()


def test_split_model(lib, tmp_path):
    rng = np.random.default_rng(5)
    groups = [[gf.Tensor(f"g{j}.t{i}", 8, [32, 3], rng.integers(0, 256, 102, dtype=np.uint8)) for i in range(3)]
              for j in range(3)]
    first = gf.write_split(str(tmp_path / "m"), [("general.architecture", "x")], groups)
    with Model(lib, first) as m:
        assert m.h, lib.gguf_last_error()
        assert lib.gguf_n_maps(m.h) == 3 and lib.gguf_n_tensors(m.h) == 9
        for g in groups:
            for t in g:
                assert m.tensor(t.name) == t.data
    # Opening a later part, or with a part missing, fails with the reason
    assert not lib.gguf_mmap_open(str(tmp_path / "m-00002-of-00003.gguf").encode())
    assert b"open the first" in lib.gguf_last_error()
    (tmp_path / "m-00003-of-00003.gguf").unlink()
    assert not lib.gguf_mmap_open(first.encode())


# ---------------------------------------------------------------- MoE layer binding

def _desc_bytes(desc, spec):
    E, NE, FE, t = spec.E, spec.NE, spec.FE, spec.qtype
    sizes = {"w_router": NE * E * 4, "w_gate": NE * FE * synth.row_size(t, E), "w_up": NE * FE * synth.row_size(t, E),
             "w_down": NE * E * synth.row_size(t, FE), "s_gate": FE * synth.row_size(t, E),
             "s_up": FE * synth.row_size(t, E), "s_down": E * synth.row_size(t, FE), "w_shexp": E * 4}
    return {k: ctypes.string_at(getattr(desc, k), n) for k, n in sizes.items() if getattr(desc, k)}


SPECS = [synth.LayerSpec(synth.QT_Q8_0, 256, 8, 2, 256, False), synth.LayerSpec(synth.QT_ROCMFP4, 512, 16, 4, 256, True),
         synth.LayerSpec(synth.QT_Q4_K, 512, 8, 3, 512, True), synth.LayerSpec(synth.QT_ROCMFP4_FAST, 256, 4, 4, 256, True)]


@pytest.mark.parametrize("spec", SPECS, ids=lambda s: f"t{s.qtype}_e{s.E}_ne{s.NE}_sh{int(s.shared)}")
def test_layer_bind_maps_every_tensor(lib, tmp_path, spec):
    layers = [synth.make_layer(spec, seed=i) for i in range(3)]
    p = gf.write_moe_model(str(tmp_path / "moe.gguf"), spec, layers)
    with Model(lib, p) as m:
        assert lib.gguf_block_count(m.h) == 3
        for i, L in enumerate(layers):
            d = moe_hip.LayerDesc()
            assert lib.moe_gguf_layer_bind(m.h, i, ctypes.byref(d)) == 0, lib.moe_gguf_error()
            assert (d.type, d.n_embd, d.n_expert, d.n_used, d.n_ff) == (spec.qtype, spec.E, spec.NE, spec.NU, spec.FE)
            got = _desc_bytes(d, spec)
            assert set(got) == set(L)
            for k, v in L.items():
                assert got[k] == np.ascontiguousarray(v).tobytes(), (i, k)
        assert lib.moe_gguf_layer_bind(m.h, 3, ctypes.byref(moe_hip.LayerDesc())) == -1
        assert b"blk.3" in lib.moe_gguf_error()


def _bind_error(lib, tmp_path, spec, L, hp=None, drop=(), retype=None, reshape=None):
    ts = gf.moe_layer_tensors(spec, L, 0)
    ts = [t for t in ts if not any(t.name.endswith(x) for x in drop)]
    for t in ts:
        if retype and t.name.endswith(retype[0]):
            t.ttype = retype[1]
        if reshape and t.name.endswith(reshape[0]):
            t.ne = reshape[1]
    kvs = gf.moe_hparams(spec)
    for k, v in (hp or {}).items():
        kvs = [(key, ty, v if key.endswith("." + k) else val) for key, ty, val in kvs]
    p = tmp_path / "bad.gguf"
    gf.write(p, kvs, ts)
    with Model(lib, p) as m:
        assert m.h, lib.gguf_last_error()
        r = lib.moe_gguf_layer_bind(m.h, 0, ctypes.byref(moe_hip.LayerDesc()))
        return r, lib.moe_gguf_error().decode()


def test_layer_bind_errors(lib, tmp_path):
    spec = synth.LayerSpec(synth.QT_ROCMFP4, 256, 8, 2, 256, True)
    L = synth.make_layer(spec, seed=1)
    cases = [
        (dict(drop=("ffn_gate_inp.weight",)), "not a MoE layer"),
        (dict(drop=("ffn_up_exps.weight",)), "missing tensor blk.0.ffn_up_exps.weight"),
        (dict(drop=("ffn_gate_inp_shexp.weight",)), "missing tensor blk.0.ffn_gate_inp_shexp.weight"),
        (dict(hp={"expert_used_count": 9}), "bad MoE hparams"),
        (dict(hp={"expert_shared_feed_forward_length": 0}), "bad MoE hparams"),
        (dict(hp={"expert_count": 4}), "ffn_gate_inp: shape 8x256, expected 4x256"),
        (dict(reshape=("ffn_down_exps.weight", [512, 128, 8])), "ffn_down_exps: shape 1024x512, expected 2048x256"),
        (dict(retype=("ffn_down_exps.weight", 101)), "different types (gate 100 up 100 down 101)"),
        (dict(reshape=("ffn_gate_exps.weight", [200, 16, 8])), "type 100 cannot hold rows of 200 values"),
        (dict(hp={"expert_shared_feed_forward_length": 512}), "ffn_gate_shexp: shape 256x256, expected 512x256"),
    ]
    for kw, want in cases:
        r, msg = _bind_error(lib, tmp_path, spec, L, **kw)
        assert r == -1 and want in msg, (kw, msg)
    # An F16 router (the right size and shape for F16) is readable but not what the router takes
    Lh = dict(L)
    Lh["w_router"] = L["w_router"].astype(np.float16)
    ts = gf.moe_layer_tensors(spec, Lh, 0)
    ts[0].ttype = 1
    p = tmp_path / "f16.gguf"
    gf.write(p, gf.moe_hparams(spec), ts)
    with Model(lib, p) as m:
        assert lib.moe_gguf_layer_bind(m.h, 0, ctypes.byref(moe_hip.LayerDesc())) == -1
        assert "router needs F32" in lib.moe_gguf_error().decode()
    # Different expert types within one layer: readable, but not one layer type
    Ld = dict(L)
    Ld["w_down"] = synth.matrix(synth.QT_ROCMFP4_FAST, spec.NE * spec.E, spec.FE, np.random.default_rng(0))
    ts = gf.moe_layer_tensors(spec, Ld, 0)
    ts[3].ttype = synth.QT_ROCMFP4_FAST
    p = tmp_path / "mixed.gguf"
    gf.write(p, gf.moe_hparams(spec), ts)
    with Model(lib, p) as m:
        assert lib.moe_gguf_layer_bind(m.h, 0, ctypes.byref(moe_hip.LayerDesc())) == -1
        assert "different types" in lib.moe_gguf_error().decode()


def test_upload_without_gpu_reports_binding_errors_first(lib, tmp_path):
    """A binding error is reported before any device call (hipErrorInvalidValue = 1, the reason kept)."""
    p = tmp_path / "none.gguf"
    gf.write(p, [("general.architecture", "x")], [])
    with Model(lib, p) as m:
        lay = moe_hip.GgufLayer()
        assert lib.moe_gguf_layer_upload(m.h, 0, 1, ctypes.byref(lay), None) == 1
        assert "not a MoE layer" in lib.moe_gguf_error().decode() and not lay.dev
