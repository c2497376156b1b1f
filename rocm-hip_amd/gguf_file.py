"""Write GGUF v3 files: synthetic MoE layers for the loader's tests and for benchmarking from a file.

GGUF v3 (little-endian): b"GGUF", u32 version 3, u64 tensor count, u64 key/value count; key/values (u64-length
string key, u32 value type, value); tensor infos (string name, u32 n_dims, n_dims x u64 ne with ne[0] the row
length, u32 tensor type, u64 offset into the data section); padding to general.alignment (32 when absent); the
data section, each tensor at an aligned offset. A model can be split in files <prefix>-0000i-of-0000N.gguf,
each with split.no / split.count and its own tensors (the layout llama.cpp's gguf-split writes, which the
reference's loader reads in src/gguf_mmap.cpp:386-425).
"""
import struct

import numpy as np

# key/value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}


def _str(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(vtype, v):
    if vtype == STRING:
        return _str(v)
    if vtype == ARRAY:
        etype, items = v
        out = struct.pack("<IQ", etype, len(items))
        return out + b"".join(_value(etype, x) for x in items)
    return struct.pack(_FMT[vtype], v)


def _infer(v):
    if isinstance(v, bool):
        return BOOL
    if isinstance(v, int):
        return U32 if 0 <= v < 2 ** 32 else I64
    if isinstance(v, float):
        return F32
    if isinstance(v, str):
        return STRING
    raise TypeError(v)


class Tensor:
    """One tensor: name, GGUF type id, ne (ne[0] first: the row length), raw bytes."""

    def __init__(self, name, ttype, ne, data):
        self.name, self.ttype, self.ne = name, int(ttype), [int(x) for x in ne]
        self.data = np.ascontiguousarray(data).view(np.uint8).reshape(-1).tobytes()


def file_bytes(kvs, tensors, alignment=32, version=3):
    """The bytes of one GGUF file. kvs: list of (key, value) or (key, type, value); tensors: list of Tensor."""
    head = bytearray(b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs)))
    for kv in kvs:
        key, vtype, v = (kv[0], _infer(kv[1]), kv[1]) if len(kv) == 2 else kv
        head += _str(key) + struct.pack("<I", vtype) + _value(vtype, v)
    offsets, off = [], 0
    for t in tensors:
        offsets.append(off)
        off = (off + len(t.data) + alignment - 1) // alignment * alignment
    for t, o in zip(tensors, offsets):
        head += _str(t.name) + struct.pack("<I", len(t.ne)) + b"".join(struct.pack("<Q", x) for x in t.ne)
        head += struct.pack("<IQ", t.ttype, o)
    head += b"\0" * ((-len(head)) % alignment)
    body = bytearray(off)
    for t, o in zip(tensors, offsets):
        body[o:o + len(t.data)] = t.data
    return bytes(head) + bytes(body)


def write(path, kvs, tensors, alignment=32):
    """One file; general.alignment is added when alignment is not 32."""
    kvs = list(kvs)
    if alignment != 32:
        kvs.append(("general.alignment", U32, alignment))
    with open(path, "wb") as f:
        f.write(file_bytes(kvs, tensors, alignment))


def write_split(prefix, kvs, tensor_groups):
    """A split model: file i holds tensor_groups[i]; the first also holds kvs. Returns the first file's path."""
    n = len(tensor_groups)
    paths = [f"{prefix}-{i + 1:05d}-of-{n:05d}.gguf" for i in range(n)]
    for i, (p, group) in enumerate(zip(paths, tensor_groups)):
        meta = (list(kvs) if i == 0 else []) + [("split.no", U16, i), ("split.count", U16, n)]
        write(p, meta, group)
    return paths[0]


def moe_hparams(spec, arch="qwen3moe", n_layers=1):
    """The "<arch>.*" hparams a MoE layer is bound with (src/inference.cpp:981-984)."""
    return [("general.architecture", STRING, arch), (f"{arch}.block_count", U32, n_layers),
            (f"{arch}.embedding_length", U32, spec.E), (f"{arch}.expert_count", U32, spec.NE),
            (f"{arch}.expert_used_count", U32, spec.NU), (f"{arch}.expert_feed_forward_length", U32, spec.FE),
            (f"{arch}.expert_shared_feed_forward_length", U32, spec.FE if spec.shared else 0)]


def moe_layer_tensors(spec, L, layer):
    """Layer `layer`'s tensors in GGUF form from synth.make_layer's host arrays: the expert stacks 3-D
    ({K, rows per expert, NE}), the shared expert 2-D, router and shared gate F32."""
    E, NE, FE, t = spec.E, spec.NE, spec.FE, spec.qtype
    b = f"blk.{layer}."
    out = [Tensor(b + "ffn_gate_inp.weight", 0, [E, NE], L["w_router"]),
           Tensor(b + "ffn_gate_exps.weight", t, [E, FE, NE], L["w_gate"]),
           Tensor(b + "ffn_up_exps.weight", t, [E, FE, NE], L["w_up"]),
           Tensor(b + "ffn_down_exps.weight", t, [FE, E, NE], L["w_down"])]
    if "s_gate" in L:
        out += [Tensor(b + "ffn_gate_shexp.weight", t, [E, FE], L["s_gate"]),
                Tensor(b + "ffn_up_shexp.weight", t, [E, FE], L["s_up"]),
                Tensor(b + "ffn_down_shexp.weight", t, [FE, E], L["s_down"]),
                Tensor(b + "ffn_gate_inp_shexp.weight", 0, [E], L["w_shexp"])]
    return out


def write_moe_model(path, spec, layers, arch="qwen3moe"):
    """A file holding several MoE layers: layers is a list of synth.make_layer dicts (blk.0, blk.1, ...)."""
    tensors = [t for i, L in enumerate(layers) for t in moe_layer_tensors(spec, L, i)]
    write(path, moe_hparams(spec, arch, len(layers)), tensors)
    return path

