"""A GGUF v3 writer for tests, and a synthetic MoE model in that format.

The layout is the one the reference loader reads (weights.c:657-842): "GGUF",
version, tensor count, metadata count (little endian); metadata as (string
key, uint32 type, value); tensor infos as (string name, uint32 n_dims, uint64
dims[n_dims], uint32 GGML type, uint64 offset relative to the data section);
the data section starts at the first multiple of the alignment after the infos,
and every tensor offset is a multiple of the alignment.
"""
import struct

import numpy as np

import roaster_amd as R

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
GT_F32, GT_F16, GT_Q8_0, GT_Q4_K, GT_Q6_K = 0, 1, 8, 12, 14
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _val(t, v):
    if t == STR:
        return _str(v)
    if t == ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_val(et, x) for x in items)
    return struct.pack(_FMT[t], v)


def write_gguf(path, metadata, tensors, alignment=32, version=3, magic=b"GGUF", truncate=None,
               offset_fix=None):
    """metadata: [(key, type, value)]; tensors: [(name, dims, ggml_type, bytes)].
    Returns (data_offset, [tensor offsets]).  truncate cuts the file to that
    many bytes; offset_fix maps a tensor index to a replacement offset."""
    head = magic + struct.pack("<IQQ", version, len(tensors), len(metadata))
    for k, t, v in metadata:
        head += _str(k) + struct.pack("<I", t) + _val(t, v)
    offs, off = [], 0
    for _, _, _, data in tensors:
        off = (off + alignment - 1) // alignment * alignment
        offs.append(off)
        off += len(data)
    for i, ((name, dims, gt, _), o) in enumerate(zip(tensors, offs)):
        o = offset_fix.get(i, o) if offset_fix else o
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", gt, o)
    data_off = (len(head) + alignment - 1) // alignment * alignment
    blob = bytearray(head) + bytearray(data_off - len(head))
    for (_, _, _, data), o in zip(tensors, offs):
        blob += bytearray(data_off + o - len(blob))
        blob += bytes(data)
    if truncate is not None:
        blob = blob[:truncate]
    with open(path, "wb") as f:
        f.write(blob)
    return data_off, offs


def quant_bytes(q6, seed, stream, rows, cols):
    nb = rows * (cols // 256)
    return R.synth_q6k(seed, stream, nb) if q6 else R.synth_q4k(seed, stream, nb)


class MoeModel:
    """Synthetic MoE tensors of n_layers layers.  types[l] = (gate, up, down,
    shared gate, shared up, shared down) with 1 = Q6_K; router_types[l] is the
    GGML type of the router (F32 or F16)."""

    def __init__(self, seed, n_layers, E, H, I, types, router_types):
        self.E, self.H, self.I, self.n_layers = E, H, I, n_layers
        self.types, self.router_types = types, router_types
        self.exps, self.shared, self.router, self.gate_inp = [], [], [], []
        for l in range(n_layers):
            t = types[l]
            kinds = []
            for k in range(3):
                rows, cols = (H, I) if k == 2 else (I, H)
                kinds.append([quant_bytes(t[k], seed, R.synth_stream(l, e, k), rows, cols) for e in range(E)])
            self.exps.append(kinds)
            self.shared.append(tuple(quant_bytes(t[3 + k], seed, R.synth_stream(l, E, k), *((H, I) if k == 2 else (I, H)))
                                     for k in range(3)))
            r = R.synth_normal(seed, R.synth_stream(l, 0, 3), E * H, 0.02).reshape(E, H)
            if router_types[l] == GT_F16:
                r = r.astype(np.float16).astype(np.float32)     # the values the file can hold
            self.router.append(np.ascontiguousarray(r))
            self.gate_inp.append(R.synth_normal(seed, R.synth_stream(l, 0, 4), H, 0.02))

    def tensors(self, extra=()):
        """GGUF tensor list (name, dims, type, bytes), plus extra tensors."""
        E, H, I = self.E, self.H, self.I
        out = list(extra)
        for l in range(self.n_layers):
            t = self.types[l]
            names = ("ffn_gate_exps", "ffn_up_exps", "ffn_down_exps")
            for k in range(3):
                dims = [I, H, E] if k == 2 else [H, I, E]
                out.append((f"blk.{l}.{names[k]}.weight", dims, GT_Q6_K if t[k] else GT_Q4_K,
                            np.concatenate(self.exps[l][k]).tobytes()))
            rt = self.router_types[l]
            rb = self.router[l].astype(np.float16).tobytes() if rt == GT_F16 else self.router[l].tobytes()
            out.append((f"blk.{l}.ffn_gate_inp.weight", [H, E], rt, rb))
            out.append((f"blk.{l}.ffn_gate_inp_shexp.weight", [H], GT_F32, self.gate_inp[l].tobytes()))
            for k, nm in enumerate(("ffn_gate_shexp", "ffn_up_shexp", "ffn_down_shexp")):
                dims = [I, H] if k == 2 else [H, I]
                out.append((f"blk.{l}.{nm}.weight", dims, GT_Q6_K if t[3 + k] else GT_Q4_K,
                            self.shared[l][k].tobytes()))
        return out


METADATA = [
    ("general.architecture", STR, "qwen35moe"),
    ("general.alignment", U32, 64),
    ("qwen35moe.expert_count", U32, 8),
    ("tokenizer.ggml.tokens", ARR, (STR, ["a", "bb", "ccc"])),
    ("tokenizer.ggml.scores", ARR, (F32, [0.5, -1.0, 2.0])),
    ("some.nested", ARR, (ARR, [(U8, [1, 2, 3]), (U16, [4])])),
    ("some.flag", BOOL, True),
    ("some.f64", F64, 1.5),
]
