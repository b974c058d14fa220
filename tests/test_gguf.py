"""GGUF v3 scanning (host only, no GPU): header, metadata skipping, alignment,
tensor table, the MoE tensors of every layer, and the error cases the reference
loader rejects (weights.c:657-842)."""
import ctypes as C

import numpy as np
import pytest

import roaster_amd as R
from gguf_util import GT_F16, GT_F32, GT_Q4_K, GT_Q8_0, METADATA, MoeModel, write_gguf

E, H, I = 8, 256, 256
TYPES = [(0, 0, 1, 1, 0, 1), (1, 1, 0, 0, 1, 1)]        # layer 1 differs from layer 0


@pytest.fixture(scope="module")
def model():
    return MoeModel(21, 2, E, H, I, TYPES, [GT_F32, GT_F16])


def extra_tensors():
    """Tensors off the MoE path, one of a type the scanner does not size."""
    return [("token_embd.weight", [H, 4], GT_F32, np.zeros(4 * H, np.float32).tobytes()),
            ("blk.0.attn_q.weight", [H, 2], GT_Q8_0, bytes(2 * H // 32 * 34)),
            ("blk.0.attn_norm.weight", [H], GT_F32, np.ones(H, np.float32).tobytes())]


def scan(path):
    info = R.RoasterGgufInfo()
    rc = R.lib().roaster_gguf_scan(str(path).encode(), C.byref(info))
    return rc, info


def test_scan_reads_header_metadata_and_moe_tensors(tmp_path, model):
    path = tmp_path / "m.gguf"
    tensors = model.tensors(extra_tensors())
    data_off, _ = write_gguf(path, METADATA, tensors, alignment=64)
    rc, info = scan(path)
    assert rc == R.OK, R.last_error()
    assert info.version == 3 and info.n_tensors == len(tensors)
    assert info.alignment == 64 and info.data_offset == data_off and data_off % 64 == 0
    assert (info.n_layers, info.n_experts, info.hidden, info.inter) == (2, E, H, I)
    assert list(info.q6) == list(TYPES[0][:3]) and list(info.sh_q6) == list(TYPES[0][3:])
    assert info.mixed_types == 1 and info.router_type == GT_F32


def test_default_alignment_is_32(tmp_path, model):
    meta = [m for m in METADATA if m[0] != "general.alignment"]
    path = tmp_path / "a32.gguf"
    data_off, _ = write_gguf(path, meta, model.tensors(), alignment=32)
    rc, info = scan(path)
    assert rc == R.OK, R.last_error()
    assert info.alignment == 32 and info.data_offset == data_off


def test_uniform_types_are_not_mixed(tmp_path):
    m = MoeModel(3, 2, E, H, I, [(0, 0, 1, 0, 0, 1)] * 2, [GT_F32, GT_F32])
    path = tmp_path / "u.gguf"
    write_gguf(path, METADATA, m.tensors(), alignment=64)
    rc, info = scan(path)
    assert rc == R.OK and info.mixed_types == 0


def _mutate(model, what):
    """(metadata, tensors, write_gguf kwargs, expected message part) of a broken file."""
    meta, ts, kw = list(METADATA), model.tensors(), {"alignment": 64}
    idx = {t[0]: i for i, t in enumerate(ts)}
    if what == "magic":
        kw["magic"] = b"GGUG"
        return meta, ts, kw, "bad magic"
    if what == "version":
        kw["version"] = 2
        return meta, ts, kw, "version 2"
    if what == "no_tensors":
        return meta, [], kw, "no tensors"
    if what == "missing_shexp":
        del ts[idx["blk.1.ffn_up_shexp.weight"]]
        return meta, ts, kw, "blk.1.ffn_up_shexp.weight is missing"
    if what == "wrong_experts":
        i = idx["blk.1.ffn_down_exps.weight"]
        n, dims, gt, data = ts[i]
        ts[i] = (n, [I, H, E // 2], gt, data[: len(data) // 2])
        return meta, ts, kw, "unexpected shape"
    if what == "wrong_type":
        i = idx["blk.0.ffn_gate_exps.weight"]
        n, dims, gt, data = ts[i]
        ts[i] = (n, dims, GT_Q8_0, bytes(H * I * E // 32 * 34))
        return meta, ts, kw, "unsupported type 8"
    if what == "quant_gate_vector":
        i = idx["blk.0.ffn_gate_inp_shexp.weight"]
        n, dims, gt, data = ts[i]
        ts[i] = (n, dims, GT_Q4_K, bytes(H // 256 * 144))
        return meta, ts, kw, "unsupported type 12"
    if what == "gap_in_layers":
        ts = [(n.replace("blk.1.", "blk.2."), d, g, b) for n, d, g, b in ts]
        return meta, ts, kw, "layer 1 has no MoE tensors"
    if what == "truncated":
        kw["truncate"] = -1000
        return meta, ts, kw, "outside the file"
    if what == "misaligned_offset":
        kw["offset_fix"] = {idx["blk.0.ffn_up_exps.weight"]: 8}
        return meta, ts, kw, "outside the file"
    if what == "bad_metadata_type":
        meta.append(("bad.key", 99, None))
        return meta, ts, kw, "unknown metadata value type 99"
    if what == "duplicate":
        ts.append(ts[idx["blk.0.ffn_gate_inp.weight"]])
        return meta, ts, kw, "duplicate tensor"
    raise ValueError(what)


@pytest.mark.parametrize("what", ["magic", "version", "no_tensors", "missing_shexp", "wrong_experts", "wrong_type",
                                  "quant_gate_vector", "gap_in_layers", "truncated", "misaligned_offset",
                                  "bad_metadata_type", "duplicate"])
def test_scan_rejects(tmp_path, model, what):
    meta, ts, kw, msg = _mutate(model, what)
    path = tmp_path / f"{what}.gguf"
    if what == "bad_metadata_type":
        # an unknown value type: key, type 99, then nothing the reader can skip
        import struct
        from gguf_util import _str
        good = [m for m in meta if m[2] is not None]
        write_gguf(path, good, ts, **kw)
        raw = bytearray(open(path, "rb").read())
        n_meta = struct.unpack_from("<Q", raw, 16)[0]
        struct.pack_into("<Q", raw, 16, n_meta + 1)
        hdr = 24
        raw[hdr:hdr] = _str("bad.key") + struct.pack("<I", 99)
        open(path, "wb").write(raw)
    else:
        if kw.get("truncate") is not None and kw["truncate"] < 0:
            write_gguf(path, meta, ts, alignment=kw["alignment"])
            size = path.stat().st_size
            kw["truncate"] = size + kw["truncate"]
        write_gguf(path, meta, ts, **kw)
    rc, _ = scan(path)
    assert rc == R.EINVAL
    assert msg in R.last_error(), R.last_error()


def test_scan_missing_file(tmp_path):
    rc, _ = scan(tmp_path / "nope.gguf")
    assert rc == R.EINVAL and "cannot open" in R.last_error()
