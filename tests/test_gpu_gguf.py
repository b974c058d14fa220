"""GGUF file -> HBM expert table -> decode / prefill on the GPU.

A three-layer synthetic model at the real hidden / inter sizes with 16 experts;
layer 1 flips every matrix type of layer 0 (so Q4_K down and Q6_K gate/up run
too) and stores its router in F16; layer 2 gives gate and up different types
(routed Q6_K gate / Q4_K up, shared the other way round), which caps prefill
tiles at 64 rows.  The loaded table must hold the file's
bytes, and decode / prefill through it must match the oracle on the same
weights (tolerance max|d|/max|y| <= 2e-3, the FFN bar; decode also <= 1e-4)."""
import ctypes as C

import numpy as np
import pytest

import roaster_amd as R
from gguf_util import GT_F16, GT_F32, METADATA, MoeModel, write_gguf
from gpu_util import Dev, log, rel_err
from oracle import oracle as O

pytestmark = pytest.mark.gpu

E, H, I = 16, 2048, 512
TYPES = [(0, 0, 1, 0, 0, 1), (1, 1, 0, 1, 1, 0), (1, 0, 1, 0, 1, 0)]
NL = len(TYPES)
TOL, TIGHT = 2e-3, 1e-4


@pytest.fixture(scope="module")
def loaded(tmp_path_factory):
    log(f"gguf: writing a {NL}-layer, {E}-expert model")
    m = MoeModel(31, NL, E, H, I, TYPES, [GT_F32, GT_F16, GT_F32])
    path = tmp_path_factory.mktemp("gguf") / "moe.gguf"
    write_gguf(path, METADATA, m.tensors(), alignment=64)
    info = R.RoasterGgufInfo()
    log("gguf: roaster_table_load_gguf")
    t = R.lib().roaster_table_load_gguf(str(path).encode(), C.byref(info))
    assert t, R.last_error()
    yield m, t, info
    R.lib().roaster_table_destroy(t)


def oracle_layer(m, l):
    exps = [tuple(m.exps[l][k][e] for k in range(3)) for e in range(E)]
    return O.Layer(H, I, m.router[l], m.gate_inp[l], exps, m.shared[l], TYPES[l][:3], TYPES[l][3:])


def test_info_and_bytes(loaded):
    m, t, info = loaded
    assert (info.n_layers, info.n_experts, info.hidden, info.inter, info.mixed_types) == (NL, E, H, I, 1)
    for l in range(NL):
        for e in (0, 5, E - 1, E):
            ptrs = [C.c_void_p() for _ in range(3)]
            R.check(R.lib().roaster_table_expert_ptrs(t, l, e, *[C.byref(p) for p in ptrs]))
            want = m.shared[l] if e == E else tuple(m.exps[l][k][e] for k in range(3))
            for k in range(3):
                got = np.empty(want[k].nbytes, np.uint8)
                R.check(R.lib().roaster_d2h(got.ctypes.data, ptrs[k].value, got.nbytes))
                assert np.array_equal(got, want[k]), (l, e, k)


@pytest.mark.parametrize("layer", range(NL))
def test_decode_from_gguf(loaded, layer):
    m, t, _ = loaded
    log(f"gguf decode layer {layer} (types {TYPES[layer]})")
    x = R.synth_normal(7, R.synth_stream(layer, 0, 5), H)
    dx, dy = Dev(x[None, :]), Dev(nbytes=H * 4, shape=(1, H))
    dl = Dev(nbytes=E * 4, shape=(1, E))
    di = Dev(nbytes=8 * 4, dtype=np.int32, shape=(1, 8))
    dw = Dev(nbytes=8 * 4, shape=(1, 8))
    io = R.RoasterDecodeIO(None, dl.p, di.p, dw.p)
    R.check(R.lib().roaster_moe_decode(t, layer, dx.p, 1, dy.p, C.byref(io)), "decode")
    R.check(R.lib().roaster_sync(), "sync")
    y, lg, ids = dy.get()[0], dl.get()[0], di.get()[0]
    assert rel_err(lg, O.matvec_f32(m.router[layer], x)) <= 1e-5
    ids_ref, _ = O.select_top8(lg)
    assert ids.tolist() == ids_ref.tolist()
    rc, y_ref, _, _, _ = oracle_layer(m, layer).decode(x, logits_in=lg)
    assert rc == 0
    err = rel_err(y, y_ref)
    log(f"gguf decode layer {layer}: max|d|/max|y| = {err:.3e}")
    assert err <= TOL and err <= TIGHT


@pytest.mark.parametrize("layer", range(NL))
def test_prefill_from_gguf(loaded, layer):
    m, t, _ = loaded
    T = 200
    log(f"gguf prefill layer {layer}, T={T}")
    X = np.stack([R.synth_normal(9, R.synth_stream(layer, tok, 5), H) for tok in range(T)])
    dx, dy = Dev(X), Dev(nbytes=T * H * 4, shape=(T, H))
    dl = Dev(nbytes=T * E * 4, shape=(T, E))
    o = R.RoasterPrefillOpts(R.PREC_F16, None, None, dl.p, None, None, None)
    R.check(R.lib().roaster_moe_prefill(t, layer, dx.p, T, dy.p, C.byref(o)), "prefill")
    R.check(R.lib().roaster_sync(), "sync")
    Y, lg = dy.get(), dl.get()
    lg_ref = np.stack([O.matvec_f32(m.router[layer], X[t]) for t in range(T)])   # T, E not multiples of 32
    assert rel_err(lg, lg_ref) <= 1e-5
    rc, Y_ref, _, _, _ = oracle_layer(m, layer).prefill(X, logits_in=lg)
    assert rc == 0
    err = rel_err(Y, Y_ref)
    log(f"gguf prefill layer {layer}: max|d|/max|y| = {err:.3e}")
    assert err <= TOL
