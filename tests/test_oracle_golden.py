"""The oracle reproduces, bit for bit, the reference's own CPU kernels on the
golden cases (tests/golden/golden.json, written by make_golden.py from the
reference tree compiled into oracle/_ref)."""
import ctypes as C
import hashlib

import numpy as np
import pytest

import roaster_amd as R
from oracle import oracle as O
import tk_gen


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def test_cfg1_q4k_matvec(golden):
    g = golden["cases"]["cfg1_q4k_matvec"]
    W = R.synth_q4k(0, R.synth_stream(0, 0, 0), 512 * 8)
    x = R.synth_normal(0, R.synth_stream(0, 0, 5), 2048)
    assert sha(W, x) == g["inputs"], "generator changed"
    y = O.matvec(0, W, x, 512, 2048)
    assert sha(y) == g["y"], (y[:4], g["excerpt"][:4])


def test_q6k_matvec_down_shape(golden):
    g = golden["cases"]["q6k_matvec_down_shape"]
    W = R.synth_q6k(0, R.synth_stream(0, 0, 2), 2048 * 2)
    e = R.synth_normal(0, R.synth_stream(0, 1, 5), 512)
    assert sha(W, e) == g["inputs"]
    assert sha(O.matvec(1, W, e, 2048, 512)) == g["y"]


def test_cfg2_decode_block_steps(golden):
    """Router logits, top-8, the shared gate dot and each selected expert's
    gate / up / SiLU*up / down equal the reference's kernels on config 2."""
    g = golden["cases"]["cfg2_decode_block"]
    desc = R.table_desc()
    router, gate_inp = R.host_router(1, 0, desc)
    x = R.synth_normal(1, R.synth_stream(0, 0, 5), 2048)
    assert sha(router, gate_inp, x) == g["inputs"]
    logits = O.matvec_f32(router, x)
    assert sha(logits) == g["logits"]
    ids, w = O.select_top8(logits)
    assert ids.tolist() == g["ids"]
    assert sha(w) == g["w"]
    raw = O.orc().orc_dot_f32(gate_inp.ctypes.data, x.ctypes.data, 2048)
    assert raw == g["shared_gate_raw"]
    layer_experts = {}
    for eid in list(ids) + [256]:
        ge, ue, de = R.host_expert(1, 0, int(eid), desc)
        ref = g["experts"][str(int(eid))]
        assert sha(ge, ue, de) == ref["weights"]
        gv = O.matvec(0, ge, x, 512, 2048)
        uv = O.matvec(0, ue, x, 512, 2048)
        assert sha(gv) == ref["gate"] and sha(uv) == ref["up"]
        layer_experts[int(eid)] = (ge, ue, de)
        # whole expert through the oracle's decode expert path
        out = np.empty(2048, np.float32)
        ex = O.OrcExpert(ge.ctypes.data, ue.ctypes.data, de.ctypes.data, 0, 0, 1)
        O.orc().orc_expert_decode(C.byref(ex), x.ctypes.data, 512, 2048, out.ctypes.data)
        assert sha(out) == ref["down"]


def test_rmsnorm(golden):
    g = golden["cases"]["rmsnorm"]
    h = R.synth_normal(3, R.synth_stream(0, 0, 5), 2048)
    nw = (R.synth_normal(3, R.synth_stream(0, 1, 6), 2048, 0.1) + np.float32(1.0)).astype(np.float32)
    assert sha(h, nw) == g["inputs"]
    r = np.empty(2048, np.float32)
    O.orc().orc_rmsnorm(r.ctypes.data, h.ctypes.data, nw.ctypes.data, 2048, C.c_float(1e-6))
    assert sha(r) == g["y"]


def test_top8_special_cases(golden):
    from make_golden import top8_cases
    for name, lg in top8_cases().items():
        ref = golden["cases"]["top8"][name]
        assert sha(lg) == ref["inputs"]
        ids, w = O.select_top8(lg)
        assert ids.tolist() == ref["ids"], name
        assert w.view(np.uint32).tolist() == ref["w_bits"], name


def test_reference_test_kernels_cases(golden):
    """src/test_kernels.c's inputs: the oracle's folded row dot equals the
    reference's kernel_dot_q*_k and its matmul equals matmul_quant_cpu; the
    MoE batch equals moe_cpu -- all bit for bit."""
    ref = golden["cases"]["test_kernels"]
    i = 0
    for c in tk_gen.matmul_cases():
        if c[0] == "mm":
            _, q6, rows, cols, T, W, X = c
            jobs = [(q6, rows, cols, W, X)]
        elif c[0] == "shared":
            _, X, js = c
            jobs = [(q6, rows, 2048, W, X) for q6, rows, W in js]
        else:
            _, X, experts, ns = c
            g = ref[i]
            i += 1
            assert g["kind"] == "moe"
            assert sha(X, *[a for ex in experts for a in ex[:3]]) == g["inputs"]
            arr = (O.OrcMoeGroup * 6)()
            for k, (gw, uw, dw, g6, u6, d6) in enumerate(experts):
                arr[k] = O.OrcMoeGroup(gw.ctypes.data, uw.ctypes.data, dw.ctypes.data, g6, u6, d6, ns[k])
            D = np.zeros((sum(ns), 2048), np.float32)
            O.orc().orc_moe_groups(arr, 6, X.ctypes.data, D.ctypes.data, 512, 2048)
            assert sha(D) == g["D"]
            continue
        for q6, rows, cols, W, X in jobs:
            g = ref[i]
            i += 1
            assert (g["q6"], g["rows"], g["T"]) == (q6, rows, X.shape[0])
            assert sha(W, X) == g["inputs"]
            Yd = np.stack([O.matvec(q6, W, np.ascontiguousarray(X[t]), rows, cols) for t in range(X.shape[0])])
            assert sha(Yd) == g["rowdot"], (q6, rows, cols, X.shape[0])
            assert sha(O.matmul(q6, W, X, rows, cols)) == g["matmul_cpu"], (q6, rows, cols, X.shape[0])
    assert i == len(ref)
