"""Writes tests/golden/golden.json: outputs of the REFERENCE's own CPU kernels
(src/kernels.c CPU subset and model.c select_top8, compiled from the reference
tree into oracle/_ref/libref.so by `make -C oracle ref`) on deterministic inputs.

Inputs are not stored: they are regenerated from seeds (roaster_amd's counter-
based generator, and the replayed src/test_kernels.c generator in tk_gen.c).
Each case stores the SHA-256 of its inputs (so a changed generator is caught),
the SHA-256 of every output array (bit-exact check) and a short excerpt.

Run in the container that holds the reference:  python tests/golden/make_golden.py
"""
import ctypes as C
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, HERE)

import roaster_amd as R  # noqa: E402  (host-side generator only)
from oracle import oracle as O  # noqa: E402
import tk_gen  # noqa: E402

_libm = C.CDLL("libm.so.6")
_libm.expf.restype = C.c_float
_libm.expf.argtypes = [C.c_float]


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def excerpt(a, n=16):
    a = np.asarray(a).ravel()[:n]
    return [float(v) if a.dtype.kind == "f" else int(v) for v in a]


def silu_mul(g, u):
    """(g / (1 + expf(-g))) * u in f32 with glibc expf (model.c:1124)."""
    e = np.array([_libm.expf(float(-v)) for v in g], np.float32)
    return ((g / (np.float32(1.0) + e)).astype(np.float32) * u).astype(np.float32)


def ref_matvec(q6, W, x, rows, cols):
    y = np.empty(rows, np.float32)
    f = O.ref().ref_matvec_q6_cpu if q6 else O.ref().ref_matvec_q4_cpu
    f(W.ctypes.data, x.ctypes.data, y.ctypes.data, rows, cols)
    return y


def ref_rowdot_matmul(q6, W, X, rows, cols):
    """test_kernels.c:33-40 (ref_matmul via kernel_dot_q4_k / kernel_dot_q6_k)."""
    T = X.shape[0]
    Y = np.empty((T, rows), np.float32)
    rb = (cols // 256) * (210 if q6 else 144)
    f = O.ref().kernel_dot_q6_k if q6 else O.ref().kernel_dot_q4_k
    for t in range(T):
        xt = np.ascontiguousarray(X[t])
        for r in range(rows):
            Y[t, r] = f(W.ctypes.data + r * rb, xt.ctypes.data, cols)
    return Y


def ref_matmul_cpu(q6, W, X, rows, cols):
    T = X.shape[0]
    Y = np.empty((T, rows), np.float32)
    X = np.ascontiguousarray(X, np.float32)
    O.ref().ref_matmul_quant_cpu(int(q6), W.ctypes.data, X.ctypes.data, Y.ctypes.data, rows, cols, T)
    return Y


def ref_top8(lg):
    lg = np.ascontiguousarray(lg, np.float32)
    ids = np.empty(8, np.int32)
    w = np.empty(8, np.float32)
    O.ref().ref_select_top8(lg.ctypes.data, ids.ctypes.data, w.ctypes.data)
    return ids, w


def top8_cases():
    """Crafted router logits: ties, NaN, +/-inf, fewer than 8 finite values."""
    base = R.synth_normal(7, R.synth_stream(0, 0, 7), 256)
    cases = {}
    a = base.copy()
    a[[3, 9, 200, 17]] = 4.0
    cases["ties_lower_index_first"] = a
    b = base.copy()
    b[[1, 50, 51]] = np.nan
    b[0] = np.inf
    b[255] = np.inf
    cases["nan_and_inf"] = b
    c = np.full(256, -np.inf, np.float32)
    c[[10, 20, 30, 40, 50]] = [1, 2, 3, 4, 5]
    cases["fewer_than_8_finite"] = c
    d = np.zeros(256, np.float32)
    cases["all_equal"] = d
    e = base.copy()
    e[77] = 200.0
    cases["one_dominant"] = e
    return cases


def main():
    if not O.ref_available():
        sys.exit("oracle/_ref/libref.so missing: run `make -C oracle ref` where the reference tree exists")
    out = {"generator": "roaster_amd synth (splitmix64 counter streams) + tk_gen.c replay of src/test_kernels.c",
           "source": "reference src/kernels.c CPU subset + model.c select_top8 via oracle/_ref",
           "cases": {}}
    cases = out["cases"]

    # config 1: Q4_K matvec [512 x 2048], seed 0
    W = R.synth_q4k(0, R.synth_stream(0, 0, 0), 512 * 8)
    x = R.synth_normal(0, R.synth_stream(0, 0, 5), 2048)
    y = ref_matvec(0, W, x, 512, 2048)
    cases["cfg1_q4k_matvec"] = {"inputs": sha(W, x), "y": sha(y), "excerpt": excerpt(y)}

    # Q6_K matvec [2048 x 512] (the down shape), seed 0
    W6 = R.synth_q6k(0, R.synth_stream(0, 0, 2), 2048 * 2)
    e = R.synth_normal(0, R.synth_stream(0, 1, 5), 512)
    y6 = ref_matvec(1, W6, e, 2048, 512)
    cases["q6k_matvec_down_shape"] = {"inputs": sha(W6, e), "y": sha(y6), "excerpt": excerpt(y6)}

    # config 2: one decode MoE block, seed 1 (kernel-level outputs of moe_forward's steps)
    desc = R.table_desc()
    router, gate_inp = R.host_router(1, 0, desc)
    x = R.synth_normal(1, R.synth_stream(0, 0, 5), 2048)
    logits = np.empty(256, np.float32)
    O.ref().kernel_matvec_f32(router.ctypes.data, x.ctypes.data, logits.ctypes.data, 256, 2048)
    ids, w = ref_top8(logits)
    raw = O.ref().kernel_dot_f32(gate_inp.ctypes.data, x.ctypes.data, 2048)
    entry = {"inputs": sha(router, gate_inp, x), "logits": sha(logits), "ids": ids.tolist(),
             "w": sha(w), "w_excerpt": excerpt(w), "shared_gate_raw": float(raw), "experts": {}}
    for k, eid in enumerate(list(ids) + [256]):
        g, u, d = R.host_expert(1, 0, int(eid), desc)
        gv = ref_matvec(0, g, x, 512, 2048)
        uv = ref_matvec(0, u, x, 512, 2048)
        eh = silu_mul(gv, uv)
        dv = ref_matvec(1, d, eh, 2048, 512)
        entry["experts"][str(int(eid))] = {"weights": sha(g, u, d), "gate": sha(gv), "up": sha(uv),
                                           "eh": sha(eh), "down": sha(dv), "down_excerpt": excerpt(dv, 8)}
    cases["cfg2_decode_block"] = entry

    # RMSNorm (kernels.c:584-605), eps 1e-6
    h = R.synth_normal(3, R.synth_stream(0, 0, 5), 2048)
    nw = R.synth_normal(3, R.synth_stream(0, 1, 6), 2048, 0.1) + np.float32(1.0)
    nw = nw.astype(np.float32)
    r = np.empty(2048, np.float32)
    O.ref().kernel_rmsnorm(r.ctypes.data, h.ctypes.data, nw.ctypes.data, 2048, C.c_float(1e-6))
    cases["rmsnorm"] = {"inputs": sha(h, nw), "y": sha(r), "excerpt": excerpt(r)}

    # select_top8 special cases (model.c:869-897)
    t8 = {}
    for name, lg in top8_cases().items():
        i8, w8 = ref_top8(lg)
        t8[name] = {"inputs": sha(lg), "ids": i8.tolist(), "w_bits": w8.view(np.uint32).tolist()}
    cases["top8"] = t8

    # src/test_kernels.c cases: row-dot oracle (its ref_matmul) and matmul_quant_cpu
    tk = []
    for c in tk_gen.matmul_cases():
        if c[0] == "mm":
            _, q6, rows, cols, T, W, X = c
            tk.append({"kind": "mm", "q6": q6, "rows": rows, "cols": cols, "T": T, "inputs": sha(W, X),
                       "rowdot": sha(ref_rowdot_matmul(q6, W, X, rows, cols)),
                       "matmul_cpu": sha(ref_matmul_cpu(q6, W, X, rows, cols))})
        elif c[0] == "shared":
            _, X, jobs = c
            for q6, rows, W in jobs:
                tk.append({"kind": "shared", "q6": q6, "rows": rows, "cols": 2048, "T": 40, "inputs": sha(W, X),
                           "rowdot": sha(ref_rowdot_matmul(q6, W, X, rows, 2048)),
                           "matmul_cpu": sha(ref_matmul_cpu(q6, W, X, rows, 2048))})
        else:
            _, X, experts, ns = c
            arr = (O.OrcMoeGroup * 6)()
            for i, (g, u, d, g6, u6, d6) in enumerate(experts):
                arr[i] = O.OrcMoeGroup(g.ctypes.data, u.ctypes.data, d.ctypes.data, g6, u6, d6, ns[i])
            D = np.zeros((sum(ns), 2048), np.float32)
            # KernelMoeExpert and OrcMoeGroup share one layout
            O.ref().ref_moe_cpu(C.cast(arr, C.c_void_p), 6, X.ctypes.data, D.ctypes.data, 512, 2048)
            tk.append({"kind": "moe", "ns": ns, "inputs": sha(X, *[a for ex in experts for a in ex[:3]]),
                       "D": sha(D), "excerpt": excerpt(D)})
    cases["test_kernels"] = tk

    path = os.path.join(HERE, "golden.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print("wrote", path)


if __name__ == "__main__":
    main()
