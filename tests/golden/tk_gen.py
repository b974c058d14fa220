"""Replays the inputs of the reference's src/test_kernels.c (via tk_gen.c,
compiled on first use into tests/golden/_build/).  Test infrastructure only."""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SO = os.path.join(HERE, "_build", "libtkgen.so")
_L = None


def _lib():
    global _L
    if _L is None:
        src = os.path.join(HERE, "tk_gen.c")
        if not os.path.exists(SO) or os.path.getmtime(SO) < os.path.getmtime(src):
            os.makedirs(os.path.dirname(SO), exist_ok=True)
            subprocess.check_call(["gcc", "-O2", "-fPIC", "-shared", "-o", SO, src])
        _L = C.CDLL(SO)
        _L.tk_make_w.argtypes = [C.c_int, C.c_size_t, C.c_size_t, C.c_void_p]
        _L.tk_frnd.argtypes = [C.c_void_p, C.c_size_t]
    return _L


def reset():
    _lib().tk_reset()


def make_w(q6, rows, cols):
    n = rows * (cols // 256) * (210 if q6 else 144)
    w = np.empty(n, np.uint8)
    _lib().tk_make_w(int(q6), rows, cols, w.ctypes.data)
    return w


def frnd(n):
    x = np.empty(n, np.float32)
    _lib().tk_frnd(x.ctypes.data, n)
    return x


TS = [1, 3, 8, 9, 16, 17, 100, 257]


def matmul_cases():
    """Yields (q6, rows, cols, T, W, X) in test_kernels.c:47-62 order, then the
    shared-X jobs (64-70) as ('shared', X, [(q6, rows, W)...]), then the MoE
    batch (72-92) as ('moe', X, experts, ns)."""
    reset()
    for q6 in (0, 1):
        for ri in range(3):
            rows = (512, 2048, 37)[ri]
            cols = 512 if ri == 1 else 2048
            W = make_w(q6, rows, cols)
            for T in TS:
                X = frnd(T * cols).reshape(T, cols)
                yield ("mm", q6, rows, cols, T, W, X)
    T, cols = 40, 2048
    X = frnd(T * cols).reshape(T, cols)
    jobs = []
    for rw, q in zip((256, 64, 32), (0, 1, 0)):
        jobs.append((q, rw, make_w(q, rw, cols)))
    yield ("shared", X, jobs)
    inter, hidden = 512, 2048
    ns = [5, 1, 0, 17, 9, 30]
    tot = sum(ns)
    X = frnd(tot * hidden).reshape(tot, hidden)
    experts = []
    for i in range(6):
        g6, d6 = i % 2, (i // 2) % 2
        experts.append((make_w(g6, inter, hidden), make_w(0, inter, hidden), make_w(d6, hidden, inter), g6, 0, d6))
    yield ("moe", X, experts, ns)
