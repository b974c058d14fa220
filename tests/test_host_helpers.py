"""CPU checks of the kernels.h helpers that run on the host, as the
reference runs them (kernels.c:102-129, 584-720: per-head dots and norms, one
conv step, one embedding row), and of the host-memory write tracker behind the
weight registry.  No device calls."""
import ctypes as C
import os
import subprocess
import sys

import numpy as np

import roaster_amd as R
from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def rel(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / max(np.max(np.abs(b)), 1e-30))


def test_rmsnorm_l2norm_against_oracle_and_fp64():
    L = R.lib()
    for n in (128, 256, 2048, 3):
        x = R.synth_normal(3, R.synth_stream(0, 0, 5), n)
        w = (R.synth_normal(3, R.synth_stream(0, 1, 6), n, 0.1) + np.float32(1)).astype(np.float32)
        y = np.empty(n, np.float32)
        L.kernel_rmsnorm(y.ctypes.data, x.ctypes.data, w.ctypes.data, n, C.c_float(1e-6))
        ref = np.empty(n, np.float32)
        O.orc().orc_rmsnorm(ref.ctypes.data, x.ctypes.data, w.ctypes.data, n, C.c_float(1e-6))
        assert rel(y, ref) <= 1e-6
        x64 = x.astype(np.float64)
        assert rel(y, x64 / np.sqrt(np.mean(x64 ** 2) + 1e-6) * w) <= 2e-6
        L.kernel_l2norm(y.ctypes.data, x.ctypes.data, n, C.c_float(1e-6))
        assert rel(y, x64 / np.sqrt(np.sum(x64 ** 2) + 1e-6)) <= 2e-6


def test_dot_f32_matches_fp64():
    L = R.lib()
    for n in (0, 1, 15, 16, 17, 256, 1000, 4096):
        a = R.synth_normal(4, 1, max(n, 1))[:n].copy()
        b = R.synth_normal(4, 2, max(n, 1))[:n].copy()
        got = L.kernel_dot_f32(a.ctypes.data, b.ctypes.data, n)
        exact = float(a.astype(np.float64) @ b.astype(np.float64)) if n else 0.0
        bound = 1e-6 * n * float(np.max(np.abs(a), initial=0) * np.max(np.abs(b), initial=0)) + 1e-7
        assert abs(got - exact) <= bound, (n, got, exact)


def test_silu_sigmoid_closed_forms():
    L = R.lib()
    x = np.concatenate([R.synth_normal(5, 1, 1000) * 8, np.array([0, -0.0, 88, -88, 1e-30], np.float32)])
    x = x.astype(np.float32)
    s = x.copy()
    L.kernel_silu_array(s.ctypes.data, s.size)
    x64 = x.astype(np.float64)
    ref = x64 / (1 + np.exp(-x64))
    assert np.max(np.abs(s - ref) / np.maximum(np.abs(ref), 1e-30)) <= 1e-6
    assert abs(L.kernel_sigmoid(C.c_float(0.0)) - 0.5) == 0
    assert abs(L.kernel_silu(C.c_float(2.0)) - 2 / (1 + np.exp(-2))) <= 1e-6


def test_embedding_row_bit_exact_vs_oracle_dequant():
    L = R.lib()
    emb = R.synth_q4k(5, 1, 3 * 8)
    for tok in range(3):
        row = np.empty(2048, np.float32)
        L.kernel_embedding_row_q4_k(emb.ctypes.data, tok, row.ctypes.data, 2048)
        ref = np.empty(2048, np.float32)
        for k in range(8):
            blk = np.ascontiguousarray(emb[(8 * tok + k) * 144:(8 * tok + k + 1) * 144])
            O.orc().orc_dequant_q4k_block(blk.ctypes.data, ref[256 * k:].ctypes.data)
        np.testing.assert_array_equal(row, ref)
    bad = np.empty(300, np.float32)
    L.kernel_embedding_row_q4_k(emb.ctypes.data, 0, bad.ctypes.data, 300)
    assert np.all(np.isnan(bad))


def test_conv1d_causal_step():
    L = R.lib()
    Cn, K = 64, 4
    inp = R.synth_normal(6, 1, Cn)
    hist = R.synth_normal(6, 2, (K - 1) * Cn)
    ker = R.synth_normal(6, 3, Cn * K)
    out = np.empty(Cn, np.float32)
    L.kernel_conv1d_causal_f32(inp.ctypes.data, hist.ctypes.data, ker.ctypes.data, out.ctypes.data, Cn, K)
    full = np.concatenate([hist.reshape(K - 1, Cn), inp[None]], 0).astype(np.float64)   # [K][C]
    ref = np.einsum("kc,ck->c", full, ker.reshape(Cn, K).astype(np.float64))
    assert rel(out, ref) <= 1e-6


def test_write_tracking_probe_and_override():
    """The probe (wtrack.hip) must report pages written by a store, by a store
    to a never-touched page and by read(2) into a page, and nothing after its
    own scan re-protected them; ROASTER_WEIGHT_SYNC=copy switches it off, and
    so does roaster_weight_tracking(0)."""
    L = R.lib()
    avail = L.roaster_weight_tracking(-1)
    assert avail in (0, 1)
    if avail:
        assert L.roaster_weight_tracking(0) == 0
        assert L.roaster_weight_tracking(-1) == 0
        assert L.roaster_weight_tracking(1) == 1
    code = ("import ctypes;L=ctypes.CDLL(%r);print(L.roaster_weight_tracking(-1))" % R.LIB_PATH)
    out = subprocess.run([sys.executable, "-c", code], env=dict(os.environ, ROASTER_WEIGHT_SYNC="copy"),
                         capture_output=True, text=True, check=True).stdout.strip()
    assert out == "0"
