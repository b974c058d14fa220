"""GPU parity of the kernels.h entry points (host buffers in, host buffers out)
against the oracle, on the reference's own test cases (src/test_kernels.c)
and on config 1 / config 2 shapes.  Tolerance: the reference test's
max|d| / max|ref| <= 2e-4 (test_kernels.c:31, 43); the f32 decode paths are
held to 2e-5."""
import ctypes as C

import numpy as np
import pytest

import roaster_amd as R
from oracle import oracle as O
from gpu_util import alloc_w, log, rel_err
import tk_gen

pytestmark = pytest.mark.gpu


def test_cfg1_q4k_matvec():
    log("cfg1 q4k matvec")
    W = R.synth_q4k(0, R.synth_stream(0, 0, 0), 512 * 8)
    x = R.synth_normal(0, R.synth_stream(0, 0, 5), 2048)
    y = np.full(512, np.nan, np.float32)
    R.lib().kernel_matvec_q4_k(alloc_w(W), x.ctypes.data, y.ctypes.data, 512, 2048)
    ref = O.matvec(0, W, x, 512, 2048)
    assert rel_err(y, ref) <= 2e-5, rel_err(y, ref)


def test_q6k_matvec_and_dots():
    log("q6k matvec / dots")
    W = R.synth_q6k(0, R.synth_stream(0, 0, 2), 2048 * 2)
    e = R.synth_normal(0, R.synth_stream(0, 1, 5), 512)
    y = np.full(2048, np.nan, np.float32)
    Wp = alloc_w(W)
    R.lib().kernel_matvec_q6_k(Wp, e.ctypes.data, y.ctypes.data, 2048, 512)
    ref = O.matvec(1, W, e, 2048, 512)
    assert rel_err(y, ref) <= 2e-5
    d = R.lib().kernel_dot_q6_k(Wp, e.ctypes.data, 512)
    assert abs(d - ref[0]) <= 2e-5 * np.max(np.abs(ref))
    assert np.isnan(R.lib().kernel_dot_q4_k(Wp, e.ctypes.data, 300))   # partial blocks rejected


def test_matvec_batch_split_phase():
    log("matvec batch begin/end")
    x = R.synth_normal(2, 1, 2048)
    mats = [(0, R.synth_q4k(2, 10 + i, 37 * 8), 37) for i in range(3)] + [(1, R.synth_q6k(2, 20, 64 * 8), 64)]
    outs = [np.full(r, np.nan, np.float32) for _, _, r in mats]
    jobs = (R.KernelMatvecJob * len(mats))()
    for i, ((q6, W, rows), o) in enumerate(zip(mats, outs)):
        jobs[i] = R.KernelMatvecJob(q6, alloc_w(W), x.ctypes.data, o.ctypes.data, rows, 2048)
    assert R.lib().kernel_matvec_quant_begin(jobs, len(mats)) == 1
    R.lib().kernel_matvec_quant_end()
    for (q6, W, rows), o in zip(mats, outs):
        assert rel_err(o, O.matvec(q6, W, x, rows, 2048)) <= 2e-5


def test_reference_matmul_cases():
    """test_kernels.c:47-70: q4/q6 x rows {512, 2048, 37} x T {1..257}, then three
    jobs sharing X in one call."""
    for c in tk_gen.matmul_cases():
        if c[0] == "mm":
            _, q6, rows, cols, T, W, X = c
            log(f"matmul q{6 if q6 else 4} rows={rows} cols={cols} T={T}")
            Y = np.full((T, rows), np.nan, np.float32)
            if T == 1:
                Wp = alloc_w(W)
            j = R.KernelMatmulJob(q6, Wp, X.ctypes.data, Y.ctypes.data, rows, cols, T)
            assert R.lib().kernel_matmul_quant_batch(C.byref(j), 1) == 0
            ref = np.stack([O.matvec(q6, W, np.ascontiguousarray(X[t]), rows, cols) for t in range(T)])
            assert rel_err(Y, ref) <= 2e-4, (q6, rows, cols, T, rel_err(Y, ref))
        elif c[0] == "shared":
            _, X, jobs = c
            log("matmul shared-X jobs")
            arr = (R.KernelMatmulJob * 3)()
            Ys = []
            for i, (q6, rows, W) in enumerate(jobs):
                Ys.append(np.full((40, rows), np.nan, np.float32))
                arr[i] = R.KernelMatmulJob(q6, alloc_w(W), X.ctypes.data, Ys[i].ctypes.data, rows, 2048, 40)
            assert R.lib().kernel_matmul_quant_batch(arr, 3) == 0
            for (q6, rows, W), Y in zip(jobs, Ys):
                ref = np.stack([O.matvec(q6, W, np.ascontiguousarray(X[t]), rows, 2048) for t in range(40)])
                assert rel_err(Y, ref) <= 2e-4


def test_matmul_invalid_arguments():
    W = alloc_w(R.synth_q4k(0, 1, 8))
    X = np.zeros((1, 2048), np.float32)
    Y = np.zeros((1, 1), np.float32)
    bad = R.KernelMatmulJob(0, W, X.ctypes.data, Y.ctypes.data, 1, 2000, 1)   # cols % 256
    assert R.lib().kernel_matmul_quant_batch(C.byref(bad), 1) == -1
    assert R.lib().kernel_matmul_quant_batch(None, 1) == -1
    assert R.lib().kernel_matmul_quant_batch(C.byref(bad), 0) == 0


def test_reference_moe_prefill_case():
    """test_kernels.c:72-92: 6 experts, n = {5, 1, 0, 17, 9, 30}, mixed q4/q6."""
    log("moe prefill 6 experts")
    for c in tk_gen.matmul_cases():
        if c[0] != "moe":
            continue
        _, X, experts, ns = c
        arr = (R.KernelMoeExpert * 6)()
        grp = (O.OrcMoeGroup * 6)()
        for i, (g, u, d, g6, u6, d6) in enumerate(experts):
            arr[i] = R.KernelMoeExpert(alloc_w(g), alloc_w(u), alloc_w(d), g6, u6, d6, ns[i])
            grp[i] = O.OrcMoeGroup(g.ctypes.data, u.ctypes.data, d.ctypes.data, g6, u6, d6, ns[i])
        D = np.full((sum(ns), 2048), np.nan, np.float32)
        assert R.lib().kernel_moe_prefill(arr, 6, X.ctypes.data, D.ctypes.data, 512, 2048) == 0
        ref = np.zeros_like(D)
        O.orc().orc_moe_groups(grp, 6, X.ctypes.data, ref.ctypes.data, 512, 2048)
        assert rel_err(D, ref) <= 2e-4, rel_err(D, ref)
        # invalid arguments
        assert R.lib().kernel_moe_prefill(arr, 6, X.ctypes.data, D.ctypes.data, 500, 2048) == -1


def test_ffn_fused_nine_experts():
    """kernel_ffn_fused for the 8 routed + shared experts of config 2 (model.c:1095-1103)."""
    log("ffn_fused 9 experts")
    desc = R.table_desc()
    x = R.synth_normal(1, R.synth_stream(0, 0, 5), 2048)
    ids = [6, 119, 104, 200, 49, 247, 216, 123, 256]
    mats = [R.host_expert(1, 0, e, desc) for e in ids]
    outs = [np.full(2048, np.nan, np.float32) for _ in ids]
    fx = (R.KernelFfnExpert * 9)()
    for i, ((g, u, d), o) in enumerate(zip(mats, outs)):
        fx[i] = R.KernelFfnExpert(alloc_w(g), alloc_w(u), alloc_w(d), 0, 0, 1, o.ctypes.data)
    assert R.lib().kernel_ffn_fused(fx, 9, x.ctypes.data, 512, 2048) == 1
    for (g, u, d), o in zip(mats, outs):
        ref = np.empty(2048, np.float32)
        ex = O.OrcExpert(g.ctypes.data, u.ctypes.data, d.ctypes.data, 0, 0, 1)
        O.orc().orc_expert_decode(C.byref(ex), x.ctypes.data, 512, 2048, ref.ctypes.data)
        assert rel_err(o, ref) <= 2e-5, rel_err(o, ref)
    assert R.lib().kernel_ffn_fused(fx, 10, x.ctypes.data, 512, 2048) == 0     # n <= 9
    assert R.lib().kernel_ffn_fused(fx, 9, x.ctypes.data, 500, 2048) == 0      # multiples of 256


def test_router_matvec_f32():
    """kernel_matvec_f32 (the router product, kernels.c:131-148) on the GPU."""
    log("matvec_f32")
    x = R.synth_normal(3, R.synth_stream(0, 0, 5), 2048)
    Wf = R.synth_normal(4, 3, 64 * 2048).reshape(64, 2048)
    yy = np.empty(64, np.float32)
    R.lib().kernel_matvec_f32(Wf.ctypes.data, x.ctypes.data, yy.ctypes.data, 64, 2048)
    assert rel_err(yy, O.matvec_f32(Wf, x)) <= 1e-5
    Wr = R.synth_normal(1, 9, 256 * 2048, 0.02).reshape(256, 2048)
    yr = np.empty(256, np.float32)
    R.lib().kernel_matvec_f32(Wr.ctypes.data, x.ctypes.data, yr.ctypes.data, 256, 2048)
    assert rel_err(yr, O.matvec_f32(Wr, x)) <= 1e-5
