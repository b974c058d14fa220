"""Dense quantised projections on device buffers (roaster_matvec_q) against the
oracle's matvec (kernels.c:407-432, 553-578): Q4_K / Q6_K, widths of 1..8
super-blocks (3, 5, 6, 7 included: row lane groups rounded up to a power of
two) and 9..16 super-blocks (two per lane: the attention output and
DeltaNet ssm_out projections are [2048 x 4096], model.c:862, 1344-1347), 1..8
tokens, ragged row counts, the MFMA route for several tokens switched off
and on (roaster_dense_mfma_min_tokens), and an LM-head-sized Q6_K matrix
[248320 x 2048] checked on sampled rows.  Tolerance: max|d|/max|y| <= 2e-5
(fp32 accumulation in another order; the reference test allows 2e-4).
Two or more tokens run with the quants as MFMA operands; small matrices and
large ones take its two work splits."""
import ctypes as C

import numpy as np
import pytest

import roaster_amd as R
from gpu_util import Dev, log, rel_err
from oracle import oracle as O

pytestmark = pytest.mark.gpu
TOL = 2e-5


def weights(q6, rows, cols, seed):
    nb = rows * (cols // 256)
    return R.synth_q6k(seed, R.synth_stream(0, 0, 9), nb) if q6 else R.synth_q4k(seed, R.synth_stream(0, 0, 9), nb)


def run(q6, W, X, rows, cols):
    T = X.shape[0]
    dw, dx = Dev(W), Dev(X)
    dy = Dev(nbytes=T * rows * 4, shape=(T, rows))
    R.check(R.lib().roaster_matvec_q(dw.p, int(q6), dx.p, dy.p, rows, cols, T), "matvec_q")
    R.check(R.lib().roaster_sync(), "sync")
    return dy.get()


@pytest.mark.parametrize("q6", [0, 1])
@pytest.mark.parametrize("cols", [256, 512, 768, 1280, 1536, 2048, 2304, 3328, 4096])
@pytest.mark.parametrize("T", [1, 3, 8])
def test_dense_matvec(q6, cols, T):
    rows = 1001
    log(f"dense matvec q6={q6} rows={rows} cols={cols} T={T}")
    W = weights(q6, rows, cols, 40 + cols + T)
    X = np.stack([R.synth_normal(41, R.synth_stream(t, cols, 5), cols) for t in range(T)])
    Y = run(q6, W, X, rows, cols)
    for t in range(T):
        err = rel_err(Y[t], O.matvec(q6, W, X[t], rows, cols))
        assert err <= TOL, (t, err)


def test_dense_matvec_invalid():
    dw, dx, dy = Dev(nbytes=256), Dev(nbytes=256), Dev(nbytes=256)
    L = R.lib()
    assert L.roaster_matvec_q(dw.p, 1, dx.p, dy.p, 4, 300, 1) == R.EINVAL     # cols not a multiple of 256
    assert L.roaster_matvec_q(dw.p, 1, dx.p, dy.p, 4, 4352, 1) == R.EINVAL    # cols > 4096
    assert L.roaster_matvec_q(dw.p, 1, dx.p, dy.p, 4, 256, 9) == R.EINVAL     # T > 8


@pytest.mark.parametrize("q6", [0, 1])
@pytest.mark.parametrize("cols", [2048, 4096])
def test_dense_mfma_route(q6, cols):
    """8 tokens with the MFMA route switched off (threshold 9: the
    dequantising matvec) and on (threshold 2, the default), rows a multiple
    of 16 and 7 rows short of one."""
    L = R.lib()
    old = L.roaster_dense_mfma_min_tokens(0)
    try:
        for thr in (9, 2):
            L.roaster_dense_mfma_min_tokens(thr)
            for rows in (1024, 1017):
                W = weights(q6, rows, cols, 60 + cols)
                X = np.stack([R.synth_normal(61, R.synth_stream(t, cols, 5), cols) for t in range(8)])
                Y = run(q6, W, X, rows, cols)
                for t in range(8):
                    err = rel_err(Y[t], O.matvec(q6, W, X[t], rows, cols))
                    assert err <= TOL, (thr, rows, t, err)
    finally:
        L.roaster_dense_mfma_min_tokens(old)


@pytest.mark.parametrize("q6", [0, 1])
def test_kernels_h_matvec_odd_block_count(q6):
    """kernel_matvec_q*_k with 3 super-blocks per row (the lane group is rounded
    up to 32 lanes; 24 would mix rows)."""
    rows, cols = 517, 768
    W = weights(q6, rows, cols, 77)
    x = R.synth_normal(78, R.synth_stream(0, 1, 5), cols)
    y = np.zeros(rows, np.float32)
    fn = R.lib().kernel_matvec_q6_k if q6 else R.lib().kernel_matvec_q4_k
    fn(W.ctypes.data, x.ctypes.data, y.ctypes.data, rows, cols)
    assert rel_err(y, O.matvec(q6, W, x, rows, cols)) <= TOL


@pytest.mark.parametrize("q6,rows,cols,T", [(1, 40009, 4096, 8), (0, 65543, 2048, 3)])
def test_dense_mfma_many_groups(q6, rows, cols, T):
    """Matrices with more 16-row groups than the grid has waves: the
    wave-strided mode of the multi-token MFMA kernel (smaller matrices split
    a group's super-blocks over a workgroup's waves), checked on sampled
    rows for every token."""
    log(f"dense MFMA, many groups: q6={q6} rows={rows} cols={cols} T={T}")
    W = weights(q6, rows, cols, 70 + T)
    X = np.stack([R.synth_normal(71, R.synth_stream(t, cols, 5), cols) for t in range(T)])
    Y = run(q6, W, X, rows, cols)
    pick = np.sort(np.random.default_rng(7).choice(rows, 1500, replace=False))
    pick[-1] = rows - 1
    Wr = np.ascontiguousarray(W.reshape(rows, -1)[pick].reshape(-1))
    for t in range(T):
        err = rel_err(Y[t][pick], O.matvec(q6, Wr, X[t], len(pick), cols))
        assert err <= TOL, (t, err)


def test_lm_head_q6k_sampled_rows():
    rows, cols = 248320, 2048
    log(f"LM head Q6_K {rows} x {cols} ({rows * 8 * 210 / 1e6:.0f} MB)")
    W = weights(1, rows, cols, 99)
    x = R.synth_normal(98, R.synth_stream(0, 2, 5), cols)
    y = run(1, W, x[None, :], rows, cols)[0]
    pick = np.random.default_rng(5).choice(rows, 2000, replace=False)
    pick.sort()
    Wr = W.reshape(rows, -1)[pick].reshape(-1)
    err = rel_err(y[pick], O.matvec(1, np.ascontiguousarray(Wr), x, len(pick), cols))
    log(f"LM head sampled rows: max|d|/max|y| = {err:.3e}")
    assert err <= TOL
