"""GPU parity of roaster_moe_prefill (the MoE block over T tokens,
model.c:1671-1791) against the oracle.

Bars: top-8 ids bit-exact given identical router logits (the oracle is fed the
GPU's biased logits); expert counts equal the histogram of the ids; FFN
outputs within max|d| / max|y| <= 2e-3 in the default fp16-operand mode, and
<= 2e-4 in the bf16x3 split mode.  The all-Q6_K 2048-token case is checked
on every token of its first layer (the oracle's grouped products run on a
thread pool, one expert group or 128-token chunk of the shared expert per
task) and on a token sample of the other three; a token's output depends on
its own input and logits alone (model.c computes every (token, expert) row
independently), which the permutation tests check bit for bit on the GPU,
at T = 300 on the Q4_K / Q6_K table and at T = 2048 on the all-Q6_K one.
The fp16 mode keeps each (token, expert) down row in fp16 scaled by a power
of two of its bound; a table whose down products reach ~1e7 checks that
scaling against the oracle.
"""
import ctypes as C
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import roaster_amd as R
from oracle import oracle as O
from gpu_util import Dev, SynthTable, bf16_round, log, prefill, rel_err, zipf_bias

pytestmark = pytest.mark.gpu

TOL = 2e-3
TOL_SPLIT = 2e-4


def tokens(seed, T, H=2048, start=0):
    return bf16_round(np.stack([R.synth_normal(seed, R.synth_stream(0, start + t, 5), H) for t in range(T)]))


def check_routing(lg, ids, w, counts, E):
    for t in range(lg.shape[0]):
        ids_ref, w_ref = O.select_top8(np.ascontiguousarray(lg[t]))
        assert ids[t].tolist() == ids_ref.tolist(), t
        np.testing.assert_allclose(w[t], w_ref, rtol=1e-6, atol=1e-7)
    assert np.array_equal(counts, np.bincount(ids[ids >= 0].ravel(), minlength=E))


@pytest.fixture(scope="module")
def cfg3():
    log("building config-3 table (seed 2)")
    t = SynthTable(2)
    yield t
    t.destroy()


@pytest.fixture(scope="module")
def cfg3_oracle(cfg3):
    return cfg3.oracle_layer(0)


@pytest.fixture(scope="module")
def q6tab():
    log("building the all-Q6_K table (seed 4)")
    t = SynthTable(4, n_layers=1, q6=(1, 1, 1), sh_q6=(1, 1, 1))
    yield t
    t.destroy()


def test_prefill_config3_zipf(cfg3, cfg3_oracle):
    """T = 512, Zipf-biased routing (expert lists 0 .. ~200 rows), F16 operands."""
    T = 512
    X = tokens(2, T)
    b = zipf_bias(256, 2)
    Y, lg, ids, w, counts = prefill(cfg3, X, bias=b)
    log(f"config 3: expert rows max {counts.max()}, empty experts {(counts == 0).sum()}")
    router, _ = cfg3.router(0)
    lg_ref = X @ router.T.astype(np.float64)
    assert rel_err(lg - b, lg_ref) <= 1e-5
    check_routing(lg, ids, w, counts, 256)
    assert counts.max() >= 100 and (counts == 0).sum() >= 1      # the skew the workload asks for
    rc, Y_ref, ids_ref, _, _ = cfg3_oracle.prefill(X, logits_in=lg)
    assert rc == 0 and np.array_equal(ids_ref, ids)
    err = rel_err(Y, Y_ref)
    log(f"config 3 (f16 operands): max|d|/max|y| = {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("prec,tol", [(R.PREC_SPLIT, TOL_SPLIT), (R.PREC_BF16, None)])
def test_prefill_precision_modes(cfg3, cfg3_oracle, prec, tol):
    T = 192
    X = tokens(2, T, start=1000)
    Y, lg, ids, w, counts = prefill(cfg3, X, precision=prec)
    check_routing(lg, ids, w, counts, 256)
    rc, Y_ref, _, _, _ = cfg3_oracle.prefill(X, logits_in=lg)
    assert rc == 0
    err = rel_err(Y, Y_ref)
    log(f"precision {prec}: max|d|/max|y| = {err:.3e}")
    if tol is not None:
        assert err <= tol
    else:
        assert err <= 2e-2          # bf16 operands: about 8 significant bits, reported only


@pytest.mark.parametrize("T", [1, 3, 64, 65, 130])
def test_prefill_ragged_given_logits(cfg3, cfg3_oracle, T):
    """Token counts that are not tile multiples, experts with one row, ties and
    NaN / -inf logits (given directly, as the all-Q6_K workload does)."""
    X = tokens(7, T, start=2000)
    lg_in = np.stack([R.synth_normal(8, R.synth_stream(0, t, 7), 256) for t in range(T)])
    lg_in[0, [3, 4, 200]] = 5.0                      # three-way tie at the top
    if T > 1:
        lg_in[1, :] = 0.0                            # all equal: ids 0..7
        lg_in[1, 9] = -0.0                           # -0 ties +0
    if T > 2:
        lg_in[2, :10] = np.nan
        lg_in[2, 10:20] = -np.inf
    Y, lg, ids, w, counts = prefill(cfg3, X, logits_in=lg_in)
    np.testing.assert_array_equal(lg, lg_in)
    check_routing(lg, ids, w, counts, 256)
    rc, Y_ref, _, _, _ = cfg3_oracle.prefill(X, logits_in=lg_in)
    assert rc == 0
    assert rel_err(Y, Y_ref) <= TOL
    for t in range(T):                               # every token, not just the largest outputs
        assert rel_err(Y[t], Y_ref[t]) <= 4 * TOL, t


@pytest.mark.parametrize("levels", [2, 5, 40])
def test_prefill_topk_tie_stress(cfg3, levels):
    """Logits drawn from a few values, so most tokens have ties at the 8th
    slot (and some at every slot): ids bit-exact against the oracle for every
    token, including rows with exactly 8 and with 9 finite logits, and rows
    mixing -0 / +0."""
    T = 192
    rng = np.random.default_rng(100 + levels)
    lg = (rng.integers(0, levels, size=(T, 256)) * 0.25 - 1.0).astype(np.float32)
    lg[0, :] = -np.inf
    lg[0, rng.choice(256, 8, replace=False)] = 0.5            # exactly 8 selectable
    lg[1, :] = np.nan
    lg[1, rng.choice(256, 9, replace=False)] = -2.0           # 9 selectable, all tied
    lg[2, ::2] = -0.0
    lg[2, 1::2] = 0.0                                         # -0 and +0 tie
    lg[3, :] = rng.standard_normal(256).astype(np.float32)    # distinct values
    X = tokens(9, T, start=3000)
    Y, lg_out, ids, w, counts = prefill(cfg3, X, logits_in=lg)
    np.testing.assert_array_equal(lg_out, lg)
    check_routing(lg, ids, w, counts, 256)


def test_prefill_token_permutation_bit_exact(cfg3):
    """A token's output does not depend on which tile or slot it lands in."""
    T = 300
    X = tokens(9, T, start=3000)
    Y, lg, ids, _, _ = prefill(cfg3, X)
    perm = np.random.default_rng(9).permutation(T)
    Yp, lgp, idsp, _, _ = prefill(cfg3, np.ascontiguousarray(X[perm]))
    np.testing.assert_array_equal(idsp, ids[perm])
    np.testing.assert_array_equal(lgp, lg[perm])
    np.testing.assert_array_equal(Yp, Y[perm])


@pytest.mark.parametrize("T", [512, 37])
def test_prefill_balanced_down_bit_exact(cfg3, T):
    """The down GEMM on one workgroup per CU over an even split of its output
    tiles gives the bits of the grid with one workgroup per four tiles
    (Zipf routing: tiles of 1..96 rows; T = 37: fewer output tiles than CUs)."""
    X = tokens(12, T, start=5000)
    b = zipf_bias(256, 2)
    lib = R.lib()
    assert lib.roaster_prefill_balanced_down(-1) == 1
    Y1, _, ids1, _, _ = prefill(cfg3, X, bias=b)
    try:
        assert lib.roaster_prefill_balanced_down(0) == 0
        Y0, _, ids0, _, _ = prefill(cfg3, X, bias=b)
    finally:
        lib.roaster_prefill_balanced_down(1)
    np.testing.assert_array_equal(ids0, ids1)
    np.testing.assert_array_equal(Y0, Y1)


@pytest.mark.parametrize("which,T", [("cfg3", 512), ("cfg3", 37), ("q6", 2048)])
def test_prefill_persistent_gate_up_bit_exact(request, which, T):
    """The gate/up GEMM on its persistent grid (work counters, the next unit
    prepared during the current one) gives the bits of one workgroup per
    unit: Zipf routing on the Q4_K table (tiles of 1..96 rows; T = 37: fewer
    units than CUs) and the all-Q6_K table at 2048 tokens."""
    tab = request.getfixturevalue("cfg3" if which == "cfg3" else "q6tab")
    X = tokens(14, T, start=7000)
    b = zipf_bias(256, 2) if which == "cfg3" else None
    lib = R.lib()
    assert lib.roaster_prefill_persistent_gate_up(-1) == 1
    Y1, _, ids1, _, _ = prefill(tab, X, bias=b)
    try:
        assert lib.roaster_prefill_persistent_gate_up(0) == 0
        Y0, _, ids0, _, _ = prefill(tab, X, bias=b)
    finally:
        lib.roaster_prefill_persistent_gate_up(1)
    np.testing.assert_array_equal(ids0, ids1)
    np.testing.assert_array_equal(Y0, Y1)


@pytest.mark.parametrize("which,T", [("cfg3", 512), ("cfg3", 37), ("cfg3", 3), ("cfg3", 1), ("q6", 2048), ("q6", 300)])
def test_prefill_fused_gemm_bit_exact(request, which, T):
    """Both GEMMs in one persistent kernel (each XCD's workgroups take its
    tiles' gate/up units, then their down chunks once a tile's units are all
    counted) gives the bits of the two-kernel path: Zipf routing on the Q4_K
    table (T = 37, 3, 1: XCDs with one tile or none) and the all-Q6_K table,
    twice in a row (the counters are re-zeroed by each call's plan kernel);
    no tile wait gives up (the call reports no error)."""
    tab = request.getfixturevalue("cfg3" if which == "cfg3" else "q6tab")
    X = tokens(15, T, start=9000)
    b = zipf_bias(256, 2) if which == "cfg3" else None
    lib = R.lib()
    assert lib.roaster_prefill_fused_gemm(-1) == 0
    Y0, _, ids0, _, _ = prefill(tab, X, bias=b)
    try:
        assert lib.roaster_prefill_fused_gemm(1) == 1
        Y1, _, ids1, _, _ = prefill(tab, X, bias=b)
        Y2, _, _, _, _ = prefill(tab, X, bias=b)
        R.check(lib.roaster_sync(), "sync after the fused calls")
    finally:
        lib.roaster_prefill_fused_gemm(0)
    np.testing.assert_array_equal(ids0, ids1)
    np.testing.assert_array_equal(Y0, Y1)
    np.testing.assert_array_equal(Y0, Y2)


def test_prefill_fp16_products_scaled_by_their_bound():
    """Down products far outside the fp16 range: expert 3's down matrix with
    every Q6_K block's d scaled by 2^12 and activations 8x larger, so that its
    per-(token, expert) rows reach ~1e7 (fp16 ends at 65504).  The fp16 mode
    stores each row scaled by a power of two of its bound (max activation
    times the table's bound on the down rows' L1 norm, rebuilt by
    roaster_table_set_expert), so every output stays finite and within the
    bar against the oracle."""
    E, T = 16, 64
    t = SynthTable(31, n_experts=E)
    try:
        g, u, d = t.expert(0, 3)
        blk = d.copy().reshape(-1, 210)
        dd = blk[:, 208:210].copy().view(np.float16).astype(np.float32) * 4096.0
        blk[:, 208:210] = dd.astype(np.float16).view(np.uint8).reshape(-1, 2)
        d = np.ascontiguousarray(blk.ravel())
        R.check(R.lib().roaster_table_set_expert(t.t, 0, 3, g.ctypes.data, u.ctypes.data, d.ctypes.data), "set_expert")
        t._experts[(0, 3)] = (g, u, d)
        X = (tokens(32, T) * 8.0).astype(np.float32)
        lg_in = np.stack([R.synth_normal(33, R.synth_stream(0, i, 7), E) for i in range(T)])
        lg_in[:, 3] = 2.0                            # expert 3 in every token's top 8
        Y, lg, ids, w, counts = prefill(t, X, logits_in=lg_in)
        assert (ids == 3).any(axis=1).all()
        assert np.isfinite(Y).all()
        rc, Y_ref, _, _, _ = t.oracle_layer(0).prefill(X, logits_in=lg_in)
        assert rc == 0
        err = rel_err(Y, Y_ref)
        log(f"large down products: max|y| = {np.abs(Y_ref).max():.3e}, max|d|/max|y| = {err:.3e}")
        assert np.abs(Y_ref).max() > 1e6
        assert err <= TOL
    finally:
        t.destroy()


def test_prefill_reports_routing_failure(cfg3, cfg3_oracle):
    T = 70
    X = tokens(10, T, start=4000)
    lg_in = np.stack([R.synth_normal(11, R.synth_stream(0, t, 7), 256) for t in range(T)])
    lg_in[5, :] = -np.inf
    lg_in[5, :3] = 1.0                               # only 3 routable experts
    dY = Dev(nbytes=T * 2048 * 4, shape=(T, 2048))
    dX = Dev(X)
    dL = Dev(lg_in)
    o = R.RoasterPrefillOpts(R.PREC_F16, dL.p, None, None, None, None, None)
    R.check(R.lib().roaster_moe_prefill(cfg3.t, 0, dX.p, T, dY.p, C.byref(o)))
    assert R.lib().roaster_sync() == R.EROUTE
    assert R.lib().roaster_sync() == 0
    Y = dY.get()
    ok = [t for t in range(T) if t != 5]
    rc, Y_ref, _, _, _ = cfg3_oracle.prefill(np.ascontiguousarray(X[ok]), logits_in=np.ascontiguousarray(lg_in[ok]))
    assert rc == 0
    assert rel_err(Y[ok], Y_ref) <= TOL


def test_prefill_all_q6k_2048_tokens_4_layers():
    """All-Q6_K experts, T = 2048, uniform N(0,1) logits given directly, 4 layers."""
    T, NL = 2048, 4
    tab = SynthTable(4, n_layers=NL, q6=(1, 1, 1), sh_q6=(1, 1, 1))
    try:
        rng = np.random.default_rng(4)
        sample = np.sort(rng.choice(T, 24, replace=False))
        for layer in range(NL):
            X = tokens(4, T, start=10000 * layer)
            lg_in = np.stack([R.synth_normal(4, R.synth_stream(layer, t, 7), 256) for t in range(T)])
            Y, lg, ids, w, counts = prefill(tab, X, layer=layer, logits_in=lg_in)
            check_routing(lg, ids, w, counts, 256)
            assert counts.sum() == 8 * T
            L = tab.oracle_layer(layer, set(ids[sample].ravel().tolist()))
            rc, Y_ref, _, _, _ = L.prefill(np.ascontiguousarray(X[sample]), logits_in=np.ascontiguousarray(lg_in[sample]))
            assert rc == 0
            err = rel_err(Y[sample], Y_ref)
            log(f"all-Q6_K layer {layer}: rows/expert {counts.min()}..{counts.max()}, sample max|d|/max|y| = {err:.3e}")
            assert err <= TOL
    finally:
        tab.destroy()


def oracle_prefill_all_tokens(tab, layer, X, ids, w):
    """The oracle's MoE block for every token with the given routing (ids, w
    [T x 8]: the oracle's select_top8 of the logits, equal to the GPU's ids): the
    reference's grouped products (orc_moe_groups: per expert its tokens in
    ascending order, model.c:1713-1771; the shared expert over all tokens,
    1694-1711) as independent tasks on a thread pool, then the combine in
    the reference order -- sigmoid(gate_inp . x) times the shared row, then
    each expert's weighted row in ascending expert id (1707-1711, 1776-1788)."""
    T, H = X.shape
    I, E = tab.desc.inter, tab.desc.n_experts
    X = np.ascontiguousarray(X, np.float32)
    groups = []
    for e in range(E):
        rows = np.nonzero((ids == e).any(axis=1))[0]
        if len(rows):
            groups.append((e, rows))
    shared = tab.expert(layer, E)
    chunks = [np.arange(a, min(a + 128, T)) for a in range(0, T, 128)]
    tasks = [(tab.expert(layer, e), rows, tuple(tab.desc.q6)) for e, rows in groups] + \
            [(shared, rows, tuple(tab.desc.sh_q6)) for rows in chunks]

    def run(task):
        (g, u, d), rows, q6 = task
        Xg = np.ascontiguousarray(X[rows])
        Dg = np.empty((len(rows), H), np.float32)
        grp = (O.OrcMoeGroup * 1)()
        grp[0] = O.OrcMoeGroup(g.ctypes.data, u.ctypes.data, d.ctypes.data, q6[0], q6[1], q6[2], len(rows))
        O.orc().orc_moe_groups(grp, 1, Xg.ctypes.data, Dg.ctypes.data, I, H)
        return Dg

    with ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1)) as pool:
        outs = list(pool.map(run, tasks))
    _, gate_inp = tab.router(layer)
    Y = np.empty((T, H), np.float32)
    sd = np.concatenate(outs[len(groups):])
    for t in range(T):
        raw = O.orc().orc_dot_f32(gate_inp.ctypes.data, X[t].ctypes.data, H)
        Y[t] = np.float32(1.0 / (1.0 + np.exp(-np.float32(raw)))) * sd[t]
    for (e, rows), D in zip(groups, outs):
        k = np.argmax(ids[rows] == e, axis=1)
        Y[rows] = Y[rows] + w[rows, k][:, None].astype(np.float32) * D
    return Y


def test_prefill_all_q6k_2048_every_token():
    """The all-Q6_K 2048-token layer (config 5's first layer, seed 4) checked
    on all 2048 tokens against the oracle's grouped products, and its outputs
    invariant, bit for bit, under a permutation of the tokens."""
    T = 2048
    tab = SynthTable(4, n_layers=1, q6=(1, 1, 1), sh_q6=(1, 1, 1))
    try:
        X = tokens(4, T, start=0)
        lg_in = np.stack([R.synth_normal(4, R.synth_stream(0, t, 7), 256) for t in range(T)])
        Y, lg, ids, w, counts = prefill(tab, X, layer=0, logits_in=lg_in)
        check_routing(lg, ids, w, counts, 256)
        w_ref = np.stack([O.select_top8(np.ascontiguousarray(lg_in[t]))[1] for t in range(T)])
        Y_ref = oracle_prefill_all_tokens(tab, 0, X, ids, w_ref)
        err = rel_err(Y, Y_ref)
        per_tok = np.max(np.abs(Y.astype(np.float64) - Y_ref), axis=1) / np.max(np.abs(Y_ref))
        log(f"all-Q6_K 2048 tokens, every token: max|d|/max|y| = {err:.3e} "
            f"(worst token {int(np.argmax(per_tok))}), rows/expert {counts.min()}..{counts.max()}")
        assert err <= TOL
        perm = np.random.default_rng(44).permutation(T)
        Yp, _, idsp, _, _ = prefill(tab, np.ascontiguousarray(X[perm]), layer=0,
                                    logits_in=np.ascontiguousarray(lg_in[perm]))
        np.testing.assert_array_equal(idsp, ids[perm])
        np.testing.assert_array_equal(Yp.view(np.uint32), Y[perm].view(np.uint32))
    finally:
        tab.destroy()


@pytest.mark.parametrize("E,H,I", [(64, 1024, 256), (64, 2048, 256), (32, 1536, 1024)])
def test_prefill_other_shapes(E, H, I):
    """Shapes beside the model's: inter 256 (the down GEMM's one-K-step
    tile ranges, four part maxima per row) at hidden 1024 (four output tiles
    per tile; the gate/up GEMM one workgroup per unit) and 2048 (the
    persistent gate/up grid, two units per tile), and inter 1024 at hidden
    1536 (the down GEMM's per-tile grid over four K steps).  fp16 mode
    against the oracle at the prefill bar, and the down GEMM's balanced
    split, its per-tile grid and the one-kernel GEMMs bit for bit against
    each other where they apply."""
    T = 150
    tab = SynthTable(41, n_experts=E, hidden=H, inter=I)
    lib = R.lib()
    try:
        X = tokens(16, T, H=H, start=500)
        lg_in = np.stack([R.synth_normal(17, R.synth_stream(0, t, 7), E) for t in range(T)]).astype(np.float32)
        Y, lg, ids, w, counts = prefill(tab, X, logits_in=lg_in)
        rc, Y_ref, ids_ref, _, _ = tab.oracle_layer(0).prefill(X, logits_in=lg_in)
        assert rc == 0 and np.array_equal(ids_ref, ids)
        err = rel_err(Y, Y_ref)
        log(f"prefill E {E} hidden {H} inter {I}: max|d|/max|y| = {err:.3e}")
        assert err <= TOL
        try:
            assert lib.roaster_prefill_balanced_down(0) == 0
            Y0, _, _, _, _ = prefill(tab, X, logits_in=lg_in)
        finally:
            lib.roaster_prefill_balanced_down(1)
        np.testing.assert_array_equal(Y0, Y)
        try:
            assert lib.roaster_prefill_fused_gemm(1) == 1
            Y1, _, _, _, _ = prefill(tab, X, logits_in=lg_in)
        finally:
            lib.roaster_prefill_fused_gemm(0)
        np.testing.assert_array_equal(Y1, Y)
    finally:
        tab.destroy()
