"""One launch per decode stack call for one token against the three-kernel path
(roaster_decode_fused_layer(0)) and the oracle.

Two one-launch kernels take one token.  dec_stack1r_kernel (mode 1, the
default, 256 experts / hidden 2048 / inter 512) folds the router into the
combine: its logits and 1/rms are sums of per-workgroup partials, so they
differ from the three-kernel path's in summation order only; its ids must be
equal, and hidden states, logits and routing weights within 1e-5 (the
non-router arithmetic is the same: with given logits and no norm its results
are equal bit for bit).  dec_stack1_kernel (mode 2, and mode 1 for the other
shapes) computes every dot, reduction, softmax and combine with the
three-kernel path's arithmetic, so its results must be equal bit for bit.
Both are held to the oracle bars of the decode tests (ids exact,
max|d|/max|ffn| <= 2e-3 and the 1e-4 regression bound).  Cases: the
256-expert shapes over 4 stacked layers with norm weights; hidden 768 /
inter 256 / 64 experts and hidden 1024 / inter 1024 / 32 experts (other lane
layouts and task counts); per-layer matrix types (Q6_K gate/up, Q4_K down);
given logits with ties; fewer than 8 routable experts; a wait that gives up
(spin limit forced to 1 poll from the host, so every kernel still ends)
reported as ROASTER_EDEVICE, then normal results again, and a stack call
that gives up leaving the caller's h as it was (every one-launch kernel);
cooperative launches giving the same results.""" 
import ctypes as C

import numpy as np
import pytest

import roaster_amd as R
from gpu_util import Dev, SynthTable, log, rel_err
from test_gpu_decode import oracle_stack, decode

pytestmark = pytest.mark.gpu

EPS = C.c_float(1e-6)


def _stack(t, h0, NL, nw=None, noalloc=False):
    B = h0.shape[0]
    dh = Dev(h0)
    dn = Dev(nw) if nw is not None else None
    di = Dev(nbytes=NL * B * 8 * 4, dtype=np.int32, shape=(NL, B, 8))
    dw = Dev(nbytes=NL * B * 8 * 4, shape=(NL, B, 8))
    f = R.lib().roaster_moe_decode_stack_noalloc if noalloc else R.lib().roaster_moe_decode_stack
    R.check(f(t.t, dh.p, B, 0, NL, dn.p if dn else None, EPS, di.p, dw.p), "stack")
    R.check(R.lib().roaster_sync(), "sync")
    return dh.get(), di.get(), dw.get()


R1_SHAPE = (256, 2048, 512)                 # the shapes dec_stack1r_kernel takes


def _in_mode(m, fn):
    """fn() with roaster_decode_fused_layer(m), then the default (1) again."""
    L = R.lib()
    assert L.roaster_decode_fused_layer(-1) == 1
    L.roaster_decode_fused_layer(m)
    try:
        return fn()
    finally:
        L.roaster_decode_fused_layer(1)


def _both(fn):
    """fn() with the one-launch layer, then with three kernels per layer."""
    return fn(), _in_mode(0, fn)


def _modes(fn):
    """fn() with the default one-launch kernel, the bit-compatible one-launch
    kernel and three kernels per layer."""
    return fn(), _in_mode(2, fn), _in_mode(0, fn)


def _same(a, b):
    for x, y in zip(a, b):
        assert x.dtype == y.dtype and x.shape == y.shape
        assert np.array_equal(np.ascontiguousarray(x).view(np.uint32), np.ascontiguousarray(y).view(np.uint32))


def _near(a, b, ref=None, tol=1e-5):
    """Integer arrays equal; float arrays within tol of b relative to max|b|
    (max|b - ref| when ref, the input, is given for the first array)."""
    for i, (x, y) in enumerate(zip(a, b)):
        assert x.dtype == y.dtype and x.shape == y.shape
        if x.dtype.kind in "iu":
            assert np.array_equal(x, y)
        else:
            base = ref if (ref is not None and i == 0) else 0.0
            assert rel_err(x - base, y - base) <= tol, (i, rel_err(x - base, y - base))


@pytest.mark.parametrize("shape", [(256, 2048, 512), (64, 768, 256), (32, 1024, 1024)])
def test_layer1_matches_three_kernels_and_oracle(shape):
    E, H, I = shape
    NL = 4 if E == 256 else 2
    log(f"one-launch layer vs three kernels: E={E} H={H} I={I}, {NL} layers")
    t = SynthTable(21, n_layers=NL, n_experts=E, hidden=H, inter=I)
    try:
        h0 = R.synth_normal(21, R.synth_stream(0, 0, 5), H)[None, :]
        nw = np.stack([1.0 + 0.25 * R.synth_normal(22, R.synth_stream(l, 0, 6), H) for l in range(NL)]).astype(np.float32)
        a, a2, b = _modes(lambda: _stack(t, h0, NL, nw))
        _same(a2, b)
        if shape == R1_SHAPE:
            _near(a, b, ref=h0)
        else:
            _same(a, b)
        h_ref, ids_ref = oracle_stack(t, h0, NL, norm_w=nw)
        for h, ids, _ in (a, a2):
            assert np.array_equal(ids, ids_ref)
            err = rel_err(h - h0, h_ref - h0)
            log(f"E={E} H={H} I={I}: max|d|/max|ffn| = {err:.3e}")
            assert err <= 2e-3 and err <= 1e-4
    finally:
        t.destroy()


def test_layer1_per_layer_types():
    """Layer 1 stores routed and shared gate/up as Q6_K and down as Q4_K."""
    log("one-launch layer: per-layer matrix types")
    desc = R.table_desc(2, 64, 2048, 512)
    types = (C.c_int * 12)(0, 0, 1, 0, 0, 1, 1, 1, 0, 1, 1, 0)
    L = R.lib()
    tp = L.roaster_table_create_layers(C.byref(desc), types)
    assert tp, R.last_error()
    try:
        R.check(L.roaster_table_synth(tp, 23, None), "synth")

        class T:
            t = tp
        h0 = R.synth_normal(23, R.synth_stream(0, 0, 5), 2048)[None, :]
        a, b = _both(lambda: _stack(T, h0, 2))
        _same(a, b)
        assert np.isfinite(a[0]).all()
    finally:
        L.roaster_table_destroy(tp)


@pytest.fixture(scope="module")
def cfg2():
    t = SynthTable(1)
    yield t
    t.destroy()


def test_layer1_single_layer_router_and_given_logits(cfg2):
    """roaster_moe_decode at B = 1: with the router (logits returned) and with
    given logits holding ties and NaN."""
    x = R.synth_normal(1, R.synth_stream(0, 0, 5), 2048)[None, :]
    a, a2, b = _modes(lambda: decode(cfg2, x, 1))
    _same(a2, b)
    _near(a, b)
    lg = R.synth_normal(12, R.synth_stream(0, 1, 7), 256)[None, :]
    lg[0, [5, 9, 13, 40]] = 4.0
    lg[0, [1, 2]] = np.nan
    a, a2, b = _modes(lambda: decode(cfg2, x, 1, logits_in=lg))
    _same(a, b)
    _same(a2, b)
    assert a[2][0, :4].tolist() == [5, 9, 13, 40]


def test_layer1_routing_failure(cfg2):
    """Three routable experts: ROASTER_EROUTE from roaster_sync, outputs equal
    to the three-kernel path's."""
    x = R.synth_normal(1, 3, 2048)[None, :]
    lg = np.full((1, 256), -np.inf, np.float32)
    lg[0, :3] = 1.0

    def run():
        dx, dy, dl = Dev(x), Dev(nbytes=2048 * 4, shape=(1, 2048)), Dev(lg)
        io = R.RoasterDecodeIO(dl.p, None, None, None)
        R.check(R.lib().roaster_moe_decode(cfg2.t, 0, dx.p, 1, dy.p, C.byref(io)))
        assert R.lib().roaster_sync() == R.EROUTE
        return (dy.get(),)

    a, b = _both(run)
    _same(a, b)
    assert np.isfinite(a[0]).all()


def test_layer1_wait_gives_up_and_recovers(cfg2):
    """Spin limit of one poll: the waits give up instead of waiting, the
    launch ends, roaster_sync reports ROASTER_EDEVICE once; with the default
    limit restored the next call is exact again."""
    L = R.lib()
    x = R.synth_normal(1, R.synth_stream(0, 0, 5), 2048)[None, :]
    ref = decode(cfg2, x, 1)
    old = L.roaster_decode_spin_limit(0)
    L.roaster_decode_spin_limit(1)
    try:
        dx, dy = Dev(x), Dev(nbytes=2048 * 4, shape=(1, 2048))
        R.check(L.roaster_moe_decode(cfg2.t, 0, dx.p, 1, dy.p, None))
        rc = L.roaster_sync()
    finally:
        L.roaster_decode_spin_limit(old)
    if rc == 0:
        pytest.skip("every slot was already published at the first poll (no wait gave up)")
    assert rc == R.EDEVICE and "timed out" in R.last_error()
    assert L.roaster_sync() == 0
    _same(decode(cfg2, x, 1), ref)


@pytest.mark.parametrize("mode,B", [(1, 1), (2, 1), (1, 3), (1, 8)])
def test_stack_gives_up_leaves_h(mode, B):
    """A 4-layer stack call whose waits give up (spin limit of one poll) in
    each one-launch kernel (one token folded-router and bit-compatible, 3 and
    8 tokens batched): ROASTER_EDEVICE, and the caller's h is left as it was
    (the final state is staged and copied only when no wait anywhere gave
    up), so the call can be run again from the same input; with the default
    limit restored the next call is exact again."""
    L = R.lib()
    t = SynthTable(3, n_layers=4)
    try:
        h0 = np.stack([R.synth_normal(3, R.synth_stream(0, b, 5), 2048) for b in range(B)])
        ref = _in_mode(mode, lambda: _stack(t, h0, 4))
        old = L.roaster_decode_spin_limit(0)
        L.roaster_decode_spin_limit(1)
        try:
            dh = Dev(h0)
            _in_mode(mode, lambda: R.check(L.roaster_moe_decode_stack(t.t, dh.p, B, 0, 4, None, EPS, None, None)))
            rc = L.roaster_sync()
        finally:
            L.roaster_decode_spin_limit(old)
        if rc == 0:
            pytest.skip("every slot was already published at the first poll (no wait gave up)")
        assert rc == R.EDEVICE and "timed out" in R.last_error()
        assert L.roaster_sync() == 0
        assert np.array_equal(dh.get().view(np.uint32), h0.view(np.uint32))
        _same(_in_mode(mode, lambda: _stack(t, h0, 4)), ref)
    finally:
        t.destroy()


def test_cooperative_launch_same_results():
    """roaster_decode_cooperative_launch(1): the one-launch kernels (one token
    and 4 tokens) launched cooperatively give the results of ordinary launches
    bit for bit."""
    L = R.lib()
    t = SynthTable(3, n_layers=4)
    try:
        for B in (1, 4):
            h0 = np.stack([R.synth_normal(3, R.synth_stream(0, b, 5), 2048) for b in range(B)])
            ref = _stack(t, h0, 4)
            assert L.roaster_decode_cooperative_launch(-1) == 0
            L.roaster_decode_cooperative_launch(1)
            try:
                got = _stack(t, h0, 4)
            finally:
                L.roaster_decode_cooperative_launch(0)
            _same(got, ref)
    finally:
        t.destroy()


def test_layer1_noalloc_one_token():
    """The allocation-free entry at B = 1 runs the one-launch layer on its
    fixed array: equal to the allocating entry, twice in a row."""
    R.check(R.lib().roaster_init(), "init")
    t = SynthTable(3, n_layers=4)
    try:
        for NL in (4, 2):
            h0 = R.synth_normal(3, R.synth_stream(0, NL, 5), 2048)[None, :]
            _same(_stack(t, h0, NL, noalloc=True), _stack(t, h0, NL))
    finally:
        t.destroy()
