"""One launch for a run of decode layers of 2..8 tokens (dec_stackB*_kernel)
against the three-kernel path (roaster_decode_fused_layer(0)), the one-token
launch and the oracle.

The batched launch computes every dot, sum of squares, softmax and combine of
each token in the three-kernel path's order, so each token's hidden state,
ids and routing weights must equal, bit for bit, both the three-kernel path's
for the whole batch and the bit-compatible one-token launch's
(roaster_decode_fused_layer(2)) for that token alone; the
oracle bars of the decode tests (ids exact, max|d|/max|ffn| <= 2e-3 and the
1e-4 regression bound) are held as well.  Cases: 8 tokens (8 token slots), 3
and 5 tokens (4 and 8 slots, some unused), 2, 4 and 6 tokens; the 256-expert
shape with norm weights, hidden 768 / 64 experts (activations stored plainly
in LDS), hidden 1280 / 128 experts, hidden 512 / 32 experts (the smallest
shape taken: one logit per workgroup of a group) and hidden 1024; one layer
through roaster_moe_decode with the router and with given logits holding
ties and NaN; fewer than 8 routable
experts for one token of four; per-layer matrix types the launch does not
take (the three-kernel path runs); a wait that gives up (spin limit forced to
1 poll from the host, so every kernel still ends)."""
import ctypes as C

import numpy as np
import pytest

import roaster_amd as R
from gpu_util import Dev, SynthTable, log, rel_err
from test_gpu_decode import oracle_stack, decode
from test_gpu_decode_layer1 import _stack, _both, _same, _in_mode

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape", [(256, 2048, 8, 4), (256, 2048, 3, 3), (64, 768, 2, 2), (128, 1280, 5, 2),
                                   (32, 512, 4, 2), (256, 1024, 6, 2)])
def test_stackB_matches_three_kernels_one_token_and_oracle(shape):
    E, H, B, NL = shape
    log(f"batched one-launch stack: E={E} H={H} B={B}, {NL} layers")
    t = SynthTable(31, n_layers=NL, n_experts=E, hidden=H, inter=512)
    try:
        h0 = np.stack([R.synth_normal(31, R.synth_stream(0, b, 5), H) for b in range(B)])
        nw = np.stack([1.0 + 0.25 * R.synth_normal(32, R.synth_stream(l, 0, 6), H) for l in range(NL)]).astype(np.float32)
        a, b = _both(lambda: _stack(t, h0, NL, nw))
        _same(a, b)
        h, ids, w = a
        for tok in range(B):
            # the one-token launch with the three-kernel path's arithmetic
            h1, ids1, w1 = _in_mode(2, lambda: _stack(t, h0[tok:tok + 1], NL, nw))
            _same((h[tok:tok + 1], ids[:, tok:tok + 1], w[:, tok:tok + 1]), (h1, ids1, w1))
        h_ref, ids_ref = oracle_stack(t, h0, NL, norm_w=nw)
        assert np.array_equal(ids, ids_ref)
        err = rel_err(h - h0, h_ref - h0)
        log(f"E={E} H={H} B={B}: max|d|/max|ffn| = {err:.3e}")
        assert err <= 2e-3 and err <= 1e-4
    finally:
        t.destroy()


@pytest.fixture(scope="module")
def cfg2():
    t = SynthTable(1)
    yield t
    t.destroy()


def test_stackB_single_layer_router_and_given_logits(cfg2):
    """roaster_moe_decode at B = 4: with the router (logits returned) and with
    given logits holding ties and NaN."""
    x = np.stack([R.synth_normal(1, R.synth_stream(0, b, 5), 2048) for b in range(4)])
    a, b = _both(lambda: decode(cfg2, x, 4))
    _same(a, b)
    lg = np.stack([R.synth_normal(12, R.synth_stream(0, b, 7), 256) for b in range(4)])
    lg[2, [5, 9, 13, 40]] = 4.0
    lg[1, [1, 2]] = np.nan
    a, b = _both(lambda: decode(cfg2, x, 4, logits_in=lg))
    _same(a, b)
    assert a[2][2, :4].tolist() == [5, 9, 13, 40]


def test_stackB_routing_failure(cfg2):
    """One token of four with three routable experts: ROASTER_EROUTE from
    roaster_sync, outputs equal to the three-kernel path's."""
    x = np.stack([R.synth_normal(1, 3 + b, 2048) for b in range(4)])
    lg = np.stack([R.synth_normal(13, R.synth_stream(0, b, 7), 256) for b in range(4)])
    lg[1] = -np.inf
    lg[1, :3] = 1.0

    def run():
        dx, dy, dl = Dev(x), Dev(nbytes=4 * 2048 * 4, shape=(4, 2048)), Dev(lg)
        io = R.RoasterDecodeIO(dl.p, None, None, None)
        R.check(R.lib().roaster_moe_decode(cfg2.t, 0, dx.p, 4, dy.p, C.byref(io)))
        assert R.lib().roaster_sync() == R.EROUTE
        return (dy.get(),)

    a, b = _both(run)
    _same(a, b)
    assert np.isfinite(a[0]).all()


def test_stackB_per_layer_types_fall_back():
    """Layer 1 stores gate/up as Q6_K and down as Q4_K: the launch is not
    taken and the three-kernel path's results come back."""
    desc = R.table_desc(2, 64, 2048, 512)
    types = (C.c_int * 12)(0, 0, 1, 0, 0, 1, 1, 1, 0, 1, 1, 0)
    L = R.lib()
    tp = L.roaster_table_create_layers(C.byref(desc), types)
    assert tp, R.last_error()
    try:
        R.check(L.roaster_table_synth(tp, 23, None), "synth")

        class T:
            t = tp
        h0 = np.stack([R.synth_normal(23, R.synth_stream(0, b, 5), 2048) for b in range(4)])
        a, b = _both(lambda: _stack(T, h0, 2))
        _same(a, b)
        assert np.isfinite(a[0]).all()
    finally:
        L.roaster_table_destroy(tp)


def test_stackB_wait_gives_up_and_recovers(cfg2):
    """Spin limit of one poll at B = 8: the waits give up instead of waiting,
    the launch ends, roaster_sync reports ROASTER_EDEVICE once; with the
    default limit restored the next call is exact again."""
    L = R.lib()
    x = np.stack([R.synth_normal(1, R.synth_stream(0, b, 5), 2048) for b in range(8)])
    ref = decode(cfg2, x, 8)
    old = L.roaster_decode_spin_limit(0)
    L.roaster_decode_spin_limit(1)
    try:
        dx, dy = Dev(x), Dev(nbytes=8 * 2048 * 4, shape=(8, 2048))
        R.check(L.roaster_moe_decode(cfg2.t, 0, dx.p, 8, dy.p, None))
        rc = L.roaster_sync()
    finally:
        L.roaster_decode_spin_limit(old)
    if rc == 0:
        pytest.skip("every slot was already published at the first poll (no wait gave up)")
    assert rc == R.EDEVICE and "timed out" in R.last_error()
    assert L.roaster_sync() == 0
    _same(decode(cfg2, x, 8), ref)
