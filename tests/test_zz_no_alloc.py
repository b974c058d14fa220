"""roaster_moe_decode_stack_noalloc: the layer stack with every intermediate in
the library's fixed device array instead of allocated scratch.

It runs the same kernels as roaster_moe_decode_stack, so its hidden states,
ids and routing weights must equal that entry point's bit for bit; the first
call is also held to the oracle's bars (ids exact, max|d|/max|ffn| <= 2e-3).
Two calls in a row, the second with fewer tokens and layers, check that the
array's leftovers from the first call do not leak into the second.  Sizes
beyond the array are rejected with ROASTER_EINVAL before anything runs.
"""
import ctypes as C

import numpy as np
import pytest

import roaster_amd as R
from gpu_util import Dev, SynthTable, log, rel_err
from test_gpu_decode import oracle_stack

pytestmark = pytest.mark.gpu

EPS = C.c_float(1e-6)


def _run(entry, t, h0, B, NL, nw):
    dh = Dev(h0)
    dn = Dev(nw) if nw is not None else None
    di = Dev(nbytes=NL * B * 8 * 4, dtype=np.int32, shape=(NL, B, 8))
    dw = Dev(nbytes=NL * B * 8 * 4, shape=(NL, B, 8))
    rc = entry(t.t, dh.p, B, 0, NL, dn.p if dn else None, EPS, di.p, dw.p)
    R.check(rc, entry.__name__)
    R.check(R.lib().roaster_sync(), "sync")
    return dh.get(), di.get(), dw.get()


def test_noalloc_stack_matches_allocating_entry_twice():
    L = R.lib()
    R.check(L.roaster_init(), "init")
    log("noalloc decode stack: 4 layers x 256 experts, seed 3")
    t = SynthTable(3, n_layers=4)
    try:
        for B, NL in ((8, 4), (2, 2)):
            log(f"noalloc call B={B} layers={NL}")
            h0 = np.stack([R.synth_normal(3, R.synth_stream(0, b, 5), 2048) for b in range(B)])
            nw = np.stack([1.0 + 0.25 * R.synth_normal(6, R.synth_stream(l, 0, 6), 2048)
                           for l in range(NL)]).astype(np.float32)
            h, ids, w = _run(L.roaster_moe_decode_stack_noalloc, t, h0, B, NL, nw)
            h_r, ids_r, w_r = _run(L.roaster_moe_decode_stack, t, h0, B, NL, nw)
            assert np.array_equal(ids, ids_r)
            assert np.array_equal(w.view(np.uint32), w_r.view(np.uint32))
            assert np.array_equal(h.view(np.uint32), h_r.view(np.uint32))
            if B == 8:
                h_o, ids_o = oracle_stack(t, h0, NL, norm_w=nw)
                assert np.array_equal(ids, ids_o)
                err = rel_err(h - h0, h_o - h0)
                log(f"noalloc B={B}: max|d|/max|ffn| vs oracle = {err:.3e}")
                assert err <= 2e-3
    finally:
        t.destroy()


def test_noalloc_one_token_after_eight():
    """A call of 8 tokens (three kernels per layer, their intermediates over
    the bytes where the one-token launch keeps its exchange slots), then one
    token (the one-launch kernel on those slots), then 8 again and one again:
    each equal to the allocating entry bit for bit."""
    L = R.lib()
    R.check(L.roaster_init(), "init")
    t = SynthTable(3, n_layers=4)
    try:
        for B, NL in ((8, 2), (1, 4), (8, 1), (1, 3)):
            log(f"noalloc call B={B} layers={NL}")
            h0 = np.stack([R.synth_normal(4, R.synth_stream(0, b + 10 * NL, 5), 2048) for b in range(B)])
            got = _run(L.roaster_moe_decode_stack_noalloc, t, h0, B, NL, None)
            ref = _run(L.roaster_moe_decode_stack, t, h0, B, NL, None)
            for x, y in zip(got, ref):
                assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    finally:
        t.destroy()


def test_noalloc_rejects_sizes_beyond_its_array():
    """inter 2048 at 8 tokens needs 8 x 9 x 2048 x 4 B of SiLU*up rows alone,
    more than the 576 KiB array: the call is refused before any launch (the
    table is created but never filled, so no kernel runs in this test)."""
    L = R.lib()
    R.check(L.roaster_init(), "init")
    log("noalloc size limit: hidden 2048, inter 2048, 8 experts, 8 tokens")
    desc = R.table_desc(1, 8, 2048, 2048)
    t = L.roaster_table_create(C.byref(desc))
    assert t, R.last_error()
    try:
        h0 = np.stack([R.synth_normal(7, R.synth_stream(0, b, 5), 2048) for b in range(8)])
        dh = Dev(h0)
        rc = L.roaster_moe_decode_stack_noalloc(t, dh.p, 8, 0, 1, None, EPS, None, None)
        assert rc == R.EINVAL, rc
        assert "maximum" in R.last_error()
        R.check(L.roaster_sync(), "sync")
        assert np.array_equal(dh.get(), h0)          # nothing ran
    finally:
        L.roaster_table_destroy(t)
