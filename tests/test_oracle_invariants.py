"""Checks of the oracle that do not depend on the reference build: known-answer
blocks, brute-force fp64 dequant-then-dot of the GGML Q4_K / Q6_K formats,
top-8 against a stable sort, counting-sort invariants, and linearity of the
decode / prefill combines."""
import ctypes as C

import numpy as np
import pytest

import roaster_amd as R
from oracle import oracle as O

rng = np.random.default_rng(1234)


# ---- independent fp64 decoders of the two super-block formats ---------------
def f16(b, off):
    return float(np.frombuffer(bytes(b[off:off + 2]), np.float16)[0])


def q4k_scales(s):
    sc, mn = [], []
    for j in range(8):
        if j < 4:
            sc.append(s[j] & 63)
            mn.append(s[j + 4] & 63)
        else:
            sc.append((s[j + 4] & 15) | ((s[j - 4] >> 6) << 4))
            mn.append((s[j + 4] >> 4) | ((s[j] >> 6) << 4))
    return sc, mn


def dec_q4k(blk):
    blk = np.asarray(blk, np.uint8)
    d, dmin = f16(blk, 0), f16(blk, 2)
    sc, mn = q4k_scales([int(v) for v in blk[4:16]])
    qs = blk[16:144].astype(np.int64)
    w = np.empty(256)
    for g in range(4):
        q = qs[32 * g:32 * g + 32]
        w[64 * g:64 * g + 32] = d * sc[2 * g] * (q & 15) - dmin * mn[2 * g]
        w[64 * g + 32:64 * g + 64] = d * sc[2 * g + 1] * (q >> 4) - dmin * mn[2 * g + 1]
    return w


def dec_q6k(blk):
    blk = np.asarray(blk, np.uint8)
    ql, qh = blk[0:128].astype(np.int64), blk[128:192].astype(np.int64)
    sc = blk[192:208].astype(np.int8).astype(np.int64)
    d = f16(blk, 208)
    w = np.empty(256)
    for n in range(2):
        L, Hh, S = ql[64 * n:], qh[32 * n:], sc[8 * n:]
        for l in range(32):
            is_ = l // 16
            w[128 * n + l] = d * S[is_] * (((L[l] & 15) | ((Hh[l] & 3) << 4)) - 32)
            w[128 * n + l + 32] = d * S[is_ + 2] * (((L[l + 32] & 15) | (((Hh[l] >> 2) & 3) << 4)) - 32)
            w[128 * n + l + 64] = d * S[is_ + 4] * (((L[l] >> 4) | (((Hh[l] >> 4) & 3) << 4)) - 32)
            w[128 * n + l + 96] = d * S[is_ + 6] * (((L[l + 32] >> 4) | (((Hh[l] >> 6) & 3) << 4)) - 32)
    return w


def dequant_matrix(q6, W, rows, cols):
    bs = 210 if q6 else 144
    nb = cols // 256
    dec = dec_q6k if q6 else dec_q4k
    return np.stack([np.concatenate([dec(W[(r * nb + b) * bs:(r * nb + b + 1) * bs]) for b in range(nb)])
                     for r in range(rows)])


# ---- known-answer blocks -------------------------------------------------------
def q4_block(d, dmin, sc, mn, q):
    """Encode a Q4_K block from 8 scales, 8 mins (6-bit) and 256 4-bit quants."""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.float16(dmin).tobytes(), np.uint8)
    s = np.zeros(12, np.int64)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    b[4:16] = s.astype(np.uint8)
    for g in range(4):
        lo, hi = q[64 * g:64 * g + 32], q[64 * g + 32:64 * g + 64]
        b[16 + 32 * g:16 + 32 * g + 32] = (lo | (hi << 4)).astype(np.uint8)
    return b


def test_q4k_known_answers():
    x = rng.standard_normal(256).astype(np.float32)
    out = np.empty(256, np.float32)
    # all quants zero: w = -dmin * m_j
    mn = [1, 2, 3, 4, 5, 6, 7, 8]
    b = q4_block(0.5, 0.25, [9] * 8, mn, np.zeros(256, np.int64))
    O.orc().orc_dequant_q4k_block(b.ctypes.data, out.ctypes.data)
    np.testing.assert_array_equal(out, np.repeat(-0.25 * np.array(mn, np.float32), 32))
    # d = 1, sc = 1, m = 0, q = i % 16 reproduces the index pattern
    q = np.arange(256) % 16
    b = q4_block(1.0, 0.0, [1] * 8, [0] * 8, q)
    O.orc().orc_dequant_q4k_block(b.ctypes.data, out.ctypes.data)
    np.testing.assert_array_equal(out, q.astype(np.float32))
    # scales above 15 and 31 exercise the packed high bits of sub-blocks 4..7
    sc = [1, 17, 33, 63, 16, 47, 62, 5]
    b = q4_block(1.0, 0.0, sc, [0] * 8, np.ones(256, np.int64))
    O.orc().orc_dequant_q4k_block(b.ctypes.data, out.ctypes.data)
    np.testing.assert_array_equal(out, np.repeat(np.array(sc, np.float32), 32))
    # single non-zero quant: the dot picks exactly x[i] * d * sc
    for i in (0, 31, 32, 63, 64, 200, 255):
        q = np.zeros(256, np.int64)
        q[i] = 7
        b = q4_block(0.125, 0.0, [3] * 8, [0] * 8, q)
        # folded form: (d*sc) * (q*x), each product rounded once
        assert O.orc().orc_dot_q4k(b.ctypes.data, x.ctypes.data, 256) == np.float32(0.375) * (np.float32(7) * x[i])


def q6_block(d, sc, q):
    """Encode a Q6_K block from 16 int8 scales and 256 6-bit quants (0..63)."""
    b = np.zeros(210, np.uint8)
    for n in range(2):
        for l in range(32):
            q1, q2, q3, q4 = (q[128 * n + l], q[128 * n + l + 32], q[128 * n + l + 64], q[128 * n + l + 96])
            b[64 * n + l] = (q1 & 15) | ((q3 & 15) << 4)
            b[64 * n + l + 32] = (q2 & 15) | ((q4 & 15) << 4)
            b[128 + 32 * n + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    b[192:208] = np.asarray(sc, np.int8).view(np.uint8)
    b[208:210] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    return b


def test_q6k_known_answers():
    out = np.empty(256, np.float32)
    # q = 32 everywhere: all weights are exactly zero
    b = q6_block(0.5, [5] * 16, np.full(256, 32, np.int64))
    O.orc().orc_dequant_q6k_block(b.ctypes.data, out.ctypes.data)
    assert not out.any()
    # d = 1, sc = 1: w = q - 32 reproduces the index pattern
    q = np.arange(256) % 64
    b = q6_block(1.0, [1] * 16, q)
    O.orc().orc_dequant_q6k_block(b.ctypes.data, out.ctypes.data)
    np.testing.assert_array_equal(out, (q - 32).astype(np.float32))
    # each of the 16 signed scales owns 16 consecutive weights
    sc = [-32, -7, 1, 31, 2, -3, 4, -5, 6, -8, 9, 10, -11, 12, 13, -14]
    b = q6_block(1.0, sc, np.full(256, 33, np.int64))
    O.orc().orc_dequant_q6k_block(b.ctypes.data, out.ctypes.data)
    np.testing.assert_array_equal(out, np.repeat(np.array(sc, np.float32), 16))


@pytest.mark.parametrize("q6", [0, 1])
@pytest.mark.parametrize("rows,cols", [(7, 256), (5, 2048), (3, 512)])
def test_dot_matches_fp64_bruteforce(q6, rows, cols):
    """Folded row dots and the tiled matmul against an fp64 dequant-then-dot."""
    nb = rows * cols // 256
    W = R.synth_q6k(5, 11, nb) if q6 else R.synth_q4k(5, 11, nb)
    X = rng.standard_normal((4, cols)).astype(np.float32)
    Wd = dequant_matrix(q6, W, rows, cols)
    ref = X.astype(np.float64) @ Wd.T
    scale = np.abs(X.astype(np.float64)) @ np.abs(Wd).T
    got_dot = np.stack([O.matvec(q6, W, np.ascontiguousarray(X[t]), rows, cols) for t in range(4)])
    got_mm = O.matmul(q6, W, X, rows, cols)
    assert np.all(np.abs(got_dot - ref) <= 1e-6 * scale + 1e-30)
    assert np.all(np.abs(got_mm - ref) <= 1e-6 * scale + 1e-30)


def test_top8_against_stable_sort():
    for trial in range(200):
        n = 256
        lg = rng.standard_normal(n).astype(np.float32)
        if trial % 3 == 0:
            lg = np.round(lg * 2) / 2            # many ties
        if trial % 5 == 0:
            lg[rng.integers(0, n, 10)] = np.nan
        if trial % 7 == 0:
            lg[rng.integers(0, n, 10)] = -np.inf
        ids, w = O.select_top8(lg)
        cand = [(-float(v), i) for i, v in enumerate(lg) if v > -np.inf]
        cand.sort()
        want = [i for _, i in cand[:8]]
        assert ids.tolist() == want
        v = lg[ids].astype(np.float64)
        sm = np.exp(v - v.max())
        np.testing.assert_allclose(w, sm / sm.sum(), rtol=2e-6, atol=1e-7)
        assert abs(float(w.sum()) - 1.0) < 1e-6


def test_top8_fewer_than_8_finite_leaves_minus_one():
    lg = np.full(256, -np.inf, np.float32)
    lg[[4, 8]] = [1.0, 2.0]
    ids, w = O.select_top8(lg)
    assert ids.tolist() == [8, 4, -1, -1, -1, -1, -1, -1]
    assert w[2:].tolist() == [0.0] * 6


def test_bucketing_invariants():
    T, E = 300, 256
    ids = np.stack([rng.choice(E, 8, replace=False) for _ in range(T)]).astype(np.int32)
    cnt = np.empty(E, np.int32)
    off = np.empty(E + 1, np.int32)
    lt = np.empty(T * 8, np.int32)
    lk = np.empty(T * 8, np.int32)
    O.orc().orc_bucket(ids.ctypes.data, T, E, cnt.ctypes.data, off.ctypes.data, lt.ctypes.data, lk.ctypes.data)
    np.testing.assert_array_equal(cnt, np.bincount(ids.ravel(), minlength=E))
    np.testing.assert_array_equal(off, np.concatenate([[0], np.cumsum(cnt)]))
    for e in range(E):
        seg = list(zip(lt[off[e]:off[e + 1]], lk[off[e]:off[e + 1]]))
        assert all(ids[t, k] == e for t, k in seg)
        assert seg == sorted(seg)                               # stable over (t, k)
    assert sorted(zip(lt, lk)) == [(t, k) for t in range(T) for k in range(8)]   # complete


def small_layer(seed, E=16, H=512, I=256, types=(0, 0, 1), sh_types=(0, 0, 1)):
    desc = R.table_desc(1, E, H, I, types, sh_types)
    experts = [R.host_expert(seed, 0, e, desc) for e in range(E)]
    shared = R.host_expert(seed, 0, E, desc)
    router, gate_inp = R.host_router(seed, 0, desc)
    return O.Layer(H, I, router, gate_inp, experts, shared, types, sh_types), experts, shared


def test_decode_combine_one_hot():
    """With one dominant logit the routing weights are exactly (1, 0, ..., 0), and
    a shared-gate logit of -200 / +200 gives sigmoid exactly 0 / 1, so the block
    output reduces to known single-expert outputs."""
    L, experts, shared = small_layer(21)
    x = rng.standard_normal(512).astype(np.float32)
    lg = rng.standard_normal(16).astype(np.float32)
    lg[11] = 500.0
    e11 = np.empty(512, np.float32)
    esh = np.empty(512, np.float32)
    g, u, d = experts[11]
    O.orc().orc_expert_decode(C.byref(O.OrcExpert(g.ctypes.data, u.ctypes.data, d.ctypes.data, 0, 0, 1)),
                              x.ctypes.data, 256, 512, e11.ctypes.data)
    g, u, d = shared
    O.orc().orc_expert_decode(C.byref(O.OrcExpert(g.ctypes.data, u.ctypes.data, d.ctypes.data, 0, 0, 1)),
                              x.ctypes.data, 256, 512, esh.ctypes.data)
    for s, want in ((-200.0, e11), (200.0, (e11 + esh).astype(np.float32))):
        gi = (x * np.float32(s / float(x @ x))).astype(np.float32)
        L.c.shexp_gate_inp = gi.ctypes.data
        rc, y, _, ids, w = L.decode(x, logits_in=lg)
        assert rc == 0 and ids[0] == 11 and w[0] == 1.0 and not w[1:].any()
        np.testing.assert_array_equal(y, want)


def test_decode_block_fp64():
    L, experts, shared = small_layer(22)
    x = rng.standard_normal(512).astype(np.float32)
    rc, y, lg, ids, w = L.decode(x)
    assert rc == 0
    gi = np.frombuffer((C.c_float * 512).from_address(L.c.shexp_gate_inp), np.float32)
    x64 = x.astype(np.float64)

    def expert64(mats, types):
        g, u, d = mats
        gv = dequant_matrix(types[0], g, 256, 512) @ x64
        uv = dequant_matrix(types[1], u, 256, 512) @ x64
        eh = gv / (1 + np.exp(-gv)) * uv
        return dequant_matrix(types[2], d, 512, 256) @ eh

    want = sum(float(w[k]) * expert64(experts[ids[k]], (0, 0, 1)) for k in range(8))
    want = want + 1 / (1 + np.exp(-(gi.astype(np.float64) @ x64))) * expert64(shared, (0, 0, 1))
    assert np.max(np.abs(y - want)) <= 1e-5 * np.max(np.abs(want))


def test_prefill_matches_per_token_decode():
    """pf_moe (grouped, dequant-then-dot) and moe_forward (folded dots) agree to
    fp32 rounding, token by token, and the shared expert is combined first."""
    L, _, _ = small_layer(23)
    T = 24
    X = rng.standard_normal((T, 512)).astype(np.float32)
    rc, Y, ids, w, lg = L.prefill(X)
    assert rc == 0
    for t in range(T):
        rc, y, lgt, idt, wt = L.decode(np.ascontiguousarray(X[t]))
        assert rc == 0
        np.testing.assert_array_equal(lg[t], lgt)
        np.testing.assert_array_equal(ids[t], idt)
        assert np.max(np.abs(Y[t] - y)) <= 2e-6 * np.max(np.abs(y))


def test_prefill_bias_and_given_logits():
    L, _, _ = small_layer(24)
    T = 8
    X = rng.standard_normal((T, 512)).astype(np.float32)
    bias = np.zeros(16, np.float32)
    bias[5] = 1000.0
    rc, _, ids, _, lg = L.prefill(X, bias=bias)
    assert rc == 0 and np.all(ids[:, 0] == 5)
    given = rng.standard_normal((T, 16)).astype(np.float32)
    rc, _, ids2, _, lg2 = L.prefill(X, logits_in=given)
    assert rc == 0
    np.testing.assert_array_equal(lg2, given)
    for t in range(T):
        assert ids2[t].tolist() == O.select_top8(given[t])[0].tolist()
