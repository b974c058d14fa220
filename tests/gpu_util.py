"""Helpers for the GPU tests: device buffers through the library's own C ABI
(roaster_dev_alloc / roaster_h2d / roaster_d2h), tolerance metrics and the
synthetic expert tables shared by several tests."""
import ctypes as C
import sys

import numpy as np

import roaster_amd as R
from oracle import oracle as O


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


class Dev:
    """A device allocation holding a copy of a numpy array (or zeros)."""

    def __init__(self, arr=None, nbytes=None, dtype=np.float32, shape=None):
        L = R.lib()
        if arr is not None:
            arr = np.ascontiguousarray(arr)
            nbytes, dtype, shape = arr.nbytes, arr.dtype, arr.shape
        self.nbytes, self.dtype, self.shape = nbytes, np.dtype(dtype), shape
        self.p = L.roaster_dev_alloc(max(nbytes, 1))
        assert self.p, R.last_error()
        if arr is not None:
            R.check(L.roaster_h2d(self.p, arr.ctypes.data, nbytes), "h2d")
        else:
            R.check(L.roaster_memset(self.p, 0, nbytes), "memset")

    def get(self):
        out = np.empty(self.nbytes // self.dtype.itemsize, self.dtype)
        R.check(R.lib().roaster_d2h(out.ctypes.data, self.p, self.nbytes), "d2h")
        return out.reshape(self.shape) if self.shape is not None else out

    def free(self):
        if self.p:
            R.lib().roaster_dev_free(self.p)
            self.p = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def alloc_w(arr):
    """Copy weight bytes into kernel_vk_alloc_weights memory, as the reference
    test's alloc_w does (test_kernels.c:16); returns the host address."""
    arr = np.ascontiguousarray(arr)
    granted = C.c_size_t(0)
    p = R.lib().kernel_vk_alloc_weights(arr.nbytes, C.byref(granted))
    assert p and granted.value >= arr.nbytes, R.last_error()
    C.memmove(p, arr.ctypes.data, arr.nbytes)
    return p


def rel_err(got, ref):
    """max |got - ref| / max |ref| (the reference test's metric, test_kernels.c:31)."""
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    den = np.max(np.abs(ref))
    return float(np.max(np.abs(got - ref)) / (den if den > 0 else 1.0))


class SynthTable:
    """A device expert table filled by roaster_table_synth, with lazy host copies
    of the same experts for the oracle."""

    def __init__(self, seed, n_layers=1, n_experts=256, hidden=2048, inter=512, q6=(0, 0, 1), sh_q6=(0, 0, 1)):
        self.seed = seed
        self.desc = R.table_desc(n_layers, n_experts, hidden, inter, q6, sh_q6)
        self.t = R.lib().roaster_table_create(C.byref(self.desc))
        assert self.t, R.last_error()
        R.check(R.lib().roaster_table_synth(self.t, seed, None), "table_synth")
        self._experts = {}
        self._routers = {}

    def expert(self, layer, e):
        k = (layer, e)
        if k not in self._experts:
            self._experts[k] = R.host_expert(self.seed, layer, e, self.desc)
        return self._experts[k]

    def router(self, layer):
        if layer not in self._routers:
            self._routers[layer] = R.host_router(self.seed, layer, self.desc)
        return self._routers[layer]

    def oracle_layer(self, layer, experts_needed=None):
        """An oracle Layer; only `experts_needed` get real bytes (others alias
        expert 0's buffers and must not be selected)."""
        E = self.desc.n_experts
        need = set(experts_needed if experts_needed is not None else range(E))
        base = self.expert(layer, min(need) if need else 0)
        exps = [self.expert(layer, e) if e in need else base for e in range(E)]
        router, gi = self.router(layer)
        return O.Layer(self.desc.hidden, self.desc.inter, router, gi, exps, self.expert(layer, E),
                       tuple(self.desc.q6), tuple(self.desc.sh_q6))

    def destroy(self):
        if self.t:
            R.lib().roaster_table_destroy(self.t)
            self.t = None


def bf16_round(a):
    """Round f32 values to the nearest bf16 (ties to even), kept as f32."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def zipf_bias(E, seed, s=1.1, tau=0.3):
    """Per-expert logit bias tau * ln(p_e) with p_e proportional to rank_e^-s
    (Zipf), ranks assigned to expert ids by a permutation drawn from seed.
    tau = 0.3 skews T = 512 tokens' expert lists from 0 to about 200 rows."""
    perm = np.random.default_rng(seed).permutation(E)
    rank = np.empty(E, np.float64)
    rank[perm] = np.arange(1, E + 1)
    p = rank ** -s
    p /= p.sum()
    return (tau * np.log(p)).astype(np.float32)


def prefill(table, X, layer=0, precision=R.PREC_F16, logits_in=None, bias=None):
    """roaster_moe_prefill through the C ABI; returns (Y, logits, ids, w, counts)."""
    T, H = X.shape
    E = table.desc.n_experts
    dx = Dev(X)
    dy = Dev(nbytes=T * H * 4, shape=(T, H))
    dl = Dev(nbytes=T * E * 4, shape=(T, E))
    di = Dev(nbytes=T * 8 * 4, dtype=np.int32, shape=(T, 8))
    dw = Dev(nbytes=T * 8 * 4, shape=(T, 8))
    dc = Dev(nbytes=E * 4, dtype=np.int32, shape=(E,))
    dli = Dev(logits_in) if logits_in is not None else None
    db = Dev(bias) if bias is not None else None
    o = R.RoasterPrefillOpts(precision, dli.p if dli else None, db.p if db else None, dl.p, di.p, dw.p, dc.p)
    R.check(R.lib().roaster_moe_prefill(table.t, layer, dx.p, T, dy.p, C.byref(o)), "prefill")
    R.check(R.lib().roaster_sync(), "sync")
    return dy.get(), dl.get(), di.get(), dw.get(), dc.get()
