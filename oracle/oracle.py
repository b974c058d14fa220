"""ctypes access to the CPU oracle (liboracle.so) and, where it was built, the
reference's own CPU kernels (_ref/libref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker, never by the product.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libref.so")

_P = C.c_void_p


class OrcExpert(C.Structure):
    _fields_ = [("gate", _P), ("up", _P), ("down", _P),
                ("gate_q6", C.c_int), ("up_q6", C.c_int), ("down_q6", C.c_int)]


class OrcLayer(C.Structure):
    _fields_ = [("n_experts", C.c_int), ("hidden", C.c_size_t), ("inter", C.c_size_t),
                ("router", _P), ("shexp_gate_inp", _P), ("experts", C.POINTER(OrcExpert)),
                ("shared", OrcExpert)]


class OrcMoeGroup(C.Structure):
    _fields_ = [("gate", _P), ("up", _P), ("down", _P),
                ("gate_q6", C.c_int), ("up_q6", C.c_int), ("down_q6", C.c_int), ("n", C.c_size_t)]


_SIG = {
    "orc_fp16_to_f32": (C.c_float, [C.c_uint16]),
    "orc_q4k_scales": (None, [_P, _P, _P]),
    "orc_dot_f32": (C.c_float, [_P, _P, C.c_size_t]),
    "orc_matvec_f32": (None, [_P, _P, _P, C.c_size_t, C.c_size_t]),
    "orc_dot_q4k": (C.c_float, [_P, _P, C.c_size_t]),
    "orc_dot_q6k": (C.c_float, [_P, _P, C.c_size_t]),
    "orc_matvec_q4k": (None, [_P, _P, _P, C.c_size_t, C.c_size_t]),
    "orc_matvec_q6k": (None, [_P, _P, _P, C.c_size_t, C.c_size_t]),
    "orc_matvec_quant": (None, [C.c_int, _P, _P, _P, C.c_size_t, C.c_size_t]),
    "orc_dequant_q4k_block": (None, [_P, _P]),
    "orc_dequant_q6k_block": (None, [_P, _P]),
    "orc_matmul_quant": (None, [C.c_int, _P, _P, _P, C.c_size_t, C.c_size_t, C.c_size_t]),
    "orc_rmsnorm": (None, [_P, _P, _P, C.c_size_t, C.c_float]),
    "orc_select_top8": (None, [_P, C.c_int, _P, _P]),
    "orc_expert_decode": (None, [C.POINTER(OrcExpert), _P, C.c_size_t, C.c_size_t, _P]),
    "orc_moe_decode": (C.c_int, [C.POINTER(OrcLayer), _P, _P, _P, _P, _P, _P]),
    "orc_moe_groups": (None, [C.POINTER(OrcMoeGroup), C.c_int, _P, _P, C.c_size_t, C.c_size_t]),
    "orc_bucket": (None, [_P, C.c_int, C.c_int, _P, _P, _P, _P]),
    "orc_moe_prefill": (C.c_int, [C.POINTER(OrcLayer), _P, C.c_int, _P, _P, _P, _P, _P, _P]),
}

_REF_SIG = {
    "kernel_dot_f32": (C.c_float, [_P, _P, C.c_size_t]),
    "kernel_matvec_f32": (None, [_P, _P, _P, C.c_size_t, C.c_size_t]),
    "kernel_dot_q4_k": (C.c_float, [_P, _P, C.c_size_t]),
    "kernel_dot_q6_k": (C.c_float, [_P, _P, C.c_size_t]),
    "kernel_rmsnorm": (None, [_P, _P, _P, C.c_size_t, C.c_float]),
    "ref_matvec_q4_cpu": (None, [_P, _P, _P, C.c_size_t, C.c_size_t]),
    "ref_matvec_q6_cpu": (None, [_P, _P, _P, C.c_size_t, C.c_size_t]),
    "ref_dequant_q4_k_block": (None, [_P, _P]),
    "ref_dequant_q6_k_block": (None, [_P, _P]),
    "ref_matmul_quant_cpu": (None, [C.c_int, _P, _P, _P, C.c_size_t, C.c_size_t, C.c_size_t]),
    "ref_moe_cpu": (None, [_P, C.c_int, _P, _P, C.c_size_t, C.c_size_t]),
    "ref_select_top8": (None, [_P, _P, _P]),
}

_orc = None
_ref = None


def orc():
    global _orc
    if _orc is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"{ORACLE_SO} missing: run make -C oracle")
        L = C.CDLL(ORACLE_SO)
        for n, (r, a) in _SIG.items():
            f = getattr(L, n)
            f.restype, f.argtypes = r, a
        _orc = L
    return _orc


def ref_available():
    return os.path.exists(REF_SO)


def ref():
    global _ref
    if _ref is None:
        L = C.CDLL(REF_SO)
        for n, (r, a) in _REF_SIG.items():
            f = getattr(L, n)
            f.restype, f.argtypes = r, a
        _ref = L
    return _ref


def p(a):
    return None if a is None else a.ctypes.data


# ---- convenience wrappers ------------------------------------------------------
def matvec(q6, W, x, rows, cols):
    y = np.empty(rows, np.float32)
    orc().orc_matvec_quant(int(q6), p(W), p(x), p(y), rows, cols)
    return y


def matmul(q6, W, X, rows, cols):
    T = X.shape[0]
    Y = np.empty((T, rows), np.float32)
    orc().orc_matmul_quant(int(q6), p(W), p(np.ascontiguousarray(X, np.float32)), p(Y), rows, cols, T)
    return Y


def matvec_f32(W, x):
    y = np.empty(W.shape[0], np.float32)
    orc().orc_matvec_f32(p(W), p(x), p(y), W.shape[0], W.shape[1])
    return y


def select_top8(logits):
    logits = np.ascontiguousarray(logits, np.float32)
    ids = np.empty(8, np.int32)
    w = np.empty(8, np.float32)
    orc().orc_select_top8(p(logits), logits.shape[0], p(ids), p(w))
    return ids, w


class Layer:
    """Keeps the numpy buffers of one MoE layer alive behind an OrcLayer."""

    def __init__(self, hidden, inter, router, gate_inp, experts, shared, types, sh_types):
        self.bufs = [router, gate_inp, shared] + list(experts)
        E = len(experts)
        self._ex = (OrcExpert * E)()
        for e, (g, u, d) in enumerate(experts):
            self._ex[e] = OrcExpert(p(g), p(u), p(d), types[0], types[1], types[2])
        self.c = OrcLayer()
        self.c.n_experts = E
        self.c.hidden, self.c.inter = hidden, inter
        self.c.router = p(router) if router is not None else None
        self.c.shexp_gate_inp = p(gate_inp)
        self.c.experts = self._ex
        g, u, d = shared
        self.c.shared = OrcExpert(p(g), p(u), p(d), sh_types[0], sh_types[1], sh_types[2])
        self.hidden, self.inter, self.E = hidden, inter, E

    def decode(self, x, logits_in=None):
        y = np.empty(self.hidden, np.float32)
        lg = np.empty(self.E, np.float32)
        ids = np.empty(8, np.int32)
        w = np.empty(8, np.float32)
        rc = orc().orc_moe_decode(C.byref(self.c), p(x), p(logits_in), p(y), p(lg), p(ids), p(w))
        return rc, y, lg, ids, w

    def prefill(self, X, logits_in=None, bias=None):
        T = X.shape[0]
        Y = np.empty((T, self.hidden), np.float32)
        ids = np.empty((T, 8), np.int32)
        w = np.empty((T, 8), np.float32)
        lg = np.empty((T, self.E), np.float32)
        rc = orc().orc_moe_prefill(C.byref(self.c), p(np.ascontiguousarray(X, np.float32)), T,
                                   p(logits_in), p(bias), p(Y), p(ids), p(w), p(lg))
        return rc, Y, ids, w, lg
