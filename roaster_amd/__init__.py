"""roaster_amd -- Python access to libroaster_moe.so, the MI355X MoE-FFN hot path.

The product is the C ABI declared in include/kernels.h (the reference's kernel API)
and include/roaster_moe.h (expert table, whole-layer decode / prefill).  This module
only loads that library with ctypes and declares its signatures, so that tests and
the benchmark can call the same entry points a C caller would.  It fails loudly
when the library has not been built: there is no Python or CPU fallback.
"""
import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libroaster_moe.so")

QK = 256
Q4K_BYTES = 144
Q6K_BYTES = 210

OK, EINVAL, EDEVICE, EROUTE, ENOMEM = 0, -1, -2, -3, -4
GATE, UP, DOWN = 0, 1, 2
PREC_F16, PREC_SPLIT, PREC_BF16 = 0, 1, 2


class KernelMatvecJob(C.Structure):
    _fields_ = [("is_q6", C.c_int), ("matrix", C.c_void_p), ("vector", C.c_void_p),
                ("output", C.c_void_p), ("rows", C.c_size_t), ("cols", C.c_size_t)]


class KernelMatmulJob(C.Structure):
    _fields_ = [("is_q6", C.c_int), ("matrix", C.c_void_p), ("X", C.c_void_p), ("Y", C.c_void_p),
                ("rows", C.c_size_t), ("cols", C.c_size_t), ("T", C.c_size_t)]


class KernelMoeExpert(C.Structure):
    _fields_ = [("gate", C.c_void_p), ("up", C.c_void_p), ("down", C.c_void_p),
                ("gate_q6", C.c_int), ("up_q6", C.c_int), ("down_q6", C.c_int), ("n", C.c_size_t)]


class KernelFfnExpert(C.Structure):
    _fields_ = [("gate", C.c_void_p), ("up", C.c_void_p), ("down", C.c_void_p),
                ("gate_q6", C.c_int), ("up_q6", C.c_int), ("down_q6", C.c_int), ("out", C.c_void_p)]


class RoasterTableDesc(C.Structure):
    _fields_ = [("n_layers", C.c_int), ("n_experts", C.c_int), ("hidden", C.c_size_t),
                ("inter", C.c_size_t), ("q6", C.c_int * 3), ("sh_q6", C.c_int * 3)]


class RoasterGgufInfo(C.Structure):
    _fields_ = [("version", C.c_int), ("n_tensors", C.c_uint64), ("alignment", C.c_uint64),
                ("data_offset", C.c_uint64), ("n_layers", C.c_int), ("n_experts", C.c_int),
                ("hidden", C.c_size_t), ("inter", C.c_size_t), ("q6", C.c_int * 3), ("sh_q6", C.c_int * 3),
                ("mixed_types", C.c_int), ("router_type", C.c_int)]


class RoasterSynthSpec(C.Structure):
    _fields_ = [("q4k_lo", C.c_float), ("q4k_hi", C.c_float), ("q6k_lo", C.c_float),
                ("q6k_hi", C.c_float), ("router_sigma", C.c_float), ("gate_inp_sigma", C.c_float)]


class RoasterDecodeIO(C.Structure):
    _fields_ = [("logits_in", C.c_void_p), ("logits_out", C.c_void_p), ("ids_out", C.c_void_p),
                ("w_out", C.c_void_p)]


class RoasterPrefillOpts(C.Structure):
    _fields_ = [("precision", C.c_int), ("logits_in", C.c_void_p), ("logit_bias", C.c_void_p),
                ("logits_out", C.c_void_p), ("ids_out", C.c_void_p), ("w_out", C.c_void_p),
                ("counts_out", C.c_void_p)]


_P = C.c_void_p
_SIG = {
    # kernels.h
    "kernel_dot_f32": (C.c_float, [_P, _P, C.c_size_t]),
    "kernel_matvec_f32": (None, [_P, _P, _P, C.c_size_t, C.c_size_t]),
    "kernel_dot_q4_k": (C.c_float, [_P, _P, C.c_size_t]),
    "kernel_dot_q6_k": (C.c_float, [_P, _P, C.c_size_t]),
    "kernel_matvec_q4_k": (None, [_P, _P, _P, C.c_size_t, C.c_size_t]),
    "kernel_matvec_q6_k": (None, [_P, _P, _P, C.c_size_t, C.c_size_t]),
    "kernel_rmsnorm": (None, [_P, _P, _P, C.c_size_t, C.c_float]),
    "kernel_l2norm": (None, [_P, _P, C.c_size_t, C.c_float]),
    "kernel_sigmoid": (C.c_float, [C.c_float]),
    "kernel_silu": (C.c_float, [C.c_float]),
    "kernel_silu_array": (None, [_P, C.c_size_t]),
    "kernel_embedding_row_q4_k": (None, [_P, C.c_size_t, _P, C.c_size_t]),
    "kernel_conv1d_causal_f32": (None, [_P, _P, _P, _P, C.c_size_t, C.c_size_t]),
    "kernel_matvec_quant_batch": (None, [_P, C.c_int]),
    "kernel_matvec_quant_begin": (C.c_int, [_P, C.c_int]),
    "kernel_matvec_quant_end": (None, []),
    "kernel_matmul_quant_batch": (C.c_int, [_P, C.c_int]),
    "kernel_moe_prefill": (C.c_int, [_P, C.c_int, _P, _P, C.c_size_t, C.c_size_t]),
    "kernel_ffn_fused": (C.c_int, [_P, C.c_int, _P, C.c_size_t, C.c_size_t]),
    "kernel_vk_trim_scratch": (None, []),
    "kernel_vk_shutdown": (None, []),
    "kernel_vk_release_host_ptr": (None, [_P]),
    "kernel_vk_register_region": (C.c_int, [_P, C.c_size_t]),
    "kernel_vk_alloc_weights": (_P, [C.c_size_t, C.POINTER(C.c_size_t)]),
    "kernel_vk_owns_weights": (C.c_int, [_P]),
    "kernel_vk_free_weights": (C.c_int, [_P]),
    # roaster_moe.h
    "roaster_last_error": (C.c_char_p, []),
    "roaster_init": (C.c_int, []),
    "roaster_stream": (_P, []),
    "roaster_sync": (C.c_int, []),
    "roaster_device_info": (C.c_int, [C.POINTER(C.c_int), C.POINTER(C.c_int), C.POINTER(C.c_size_t)]),
    "roaster_dev_alloc": (_P, [C.c_size_t]),
    "roaster_dev_free": (None, [_P]),
    "roaster_h2d": (C.c_int, [_P, _P, C.c_size_t]),
    "roaster_d2h": (C.c_int, [_P, _P, C.c_size_t]),
    "roaster_memset": (C.c_int, [_P, C.c_int, C.c_size_t]),
    "roaster_weight_tracking": (C.c_int, [C.c_int]),
    "roaster_weight_sync_stats": (C.c_int, [C.POINTER(C.c_ulonglong), C.POINTER(C.c_int)]),
    "roaster_table_create": (_P, [C.POINTER(RoasterTableDesc)]),
    "roaster_table_create_layers": (_P, [C.POINTER(RoasterTableDesc), _P]),
    "roaster_gguf_scan": (C.c_int, [C.c_char_p, C.POINTER(RoasterGgufInfo)]),
    "roaster_matvec_q": (C.c_int, [_P, C.c_int, _P, _P, C.c_size_t, C.c_size_t, C.c_int]),
    "roaster_table_load_gguf": (_P, [C.c_char_p, C.POINTER(RoasterGgufInfo)]),
    "roaster_table_destroy": (None, [_P]),
    "roaster_table_bytes": (C.c_size_t, [_P]),
    "roaster_table_set_expert": (C.c_int, [_P, C.c_int, C.c_int, _P, _P, _P]),
    "roaster_table_set_exps": (C.c_int, [_P, C.c_int, C.c_int, _P, C.c_size_t]),
    "roaster_table_set_router": (C.c_int, [_P, C.c_int, _P, _P]),
    "roaster_table_expert_ptrs": (C.c_int, [_P, C.c_int, C.c_int, C.POINTER(_P), C.POINTER(_P),
                                            C.POINTER(_P)]),
    "roaster_synth_stream": (C.c_uint64, [C.c_int, C.c_int, C.c_int]),
    "roaster_synth_q4k": (None, [C.c_uint64, C.c_uint64, C.c_size_t, C.c_float, C.c_float, _P]),
    "roaster_synth_q6k": (None, [C.c_uint64, C.c_uint64, C.c_size_t, C.c_float, C.c_float, _P]),
    "roaster_synth_normal": (None, [C.c_uint64, C.c_uint64, C.c_size_t, C.c_float, _P]),
    "roaster_table_synth": (C.c_int, [_P, C.c_uint64, C.POINTER(RoasterSynthSpec)]),
    "roaster_moe_decode": (C.c_int, [_P, C.c_int, _P, C.c_int, _P, C.POINTER(RoasterDecodeIO)]),
    "roaster_moe_decode_stack": (C.c_int, [_P, _P, C.c_int, C.c_int, C.c_int, _P, C.c_float, _P, _P]),
    "roaster_moe_decode_stack_noalloc": (C.c_int, [_P, _P, C.c_int, C.c_int, C.c_int, _P, C.c_float, _P, _P]),
    "roaster_decode_fused_layer": (C.c_int, [C.c_int]),
    "roaster_decode_spin_limit": (C.c_uint, [C.c_uint]),
    "roaster_decode_cooperative_launch": (C.c_int, [C.c_int]),
    "roaster_decode_stack_kernel": (C.c_char_p, [_P, C.c_int, C.c_int, C.c_int]),
    "roaster_dense_mfma_min_tokens": (C.c_int, [C.c_int]),
    "roaster_moe_prefill": (C.c_int, [_P, C.c_int, _P, C.c_int, _P, C.POINTER(RoasterPrefillOpts)]),
    "roaster_prefill_balanced_down": (C.c_int, [C.c_int]),
    "roaster_prefill_persistent_gate_up": (C.c_int, [C.c_int]),
    "roaster_prefill_fused_gemm": (C.c_int, [C.c_int]),
}

_lib = None


def lib():
    """The loaded libroaster_moe.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()')")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIG.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def last_error():
    return lib().roaster_last_error().decode(errors="replace")


def check(rc, what="call"):
    if rc != OK:
        raise RuntimeError(f"{what} failed ({rc}): {last_error()}")
    return rc


def ptr(a):
    """Address of a numpy array's data (or a torch tensor's)."""
    if a is None:
        return None
    if hasattr(a, "data_ptr"):
        return a.data_ptr()
    return a.ctypes.data


# ---- synthetic inputs (host side, identical to the device generator) ----------
def synth_stream(layer, expert, kind):
    return lib().roaster_synth_stream(layer, expert, kind)


def synth_q4k(seed, stream, nblocks, lo=1e-3, hi=2e-2):
    out = np.empty(nblocks * Q4K_BYTES, dtype=np.uint8)
    lib().roaster_synth_q4k(seed, stream, nblocks, lo, hi, out.ctypes.data)
    return out


def synth_q6k(seed, stream, nblocks, lo=1e-3, hi=1e-2):
    out = np.empty(nblocks * Q6K_BYTES, dtype=np.uint8)
    lib().roaster_synth_q6k(seed, stream, nblocks, lo, hi, out.ctypes.data)
    return out


def synth_quant(q6, seed, stream, rows, cols, spec=None):
    nb = rows * (cols // QK)
    if q6:
        lo, hi = (spec.q6k_lo, spec.q6k_hi) if spec else (1e-3, 1e-2)
        return synth_q6k(seed, stream, nb, lo, hi)
    lo, hi = (spec.q4k_lo, spec.q4k_hi) if spec else (1e-3, 2e-2)
    return synth_q4k(seed, stream, nb, lo, hi)


def synth_normal(seed, stream, n, sigma=1.0):
    out = np.empty(n, dtype=np.float32)
    lib().roaster_synth_normal(seed, stream, n, sigma, out.ctypes.data)
    return out


def default_spec():
    return RoasterSynthSpec(1e-3, 2e-2, 1e-3, 1e-2, 0.02, 0.02)


def table_desc(n_layers=1, n_experts=256, hidden=2048, inter=512, q6=(0, 0, 1), sh_q6=(0, 0, 1)):
    d = RoasterTableDesc()
    d.n_layers, d.n_experts, d.hidden, d.inter = n_layers, n_experts, hidden, inter
    for i in range(3):
        d.q6[i] = q6[i]
        d.sh_q6[i] = sh_q6[i]
    return d


def matrix_bytes(q6, rows, cols):
    return rows * (cols // QK) * (Q6K_BYTES if q6 else Q4K_BYTES)


def host_expert(seed, layer, expert, desc, spec=None):
    """Host copy of the synthetic bytes roaster_table_synth writes for one expert
    (expert == n_experts is the shared expert): (gate, up, down) uint8 arrays."""
    shared = expert == desc.n_experts
    q6 = desc.sh_q6 if shared else desc.q6
    H, I = desc.hidden, desc.inter
    return (synth_quant(q6[0], seed, synth_stream(layer, expert, 0), I, H, spec),
            synth_quant(q6[1], seed, synth_stream(layer, expert, 1), I, H, spec),
            synth_quant(q6[2], seed, synth_stream(layer, expert, 2), H, I, spec))


def host_router(seed, layer, desc, spec=None):
    s = spec or default_spec()
    r = synth_normal(seed, synth_stream(layer, 0, 3), desc.n_experts * desc.hidden, s.router_sigma)
    g = synth_normal(seed, synth_stream(layer, 0, 4), desc.hidden, s.gate_inp_sigma)
    return r.reshape(desc.n_experts, desc.hidden), g
