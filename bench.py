"""MoE-FFN hot path benchmark on one MI355X.

Headline (value): batch-1 decode through the 40-layer MoE-FFN stack -- hidden
2048, 256 routed experts (top-8) + 1 shared expert per layer, gate/up Q4_K
[512 x 2048], down Q6_K [2048 x 512], F32 router, RMSNorm (eps 1e-6) carried
between layers -- with every expert resident in HBM (21.05 GB).  A step is one
token through all 40 layers (one launch).  Inputs and weights are synthetic
(seeded) and already in HBM when timing starts.

Also reported: batch-8 decode (8 slots, one token each) and the roofline of the
decode kernel (algorithmic bytes / average kernel time from HIP events on the
library's stream), plus the reference's CPU path (its own AVX2 kernels,
compiled from the reference tree into oracle/_ref) timed on this host.
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
N_LAYERS, E, H, I = 40, 256, 2048, 512
Q4_MAT = I * (H // 256) * 144          # 589,824
Q6_MAT = H * (I // 256) * 210          # 860,160
EXPERT_BYTES = 2 * Q4_MAT + Q6_MAT     # 2,039,808
ROUTER_BYTES = E * H * 4 + H * 4       # router + shared-gate vector


def decode_bytes(ids):
    """Algorithmic HBM bytes of one decode step: per layer the router, the
    shared-gate vector, every distinct selected expert once and the shared
    expert once.  ids: [layers, B, 8]."""
    total = 0
    for l in range(ids.shape[0]):
        total += ROUTER_BYTES + (len(set(ids[l].ravel().tolist())) + 1) * EXPERT_BYTES
    return total


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-tokens", type=int, default=40)
    return ap.parse_args()


def fetch_expert(R, table, seed, layer, e, desc):
    if table is None:
        return R.host_expert(seed, layer, e, desc)
    L = R.lib()
    ptrs = [C.c_void_p() for _ in range(3)]
    R.check(L.roaster_table_expert_ptrs(table, layer, e, *[C.byref(p) for p in ptrs]))
    out = []
    for p, n in zip(ptrs, (Q4_MAT, Q4_MAT, Q6_MAT)):
        a = np.empty(n, np.uint8)
        R.check(L.roaster_d2h(a.ctypes.data, p.value, n))
        out.append(a)
    return out


def cpu_baseline(table_seed, n_tokens, table=None):
    """The reference's CPU decode path (kernels.c AVX2 kernels via oracle/_ref,
    composed as model.c:1059-1146 does, one thread as the reference's OpenMP
    thresholds keep it) on a bounded sample: n_tokens tokens through all 40
    layers.  Expert bytes are copied from the device table (or regenerated on
    the host) outside the timed region."""
    import roaster_amd as R
    from oracle import oracle as O
    kind = "reference"
    if not O.ref_available():
        kind = "port"
    desc = R.table_desc(N_LAYERS)
    libm = C.CDLL("libm.so.6")
    libm.expf.restype = C.c_float
    libm.expf.argtypes = [C.c_float]
    ones = np.ones(H, np.float32)
    routers = {}
    total = 0.0
    for tk in range(n_tokens):
        h = R.synth_normal(table_seed, R.synth_stream(0, 1000 + tk, 5), H)
        for l in range(N_LAYERS):
            if l not in routers:
                routers[l] = R.host_router(table_seed, l, desc)
            router, gi = routers[l]
            xn = np.empty(H, np.float32)
            lg = np.empty(E, np.float32)
            ids = np.empty(8, np.int32)
            w = np.empty(8, np.float32)
            if kind == "reference":
                Rf = O.ref()
                Rf.kernel_rmsnorm(xn.ctypes.data, h.ctypes.data, ones.ctypes.data, H, C.c_float(1e-6))
                Rf.kernel_matvec_f32(router.ctypes.data, xn.ctypes.data, lg.ctypes.data, E, H)
                Rf.ref_select_top8(lg.ctypes.data, ids.ctypes.data, w.ctypes.data)
            else:
                O.orc().orc_rmsnorm(xn.ctypes.data, h.ctypes.data, ones.ctypes.data, H, C.c_float(1e-6))
                lg = O.matvec_f32(router, xn)
                ids, w = O.select_top8(lg)
            mats = [fetch_expert(R, table, table_seed, l, int(e), desc) for e in list(ids) + [E]]
            outs = np.empty((9, H), np.float32)
            t0 = time.perf_counter()
            if kind == "reference":
                Rf.kernel_rmsnorm(xn.ctypes.data, h.ctypes.data, ones.ctypes.data, H, C.c_float(1e-6))
                Rf.kernel_matvec_f32(router.ctypes.data, xn.ctypes.data, lg.ctypes.data, E, H)
                Rf.ref_select_top8(lg.ctypes.data, ids.ctypes.data, w.ctypes.data)
                g = np.empty(I, np.float32)
                u = np.empty(I, np.float32)
                for k, (gw, uw, dw) in enumerate(mats):
                    Rf.ref_matvec_q4_cpu(gw.ctypes.data, xn.ctypes.data, g.ctypes.data, I, H)
                    Rf.ref_matvec_q4_cpu(uw.ctypes.data, xn.ctypes.data, u.ctypes.data, I, H)
                    with np.errstate(over="ignore"):
                        eh = (g / (np.float32(1) + np.exp(-g))) * u
                    Rf.ref_matvec_q6_cpu(dw.ctypes.data, eh.ctypes.data, outs[k].ctypes.data, H, I)
                raw = Rf.kernel_dot_f32(gi.ctypes.data, xn.ctypes.data, H)
            else:
                for k, (gw, uw, dw) in enumerate(mats):
                    ex = O.OrcExpert(gw.ctypes.data, uw.ctypes.data, dw.ctypes.data, 0, 0, 1)
                    O.orc().orc_expert_decode(C.byref(ex), xn.ctypes.data, I, H, outs[k].ctypes.data)
                raw = O.orc().orc_dot_f32(gi.ctypes.data, xn.ctypes.data, H)
            sg = np.float32(1.0 / (1.0 + np.exp(-raw)))
            y = (w[:, None] * outs[:8]).sum(0) + sg * outs[8]
            h = (h + y).astype(np.float32)
            total += time.perf_counter() - t0
    tok_s = n_tokens / total
    return {"value": round(tok_s, 3), "unit": "tokens/s", "cores": 1, "kind": kind,
            "sample": f"{n_tokens} tokens x {N_LAYERS} layers of the batch-1 decode stack (router, top-8, "
                      f"8+1 experts, combine; {total:.2f} s of CPU work), same table seed"}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU: the MoE-FFN hot path is measured "
                                   "on one MI355X; see DESIGN.md for how it would shard"}))
        sys.exit(2)
    import torch
    import roaster_amd as R

    L = R.lib()
    dev = torch.device("cuda:0")
    torch.cuda.init()
    B = args.batch
    seed = 3
    desc = R.table_desc(N_LAYERS)
    t = L.roaster_table_create(C.byref(desc))
    assert t, R.last_error()
    R.check(L.roaster_table_synth(t, seed, None), "table_synth")
    stream = torch.cuda.ExternalStream(L.roaster_stream(), device=dev)
    h0 = torch.from_numpy(np.stack([R.synth_normal(seed, R.synth_stream(0, b, 5), H) for b in range(B)])).to(dev)
    h = torch.empty_like(h0)
    ids = torch.empty((N_LAYERS, B, 8), dtype=torch.int32, device=dev)
    torch.cuda.synchronize()

    def step():
        with torch.cuda.stream(stream):
            h.copy_(h0)
        rc = L.roaster_moe_decode_stack(t, h.data_ptr(), B, 0, N_LAYERS, None, C.c_float(1e-6),
                                        ids.data_ptr(), None)
        if rc:
            raise RuntimeError(R.last_error())

    for _ in range(args.warmup):
        step()
    R.check(L.roaster_sync(), "warmup")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    R.check(L.roaster_sync(), "timed steps")
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0

    # kernel-only duration with HIP events on the library's stream
    nev = min(args.steps, 50)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(nev)]
    for a, b in evs:
        with torch.cuda.stream(stream):
            h.copy_(h0)
            a.record(stream)
        rc = L.roaster_moe_decode_stack(t, h.data_ptr(), B, 0, N_LAYERS, None, C.c_float(1e-6), ids.data_ptr(), None)
        assert rc == 0
        with torch.cuda.stream(stream):
            b.record(stream)
    R.check(L.roaster_sync(), "event steps")
    kern_ms = float(np.mean([a.elapsed_time(b) for a, b in evs]))
    ids_np = ids.cpu().numpy()
    nbytes = decode_bytes(ids_np)
    achieved = nbytes / (kern_ms * 1e-3) / 1e9

    ms = elapsed / args.steps * 1e3
    line = {
        "metric": "MoE-FFN decode tok/s (batch %d, 40-layer stack)" % B,
        "value": round(B * args.steps / elapsed, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k/q6_k weights, f32 activations and accumulation",
        "data": "synthetic (seeded random Q4_K/Q6_K experts, F32 routers, N(0,1) hidden state)",
        "config": {"workload": "40-layer MoE-FFN decode stack, batch %d" % B, "hidden": H, "inter": I,
                   "experts": E, "top_k": 8, "shared_experts": 1, "layers": N_LAYERS,
                   "gate_up": "Q4_K", "down": "Q6_K", "resident_table_bytes": int(L.roaster_table_bytes(t))},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "moe_decode_kernel", "kernel_ms": round(kern_ms, 5),
                     "algorithmic_bytes_per_launch": int(nbytes)},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(seed, args.cpu_tokens, t)
    L.roaster_table_destroy(t)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
