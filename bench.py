"""MoE-FFN hot path benchmark on one MI355X.

Headline (value): batch-1 decode through the 40-layer MoE-FFN stack -- hidden
2048, 256 routed experts (top-8) + 1 shared expert per layer, gate/up Q4_K
[512 x 2048], down Q6_K [2048 x 512], F32 router, RMSNorm (eps 1e-6) carried
between layers -- with every expert resident in HBM (21.05 GB in the GGML layout
the decode kernels read, plus the 22.9 GB MFMA tile-layout copy the prefill
GEMMs read).  A step is one token through all 40 layers (one library call: one
launch for the whole stack, at batch 1 and at batches 2-8).  Inputs
and weights are synthetic (seeded) and already in HBM when timing starts.

Also reported in the same JSON line:
  batch2, batch4, batch8 -- 2, 4, 8 slots, one token each, through the same
              stack (the batched one-launch kernels);
  prefill  -- the MoE block over T tokens: 2048 tokens through 4 all-Q6_K
              layers with N(0,1) logits given (its value, MFMA roofline and CPU
              baseline), and 512 tokens through one Q4_K/Q6_K layer with the
              router and a Zipf(1.1) per-expert logit bias (HBM-bound roofline);
  config1  -- one Q4_K [512 x 2048] matvec: cache-resident latency and the HBM
              rate over 512 rotated copies;
  config2  -- one decode MoE block: device time and isolated latency;
  dense    -- the LM head [248320 x 2048] Q6_K as a dense projection, 1 and 8
              tokens, with its HBM roofline;
  roofline / cpu_baseline -- see below; roofline.traffic is read from the
              committed rocprofv3 counter summary profiles/traffic_per_step.md.
Kernel times come from HIP events recorded on the library's stream.  The CPU
baselines run the reference's own C kernels (compiled from the reference tree
into oracle/_ref) on a bounded sample of the same workloads on this host.
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

# The prefill CPU baselines run the reference's OpenMP kernels: threads bound
# close to each other, one per physical core.  Set before torch loads: its
# bundled libgomp (which the reference build binds to as well, by soname) reads
# them once, and then binds the initial thread to the first core, so the CPUs
# this process may use are recorded first.
_CPUS0 = sorted(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else list(range(os.cpu_count() or 1))
os.environ.setdefault("OMP_PROC_BIND", "close")
os.environ.setdefault("OMP_PLACES", "cores")

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
TRAFFIC_SOURCE = "profiles/traffic_per_step.md (rocprofv3 FETCH_SIZE / WRITE_SIZE passes, copy-calibrated)"

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0          # dense fp16 / bf16
N_LAYERS, E, H, I = 40, 256, 2048, 512
Q4_MAT = I * (H // 256) * 144          # 589,824
Q6_MAT = H * (I // 256) * 210          # 860,160
Q6_GU = I * (H // 256) * 210           # 860,160 (all-Q6_K gate / up)
EXPERT_BYTES = 2 * Q4_MAT + Q6_MAT     # 2,039,808
EXPERT_BYTES_Q6 = 3 * Q6_GU            # 2,580,480
ROUTER_BYTES = E * H * 4 + H * 4       # router + shared-gate vector
FFN_FLOPS_PER_ROW = 6 * H * I          # gate + up + down per (token, expert) row


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
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill legs")
    ap.add_argument("--cpu-tokens", type=int, default=160)
    ap.add_argument("--prefill-reps", type=int, default=10)
    ap.add_argument("--fused-mode", type=int, default=None,
                    help="roaster_decode_fused_layer mode: 1 default one-launch kernels, 2 the one-token kernel "
                         "with the three-kernel path's arithmetic, 0 three kernels per layer")
    ap.add_argument("--three-kernel", action="store_true",
                    help="decode one token's layers with three launches each instead of one (for comparison)")
    ap.add_argument("--legs", default="decode,prefill,config1,config2,dense",
                    help="comma-separated legs to run (the decode headline always runs unless omitted here); "
                         "prefill5 / prefill3 run one prefill workload alone (config 5 / config 3)")
    return ap.parse_args()


def bf16_round(a):
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def zipf_bias(n, seed, s=1.1, tau=0.3):
    """tau * ln(p_e), p_e proportional to rank_e^-s, ranks permuted by seed."""
    perm = np.random.default_rng(seed).permutation(n)
    rank = np.empty(n, np.float64)
    rank[perm] = np.arange(1, n + 1)
    p = rank ** -s
    p /= p.sum()
    return (tau * np.log(p)).astype(np.float32)


def fetch_expert(R, table, seed, layer, e, desc):
    if table is None:
        return R.host_expert(seed, layer, e, desc)
    L = R.lib()
    ptrs = [C.c_void_p() for _ in range(3)]
    R.check(L.roaster_table_expert_ptrs(table, layer, e, *[C.byref(p) for p in ptrs]))
    sizes = [R.matrix_bytes(desc.q6[0] if e < desc.n_experts else desc.sh_q6[0], desc.inter, desc.hidden),
             R.matrix_bytes(desc.q6[1] if e < desc.n_experts else desc.sh_q6[1], desc.inter, desc.hidden),
             R.matrix_bytes(desc.q6[2] if e < desc.n_experts else desc.sh_q6[2], desc.hidden, desc.inter)]
    out = []
    for p, n in zip(ptrs, sizes):
        a = np.empty(n, np.uint8)
        R.check(L.roaster_d2h(a.ctypes.data, p.value, n))
        out.append(a)
    return out


def omp_threads():
    try:
        return int(C.CDLL("libgomp.so.1").omp_get_max_threads())
    except OSError:
        return int(os.environ.get("OMP_NUM_THREADS", "1"))


def socket_cores():
    """Physical cores of one socket among the CPUs this process may run on
    (the socket with the most of them): the prefill CPU baseline's thread
    count."""
    cpus = _CPUS0                    # before the OpenMP runtime bound this thread
    per_pkg = {}
    for c in cpus:
        base = "/sys/devices/system/cpu/cpu%d/topology/" % c
        try:
            with open(base + "physical_package_id") as f:
                pkg = int(f.read())
            with open(base + "core_id") as f:
                core = int(f.read())
        except (OSError, ValueError):
            pkg, core = 0, c
        per_pkg.setdefault(pkg, set()).add(core)
    return max(len(v) for v in per_pkg.values()) if per_pkg else 1


def set_omp_threads(n):
    """The reference kernels' OpenMP team size (omp_set_num_threads on the
    loaded runtime, before its parallel regions run); returns the team size in
    force."""
    try:
        g = C.CDLL("libgomp.so.1")
        g.omp_set_num_threads(int(n))
        return int(g.omp_get_max_threads())
    except OSError:
        return omp_threads()


def host_cpu():
    """CPU model and the SIMD extensions the reference's CPU kernels use
    (kernels.c picks its AVX2 / FMA / F16C paths at compile time)."""
    model, flags = None, set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if model is None and line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                elif not flags and line.startswith("flags"):
                    flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    return {"cpu_model": model, "isa": [x for x in ("avx2", "fma", "f16c") if x in flags],
            "build": "gcc -O3 -mavx2 -mfma -mf16c -fopenmp (kernels.c CPU subset compiled from the reference tree)"}


def profiled_traffic(workload):
    """HBM traffic per step of `workload` from the committed counter summary
    (profiles/traffic_per_step.md: FETCH_SIZE and WRITE_SIZE passes of
    rocprofv3, scaled by the copy-kernel calibration stated there), or None."""
    path = os.path.join(ROOT, "profiles", "traffic_per_step.md")
    try:
        with open(path) as f:
            for line in f:
                cells = [c.strip() for c in line.strip().strip("|").split("|")]
                if len(cells) >= 3 and cells[0] == workload:
                    return int(cells[1].replace(",", "")) + int(cells[2].replace(",", ""))
    except (OSError, ValueError):
        pass
    return None


def cpu_baseline_decode(table_seed, n_tokens, table=None, n_layers=N_LAYERS, x_stream=1000):
    """The reference's CPU decode path (kernels.c AVX2 kernels via oracle/_ref,
    composed as model.c:1059-1146 does, one thread as the reference's OpenMP
    thresholds keep it) on a bounded sample: n_tokens tokens through all 40
    layers.  Expert bytes are copied from the device table outside the timed
    region."""
    import roaster_amd as R
    from oracle import oracle as O
    kind = "reference" if O.ref_available() else "port"
    desc = R.table_desc(N_LAYERS)
    ones = np.ones(H, np.float32)
    routers = {}
    total = 0.0
    for tk in range(n_tokens):
        h = R.synth_normal(table_seed, R.synth_stream(0, x_stream + tk, 5), H)
        for l in range(n_layers):
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
    out = {"value": round(tok_s, 3), "unit": "tokens/s", "cores": 1, "kind": kind,
           "sample": f"{n_tokens} tokens x {n_layers} layers of the batch-1 decode stack (router, top-8, "
                     f"8+1 experts, combine; {total:.2f} s of CPU work), same table seed",
           "us_per_layer": round(total / (n_tokens * n_layers) * 1e6, 2)}
    out.update(host_cpu())
    return out


def cpu_baseline_prefill(table, desc, seed, X, ids, layer=0, with_router=True, reps=2, label=""):
    """The reference's CPU prefill block (model.c:1671-1791 composed over its
    kernels.c routines via oracle/_ref: the router matvec per token when the
    workload has one, moe_cpu over the expert row groups -- OpenMP-parallel
    over 32-row tiles as kernels.c:1882 is -- and moe_cpu for the shared
    expert over all T tokens) with the GPU's routing ids [T x 8].  Gathers and
    the combine are outside the timed region."""
    import roaster_amd as R
    from oracle import oracle as O
    if not O.ref_available():
        return None
    Rf = O.ref()
    T = X.shape[0]
    router, gi = R.host_router(seed, layer, desc)
    groups = []
    for e in range(E):
        rows = np.nonzero((ids == e).any(axis=1))[0]
        if len(rows):
            groups.append((e, rows))
    mats = {e: fetch_expert(R, table, seed, layer, e, desc) for e in [g[0] for g in groups] + [E]}
    n_tot = sum(len(r) for _, r in groups)
    Xg = np.ascontiguousarray(np.concatenate([X[r] for _, r in groups]))
    Dg = np.empty((n_tot, H), np.float32)
    exs = (R.KernelMoeExpert * len(groups))()
    for i, (e, rows) in enumerate(groups):
        g, u, d = mats[e]
        exs[i] = R.KernelMoeExpert(g.ctypes.data, u.ctypes.data, d.ctypes.data, desc.q6[0], desc.q6[1], desc.q6[2], len(rows))
    sh = (R.KernelMoeExpert * 1)()
    g, u, d = mats[E]
    sh[0] = R.KernelMoeExpert(g.ctypes.data, u.ctypes.data, d.ctypes.data, desc.sh_q6[0], desc.sh_q6[1], desc.sh_q6[2], T)
    Ds = np.empty((T, H), np.float32)
    lg = np.empty(E, np.float32)
    X = np.ascontiguousarray(X, np.float32)
    threads = set_omp_threads(socket_cores())
    best = None
    for _ in range(reps):
        t0 = time.perf_counter()
        if with_router:
            for t in range(T):
                Rf.kernel_matvec_f32(router.ctypes.data, X[t].ctypes.data, lg.ctypes.data, E, H)
        Rf.ref_moe_cpu(C.cast(sh, C.c_void_p), 1, X.ctypes.data, Ds.ctypes.data, I, H)
        Rf.ref_moe_cpu(C.cast(exs, C.c_void_p), len(groups), Xg.ctypes.data, Dg.ctypes.data, I, H)
        dt = time.perf_counter() - t0
        best = dt if best is None else min(best, dt)
    out = {"value": round(T / best, 1), "unit": "tokens/s", "cores": threads, "kind": "reference",
           "sample": f"one {T}-token {label} layer ({'router + ' if with_router else ''}{len(groups)} expert groups "
                     f"+ shared expert via the reference moe_cpu), best of {reps}: {best:.3f} s",
           "threads": f"{threads} OpenMP threads = physical cores of one socket among the "
                      f"{len(_CPUS0)} CPUs this process may use; OMP_PROC_BIND="
                      f"{os.environ.get('OMP_PROC_BIND')}, OMP_PLACES={os.environ.get('OMP_PLACES')}"}
    out.update(host_cpu())
    return out


def warm(L, R, fn, n, what):
    """n untimed calls of fn, then a synchronisation: the timed calls that follow
    see the steady state (the first timed pass after a single warm-up call
    measured about 10% slower than the following ones)."""
    for _ in range(n):
        fn()
    R.check(L.roaster_sync(), what)


def event_ms(torch, stream, fn, reps):
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(reps):
        fn()
    b.record(stream)
    b.synchronize()
    return a.elapsed_time(b) / reps


def prefill_legs(torch, L, R, dev, stream, reps, with_cpu, parts=("q6", "zipf", "api")):
    """Prefill: config 5 (all-Q6_K, 2048 tokens x 4 layers, N(0,1) logits
    given) is the line's prefill value with its MFMA roofline; config 3 (512
    Zipf-routed tokens through one Q4_K/Q6_K layer with the router) is
    HBM-bound and reported against min(MFMA peak, AI x HBM peak); "api" adds
    the kernels.h kernel_moe_prefill leg on the config-3 layer."""
    out = {}
    if "q6" in parts:
        out = prefill_q6_leg(torch, L, R, dev, stream, reps, with_cpu)
    if "zipf" in parts:
        z = prefill_zipf_leg(torch, L, R, dev, stream, reps, with_cpu, "api" in parts)
        out["zipf_512x1"] = z
        # scalar copies of the Zipf layer's figures
        out["zipf_tokens_per_s"] = z["tokens_per_s"]
        out["zipf_roofline_frac"] = z["roofline"]["frac"]
        out["zipf_traffic_bytes"] = z["roofline"]["traffic"]
        if "cpu_baseline" in z:
            out["zipf_cpu_baseline_tok_s"] = z["cpu_baseline"]["value"]
    return out


def prefill_q6_leg(torch, L, R, dev, stream, reps, with_cpu):
    """Config 5: all-Q6_K, T = 2048, 4 layers, N(0,1) logits given (no router)."""
    T, NL, seed = 2048, 4, 4
    desc = R.table_desc(NL, q6=(1, 1, 1), sh_q6=(1, 1, 1))
    t = L.roaster_table_create(C.byref(desc))
    assert t, R.last_error()
    try:
        R.check(L.roaster_table_synth(t, seed, None), "table_synth")
        Xh5 = bf16_round(np.stack([R.synth_normal(seed, R.synth_stream(0, i, 5), H) for i in range(T)]))
        X = torch.from_numpy(Xh5).to(dev)
        lg = [torch.from_numpy(np.stack([R.synth_normal(seed, R.synth_stream(l, i, 7), E) for i in range(T)])).to(dev)
              for l in range(NL)]
        Y = torch.empty_like(X)
        cnt = torch.empty((NL, E), dtype=torch.int32, device=dev)
        ids0 = torch.empty((T, 8), dtype=torch.int32, device=dev)
        torch.cuda.synchronize()
        opts = [R.RoasterPrefillOpts(R.PREC_F16, lg[l].data_ptr(), None, None, ids0.data_ptr() if l == 0 else None,
                                     None, cnt[l].data_ptr()) for l in range(NL)]

        def run():
            for l in range(NL):
                rc = L.roaster_moe_prefill(t, l, X.data_ptr(), T, Y.data_ptr(), C.byref(opts[l]))
                if rc:
                    raise RuntimeError(R.last_error())

        warm(L, R, run, reps, "prefill warmup")
        ms = event_ms(torch, stream, run, reps)
        R.check(L.roaster_sync(), "prefill")
        counts = cnt.cpu().numpy()
        rows = int(counts.sum()) + NL * T                     # routed rows + shared rows
        flops = rows * FFN_FLOPS_PER_ROW
        # algorithmic bytes: each hit expert once + shared, X read (f32) and Y written (f32), logits read
        nbytes = sum(((int((counts[l] > 0).sum()) + 1) * EXPERT_BYTES_Q6) for l in range(NL)) \
            + NL * (T * H * 4 * 2 + T * E * 4)
        tf = flops / (ms * 1e-3) / 1e12
        gbs = nbytes / (ms * 1e-3) / 1e9
        ai = flops / nbytes
        tok_s = T / (ms * 1e-3)
        out = {
            "metric": "MoE-FFN prefill tok/s (all-Q6_K experts, 2048 tokens x 4 layers, one MI355X)",
            "value": round(tok_s, 1), "unit": "tokens/s", "tokens_per_s": round(tok_s, 1), "tok_s": round(tok_s, 1),
            "higher_is_better": True, "ms_per_pass": round(ms, 4), "layers": NL, "ms_per_layer": round(ms / NL, 4),
            "dtype": "fp16 MFMA operands (activations row-scaled by powers of two), fp32 accumulation; "
                     "per-(token, expert) down rows stored in fp16 (row-scaled by a power of two of their bound), "
                     "combined in fp32",
            "config": {"workload": "all-Q6_K MoE prefill, 2048 tokens x 4 layers, logits ~ N(0,1) given, seed 4",
                       "hidden": H, "inter": I, "experts": E, "top_k": 8, "shared_experts": 1},
            "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tf / MFMA_PEAK_TFLOPS, 4), "traffic": profiled_traffic("prefill_q6_2048_layer"),
                         "kernel": "whole prefill block (6 kernels per layer)",
                         "algorithmic_flops_per_layer": int(flops // NL),
                         "algorithmic_bytes_per_layer": int(nbytes // NL), "arithmetic_intensity": round(ai, 1),
                         "frac_of_min_peak_ai_bw": round(tf / min(MFMA_PEAK_TFLOPS, ai * HBM_PEAK_GBS / 1000), 4)},
            "hbm_GBps_algorithmic": round(gbs, 1)}
        # scalar copies (a parser keeping only scalar fields keeps these)
        out["roofline_frac"] = out["roofline"]["frac"]
        out["achieved_TFLOPs"] = out["roofline"]["achieved"]
        out["frac_of_min_peak_ai_bw"] = out["roofline"]["frac_of_min_peak_ai_bw"]
        out["traffic_bytes_per_layer"] = out["roofline"]["traffic"]
        if with_cpu:
            cb = cpu_baseline_prefill(t, desc, seed, Xh5, ids0.cpu().numpy(), layer=0, with_router=False,
                                      label="all-Q6_K (logits given)")
            if cb:
                out["cpu_baseline"] = cb
                out["cpu_baseline_tok_s"] = cb["value"]
                out["cpu_threads"] = cb["cores"]
    finally:
        L.roaster_table_destroy(t)
    return out


def prefill_zipf_leg(torch, L, R, dev, stream, reps, with_cpu, with_api):
    """Config 3: Q4_K/Q6_K, T = 512, router + Zipf bias, one layer."""
    T, seed = 512, 2
    desc = R.table_desc(1)
    t = L.roaster_table_create(C.byref(desc))
    assert t, R.last_error()
    try:
        R.check(L.roaster_table_synth(t, seed, None), "table_synth")
        Xh = bf16_round(np.stack([R.synth_normal(seed, R.synth_stream(0, i, 5), H) for i in range(T)]))
        X = torch.from_numpy(Xh).to(dev)
        bias = torch.from_numpy(zipf_bias(E, seed)).to(dev)
        Y = torch.empty_like(X)
        ids = torch.empty((T, 8), dtype=torch.int32, device=dev)
        torch.cuda.synchronize()
        o = R.RoasterPrefillOpts(R.PREC_F16, None, bias.data_ptr(), None, ids.data_ptr(), None, None)

        def run3():
            rc = L.roaster_moe_prefill(t, 0, X.data_ptr(), T, Y.data_ptr(), C.byref(o))
            if rc:
                raise RuntimeError(R.last_error())

        warm(L, R, run3, reps, "prefill warmup")
        ms = event_ms(torch, stream, run3, reps)
        R.check(L.roaster_sync(), "prefill")
        idh = ids.cpu().numpy()
        n_hit = len(set(idh.ravel().tolist()))
        flops = 9 * T * FFN_FLOPS_PER_ROW + T * (E + 1) * H * 2
        nbytes = (n_hit + 1) * EXPERT_BYTES + ROUTER_BYTES + 2 * T * H * 4
        ai = flops / nbytes
        roof_tf = min(MFMA_PEAK_TFLOPS, ai * HBM_PEAK_GBS / 1000)
        tf = flops / (ms * 1e-3) / 1e12
        gbs = nbytes / (ms * 1e-3) / 1e9
        leg = {"tokens_per_s": round(T / (ms * 1e-3), 1), "ms_per_layer": round(ms, 4),
               "config": {"workload": "Q4_K/Q6_K MoE prefill, 512 tokens x 1 layer, router + Zipf(1.1) expert bias, "
                                      "seed 2", "experts_hit": n_hit},
               "roofline": {"bound": "hbm" if roof_tf < MFMA_PEAK_TFLOPS else "mfma", "achieved": round(gbs, 1),
                            "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(tf / roof_tf, 4),
                            "traffic": profiled_traffic("prefill_zipf_512_layer"),
                            "algorithmic_bytes": int(nbytes), "algorithmic_flops": int(flops),
                            "arithmetic_intensity": round(ai, 1), "achieved_TFLOPs": round(tf, 2),
                            "roof_TFLOPs": round(roof_tf, 1), "frac_mfma_peak": round(tf / MFMA_PEAK_TFLOPS, 4)}}
        if with_api:
            leg["kernels_h_moe_prefill"] = moe_prefill_hostbuf_leg(L, R, t, desc, seed, Xh, idh)
        if with_cpu:
            cb = cpu_baseline_prefill(t, desc, seed, Xh, idh, layer=0, with_router=True, label="Zipf-routed Q4_K/Q6_K")
            if cb:
                leg["cpu_baseline"] = cb
    finally:
        L.roaster_table_destroy(t)
    return leg


def moe_prefill_hostbuf_leg(L, R, table, desc, seed, X, ids, reps=3):
    """The drop-in path for the same layer: the expert row groups of the
    Zipf-routed 512 tokens through kernels.h kernel_moe_prefill on host
    buffers, in calls of at most 32 experts as pf_moe makes them
    (model.c:1736-1742), plus the shared expert over all tokens as one more
    group; weights in kernel_vk_alloc_weights memory as weights.c allocates
    them.  Host wall clock, including the X upload and D download over PCIe;
    the first pass (weight upload into HBM) is not timed."""
    T = X.shape[0]
    groups = []
    for e in range(E):
        rows = np.nonzero((ids == e).any(axis=1))[0]
        if len(rows):
            groups.append((e, rows))
    granted = C.c_size_t(0)
    host = {}
    for e in [g[0] for g in groups] + [E]:
        mats = fetch_expert(R, table, seed, 0, e, desc)
        ptrs = []
        for a in mats:
            p = L.kernel_vk_alloc_weights(a.nbytes, C.byref(granted))
            assert p, R.last_error()
            C.memmove(p, a.ctypes.data, a.nbytes)
            ptrs.append(p)
        host[e] = ptrs
    calls = []
    for c0 in range(0, len(groups), 32):
        chunk = groups[c0:c0 + 32]
        Xg = np.ascontiguousarray(np.concatenate([X[r] for _, r in chunk]), np.float32)
        Dg = np.empty_like(Xg)
        arr = (R.KernelMoeExpert * len(chunk))()
        for i, (e, r) in enumerate(chunk):
            g, u, d = host[e]
            arr[i] = R.KernelMoeExpert(g, u, d, desc.q6[0], desc.q6[1], desc.q6[2], len(r))
        calls.append((arr, len(chunk), Xg, Dg))
    g, u, d = host[E]
    sh = (R.KernelMoeExpert * 1)()
    sh[0] = R.KernelMoeExpert(g, u, d, desc.sh_q6[0], desc.sh_q6[1], desc.sh_q6[2], T)
    Xs = np.ascontiguousarray(X, np.float32)
    calls.append((sh, 1, Xs, np.empty_like(Xs)))
    best = None
    for rep in range(reps + 1):
        t0 = time.perf_counter()
        for arr, n, Xg, Dg in calls:
            if L.kernel_moe_prefill(arr, n, Xg.ctypes.data, Dg.ctypes.data, I, H) != 0:
                raise RuntimeError(R.last_error())
        dt = time.perf_counter() - t0
        if rep:
            best = dt if best is None else min(best, dt)
    rows = sum(len(r) for _, r in groups) + T
    return {"tokens_per_s": round(T / best, 1), "ms_per_layer": round(best * 1e3, 3), "calls": len(calls),
            "expert_rows": int(rows), "precision": "split bf16 hi+lo operands, fp32 accumulation (MFMA)",
            "note": "host wall clock incl. PCIe transfers of X and D; router and combine not included"}


def config1_leg(torch, L, R, dev, stream, with_cpu):
    """Config 1: one Q4_K [512 x 2048] dequant-matvec (seed 0) through
    roaster_matvec_q on device buffers.  Back-to-back calls on one copy give
    the cache-resident latency; calls rotating over 512 copies (302 MB, beyond
    the 256 MB Infinity Cache) give the HBM rate.  The reference's
    matvec_q4_cpu (kernels.c:407-432, one thread as its OpenMP threshold keeps
    it) is timed beside it."""
    rows, cols, ncopy = 512, 2048, 512
    W = R.synth_q4k(0, R.synth_stream(0, 0, 0), rows * cols // 256)
    x = R.synth_normal(0, R.synth_stream(0, 0, 5), cols)
    dW = torch.from_numpy(np.tile(W, ncopy)).to(dev)
    dx = torch.from_numpy(x).to(dev)
    dy = torch.empty(rows, dtype=torch.float32, device=dev)
    mb = W.nbytes

    def one(i):
        rc = L.roaster_matvec_q(dW.data_ptr() + i * mb, 0, dx.data_ptr(), dy.data_ptr(), rows, cols, 1)
        if rc:
            raise RuntimeError(R.last_error())

    warm(L, R, lambda: one(0), 50, "config1 warmup")
    hot_ms = event_ms(torch, stream, lambda: one(0), 200)
    it = iter(range(10 ** 9))
    rot_ms = event_ms(torch, stream, lambda: one(next(it) % ncopy), 2 * ncopy)
    # the same 512 copies as one [262144 x 2048] matrix in one launch: the kernel's streaming rate
    dY = torch.empty(rows * ncopy, dtype=torch.float32, device=dev)
    big = lambda: R.check(L.roaster_matvec_q(dW.data_ptr(), 0, dx.data_ptr(), dY.data_ptr(), rows * ncopy, cols, 1))
    one_ms = event_ms(torch, stream, big, 20)
    R.check(L.roaster_sync(), "config1")
    nbytes = mb + cols * 4 + rows * 4
    gbs = nbytes / (rot_ms * 1e-3) / 1e9
    gbs_one = ncopy * mb / (one_ms * 1e-3) / 1e9
    out = {"workload": "Q4_K [512 x 2048] matvec, seed 0", "algorithmic_bytes": int(nbytes),
           "us_per_call_cache_resident": round(hot_ms * 1e3, 3), "us_per_call_rotating_512_copies": round(rot_ms * 1e3, 3),
           "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": profiled_traffic("config1_matvec"),
                        "traffic_source": TRAFFIC_SOURCE,
                        "kernel": "dense_mv_kernel (one launch per matvec, 512 rotated copies)"},
           "streaming_512_copies_one_launch": {"us": round(one_ms * 1e3, 1), "GBps": round(gbs_one, 1),
                                               "frac_hbm_peak": round(gbs_one / HBM_PEAK_GBS, 4)}}
    if with_cpu:
        from oracle import oracle as O
        if O.ref_available():
            Rf = O.ref()
            y = np.empty(rows, np.float32)
            n = 0
            t0 = time.perf_counter()
            while time.perf_counter() - t0 < 1.0:
                Rf.ref_matvec_q4_cpu(W.ctypes.data, x.ctypes.data, y.ctypes.data, rows, cols)
                n += 1
            dt = (time.perf_counter() - t0) / n
            cb = {"value": round(1e6 * dt, 2), "unit": "us per matvec", "cores": 1, "kind": "reference",
                  "sample": f"{n} calls of matvec_q4_cpu on the same matrix (cache-resident) over 1 s",
                  "GBps": round(nbytes / dt / 1e9, 2)}
            cb.update(host_cpu())
            out["cpu_baseline"] = cb
    return out


def config2_leg(torch, L, R, dev, stream, with_cpu):
    """Config 2: one decode MoE block (router -> top-8 -> 8 + 1 experts ->
    combine, seed 1) through roaster_moe_decode.  Back-to-back calls give the
    per-block device time; single calls with a host sync around each give the
    isolated latency.  The reference's CPU block (model.c:1059-1146 over its
    kernels.c routines, one thread) is timed beside it."""
    seed = 1
    desc = R.table_desc(1)
    t = L.roaster_table_create(C.byref(desc))
    assert t, R.last_error()
    try:
        R.check(L.roaster_table_synth(t, seed, None), "table_synth")
        x = torch.from_numpy(R.synth_normal(seed, R.synth_stream(0, 0, 5), H)).to(dev)
        y = torch.empty_like(x)
        torch.cuda.synchronize()

        def run():
            rc = L.roaster_moe_decode(t, 0, x.data_ptr(), 1, y.data_ptr(), None)
            if rc:
                raise RuntimeError(R.last_error())

        warm(L, R, run, 50, "config2 warmup")
        dev_ms = event_ms(torch, stream, run, 200)
        lat = []
        for _ in range(50):
            t0 = time.perf_counter()
            run()
            R.check(L.roaster_sync(), "config2")
            lat.append(time.perf_counter() - t0)
        nbytes = ROUTER_BYTES + 9 * EXPERT_BYTES
        gbs = nbytes / (dev_ms * 1e-3) / 1e9
        out = {"workload": "one decode MoE block, 1 token, hidden 2048, 256 experts top-8 + shared, seed 1",
               "us_per_block_device": round(dev_ms * 1e3, 2), "us_per_block_isolated_median": round(
                   float(np.median(lat)) * 1e6, 1), "algorithmic_bytes": nbytes,
               "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": profiled_traffic("config2_block"),
                            "traffic_source": TRAFFIC_SOURCE,
                            "kernel": L.roaster_decode_stack_kernel(t, 1, 0, 1).decode() + " (one launch per block)",
                            "note": "the block's 20.5 MB stay in the 256 MB Infinity Cache between calls: "
                                    "a latency figure, not an HBM rate"}}
        if with_cpu:
            out["cpu_baseline"] = cpu_baseline_decode(seed, 200, t, n_layers=1, x_stream=0)
    finally:
        L.roaster_table_destroy(t)
    return out


def dense_leg(torch, L, R, dev, stream):
    """Dense quantised projections through roaster_matvec_q (model.c:113-121):
    the LM head Q6_K [248320 x 2048] (model.c:1368-1370) and the attention
    output projection Q4_K [2048 x 4096] (model.c:862) at 1 and 8 tokens (8:
    the quants-on-MFMA kernel, the default from 2 tokens, and for comparison
    the dequantising matvec, "T8_valu").
    Device time from HIP events, HBM roofline over the matrix bytes."""
    out = {}
    for name, q6, rows, cols in (("lm_head_q6k_248320x2048", 1, 248320, 2048), ("attn_out_q4k_2048x4096", 0, 2048, 4096)):
        nb = rows * (cols // 256)
        W = R.synth_q6k(5, R.synth_stream(0, 0, 9), nb) if q6 else R.synth_q4k(5, R.synth_stream(0, 0, 9), nb)
        dw = torch.from_numpy(W).to(dev)
        leg = {"matrix_bytes": int(W.nbytes)}
        for T, mfma in ((1, False), (8, True), (8, False)):
            x = torch.from_numpy(np.stack([R.synth_normal(5, R.synth_stream(0, t, 5), cols) for t in range(T)])).to(dev)
            y = torch.empty((T, rows), dtype=torch.float32, device=dev)
            old = L.roaster_dense_mfma_min_tokens(0)
            L.roaster_dense_mfma_min_tokens(2 if mfma else 9)

            def run():
                rc = L.roaster_matvec_q(dw.data_ptr(), q6, x.data_ptr(), y.data_ptr(), rows, cols, T)
                if rc:
                    raise RuntimeError(R.last_error())
            warm(L, R, run, 10, "dense warmup")
            ms = event_ms(torch, stream, run, 50 if rows > 100000 else 200)
            L.roaster_dense_mfma_min_tokens(old)
            gbs = W.nbytes / (ms * 1e-3) / 1e9
            leg["T%d%s" % (T, "_valu" if T > 1 and not mfma else "")] = {
                "us": round(ms * 1e3, 2), "tokens_per_s": round(T / (ms * 1e-3), 1),
                "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(gbs / HBM_PEAK_GBS, 4)}}
        out[name] = leg
    return out


def decode_legs(args, torch, L, R, dev, stream):
    """The headline: batch-`args.batch` decode through the 40-layer stack (host
    wall clock over --steps steps, device time from HIP events), batches 2, 4, 8 and
    the reference CPU decode beside it."""
    seed = 3
    desc = R.table_desc(N_LAYERS)
    t = L.roaster_table_create(C.byref(desc))
    assert t, R.last_error()
    R.check(L.roaster_table_synth(t, seed, None), "table_synth")

    def stack_setup(B):
        h0 = torch.from_numpy(np.stack([R.synth_normal(seed, R.synth_stream(0, b, 5), H) for b in range(B)])).to(dev)
        return h0, torch.empty_like(h0), torch.empty((N_LAYERS, B, 8), dtype=torch.int32, device=dev)

    def stack_step(B, h0, h, ids):
        with torch.cuda.stream(stream):
            h.copy_(h0)
        rc = L.roaster_moe_decode_stack(t, h.data_ptr(), B, 0, N_LAYERS, None, C.c_float(1e-6), ids.data_ptr(), None)
        if rc:
            raise RuntimeError(R.last_error())

    B = args.batch
    h0, h, ids = stack_setup(B)
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        stack_step(B, h0, h, ids)
    R.check(L.roaster_sync(), "warmup")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        stack_step(B, h0, h, ids)
    R.check(L.roaster_sync(), "timed steps")
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0

    # device time per step with HIP events on the library's stream
    kern_ms = event_ms(torch, stream, lambda: stack_step(B, h0, h, ids), min(args.steps, 50))
    R.check(L.roaster_sync(), "event steps")
    nbytes = decode_bytes(ids.cpu().numpy())
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
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": profiled_traffic("decode_b%d_step" % B),
                     "traffic_source": TRAFFIC_SOURCE,
                     "kernel": "decode stack: %s" % L.roaster_decode_stack_kernel(t, B, 0, N_LAYERS).decode(),
                     "kernel_ms": round(kern_ms, 5), "algorithmic_bytes_per_launch": int(nbytes)},
    }
    if B == 1:
        for nb in (2, 4, 8):              # the batched one-launch stack (dec_stackB<nb>_kernel)
            hb_0, hb, idsb = stack_setup(nb)
            warm(L, R, lambda: stack_step(nb, hb_0, hb, idsb), 10, "batch%d warmup" % nb)
            msb = event_ms(torch, stream, lambda: stack_step(nb, hb_0, hb, idsb), 20)
            R.check(L.roaster_sync(), "batch%d" % nb)
            bb = decode_bytes(idsb.cpu().numpy())
            line["batch%d" % nb] = {"tokens_per_s": round(nb / (msb * 1e-3), 1), "ms_per_step": round(msb, 4),
                                    "hbm_GBps": round(bb / (msb * 1e-3) / 1e9, 1),
                                    "frac_hbm_peak": round(bb / (msb * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                    "kernel": L.roaster_decode_stack_kernel(t, nb, 0, N_LAYERS).decode()}
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline_decode(seed, args.cpu_tokens, t)
    L.roaster_table_destroy(t)
    return line


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "--gpus must be 1: the MoE-FFN hot path is measured on one MI355X "
                                   "(one GPU's share of an expert-parallel layout, at its real shape)"}))
        sys.exit(2)
    import torch
    import roaster_amd as R

    L = R.lib()
    dev = torch.device("cuda:0")
    torch.cuda.init()
    stream = torch.cuda.ExternalStream(L.roaster_stream(), device=dev)
    if args.three_kernel:
        L.roaster_decode_fused_layer(0)
    if args.fused_mode is not None:
        L.roaster_decode_fused_layer(args.fused_mode)
    legs = set(args.legs.split(","))
    line = {"metric": "partial run: legs %s" % sorted(legs)}
    if "decode" in legs:
        line = decode_legs(args, torch, L, R, dev, stream)
    parts = {"prefill": ("q6", "zipf", "api"), "prefill5": ("q6",), "prefill3": ("zipf",)}
    want = tuple(p for leg in legs if leg in parts for p in parts[leg])
    if want and not args.no_prefill:
        line["prefill"] = prefill_legs(torch, L, R, dev, stream, args.prefill_reps, not args.no_cpu, want)
    if "config1" in legs:
        line["config1"] = config1_leg(torch, L, R, dev, stream, not args.no_cpu)
    if "config2" in legs:
        line["config2"] = config2_leg(torch, L, R, dev, stream, not args.no_cpu)
    if "dense" in legs:
        line["dense"] = dense_leg(torch, L, R, dev, stream)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
