/*
 * decode.hip -- MoE-FFN decode (1..8 tokens) on gfx950.
 *
 * Reference path: model.c:1059-1146 (moe_forward) and kernels.c:1703-1830
 * (kernel_ffn_fused); the layer carry h += MoE(RMSNorm(h)) is model.c:1349-1358.
 *
 * One kernel body, four phases per layer:
 *   R  RMSNorm of h (stack) into LDS, router logits W_r x (f32) and the
 *      shared-expert gate logit gate_inp . x.
 *   P  top-8 per token (strict '>' insertion order => ties to the lower index,
 *      NaN / -inf never selected; model.c:869-897) and the union of selected
 *      experts into an "active expert" plan, built redundantly in every
 *      workgroup's LDS (deterministic, no extra grid sync).
 *   GU gate and up rows of every active expert for each of its tokens,
 *      eh = silu(g) * u  (model.c:1122-1126).
 *   D  down rows; each workgroup owns a slice of output rows for all active
 *      experts and combines them in the reference order
 *      y = sum_k w_k d_k (k = 0..7) + sigmoid(s) d_shared  (model.c:1139-1144).
 * Fused mode runs all phases of all layers in one cooperative launch with grid
 * barriers between R->GU (logits complete), GU->D (eh complete) and D->R (h
 * complete).  Split mode launches one phase per kernel (same code).
 *
 * Weights are read in their native GGML layout: every super-block is read once
 * per call by 8 lanes (16-byte chunks), scales decoded in registers, lane
 * partials reduced with cross-lane shuffles.  A row is at most 8 super-blocks
 * (hidden, inter <= 2048), so one wave pass covers it.
 */
#include "internal.h"
#include "qdot.h"
#include "decode.h"

#include <stdio.h>
#include <string.h>

#define DEC_THREADS 512
#define DEC_WAVES (DEC_THREADS / 64)
#define PF 2                          /* tasks prefetched per wave in GU */

/* ---- grid barrier ----------------------------------------------------------
 * Monotonic arrival counter (zeroed before launch).  Barrier number k waits for
 * k * gridDim.x arrivals.  The wait is bounded: after ~2^26 polls the flag
 * err |= 2 is raised and the wave proceeds, so every wave always exits. */
__device__ __forceinline__ void grid_sync(unsigned *bar, unsigned &epoch, int *err)
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    epoch += 1;
    if (threadIdx.x == 0) {
        const unsigned target = epoch * gridDim.x;
        __hip_atomic_fetch_add(bar, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        unsigned polls = 0;
        while (__hip_atomic_load(bar, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) < target) {
            __builtin_amdgcn_s_sleep(1);
            if (++polls > (1u << 26)) {
                __hip_atomic_fetch_or(err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
    }
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

/* ---- LDS layout ---------------------------------------------------------- */
struct DecShared {
    DecPlan plan;
    float red[DEC_WAVES][RMAX_B];
    float inv_rms[RMAX_B];
};

__device__ __forceinline__ float silu_mul(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

/* xn[t][:] (LDS) and its 16-column run sums.  Stack mode normalises h
 * (kernels.c:584-605 semantics: x * (1/sqrt(mean(x^2)+eps)) * w). */
__device__ void phase_norm(const DecArgs &A, int l, DecShared &S, float *xn, float *xsum)
{
    const int H = A.H, B = A.B;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const float *src = A.h;
    if (A.do_norm) {
        for (int t = 0; t < B; t++) {
            float ss = 0.0f;
            for (int i = tid; i < H; i += DEC_THREADS) { float v = src[(size_t)t * H + i]; ss = fmaf(v, v, ss); }
            ss = group_sum(ss, 64);
            if (lane == 0) S.red[wv][t] = ss;
        }
        __syncthreads();
        if (tid < B) {
            float ss = 0.0f;
            for (int w = 0; w < DEC_WAVES; w++) ss += S.red[w][tid];
            S.inv_rms[tid] = 1.0f / sqrtf(ss / (float)H + A.eps);
        }
        __syncthreads();
        const float *nw = A.norm_w ? A.norm_w + (size_t)(l - A.layer0) * H : NULL;
        for (int t = 0; t < B; t++) {
            const float inv = S.inv_rms[t];
            for (int i = tid; i < H; i += DEC_THREADS) {
                float v = src[(size_t)t * H + i] * inv;
                xn[t * H + i] = nw ? v * nw[i] : v;
            }
        }
    } else {
        for (int t = 0; t < B; t++)
            for (int i = tid; i < H; i += DEC_THREADS) xn[t * H + i] = src[(size_t)t * H + i];
    }
    __syncthreads();
    for (int r = tid; r < B * (H / 16); r += DEC_THREADS) xsum[r] = sum16(xn + r * 16);
    __syncthreads();
}

/* Router logits and shared gate logits: row e < E is W_r[e], row E is gate_inp.
 * Rows are spread over all waves of the grid; each row is one wave, lane owns
 * columns 4*lane + 256*m. */
__device__ void phase_router(const DecArgs &A, const DecLayer &L, const float *xn)
{
    const int H = A.H, B = A.B, E = A.E;
    const int lane = threadIdx.x & 63;
    const int gw = blockIdx.x * DEC_WAVES + (threadIdx.x >> 6), nw = gridDim.x * DEC_WAVES;
    const int first = A.logits_in ? E : 0;
    for (int e = first + gw; e <= E; e += nw) {
        const float *row = e < E ? L.router + (size_t)e * H : L.gate_inp;
        float acc[RMAX_B];
#pragma unroll
        for (int t = 0; t < RMAX_B; t++) acc[t] = 0.0f;
        for (int c0 = 4 * lane; c0 < H; c0 += 256) {
            float4 w = *(const float4 *)(row + c0);
#pragma unroll
            for (int t = 0; t < RMAX_B; t++) {
                if (t < B) {
                    float4 x = *(const float4 *)(xn + t * H + c0);
                    acc[t] = fmaf(w.x, x.x, acc[t]);
                    acc[t] = fmaf(w.y, x.y, acc[t]);
                    acc[t] = fmaf(w.z, x.z, acc[t]);
                    acc[t] = fmaf(w.w, x.w, acc[t]);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < RMAX_B; t++) {
            if (t < B) {
                float s = group_sum(acc[t], 64);
                if (lane == 0) {
                    if (e < E) A.logits[(size_t)t * E + e] = s;
                    else A.sgate_raw[t] = s;
                }
            }
        }
    }
}

/* Wave-level top-8 of one token (model.c:869-897) into ids / w. */
__device__ void topk8_wave(const float *lg, int E, int *ids, float *w, int *bad)
{
    const int lane = threadIdx.x & 63;
    float val[8];
    int idx[8];
#pragma unroll
    for (int k = 0; k < RTOPK; k++) {
        /* best candidate of this lane not yet taken: larger value, then lower index */
        float bv = -INFINITY;
        int bi = 0x7FFFFFFF;
        for (int e = lane; e < E; e += 64) {
            float v = lg[e];
            bool taken = false;
#pragma unroll
            for (int j = 0; j < RTOPK; j++) taken |= (j < k && idx[j] == e);
            if (taken || !(v > -INFINITY)) continue;       /* NaN and -inf never enter */
            if (v > bv || (v == bv && e < bi)) { bv = v; bi = e; }
        }
        for (int off = 32; off > 0; off >>= 1) {
            float ov = __shfl_xor(bv, off, 64);
            int oi = __shfl_xor(bi, off, 64);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        val[k] = bv;
        idx[k] = bi == 0x7FFFFFFF ? -1 : bi;
    }
    if (lane == 0) {
        int ok = 1;
        for (int k = 0; k < RTOPK; k++) ok &= idx[k] >= 0;
        float mx = val[0], sum = 0.0f, e8[8];
        for (int k = 0; k < RTOPK; k++) { e8[k] = expf(val[k] - mx); sum += e8[k]; }
        float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        for (int k = 0; k < RTOPK; k++) { ids[k] = idx[k]; w[k] = e8[k] * inv; }
        if (!ok) *bad = 1;
    }
}

/* Active-expert plan in LDS: union of the tokens' experts in first-appearance
 * order over (t, k), then the shared expert.  pair p = t*9 + k (k = 8: shared). */
__device__ void phase_plan(const DecArgs &A, const DecLayer &L, int l, DecShared &S)
{
    DecPlan &P = S.plan;
    const int B = A.B, E = A.E, tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
    const float *lg = A.logits_in ? A.logits_in : A.logits;
    if (tid == 0) P.err = 0;
    __syncthreads();
    for (int t = wv; t < B; t += DEC_WAVES) topk8_wave(lg + (size_t)t * E, E, P.ids[t], P.w[t], &P.err);
    if (tid < B) P.w[tid][8] = 1.0f / (1.0f + expf(-A.sgate_raw[tid]));
    __syncthreads();
    if (wv == 0) {
        /* lane i = pair (t, k) = (i / 8, i % 8) */
        const int n = B * RTOPK;
        int e = lane < n ? P.ids[lane >> 3][lane & 7] : -1;
        if (e < 0) e = -1;
        /* lanes with the same expert: compare across the wave */
        unsigned long long same = 0ull;
        for (int j = 0; j < n; j++) {
            int ej = __shfl(e, j, 64);
            if (ej == e && e >= 0) same |= 1ull << j;
        }
        const bool valid = e >= 0;
        const bool leader = valid && ((same & ((1ull << lane) - 1ull)) == 0ull);
        unsigned long long lead_mask = __ballot(leader);
        const int a = __popcll(lead_mask & ((1ull << lane) - 1ull));
        const int nroute = __popcll(lead_mask);
        if (leader) {
            DecActive &X = P.a[a];
            X.g = L.gate + (size_t)e * A.bytes_g;
            X.u = L.up + (size_t)e * A.bytes_u;
            X.d = L.down + (size_t)e * A.bytes_d;
            X.gq6 = A.q6g; X.uq6 = A.q6u; X.dq6 = A.q6d;
            int nt = 0;
            for (int j = 0; j < n; j++)
                if (same & (1ull << j)) X.tk[nt++] = (j >> 3) * 9 + (j & 7);
            X.ntok = nt;
        }
        if (lane == 0) {
            DecActive &X = P.a[nroute];
            X.g = L.sgate; X.u = L.sup; X.d = L.sdown;
            X.gq6 = A.sq6g; X.uq6 = A.sq6u; X.dq6 = A.sq6d;
            X.ntok = B;
            for (int t = 0; t < B; t++) X.tk[t] = t * 9 + 8;
            P.nact = nroute + 1;
        }
    }
    __syncthreads();
    if (blockIdx.x == 0 && tid < B * RTOPK) {
        const size_t o = ((size_t)(l - A.layer0) * B + (tid >> 3)) * RTOPK + (tid & 7);
        if (A.ids_out) A.ids_out[o] = P.ids[tid >> 3][tid & 7];
        if (A.w_out) A.w_out[o] = P.w[tid >> 3][tid & 7];
    }
    if (blockIdx.x == 0 && tid == 0 && P.err) atomicOr(A.err, 1);
}

/* First index >= begin that is congruent to w modulo n. */
__device__ __forceinline__ int first_of(int begin, int w, int n)
{
    return begin + ((w - begin) % n + n) % n;
}

/* Length of the run of active experts starting at a0 that share the given
 * matrix types (all routed experts of a table share them; the shared expert
 * may differ; kernel_ffn_fused experts may each differ). */
__device__ __forceinline__ int type_run_end(const DecPlan &P, int a0, bool gu)
{
    const DecActive &X0 = P.a[a0];
    int a1 = a0 + 1;
    while (a1 < P.nact && (gu ? (P.a[a1].gq6 == X0.gq6 && P.a[a1].uq6 == X0.uq6) : (P.a[a1].dq6 == X0.dq6))) a1++;
    return a1;
}

/* Gate/up tasks q = a*I + j for q in [q0, q1), all with types (G6, U6).  The
 * wave loads the chunks of PF tasks first, then computes:
 * eh[p][j] = silu(gate_j . x_t) * (up_j . x_t) for each (t, slot) pair p of a. */
template <bool G6, bool U6>
__device__ void gu_tasks(const DecArgs &A, const DecPlan &P, int q0, int q1, const float *xn, const float *xsum)
{
    const int H = A.H, I = A.I, nb = H / RQK;
    const int lane = threadIdx.x & 63, c = lane & 7, lb = lane >> 3;
    const int gw = blockIdx.x * DEC_WAVES + (threadIdx.x >> 6), nw = gridDim.x * DEC_WAVES;
    const bool lane_live = lb < nb;
    const size_t gbs = G6 ? RQ6K_BYTES : RQ4K_BYTES, ubs = U6 ? RQ6K_BYTES : RQ4K_BYTES;
    const int ga = lb * RQK + q_run_a<G6>(c), gb = ga + q_run_b_off<G6>();
    const int ua = lb * RQK + q_run_a<U6>(c), ub = ua + q_run_b_off<U6>();
    for (int qs = first_of(q0, gw, nw); qs < q1; qs += nw * PF) {
        QChunk cg[PF], cu[PF];
#pragma unroll
        for (int f = 0; f < PF; f++) {
            const int q = qs + f * nw;
            if (q < q1 && lane_live) {
                const DecActive &X = P.a[q / I];
                const int j = q % I;
                cg[f] = q_load<G6>(X.g + ((size_t)j * nb + lb) * gbs, c);
                cu[f] = q_load<U6>(X.u + ((size_t)j * nb + lb) * ubs, c);
            }
        }
#pragma unroll
        for (int f = 0; f < PF; f++) {
            const int q = qs + f * nw;
            if (q >= q1) break;
            const DecActive &X = P.a[q / I];
            const int j = q % I;
            for (int i = 0; i < X.ntok; i++) {
                const int p = X.tk[i], t = p / 9;
                const float *x = xn + t * H;
                const float *xs = xsum + t * (H / 16);
                float pg = 0.0f, pu = 0.0f;
                if (lane_live) {
                    pg = q_chunk_dot<G6>(cg[f], c, x + ga, x + gb, xs[ga >> 4], xs[gb >> 4]);
                    pu = q_chunk_dot<U6>(cu[f], c, x + ua, x + ub, xs[ua >> 4], xs[ub >> 4]);
                }
                pg = group_sum(pg, 64);
                pu = group_sum(pu, 64);
                if (lane == 0) A.eh[(size_t)p * I + j] = silu_mul(pg, pu);
            }
        }
    }
}

__device__ void phase_gu(const DecArgs &A, const DecPlan &P, const float *xn, const float *xsum)
{
    const int I = A.I;
    for (int a0 = 0; a0 < P.nact;) {
        const int a1 = type_run_end(P, a0, true);
        const int kind = (P.a[a0].gq6 ? 2 : 0) | (P.a[a0].uq6 ? 1 : 0);
        if (kind == 0) gu_tasks<false, false>(A, P, a0 * I, a1 * I, xn, xsum);
        else if (kind == 3) gu_tasks<true, true>(A, P, a0 * I, a1 * I, xn, xsum);
        else if (kind == 2) gu_tasks<true, false>(A, P, a0 * I, a1 * I, xn, xsum);
        else gu_tasks<false, true>(A, P, a0 * I, a1 * I, xn, xsum);
        a0 = a1;
    }
}

/* Down tasks q = a*ngroups + g for q in [q0, q1) (all with type D6): rows
 * r0 + g*rpw + (lane / lpr) of expert a, for each of its (t, slot) pairs, into
 * dbuf[p][row - r0]. */
template <bool D6>
__device__ void down_tasks(const DecArgs &A, const DecPlan &P, int q0, int q1, float *dbuf, int R, int ngroups)
{
    const int H = A.H, I = A.I, nb = I / RQK;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int lpr = nb >= 8 ? 64 : 8 * nb, rpw = 64 / lpr;
    const int rw = lane / lpr, lr = lane % lpr, c = lr & 7, lb = lr >> 3;
    const size_t dbs = D6 ? RQ6K_BYTES : RQ4K_BYTES;
    const int r0 = blockIdx.x * R;
    const int ca = lb * RQK + q_run_a<D6>(c), cb = ca + q_run_b_off<D6>();
    for (int q = first_of(q0, wv, DEC_WAVES); q < q1; q += DEC_WAVES) {
        const int a = q / ngroups, g = q % ngroups;
        const DecActive &X = P.a[a];
        const int rl = g * rpw + rw, row = r0 + rl;
        const bool live = rl < R && row < H;
        const uint8_t *drow = X.d + (size_t)(live ? row : 0) * nb * dbs;
        QChunk ch0;
        if (live && lb < nb) ch0 = q_load<D6>(drow + (size_t)lb * dbs, c);
        for (int i = 0; i < X.ntok; i++) {
            const int p = X.tk[i];
            const float *x = A.eh + (size_t)p * I;
            float part = 0.0f;
            if (live && lb < nb) part = q_chunk_dot<D6>(ch0, c, x + ca, x + cb, sum16(x + ca), sum16(x + cb));
            part = group_sum(part, lpr);
            if (live && lr == 0) dbuf[p * R + rl] = part;
        }
    }
}

/* Down rows [r0, r0 + R) of every active expert, then the combine. */
__device__ void phase_down(const DecArgs &A, const DecPlan &P, float *dbuf, int R)
{
    const int H = A.H, I = A.I, B = A.B, nb = I / RQK;
    const int tid = threadIdx.x;
    const int lpr = nb >= 8 ? 64 : 8 * nb, rpw = 64 / lpr;
    const int ngroups = (R + rpw - 1) / rpw;
    const int r0 = blockIdx.x * R;
    for (int a0 = 0; a0 < P.nact;) {
        const int a1 = type_run_end(P, a0, false);
        if (P.a[a0].dq6) down_tasks<true>(A, P, a0 * ngroups, a1 * ngroups, dbuf, R, ngroups);
        else down_tasks<false>(A, P, a0 * ngroups, a1 * ngroups, dbuf, R, ngroups);
        a0 = a1;
    }
    __syncthreads();
    if (A.ffn_out) {                    /* kernel_ffn_fused: per-expert outputs, token 0 */
        for (int idx = tid; idx < A.ffn_n * R; idx += DEC_THREADS) {
            const int k = idx / R, rl = idx % R, row = r0 + rl;
            if (row < H) A.ffn_out[(size_t)k * H + row] = dbuf[k * R + rl];
        }
    } else {
        for (int idx = tid; idx < B * R; idx += DEC_THREADS) {
            const int t = idx / R, rl = idx % R, row = r0 + rl;
            if (row >= H) continue;
            float y = 0.0f;
            for (int k = 0; k < RTOPK; k++) y = fmaf(P.w[t][k], dbuf[(t * 9 + k) * R + rl], y);
            y = fmaf(P.w[t][8], dbuf[(t * 9 + 8) * R + rl], y);
            if (A.y) A.y[(size_t)t * H + row] = y;
            else A.h[(size_t)t * H + row] = A.h[(size_t)t * H + row] + y;
        }
    }
}

__device__ void load_ffn_plan(const DecArgs &A, DecShared &S)
{
    if (threadIdx.x == 0) {
        S.plan.nact = A.ffn_n;
        S.plan.err = 0;
        for (int k = 0; k < A.ffn_n; k++) {
            S.plan.a[k] = A.ffn_ex[k];
            S.plan.a[k].ntok = 1;
            S.plan.a[k].tk[0] = k;
        }
    }
    __syncthreads();
}

__device__ __forceinline__ int rows_per_wg(int H)
{
    int R = (H + (int)gridDim.x - 1) / (int)gridDim.x;
    return (R + 3) & ~3;
}

/* phase_mask bit 0: R, 1: GU (with plan), 2: D (with plan).  fused != 0 runs
 * all phases of all layers with grid barriers. */
extern "C" __global__ void __launch_bounds__(DEC_THREADS)
moe_decode_kernel(DecArgs A, int phase_mask, int fused)
{
    extern __shared__ __align__(16) float lds[];
    __shared__ DecShared S;
    const int H = A.H, B = A.B;
    float *xn = lds;                           /* [B x H] */
    float *xsum = xn + B * H;                  /* [B x H/16] */
    float *dbuf = xsum + B * (H / 16);         /* [B*9 x R] */
    const int R = rows_per_wg(H);
    unsigned epoch = 0;
    if (A.ffn_out) {
        phase_norm(A, 0, S, xn, xsum);
        load_ffn_plan(A, S);
        phase_gu(A, S.plan, xn, xsum);
        grid_sync(A.bar, epoch, A.err);
        phase_down(A, S.plan, dbuf, R);
        return;
    }
    for (int l = A.layer0; l < A.layer0 + A.nlayers; l++) {
        const DecLayer L = A.layers[l];
        if (fused || (phase_mask & 1)) {
            phase_norm(A, l, S, xn, xsum);
            phase_router(A, L, xn);
        }
        if (fused) grid_sync(A.bar, epoch, A.err);
        if (fused || (phase_mask & 2)) {
            if (!fused) phase_norm(A, l, S, xn, xsum);
            phase_plan(A, L, l, S);
            phase_gu(A, S.plan, xn, xsum);
        }
        if (fused) grid_sync(A.bar, epoch, A.err);
        if (fused || (phase_mask & 4)) {
            if (!fused) phase_plan(A, L, l, S);
            phase_down(A, S.plan, dbuf, R);
        }
        if (fused && l + 1 < A.layer0 + A.nlayers) grid_sync(A.bar, epoch, A.err);
    }
}

/* ---- host side ------------------------------------------------------------ */
size_t dec_lds_bytes(int B, int H)
{
    /* xn + xsum + dbuf (R <= H rows of 9*B pairs; R is small, size for 64 rows) */
    return (size_t)B * H * 4 + (size_t)B * (H / 16) * 4 + (size_t)B * 9 * 64 * 4;
}

int dec_launch(DecArgs &A, int fused)
{
    RtState &R = rt();
    const size_t lds = dec_lds_bytes(A.B, A.H);
    unsigned *ctrl = rt_ctrl();
    if (!ctrl) return ROASTER_ENOMEM;
    A.bar = ctrl;
    A.err = (int *)(ctrl + 16);
    if (fused) {
        if (rt_check(hipMemsetAsync(ctrl, 0, 4, R.stream), "barrier reset")) return ROASTER_EDEVICE;
        int blocks = 0;
        if (rt_coop_grid((const void *)moe_decode_kernel, DEC_THREADS, lds, &blocks)) return ROASTER_EDEVICE;
        blocks = R.n_cu < blocks ? R.n_cu : blocks;     /* one workgroup per CU */
        if (((A.H + blocks - 1) / blocks + 3) / 4 * 4 > 64) return rt_fail(ROASTER_EINVAL, "hidden too large");
        int mask = 7, fz = 1;
        void *args[] = { &A, &mask, &fz };
        return rt_check(hipLaunchCooperativeKernel((const void *)moe_decode_kernel, dim3(blocks), dim3(DEC_THREADS),
                                                   args, lds, R.stream), "cooperative decode launch");
    }
    const int blocks = R.n_cu;
    for (int l = A.layer0; l < A.layer0 + A.nlayers; l++) {
        DecArgs a1 = A;
        a1.layer0 = l;
        a1.nlayers = 1;
        for (int ph = 0; ph < 3; ph++) {
            hipLaunchKernelGGL(moe_decode_kernel, dim3(blocks), dim3(DEC_THREADS), lds, R.stream, a1, 1 << ph, 0);
            if (rt_check(hipGetLastError(), "decode launch")) return ROASTER_EDEVICE;
        }
    }
    return 0;
}

int dec_ffn_launch(DecArgs &A)
{
    RtState &R = rt();
    const size_t lds = dec_lds_bytes(1, A.H);
    unsigned *ctrl = rt_ctrl();
    if (!ctrl) return ROASTER_ENOMEM;
    A.bar = ctrl;
    A.err = (int *)(ctrl + 16);
    if (rt_check(hipMemsetAsync(ctrl, 0, 4, R.stream), "barrier reset")) return ROASTER_EDEVICE;
    int blocks = 0;
    if (rt_coop_grid((const void *)moe_decode_kernel, DEC_THREADS, lds, &blocks)) return ROASTER_EDEVICE;
    blocks = R.n_cu < blocks ? R.n_cu : blocks;
    int mask = 7, fz = 1;
    void *args[] = { &A, &mask, &fz };
    return rt_check(hipLaunchCooperativeKernel((const void *)moe_decode_kernel, dim3(blocks), dim3(DEC_THREADS),
                                               args, lds, R.stream), "cooperative ffn launch");
}
