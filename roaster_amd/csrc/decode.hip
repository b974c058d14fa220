/*
 * decode.hip -- MoE-FFN decode (1..8 tokens) on gfx950.
 *
 * Reference path: model.c:1059-1146 (moe_forward) and kernels.c:1703-1830
 * (kernel_ffn_fused); the layer carry h += MoE(RMSNorm(h)) is model.c:1349-1358.
 *
 * Two ways to run a call's layers:
 *
 * One launch for the whole call (a run of up to 64 layers): 256 workgroups,
 * one per CU, that pass values to each other through exchange slots in
 * memory (64-bit (epoch, value) words, every wait bounded).  XCD k's 32
 * workgroups serve routed slot k of every token (the k-th selected expert);
 * the shared expert and the router are spread over all 256.
 *   dec_stack1r_kernel   one token, 256 experts / hidden 2048 / inter 512,
 *                        gate/up Q4_K and down Q6_K: the router folded into
 *                        the previous layer's combine (partial logits over
 *                        each workgroup's combined rows, summed across XCDs);
 *   dec_stack1_kernel,   one token, any other shape the launch takes (2x2:
 *   dec_stack1_2x2_kernel  two gate/up pairs and two down tasks per wave),
 *                        with the three-kernel path's arithmetic;
 *   dec_stackB2/4/8_kernel  2..8 tokens, each token's results equal to its
 *                        one-token result on the three-kernel arithmetic.
 * A stack call's final h is staged and copied over the caller's only when no
 * wait gave up anywhere (k1_finish).
 *
 * Three kernels per layer (kernels.h calls, other shapes, or
 * roaster_decode_fused_layer(0)):
 *   R   RMSNorm of h into LDS (each workgroup, redundantly), router logits
 *       W_r x (f32), the shared-gate logit gate_inp . x and the shared
 *       expert's gate/up rows (they need no routing): eh_shared = silu(g)*u.
 *   GU  top-8 per token from the logits (strict '>' insertion order: ties go
 *       to the lower index, NaN / -inf never enter; model.c:869-897), the
 *       union of the tokens' experts as an "active expert" plan (built
 *       identically in every workgroup; workgroup 0 publishes it), and every
 *       routed expert's gate/up rows: eh = silu(g) * u  (model.c:1122-1126).
 *   D   down rows: each workgroup owns one token and a block of output rows
 *       (4, or 8 with several tokens) for that token's nine slots, with their
 *       SiLU*up vectors staged in LDS, and combines them in the reference
 *       order y = sum_{k=0..7} w_k d_k + sigmoid(s) d_shared
 *       (model.c:1139-1144).
 *
 * Weights are read in their native GGML layout: each super-block is read once
 * per call by 8 lanes (16-byte chunks), scales decoded in registers, lane
 * partials reduced with cross-lane shuffles.  A row is at most 8 super-blocks
 * (hidden, inter <= 2048), so one wave pass covers it.  Every wave issues all
 * loads of its task set before consuming any (one memory round trip per
 * dependency instead of one per loop iteration).
 */
#include "internal.h"
#include "qdot.h"
#include "topk.h"
#include "decode.h"

#include <stdio.h>
#include <string.h>

#define DT 256                        /* threads per workgroup */
#define DW (DT / 64)                  /* waves per workgroup */
#define GU_PF 2                       /* tasks in flight per wave, one token */
#define GU_PF_B 4                     /* the same with several tokens (activations from LDS) */
#define D_ROWS 4                      /* output rows per down workgroup, one token */
#define D_ROWS_B 8                    /* the same with several tokens (one workgroup per token) */
#define D_MAXR 8
#ifndef D_PF
#define D_PF 4                        /* down tasks in flight per wave */
#endif
#define LGKM_ONLY 0xC07F              /* s_waitcnt lgkmcnt(0), leaving vector-memory loads in flight */

/* Opt-in phase tracing (build with -DROASTER_PHASE_TS): thread 0 of every
 * workgroup records the 100 MHz real-time counter at phase boundaries;
 * roaster_phase_ts() copies the [kernel][workgroup][mark] table out. */
#ifdef ROASTER_PHASE_TS
__device__ unsigned long long g_phase_ts[4][1024][8];
#define PHASE_TS(k, i)                                                                      \
    do {                                                                                    \
        if (threadIdx.x == 0 && blockIdx.x < 1024)                                          \
            g_phase_ts[k][blockIdx.x][i] = __builtin_amdgcn_s_memrealtime();                \
    } while (0)
extern "C" int roaster_phase_ts(unsigned long long *out)
{
    return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(g_phase_ts), sizeof(g_phase_ts));
}
/* one-launch stack: [last two layers][workgroup][wave 0, 1, 3][mark] */
__device__ unsigned long long g_k1_ts[2][256][3][16];
extern "C" int roaster_phase_ts_k1(unsigned long long *out)
{
    return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(g_k1_ts), sizeof(g_k1_ts));
}
#else
#define PHASE_TS(k, i) do { } while (0)
#endif

/* This thread's wave index, as a wave-uniform (scalar) value: branches on it
 * are scalar branches, not exec-masked regions. */
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

/* A pointer every lane of the wave holds (read from LDS), as a scalar value. */
__device__ __forceinline__ const uint8_t *uniform_ptr(const uint8_t *p)
{
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return (const uint8_t *)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ float silu_mul(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

__device__ __forceinline__ int first_of(int begin, int w, int n)
{
    return begin + ((w - begin) % n + n) % n;
}

/* Copy n16 16-byte units global -> LDS, 8 units per thread per round: all
 * loads of a round are issued before its first store, so a round costs one
 * memory round trip (one round covers 32 KB).  Loads and stores are
 * unconditional, of units clamped to the last one (lanes past the end load
 * and store that unit again, the same value), so the compiler neither sinks a
 * load into a guarded store nor places a wait before the loads are issued:
 * the first round shares a round trip with whatever the caller issued just
 * before. */
__device__ __forceinline__ void block_copy16(void *dst, const void *src, int n16)
{
    for (int base = 0; base < n16; base += 8 * DT) {
        uint4 v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = ((const uint4 *)src)[min(base + (int)threadIdx.x + k * DT, n16 - 1)];
#pragma unroll
        for (int k = 0; k < 8; k++) ((uint4 *)dst)[min(base + (int)threadIdx.x + k * DT, n16 - 1)] = v[k];
    }
}

/* Storage position of 16-byte unit u of the gate/up kernel's activations in
 * LDS: bits 4..6 of u are folded into bits 0, 1 and 3 (an involution that
 * keeps every run of 16 units in place).  The 16 lanes of one ds_read_b128
 * pass read units 64 lb + 16 g + 4 h + i of a Q4_K row chunk (qdot.h lane
 * layout): stored plainly they share 2 of the 16 bank groups (8-way
 * conflicts), swizzled they cover all 16 (Q6_K chunks: 2 lanes per group). */
__device__ __forceinline__ int xsw(int u) { return u ^ ((u >> 4) & 3) ^ (((u >> 6) & 1) << 3); }

/* Storage position of unit u: swizzled when the rows fill whole 128-unit
 * blocks (xsw permutes within aligned blocks of 128 units), plain otherwise. */
__device__ __forceinline__ int xpos(int u, bool swz) { return swz ? xsw(u) : u; }

/* block_copy16 with units below nsw stored at xsw(unit). */
__device__ __forceinline__ void block_copy16_sw(void *dst, const void *src, int n16, int nsw)
{
    for (int base = 0; base < n16; base += 8 * DT) {
        uint4 v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = ((const uint4 *)src)[min(base + (int)threadIdx.x + k * DT, n16 - 1)];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int i = min(base + (int)threadIdx.x + k * DT, n16 - 1);
            ((uint4 *)dst)[i < nsw ? xsw(i) : i] = v[k];
        }
    }
}

/* The 16 activations at float offset off (a multiple of 16) of an LDS copy. */
__device__ __forceinline__ void load_x16(const float *xn, int off, float4 (&x)[4], bool swz)
{
#pragma unroll
    for (int i = 0; i < 4; i++) x[i] = ((const float4 *)xn)[xpos((off >> 2) + i, swz)];
}

/* xn[t][:] (LDS) = RMSNorm(h[t]) or a copy of x, and its 16-column run sums.
 * RMSNorm follows kernels.c:584-605: x * (1/sqrt(mean(x^2) + eps)) * w. */
/* xn[t][:] (LDS) = RMSNorm(h[t]) or a copy of x, stored at xpos (16-byte
 * unit u of the B x H block at xsw(u) when A.xswz), and xsum[t][r] = the sum of the 16
 * logical elements 16 r .. 16 r + 15 (plain index), added in element order.
 * RMSNorm follows kernels.c:584-605: x * (1/sqrt(mean(x^2) + eps)) * w.  All
 * LDS traffic is in 16-byte units (4-byte LDS accesses issue at an eighth of
 * the rate); H <= 2048 = 2 units per thread per token. */
/* Norm weights of this thread's storage units (logical units xsw(u)), or
 * NULL (then wq holds ones). */
__device__ __forceinline__ const float *norm_weights(const DecArgs &A, int l, float4 (&wq)[2])
{
    const int HU = A.H / 4;
    const float *nw = A.do_norm && A.norm_w ? A.norm_w + (size_t)(l - A.layer0) * A.H : NULL;
#pragma unroll
    for (int k = 0; k < 2; k++)
        wq[k] = nw ? ((const float4 *)nw)[xpos(min((int)threadIdx.x + k * DT, HU - 1), A.xswz)]
                   : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
    return nw;
}

__device__ void block_norm_tail(const DecArgs &A, float *xn, float *xsum, float (*red)[RMAX_B], float *inv_rms,
                                const float4 (&wq)[2], const float *nw);

__device__ void block_norm(const DecArgs &A, int l, float *xn, float *xsum, float (*red)[RMAX_B], float *inv_rms)
{
    float4 wq[2];
    const float *nw = norm_weights(A, l, wq);          /* loaded with h */
    block_copy16_sw(xn, A.h, A.B * (A.H / 4), A.xswz ? A.B * (A.H / 4) : 0);
    block_norm_tail(A, xn, xsum, red, inv_rms, wq, nw);
}

/* block_norm after h is stored in LDS (not yet synchronised) */
__device__ __forceinline__ void block_norm_tail(const DecArgs &A, float *xn, float *xsum, float (*red)[RMAX_B],
                                                float *inv_rms, const float4 (&wq)[2], const float *nw)
{
    const int H = A.H, B = A.B, HU = H / 4;     /* 16-byte units per token */
    const int tid = threadIdx.x, lane = tid & 63, wv = wave_id();
    const bool swz = A.xswz;
    float4 *x4 = (float4 *)xn;
    __syncthreads();
    PHASE_TS(0, 3);
    if (A.do_norm) {
        /* sums of squares of every token first, then their reductions (the
         * tokens' reduction chains are independent and interleave) */
        float ss[RMAX_B];
#pragma unroll
        for (int t = 0; t < RMAX_B; t++) {
            ss[t] = 0.0f;
            if (t < B) {
#pragma unroll
                for (int k = 0; k < 2; k++) {
                    const int u = tid + k * DT;
                    if (u < HU) {
                        const float4 v = x4[t * HU + u];
                        ss[t] = fmaf(v.x, v.x, ss[t]);
                        ss[t] = fmaf(v.y, v.y, ss[t]);
                        ss[t] = fmaf(v.z, v.z, ss[t]);
                        ss[t] = fmaf(v.w, v.w, ss[t]);
                    }
                }
            }
        }
#pragma unroll
        for (int t = 0; t < RMAX_B; t++) {
            if (t < B) {
                ss[t] = group_sum<64>(ss[t]);
                if (lane == 0) red[wv][t] = ss[t];
            }
        }
        __syncthreads();
        PHASE_TS(0, 4);
        if (tid < B) {
            float s2 = 0.0f;
            for (int w = 0; w < DW; w++) s2 += red[w][tid];
            inv_rms[tid] = 1.0f / sqrtf(s2 / (float)H + A.eps);
        }
        __syncthreads();
        for (int t = 0; t < B; t++) {
            const float inv = inv_rms[t];
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const int u = tid + k * DT;
                if (u < HU) {
                    float4 v = x4[t * HU + u];
                    v.x *= inv; v.y *= inv; v.z *= inv; v.w *= inv;
                    if (nw) { v.x *= wq[k].x; v.y *= wq[k].y; v.z *= wq[k].z; v.w *= wq[k].w; }
                    x4[t * HU + u] = v;
                }
            }
        }
        __syncthreads();
        PHASE_TS(0, 5);
    }
    for (int r = tid; r < B * (H / 16); r += DT) {       /* the order of sum16 (qdot.h) */
        const float4 a = x4[xpos(4 * r, swz)], b = x4[xpos(4 * r + 1, swz)];
        const float4 c = x4[xpos(4 * r + 2, swz)], d = x4[xpos(4 * r + 3, swz)];
        xsum[r] = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w)) +
                  (((c.x + c.y) + (c.z + c.w)) + ((d.x + d.y) + (d.z + d.w)));
    }
    __syncthreads();
}

/* The lane's chunks of gate row j and up row j.  Lanes past the row's last
 * super-block (lb >= nb) load the last one again: loads stay unconditional
 * (a lane-dependent guard would make them exec-masked, with a wait after
 * each), and those lanes' products are never used. */
template <bool G6, bool U6>
__device__ __forceinline__ QChunk2 load_gu_pair(const uint8_t *g, const uint8_t *u, int j, int nb, int lb, int c)
{
    const int lbc = lb < nb ? lb : nb - 1;
    QChunk2 r;
    r.g = q_load<G6>(g + ((size_t)j * nb + lbc) * (G6 ? RQ6K_BYTES : RQ4K_BYTES), c);
    r.u = q_load<U6>(u + ((size_t)j * nb + lbc) * (U6 ? RQ6K_BYTES : RQ4K_BYTES), c);
    return r;
}

/* eh[p][j] = silu(gate_j . x_t) * (up_j . x_t) for the (t, slot) pairs p of one
 * expert, given the lane's chunks of gate row j and up row j. */
template <bool G6, bool U6>
__device__ __forceinline__ void gu_row(const DecArgs &A, int j, const QChunk2 &ch, int ntok, const int *tk,
                                       const float *xn, const float *xsum)
{
    const int H = A.H, I = A.I, nb = H / RQK;
    const int lane = threadIdx.x & 63, c = lane & 7, lb = lane >> 3;
    const int ga = lb * RQK + q_run_a<G6>(c), gb = ga + q_run_b_off<G6>();
    const int ua = lb * RQK + q_run_a<U6>(c), ub = ua + q_run_b_off<U6>();
    for (int i = 0; i < ntok; i++) {
        const int p = tk[i], t = p / 9;
        const float *xs = xsum + t * (H / 16);
        float pg = 0.0f, pu = 0.0f;
        if (lb < nb) {
            float4 x0[4], x1[4];
            load_x16(xn, t * H + ga, x0, A.xswz);
            load_x16(xn, t * H + gb, x1, A.xswz);
            pg = q_chunk_dot_r<G6>(ch.g, c, x0, x1, xs[ga >> 4], xs[gb >> 4]);
            load_x16(xn, t * H + ua, x0, A.xswz);
            load_x16(xn, t * H + ub, x1, A.xswz);
            pu = q_chunk_dot_r<U6>(ch.u, c, x0, x1, xs[ua >> 4], xs[ub >> 4]);
        }
        pg = group_sum<64>(pg);
        pu = group_sum<64>(pu);
        if (lane == 0) A.eh[(size_t)p * I + j] = silu_mul(pg, pu);
    }
}

/* ---- R: router + shared-gate logit + shared expert gate/up ------------------ */
/* Router kernel body; ONE: one token (B == 1), whose h is loaded before the
 * weights (below). */
template <bool ONE>
__device__ __forceinline__ void router_body(const DecArgs &A, int l)
{
    extern __shared__ __align__(16) float lds[];
    __shared__ float red[DW][RMAX_B];
    __shared__ float inv_rms[RMAX_B];
    __shared__ int sh_tk[RMAX_B];
    const int H = A.H, E = A.E, I = A.I, B = A.B, nb = H / RQK;
    float *xn = lds, *xsum = lds + B * H;
    const DecLayer L = A.layers[l];
    const int lane = threadIdx.x & 63, c = lane & 7, lb = lane >> 3;
    PHASE_TS(0, 0);
    const int task = blockIdx.x * DW + wave_id();
    const int nrouter = A.logits_in ? 0 : E;
    /* task < nrouter: router row; == nrouter: gate_inp; then shared-expert row pairs */
    const bool is_row = task <= nrouter;
    const int j = task - nrouter - 1;
    const bool is_sh = !is_row && j < I;
    const int kind = (L.sq6[0] ? 2 : 0) | (L.sq6[1] ? 1 : 0);
    if (threadIdx.x < B) sh_tk[threadIdx.x] = threadIdx.x * 9 + 8;
    /* 1. h and the weights.  With several tokens the weight loads go first
     * (independent of h) and block_norm copies h.  With one token h (2 units
     * per thread) and the norm weights are loaded first and each branch
     * stores h to LDS after its own weight loads, so the store waits for h
     * only (a wave's loads complete in order) and the norm runs while the
     * weights are in flight.  A distinct marker after each branch's stores
     * keeps the compiler from merging them past the join (where the wait
     * would cover the weights again). */
    float4 w[8];
    QChunk2 ch;
    const int HU = H / 4;
    float4 h0, h1, wq[2];
    const float *nw = NULL;
    if (ONE) {
        h0 = ((const float4 *)A.h)[min((int)threadIdx.x, HU - 1)];
        h1 = ((const float4 *)A.h)[min((int)threadIdx.x + DT, HU - 1)];
        nw = norm_weights(A, l, wq);
    }
#define R_STORE_H(tag)                                                                           \
    do {                                                                                         \
        if (ONE) {                                                                               \
            ((float4 *)xn)[xpos(min((int)threadIdx.x, HU - 1), A.xswz)] = h0;                    \
            ((float4 *)xn)[xpos(min((int)threadIdx.x + DT, HU - 1), A.xswz)] = h1;               \
            asm volatile("; h stored, " tag);                                                    \
        }                                                                                        \
    } while (0)
    if (is_row) {
        const float *row = task < nrouter ? L.router + (size_t)task * H : L.gate_inp;
#pragma unroll
        for (int m = 0; m < 8; m++) w[m] = gld_f4(row + min(4 * lane + 256 * m, H - 4));   /* clamped: no masked loads */
        R_STORE_H("router row");
    } else if (is_sh) {
        if (kind == 0) ch = load_gu_pair<false, false>(L.sgate, L.sup, j, nb, lb, c);
        else if (kind == 3) ch = load_gu_pair<true, true>(L.sgate, L.sup, j, nb, lb, c);
        else if (kind == 2) ch = load_gu_pair<true, false>(L.sgate, L.sup, j, nb, lb, c);
        else ch = load_gu_pair<false, true>(L.sgate, L.sup, j, nb, lb, c);
        R_STORE_H("shared rows");
    } else {
        R_STORE_H("no task");
    }
#undef R_STORE_H
    /* 2. normalised input into LDS; workgroup 0 publishes it for the gate/up kernel */
    if (ONE) block_norm_tail(A, xn, xsum, red, inv_rms, wq, nw);
    else block_norm(A, l, xn, xsum, red, inv_rms);
    if (blockIdx.x == 0)
        for (int i = threadIdx.x; i < B * (H + H / 16) / 4; i += DT) ((float4 *)A.xn_g)[i] = ((const float4 *)xn)[i];
    PHASE_TS(0, 1);
    /* 3. dots */
    if (is_row) {
        float acc[RMAX_B];
#pragma unroll
        for (int t = 0; t < RMAX_B; t++) acc[t] = 0.0f;
#pragma unroll
        for (int m = 0; m < 8; m++) {
            const int c0 = 4 * lane + 256 * m;
            if (c0 < H) {
#pragma unroll
                for (int t = 0; t < RMAX_B; t++) {
                    if (t < B) {
                        const float4 x = ((const float4 *)xn)[xpos((t * H + c0) >> 2, A.xswz)];
                        acc[t] = fmaf(w[m].x, x.x, acc[t]);
                        acc[t] = fmaf(w[m].y, x.y, acc[t]);
                        acc[t] = fmaf(w[m].z, x.z, acc[t]);
                        acc[t] = fmaf(w[m].w, x.w, acc[t]);
                    }
                }
            }
        }
#pragma unroll
        for (int t = 0; t < RMAX_B; t++) {
            if (t < B) {
                const float s = group_sum<64>(acc[t]);
                if (lane == 0) {
                    if (task < nrouter) A.logits[(size_t)t * E + task] = s;
                    else A.sgate_raw[t] = s;
                }
            }
        }
    } else if (is_sh) {
        if (kind == 0) gu_row<false, false>(A, j, ch, B, sh_tk, xn, xsum);
        else if (kind == 3) gu_row<true, true>(A, j, ch, B, sh_tk, xn, xsum);
        else if (kind == 2) gu_row<true, false>(A, j, ch, B, sh_tk, xn, xsum);
        else gu_row<false, true>(A, j, ch, B, sh_tk, xn, xsum);
    }
    PHASE_TS(0, 2);
}

extern "C" __global__ void __launch_bounds__(DT, 3) dec_router_kernel(DecArgs A, int l) { router_body<false>(A, l); }
extern "C" __global__ void __launch_bounds__(DT, 3) dec_router1_kernel(DecArgs A, int l) { router_body<true>(A, l); }

/* ---- GU: routing plan + routed experts' gate/up ----------------------------- */

/* Active-expert plan from the tokens' top-8 ids in P: union of the tokens'
 * experts in first-appearance order over (t, k), then the shared expert.
 * Pair p = t*9 + k (k = 8: shared).  emask: 256 x 64-bit LDS scratch. */
__device__ __forceinline__ void plan_from_ids(const DecArgs &A, const DecLayer &L, DecPlan &P, float sg, unsigned long long *emask)
{
    const int B = A.B, tid = threadIdx.x, wv = wave_id(), lane = tid & 63;
    if (tid < B) P.w[tid][8] = 1.0f / (1.0f + expf(-sg));
    __syncthreads();
    PHASE_TS(1, 4);
    if (wv == 0) {
        const int n = B * RTOPK;                 /* lane i = pair (i / 8, i % 8) */
        const int e = lane < n ? P.ids[lane >> 3][lane & 7] : -1;
        const bool valid = e >= 0;
        if (valid) emask[e] = 0ull;
        __builtin_amdgcn_s_waitcnt(LGKM_ONLY);
        __builtin_amdgcn_wave_barrier();
        if (valid) atomicOr(&emask[e], 1ull << lane);
        __builtin_amdgcn_s_waitcnt(LGKM_ONLY);
        __builtin_amdgcn_wave_barrier();
        const unsigned long long m = valid ? emask[e] : 0ull;
        const bool leader = valid && (__ffsll((long long)m) - 1) == lane;
        const unsigned long long lead_mask = __ballot(leader);
        const int a = __popcll(lead_mask & ((1ull << lane) - 1ull));
        const int nroute = __popcll(lead_mask);
        if (leader) {
            DecActive &X = P.a[a];
            X.g = L.gate + (size_t)e * L.eb[0];
            X.u = L.up + (size_t)e * L.eb[1];
            X.d = L.down + (size_t)e * L.eb[2];
            X.gq6 = L.q6[0]; X.uq6 = L.q6[1]; X.dq6 = L.q6[2];
            int nt = 0;
            for (unsigned long long mm = m; mm; mm &= mm - 1ull) {
                const int jj = __ffsll((long long)mm) - 1;
                X.tk[nt++] = (jj >> 3) * 9 + (jj & 7);
            }
            X.ntok = nt;
        }
        if (lane == 0) {
            DecActive &X = P.a[nroute];
            X.g = L.sgate; X.u = L.sup; X.d = L.sdown;
            X.gq6 = L.sq6[0]; X.uq6 = L.sq6[1]; X.dq6 = L.sq6[2];
            X.ntok = B;
            for (int t = 0; t < B; t++) X.tk[t] = t * 9 + 8;
            P.nroute = nroute;
            P.nact = nroute + 1;
        }
    }
    /* down slot table for the down kernel (waves 1..3, beside wave 0's list) */
    for (int i = tid - 64; i >= 0 && i < B * 9; i += DT - 64) {
        const int t = i / 9, k = i % 9;
        if (k < RTOPK) {
            const int e = P.ids[t][k];
            P.dsl[t][k] = e >= 0 ? L.down + (size_t)e * L.eb[2] : NULL;
        } else {
            P.dsl[t][k] = L.sdown;
        }
    }
    if (tid >= 64 && tid < 64 + 9) P.dq6k[tid - 64] = tid - 64 < RTOPK ? L.q6[2] : L.sq6[2];
    __syncthreads();
}

/* plan_from_ids for one token whose top-8 ids in P are visible to the whole
 * workgroup: the selected slots (a prefix of the 8: topk fills slots in
 * order) are the routed active experts in slot order, so lane k of wave 0
 * writes active expert k directly; then the shared expert, and the slot table
 * as in plan_from_ids.  Gives the same plan as plan_from_ids with B = 1. */
__device__ __forceinline__ void plan_one_token(const DecArgs &A, const DecLayer &L, DecPlan &P, float sg)
{
    const int tid = threadIdx.x, wv = wave_id(), lane = tid & 63;
    if (wv == 0) {
        const int e = lane < RTOPK ? P.ids[0][lane] : -1;
        const int nroute = __popcll(__ballot(e >= 0));
        if (e >= 0) {
            DecActive &X = P.a[lane];
            X.g = L.gate + (size_t)e * L.eb[0];
            X.u = L.up + (size_t)e * L.eb[1];
            X.d = L.down + (size_t)e * L.eb[2];
            X.gq6 = L.q6[0]; X.uq6 = L.q6[1]; X.dq6 = L.q6[2];
            X.ntok = 1;
            X.tk[0] = lane;                                 /* pair (token 0, slot lane) */
        }
        if (lane == 0) {
            P.w[0][8] = 1.0f / (1.0f + expf(-sg));
            DecActive &X = P.a[nroute];
            X.g = L.sgate; X.u = L.sup; X.d = L.sdown;
            X.gq6 = L.sq6[0]; X.uq6 = L.sq6[1]; X.dq6 = L.sq6[2];
            X.ntok = 1;
            X.tk[0] = 8;
            P.nroute = nroute;
            P.nact = nroute + 1;
        }
    } else if (tid < 64 + 9) {                              /* down slot table */
        const int k = tid - 64;
        if (k < RTOPK) {
            const int e = P.ids[0][k];
            P.dsl[0][k] = e >= 0 ? L.down + (size_t)e * L.eb[2] : NULL;
        } else {
            P.dsl[0][k] = L.sdown;
        }
        P.dq6k[k] = k < RTOPK ? L.q6[2] : L.sq6[2];
    }
    __syncthreads();
}

/* Plan of B tokens: wave w computes the top-8 of tokens w, w + 4, ... (ts:
 * one scratch per wave) */
__device__ void build_plan(const DecArgs &A, const DecLayer &L, DecPlan &P, const float (*lg4)[4], float sg,
                           unsigned long long *emask, TopkScratch *ts)
{
    if (threadIdx.x == 0) P.err = 0;
    __syncthreads();
    for (int t = wave_id(), r = 0; t < A.B; t += DW, r++)
        topk8_fast(lg4[r], A.E, P.ids[t], P.w[t], &P.err, &ts[wave_id()]);
    plan_from_ids(A, L, P, sg, emask);
}

__device__ void ffn_plan(const DecArgs &A, DecPlan &P)
{
    if (threadIdx.x == 0) {
        P.nact = A.ffn_n;
        P.nroute = A.ffn_n;
        P.err = 0;
        for (int k = 0; k < A.ffn_n; k++) {
            P.a[k] = A.ffn_ex[k];
            P.a[k].ntok = 1;
            P.a[k].tk[0] = k;
        }
        for (int k = 0; k < 9; k++) {
            P.dsl[0][k] = k < A.ffn_n ? A.ffn_ex[k].d : NULL;
            P.dq6k[k] = k < A.ffn_n ? A.ffn_ex[k].dq6 : 0;
            P.w[0][k] = 0.0f;
        }
    }
    __syncthreads();
}

__device__ __forceinline__ int type_run_end(const DecPlan &P, int a0, int a_end, bool gu)
{
    const DecActive &X0 = P.a[a0];
    int a1 = a0 + 1;
    while (a1 < a_end && (gu ? (P.a[a1].gq6 == X0.gq6 && P.a[a1].uq6 == X0.uq6) : (P.a[a1].dq6 == X0.dq6))) a1++;
    return a1;
}

/* Gate/up tasks q = a*I + j for q in [q0, q1), all with types (G6, U6).  Each
 * wave loads the chunks of PF tasks (GU_PF, or GU_PF_B with several tokens),
 * then computes them.  With one token (decode batch 1 and kernel_ffn_fused)
 * the lane's activations are loaded into registers once and reused by every
 * task. */
template <bool G6, bool U6, bool ONE>
__device__ void gu_tasks(const DecArgs &A, const DecPlan &P, int q0, int q1, const float *xn, const float *xsum)
{
    const int H = A.H, I = A.I, nb = H / RQK;
    const int lane = threadIdx.x & 63, c = lane & 7, lb = lane >> 3;
    const int gw = blockIdx.x * DW + wave_id(), nw = gridDim.x * DW;
    const int ga = lb * RQK + q_run_a<G6>(c), gb = ga + q_run_b_off<G6>();
    const int ua = lb * RQK + q_run_a<U6>(c), ub = ua + q_run_b_off<U6>();
    float4 xga[4], xgb[4], xua[4], xub[4];
    float sga = 0.0f, sgb = 0.0f, sua = 0.0f, sub = 0.0f;
    if (ONE && lb < nb) {
        load_x16(xn, ga, xga, A.xswz);
        load_x16(xn, gb, xgb, A.xswz);
        load_x16(xn, ua, xua, A.xswz);
        load_x16(xn, ub, xub, A.xswz);
        sga = xsum[ga >> 4]; sgb = xsum[gb >> 4]; sua = xsum[ua >> 4]; sub = xsum[ub >> 4];
    }
    constexpr int PF = ONE ? GU_PF : GU_PF_B;
    for (int qs = first_of(q0, gw, nw); qs < q1; qs += nw * PF) {
        QChunk2 ch[PF];
#pragma unroll
        for (int f = 0; f < PF; f++) {
            const int q = min(qs + f * nw, q1 - 1);          /* unconditional: past q1 repeats the last task */
            const DecActive &X = P.a[q / I];
            ch[f] = load_gu_pair<G6, U6>(X.g, X.u, q % I, nb, lb, c);
        }
#pragma unroll
        for (int f = 0; f < PF; f++) {
            const int q = qs + f * nw;
            if (q >= q1) break;
            const DecActive &X = P.a[q / I];
            if (ONE) {
                float pg = 0.0f, pu = 0.0f;
                if (lb < nb) {
                    pg = q_chunk_dot_r<G6>(ch[f].g, c, xga, xgb, sga, sgb);
                    pu = q_chunk_dot_r<U6>(ch[f].u, c, xua, xub, sua, sub);
                }
                pg = group_sum<64>(pg);
                pu = group_sum<64>(pu);
                if (lane == 0) A.eh[(size_t)X.tk[0] * I + q % I] = silu_mul(pg, pu);
            } else {
                gu_row<G6, U6>(A, q % I, ch[f], X.ntok, X.tk, xn, xsum);
            }
        }
    }
}

template <bool G6, bool U6>
__device__ __forceinline__ void gu_tasks_any(const DecArgs &A, const DecPlan &P, int q0, int q1, const float *xn,
                                             const float *xsum)
{
    if (A.B == 1) gu_tasks<G6, U6, true>(A, P, q0, q1, xn, xsum);
    else gu_tasks<G6, U6, false>(A, P, q0, q1, xn, xsum);
}

/* Publish the plan (workgroup 0: the plan for the down kernel, ids and
 * weights for the caller, the routing error), then warm the last-level cache
 * with this layer's down matrices (the plan's active experts): one dword per
 * 128-byte line, spread over the grid, so that the down kernel's weight loads
 * hit the cache.  Returns the loaded value, which the kernel folds into a
 * condition that is never true so the load is kept. */
__device__ __forceinline__ uint32_t publish_and_warm(const DecArgs &A, const DecPlan &P, int l)
{
    const int B = A.B, tid = threadIdx.x;
    if (blockIdx.x == 0) {
        for (int i = tid; i < (int)(sizeof(DecPlan) / 16); i += DT) ((uint4 *)A.plan_g)[i] = ((const uint4 *)&P)[i];
        if (!A.ffn_out && tid < B * RTOPK) {
            const size_t o = ((size_t)(l - A.layer0) * B + (tid >> 3)) * RTOPK + (tid & 7);
            if (A.ids_out) A.ids_out[o] = P.ids[tid >> 3][tid & 7];
            if (A.w_out) A.w_out[o] = P.w[tid >> 3][tid & 7];
        }
        if (tid == 0 && P.err) atomicOr(A.err, 1);
    }
    uint32_t warm = 0;
    if (!A.ffn_out) {
        const size_t lpe = (size_t)A.H * (A.I / RQK) * RQ6K_BYTES / 128;   /* lines per expert slot (Q6_K bound) */
        const size_t g = (size_t)blockIdx.x * DT + tid;
        const int a = (int)(g / lpe);
        if (a < P.nact) {
            const size_t lines = (size_t)A.H * (A.I / RQK) * (P.a[a].dq6 ? RQ6K_BYTES : RQ4K_BYTES) / 128;
            const size_t li = g % lpe;
            if (li < lines) warm = *(const GAS uint32_t *)(P.a[a].d + li * 128);
        }
    }
    return warm;
}

/* Gate/up rows of every routed active expert of the plan, in runs of equal
 * matrix types (ONE: the plan has one token).  Each kernel calls it from one
 * place, so that it is inlined. */
template <bool ONE>
__device__ __forceinline__ void gu_all(const DecArgs &A, const DecPlan &P, const float *xn, const float *xsum)
{
    const int I = A.I;
    for (int a0 = 0; a0 < P.nroute;) {
        const int a1 = type_run_end(P, a0, P.nroute, true);
        const int kind = (P.a[a0].gq6 ? 2 : 0) | (P.a[a0].uq6 ? 1 : 0);
        if (ONE) {
            if (kind == 0) gu_tasks<false, false, true>(A, P, a0 * I, a1 * I, xn, xsum);
            else if (kind == 3) gu_tasks<true, true, true>(A, P, a0 * I, a1 * I, xn, xsum);
            else if (kind == 2) gu_tasks<true, false, true>(A, P, a0 * I, a1 * I, xn, xsum);
            else gu_tasks<false, true, true>(A, P, a0 * I, a1 * I, xn, xsum);
        } else {
            if (kind == 0) gu_tasks_any<false, false>(A, P, a0 * I, a1 * I, xn, xsum);
            else if (kind == 3) gu_tasks_any<true, true>(A, P, a0 * I, a1 * I, xn, xsum);
            else if (kind == 2) gu_tasks_any<true, false>(A, P, a0 * I, a1 * I, xn, xsum);
            else gu_tasks_any<false, true>(A, P, a0 * I, a1 * I, xn, xsum);
        }
        a0 = a1;
    }
}

/* One token (decode batch 1): wave 0 ranks the top-8 (topk8_fast, a few
 * hundred cycles where the eight reduction rounds take thousands), then every
 * wave issues the loads of its GU_PF gate/up tasks before the plan is built,
 * so the rows' memory latency overlaps the plan, its publication and the
 * warming reads.  With one token and 8 selectable logits the routed active
 * experts are the slots in order, so task q = a*I + j is row j of slot a's
 * expert; otherwise, or when the grid has fewer than 8*I / GU_PF waves, the
 * preloaded rows are dropped, false is returned and the caller runs the
 * plan's tasks through gu_all.  Routed gate / up types are the layer's
 * (G6, U6). */
template <bool G6, bool U6>
__device__ __forceinline__ bool gu_one_token(const DecArgs &A, const DecLayer &L, DecPlan &P, const float lg[4],
                                             float sg, const float *xn, const float *xsum, int l, uint32_t &warm,
                                             TopkScratch *ts)
{
    const int I = A.I, nb = A.H / RQK, ntask = RTOPK * I;
    const int lane = threadIdx.x & 63, c = lane & 7, lb = lane >> 3, wv = wave_id();
    const int gw = blockIdx.x * DW + wv, nw = gridDim.x * DW;
    if (wv == 0) {
        if (lane == 0) P.err = 0;
        topk8_fast(lg, A.E, P.ids[0], P.w[0], &P.err, ts);
    }
    __syncthreads();
    QChunk2 ch[GU_PF];
#pragma unroll
    for (int f = 0; f < GU_PF; f++) {
        /* task f of this wave, clamped to the last task so that the load is
         * unconditional (a wave without task f loads a row it does not use);
         * an unselected slot (id -1) loads expert 0's row */
        const int q = min(gw + f * nw, ntask - 1);
        const int e = max(P.ids[0][q / I], 0);
        ch[f] = load_gu_pair<G6, U6>(L.gate + (size_t)e * L.eb[0], L.up + (size_t)e * L.eb[1], q % I, nb, lb, c);
    }
    plan_one_token(A, L, P, sg);
    PHASE_TS(1, 2);
    warm = publish_and_warm(A, P, l);
    if (P.nroute != RTOPK || GU_PF * nw < ntask) return false;      /* not every task preloaded */
    {
        const int ga = lb * RQK + q_run_a<G6>(c), gb = ga + q_run_b_off<G6>();
        const int ua = lb * RQK + q_run_a<U6>(c), ub = ua + q_run_b_off<U6>();
        float4 xga[4], xgb[4], xua[4], xub[4];
        float sga = 0.0f, sgb = 0.0f, sua = 0.0f, sub = 0.0f;
        if (lb < nb) {
            load_x16(xn, ga, xga, A.xswz);
            load_x16(xn, gb, xgb, A.xswz);
            load_x16(xn, ua, xua, A.xswz);
            load_x16(xn, ub, xub, A.xswz);
            sga = xsum[ga >> 4]; sgb = xsum[gb >> 4]; sua = xsum[ua >> 4]; sub = xsum[ub >> 4];
        }
#pragma unroll
        for (int f = 0; f < GU_PF; f++) {
            const int q = gw + f * nw;
            if (q >= ntask) break;
            float pg = 0.0f, pu = 0.0f;
            if (lb < nb) {
                pg = q_chunk_dot_r<G6>(ch[f].g, c, xga, xgb, sga, sgb);
                pu = q_chunk_dot_r<U6>(ch[f].u, c, xua, xub, sua, sub);
            }
            pg = group_sum<64>(pg);
            pu = group_sum<64>(pu);
            if (lane == 0) A.eh[(size_t)P.a[q / I].tk[0] * I + q % I] = silu_mul(pg, pu);
        }
    }
    return true;
}

extern "C" __global__ void __launch_bounds__(DT, 2) dec_gu_kernel(DecArgs A, int l)
{
    extern __shared__ __align__(16) float lds[];
    __shared__ DecPlan P;
    __shared__ float red[DW][RMAX_B];
    __shared__ float inv_rms[RMAX_B];
    __shared__ unsigned long long emask[256];
    __shared__ TopkScratch ts[DW];
    const int B = A.B, E = A.E;
    float *xn = lds, *xsum = lds + B * A.H;
    PHASE_TS(1, 0);
    if (A.ffn_out) {
        ffn_plan(A, P);
        block_norm(A, l, xn, xsum, red, inv_rms);
    } else {
        /* logits of this wave's tokens and the shared-gate logits, loaded with h */
        const int lane = threadIdx.x & 63, wv = wave_id();
        const float *lg = A.logits_in ? A.logits_in : A.logits;
        float lg4[(RMAX_B + DW - 1) / DW][4];
#pragma unroll
        for (int r = 0; r < (RMAX_B + DW - 1) / DW; r++) {
            const int t = wv + r * DW;
#pragma unroll
            for (int i = 0; i < 4; i++)
                lg4[r][i] = (t < B && lane + 64 * i < E) ? lg[(size_t)t * E + lane + 64 * i] : -INFINITY;
        }
        const float sg = threadIdx.x < B ? A.sgate_raw[threadIdx.x] : 0.0f;
        const DecLayer L = A.layers[l];
        block_copy16(xn, A.xn_g, B * (A.H + A.H / 16) / 4);     /* published swizzled by the router kernel */
        __syncthreads();
        PHASE_TS(1, 1);
        build_plan(A, L, P, lg4, sg, emask, ts);
    }
    PHASE_TS(1, 2);
    const uint32_t warm = publish_and_warm(A, P, l);
    gu_all<false>(A, P, xn, xsum);
    PHASE_TS(1, 3);
    if (warm == 0x9E3779B9u && threadIdx.x == 0) A.err[1] = (int)warm;   /* data-dependent sink, keeps the load */
}

/* The gate/up kernel for one token in the layer stack (decode batch 1): see
 * gu_one_token. */
extern "C" __global__ void __launch_bounds__(DT, 2) dec_gu1_kernel(DecArgs A, int l)
{
    extern __shared__ __align__(16) float lds[];
    __shared__ DecPlan P;
    __shared__ TopkScratch ts;
    const int E = A.E, lane = threadIdx.x & 63;
    float *xn = lds, *xsum = lds + A.H;
    PHASE_TS(1, 0);
    const float *lg = A.logits_in ? A.logits_in : A.logits;
    float lg4[4];
#pragma unroll
    for (int i = 0; i < 4; i++) lg4[i] = lane + 64 * i < E ? lg[lane + 64 * i] : -INFINITY;
    const float sg = A.sgate_raw[0];
    const DecLayer L = A.layers[l];
    /* waves 1..3 stage the normalised input (published swizzled by the router
     * kernel: (H + H/16) / 4 <= 3 * 192 16-byte units) while wave 0 ranks the
     * top-8; the barrier after the ranking covers both */
    if (wave_id() > 0) {
        const int n16 = (A.H + A.H / 16) / 4, t3 = threadIdx.x - 64;
        uint4 v[3];
#pragma unroll
        for (int k = 0; k < 3; k++) v[k] = ((const uint4 *)A.xn_g)[min(t3 + k * (DT - 64), n16 - 1)];
#pragma unroll
        for (int k = 0; k < 3; k++) ((uint4 *)xn)[min(t3 + k * (DT - 64), n16 - 1)] = v[k];
    }
    PHASE_TS(1, 1);
    const int kind = (L.q6[0] ? 2 : 0) | (L.q6[1] ? 1 : 0);
    uint32_t warm = 0;
    bool done;
    if (kind == 0) done = gu_one_token<false, false>(A, L, P, lg4, sg, xn, xsum, l, warm, &ts);
    else if (kind == 3) done = gu_one_token<true, true>(A, L, P, lg4, sg, xn, xsum, l, warm, &ts);
    else if (kind == 2) done = gu_one_token<true, false>(A, L, P, lg4, sg, xn, xsum, l, warm, &ts);
    else done = gu_one_token<false, true>(A, L, P, lg4, sg, xn, xsum, l, warm, &ts);
    if (!done) gu_all<true>(A, P, xn, xsum);
    PHASE_TS(1, 3);
    if (warm == 0x9E3779B9u && threadIdx.x == 0) A.err[1] = (int)warm;   /* data-dependent sink, keeps the load */
}

/* ---- D: down rows + combine ----------------------------------------------- */

/* Down tasks of slots [k0, k1) of this workgroup's token (all of type D6):
 * task q = (k - k0) * ngroups + g covers rows r0 + g*rpw + lane/lpr of slot
 * k's down matrix sd[k], dotted with the slot's SiLU*up vector in LDS (ehl,
 * with 16-column sums ehs), into dbuf[k][row - r0].  Every wave issues the
 * loads of D_PF tasks before computing any. */
template <bool D6>
__device__ void down_slots(const DecArgs &A, const uint8_t *const *sd, int k0, int k1, float *dbuf, int ngroups,
                           int dr, int r0, const float *ehl, const float *ehs, const uint8_t *fb)
{
    const int H = A.H, I = A.I, nb = I / RQK;
    const int lane = threadIdx.x & 63, wv = wave_id();
    const int lpr = lanes_per_row(nb), rpw = 64 / lpr;
    const int rw = lane / lpr, lr = lane % lpr, c = lr & 7, lb = lr >> 3;
    const size_t dbs = D6 ? RQ6K_BYTES : RQ4K_BYTES;
    const int ca = lb * RQK + q_run_a<D6>(c), cb = ca + q_run_b_off<D6>();
    const int q1 = (k1 - k0) * ngroups;
    for (int qs = wv; qs < q1; qs += DW * D_PF) {
        /* loads are unconditional (a guarded load is exec-masked or branched
         * around, and the compiler then waits before the next one): tasks past
         * q1 repeat the last task, rows past the matrix or the block and
         * blocks past the row read a valid chunk, an unselected slot reads fb;
         * none of those is used */
        QChunk ch[D_PF];
#pragma unroll
        for (int f = 0; f < D_PF; f++) {
            const int q = min(qs + f * DW, q1 - 1);
            const int k = k0 + q / ngroups, g = q % ngroups;
            const int row = min(r0 + g * rpw + rw, H - 1);
            const uint8_t *m = uniform_ptr(sd[k]);
            ch[f] = q_load<D6>((m ? m : fb) + ((size_t)row * nb + min(lb, nb - 1)) * dbs, c);
        }
#pragma unroll
        for (int f = 0; f < D_PF; f++) {
            const int q = qs + f * DW;
            if (q >= q1) break;
            const int k = k0 + q / ngroups, g = q % ngroups;
            const int rl = g * rpw + rw, row = r0 + rl;
            const bool live = rl < dr && row < H && lb < nb && uniform_ptr(sd[k]) != NULL;
            float part = 0.0f;
            if (live) {
                const float *x = ehl + k * I, *xs = ehs + k * (I / 16);
                part = q_chunk_dot<D6>(ch[f], c, x + ca, x + cb, xs[ca >> 4], xs[cb >> 4]);
            }
            part = group_sum_w(part, lpr);
            if (live && lr == 0) dbuf[k * D_MAXR + rl] = part;
        }
    }
}

/* Down rows and combine for one token when the 9 down matrices share one
 * type D6 (A.d1, set per launch): each wave reads its tasks' slot pointers
 * straight from the published plan and issues the weight-row loads as soon
 * as they arrive, before the SiLU*up rows are stored to LDS, so the rows'
 * memory latency overlaps the copy, the barriers and the run sums.  Tasks as
 * in down_slots (q = k * ngroups + g, wave w takes q = w, w + 4, ...; the
 * host checks that D_PF tasks per wave cover them); loads are unconditional
 * (clamped task, row and block; an unselected slot reads the shared slot's
 * matrix) and the copy's stores wait for the copy's loads only. */
template <bool D6>
__device__ __forceinline__ void down_one_token(const DecArgs &A, int dr, float *ehl, float *ehs, float *dbuf, float *sw)
{
    const int H = A.H, I = A.I, nb = I / RQK, tid = threadIdx.x, lane = tid & 63, wv = wave_id();
    const int lpr = lanes_per_row(nb), rpw = 64 / lpr, ngroups = (dr + rpw - 1) / rpw, ntask = 9 * ngroups;
    const int rw = lane / lpr, lr = lane % lpr, c = lr & 7, lb = lr >> 3;
    const int r0 = blockIdx.x * dr;
    const size_t dbs = D6 ? RQ6K_BYTES : RQ4K_BYTES;
    const int ca = lb * RQK + q_run_a<D6>(c), cb = ca + q_run_b_off<D6>();
    const DecPlan *PG = A.plan_g;
    /* the residual of this thread's output row (stack mode), read first */
    const float hv = A.y ? 0.0f : A.h[min(r0 + min(tid, dr - 1), H - 1)];
    const uint8_t *mp[D_PF];
#pragma unroll
    for (int f = 0; f < D_PF; f++) mp[f] = PG->dsl[0][min(wv + f * DW, ntask - 1) / ngroups];
    const uint8_t *fb = PG->dsl[0][8];
    const float wk = PG->w[0][min(tid, 8)];
    /* the SiLU*up rows: 9 x I / 4 16-byte units, 5 per thread (I <= 568), in
     * named registers (an array here is not kept in registers across the
     * scheduling fences) */
    const int n16 = 9 * I / 4;
    const uint4 *eh4 = (const uint4 *)A.eh;
    const uint4 e0 = eh4[min(tid, n16 - 1)], e1 = eh4[min(tid + DT, n16 - 1)], e2 = eh4[min(tid + 2 * DT, n16 - 1)];
    const uint4 e3 = eh4[min(tid + 3 * DT, n16 - 1)], e4 = eh4[min(tid + 4 * DT, n16 - 1)];
    __builtin_amdgcn_sched_barrier(0);
    QChunk ch[D_PF];
#pragma unroll
    for (int f = 0; f < D_PF; f++) {
        const int q = min(wv + f * DW, ntask - 1), g = q % ngroups;
        const int row = min(r0 + g * rpw + rw, H - 1);
        const uint8_t *m = mp[f] ? mp[f] : fb;
        ch[f] = q_load<D6>(m + ((size_t)row * nb + min(lb, nb - 1)) * dbs, c);
    }
    __builtin_amdgcn_sched_barrier(0);
    uint4 *el4 = (uint4 *)ehl;
    el4[min(tid, n16 - 1)] = e0;
    el4[min(tid + DT, n16 - 1)] = e1;
    el4[min(tid + 2 * DT, n16 - 1)] = e2;
    el4[min(tid + 3 * DT, n16 - 1)] = e3;
    el4[min(tid + 4 * DT, n16 - 1)] = e4;
    sw[min(tid, 8)] = wk;                                   /* threads past 8 store slot 8's weight again */
    for (int i = tid; i < 9 * D_MAXR; i += DT) dbuf[i] = 0.0f;
    __syncthreads();
    for (int r = tid; r < 9 * (I / 16); r += DT) ehs[r] = sum16(ehl + r * 16);
    __syncthreads();
    PHASE_TS(2, 1);
#pragma unroll
    for (int f = 0; f < D_PF; f++) {
        const int q = wv + f * DW;
        if (q >= ntask) break;
        const int k = q / ngroups, g = q % ngroups;
        const int rl = g * rpw + rw, row = r0 + rl;
        const bool live = rl < dr && row < H && lb < nb && mp[f] != NULL;
        float part = 0.0f;
        if (live) {
            const float *x = ehl + k * I, *xs = ehs + k * (I / 16);
            part = q_chunk_dot<D6>(ch[f], c, x + ca, x + cb, xs[ca >> 4], xs[cb >> 4]);
        }
        part = group_sum_w(part, lpr);
        if (live && lr == 0) dbuf[k * D_MAXR + rl] = part;
    }
    __syncthreads();
    PHASE_TS(2, 2);
    for (int rl = tid; rl < dr; rl += DT) {
        const int row = r0 + rl;
        if (row >= H) continue;
        float y = 0.0f;
        for (int k = 0; k < RTOPK; k++) y = fmaf(sw[k], dbuf[k * D_MAXR + rl], y);
        y = fmaf(sw[8], dbuf[8 * D_MAXR + rl], y);
        if (A.y) A.y[row] = y;
        else A.h[row] = hv + y;                             /* rl == tid here */
    }
    PHASE_TS(2, 3);
}

/* One workgroup per (token t, block of dr output rows): the token's nine
 * slots (8 routed experts from the plan's ids, then the shared expert), or
 * the n experts of kernel_ffn_fused for token 0.  The slots' SiLU*up vectors
 * (at most 9 x 2048 floats) are staged in LDS. */
extern "C" __global__ void __launch_bounds__(DT, 3) dec_down_kernel(DecArgs A, int l, int dr)
{
    extern __shared__ __align__(16) float lds[];
    __shared__ float dbuf[9 * D_MAXR];
    __shared__ const uint8_t *sd[9];
    __shared__ float sw[9];
    __shared__ int sq[9];
    const int H = A.H, I = A.I, nb = I / RQK;
    const int tid = threadIdx.x;
    const int nrb = (H + dr - 1) / dr, t = blockIdx.x / nrb, r0 = (blockIdx.x % nrb) * dr;
    const bool ffn = A.ffn_out != NULL;
    const int nslot = ffn ? A.ffn_n : 9;
    PHASE_TS(2, 0);
    float *ehl = lds, *ehs = lds + nslot * I;
    if (A.d1) {
        if (A.d1 == 2) down_one_token<true>(A, dr, ehl, ehs, dbuf, sw);
        else down_one_token<false>(A, dr, ehl, ehs, dbuf, sw);
        return;
    }
    /* slot table (published with the plan): its loads are unconditional,
     * issued first and consumed only after the SiLU*up copy, so both share
     * one memory round trip */
    const int ks = min(tid, 8);
    const uint8_t *pk = A.plan_g->dsl[t][ks];
    const float wk = A.plan_g->w[t][ks];
    const int qk = A.plan_g->dq6k[ks];
    for (int i = tid; i < 9 * D_MAXR; i += DT) dbuf[i] = 0.0f;
    block_copy16(ehl, A.eh + (size_t)(ffn ? 0 : t * 9) * I, nslot * I / 4);
    if (tid < 9) {
        sd[tid] = pk;
        sw[tid] = wk;
        sq[tid] = qk;
    }
    __syncthreads();
    for (int r = tid; r < nslot * (I / 16); r += DT) ehs[r] = sum16(ehl + r * 16);
    __syncthreads();
    const int lpr = lanes_per_row(nb), rpw = 64 / lpr;
    const int ngroups = (dr + rpw - 1) / rpw;
    const uint8_t *fb = uniform_ptr(sd[nslot - 1]);     /* always set: the shared expert, or the last expert */
    PHASE_TS(2, 1);
    for (int k0 = 0; k0 < nslot;) {
        int k1 = k0 + 1;
        while (k1 < nslot && sq[k1] == sq[k0]) k1++;
        if (sq[k0]) down_slots<true>(A, sd, k0, k1, dbuf, ngroups, dr, r0, ehl, ehs, fb);
        else down_slots<false>(A, sd, k0, k1, dbuf, ngroups, dr, r0, ehl, ehs, fb);
        k0 = k1;
    }
    __syncthreads();
    PHASE_TS(2, 2);
    if (ffn) {                          /* kernel_ffn_fused: per-expert outputs */
        for (int idx = tid; idx < nslot * dr; idx += DT) {
            const int k = idx / dr, rl = idx % dr, row = r0 + rl;
            if (row < H) A.ffn_out[(size_t)k * H + row] = dbuf[k * D_MAXR + rl];
        }
    } else {
        for (int rl = tid; rl < dr; rl += DT) {
            const int row = r0 + rl;
            if (row >= H) continue;
            float y = 0.0f;
            for (int k = 0; k < RTOPK; k++) y = fmaf(sw[k], dbuf[k * D_MAXR + rl], y);
            y = fmaf(sw[8], dbuf[8 * D_MAXR + rl], y);
            if (A.y) A.y[(size_t)t * H + row] = y;
            else A.h[(size_t)t * H + row] = A.h[(size_t)t * H + row] + y;
        }
    }
    PHASE_TS(2, 3);
}

/* ---- one launch for one token's layer stack ----------------------------------
 * dec_stack1_kernel runs layers [l0, l0 + n) of one token (model.c:1059-1146 per
 * layer; in stack mode with the carry h += MoE(RMSNorm(h)), model.c:1352-1358)
 * as ONE launch of 256 workgroups in 8 groups of 32, one group per XCD (the
 * group is the XCD a workgroup runs on, so a group shares one L2).  Group k
 * serves routed slot k, the k-th selected expert.  Per layer:
 *   1. every workgroup gathers h -- the caller's buffer for the first layer,
 *      the owners' rows of the previous layer after that -- and normalises it
 *      (block_norm_tail's arithmetic); wave 1 dots router row b (b < E), wave
 *      2 the shared-gate vector, waves 4.. this workgroup's pairs of the
 *      shared expert's gate/up rows; the logit and the shared SiLU*up values
 *      are published;
 *   2. wave 0 gathers the E logits and ranks the top 8 (topk8_fast: larger
 *      logit, then lower index; NaN and -inf never selected; weights by
 *      topk_finish) while wave 3 gathers the shared SiLU*up values;
 *   3. the slot's expert: this workgroup's 1/32 of its gate/up row pairs, and
 *      once those have arrived its 1/32 of the down rows (a burst of about
 *      40 KB per CU in flight completes about twice as fast as one of 64 KB);
 *      SiLU*up is published within the group and gathered; the down rows are
 *      dotted and published;
 *   4. the next layer's router row, shared-gate vector, shared expert rows and
 *      norm weights are loaded: they depend on nothing of this layer, and they
 *      arrive while this layer's outputs are exchanged;
 *   5. workgroup b owns output rows [b H/256, (b + 1) H/256): it dots the
 *      shared expert's down rows for them (after step 2), gathers the eight
 *      slots' down outputs for them, combines y = sum_{k=0..7} w_k d_k +
 *      sigmoid(s) d_shared in that order (model.c:1139-1144) and publishes
 *      h + y for the next layer (after the last layer: writes it, or y, to
 *      the caller's buffer).
 * Exchanges are 64-bit (epoch, value) slots; layer i of a launch uses epoch
 * A.epoch + i and a slot is ready once it carries that epoch, so neither
 * fences nor cache maintenance are needed and nothing is cleared between
 * launches or layers.  Slots read on other XCDs are written with agent-scope
 * stores (through to memory); slots read only within the writer's XCD (the
 * group's SiLU*up values) with workgroup-scope stores that stay in the shared
 * L2, where the readers' agent-scope loads find them (0.23 us one way against
 * 0.48 across XCDs, measured); A.xl2 = 0 writes those through to memory too.
 * A slot is rewritten by the next layer only after every reader has read it:
 * a workgroup publishes layer i + 1 values only after it has gathered h of
 * layer i + 1, which needs every owner's combine of layer i, which comes after
 * that owner's top-8 and gathers of layer i.  Every wait is bounded (A.spin
 * polls); a wait that gives up sets error bit 2 and the workgroup waits for
 * nothing else, so the launch always ends.  Sums, dot lane layouts,
 * reductions, softmax and combine are those of the three-kernel path, so
 * results are bit-identical to it.  NPG / ND: gate/up pairs and down tasks per
 * wave fixed at compile time for the common shapes (every load of a phase then
 * straight-line code), 0 = from the shapes at run time. */
#define K1_T 512
#define K1_W (K1_T / 64)
#define K1_G 8
#define K1_GW 32
#define K1_NWG (K1_G * K1_GW)
#define K1_SPIN (1u << 20)
#define K1_MAXH 2048
#define K1_MAXI 1024
#define K1_MAXPG (K1_MAXI / K1_GW / K1_W)               /* gate/up pairs per wave */
#define K1_MAXD 4                                        /* down tasks per wave */
#define K1_WR 1                                          /* wave roles: router row */
#define K1_WGI 2                                         /* shared-gate vector */
#define K1_WN 3                                          /* norm weights; shared SiLU*up gather */
#define K1_MAXL 64                                       /* layers per launch (descriptors in LDS) */

/* Back-off between polling rounds of an exchange slot, in units of 64 cycles
 * (longer back-offs measured slower). */
#ifndef K1_POLL_SLEEP
#define K1_POLL_SLEEP 1
#endif

__device__ __forceinline__ uint64_t xch_word(float v, uint32_t ep)
{
    return ((uint64_t)ep << 32) | __builtin_bit_cast(uint32_t, v);
}

/* A slot read on other XCDs: written through to memory. */
__device__ __forceinline__ void xch_put(uint64_t *p, float v, uint32_t ep)
{
    __hip_atomic_store(p, xch_word(v, ep), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* A slot read only on the writer's XCD: kept in the shared L2 (l2), else as
 * xch_put. */
__device__ __forceinline__ void xch_put_xcd(uint64_t *p, float v, uint32_t ep, bool l2)
{
    if (l2) __hip_atomic_store(p, xch_word(v, ep), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    else xch_put(p, v, ep);
}

__device__ __forceinline__ uint64_t xch_load(const uint64_t *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* The value of slot p once it carries epoch ep, polling at most spin times
 * (dead: stop waiting). */
__device__ __forceinline__ float xch_wait(const uint64_t *p, uint64_t v, uint32_t ep, int &dead, uint32_t spin)
{
    unsigned it = 0;
    while ((uint32_t)(v >> 32) != ep && !dead) {
        if (++it > spin) {
            dead = 1;
            break;
        }
        __builtin_amdgcn_s_sleep(K1_POLL_SLEEP);
        v = xch_load(p);
    }
    return __builtin_bit_cast(float, (uint32_t)v);
}

__device__ __forceinline__ float xch_get(const uint64_t *p, uint32_t ep, int &dead, uint32_t spin)
{
    return xch_wait(p, xch_load(p), ep, dead, spin);
}

/* The values of slots q[0..N) (those with need bit i) once they carry epoch
 * ep.  Every round re-polls all slots still missing, their loads in flight
 * together, so a gather costs the rounds until its last slot is published,
 * not one round trip per slot; at most spin rounds (dead: stop waiting).
 * Rounds are spaced by K1_POLL_SLEEP; a second round kept in flight measured
 * slower (the round left in flight at the end delays the wave's next load). */
template <int N>
__device__ __forceinline__ void xch_gather(const uint64_t *const (&q)[N], unsigned need, uint32_t ep, int &dead,
                                           uint32_t spin, float (&o)[N])
{
    uint64_t r[N];
#pragma unroll
    for (int i = 0; i < N; i++) r[i] = xch_load(q[i]);
    unsigned it = 0;
    for (;;) {
        unsigned miss = 0;
#pragma unroll
        for (int i = 0; i < N; i++) miss |= ((need >> i) & 1u) && (uint32_t)(r[i] >> 32) != ep ? 1u << i : 0u;
        if (!miss || dead) break;
        if (++it > spin) {
            dead = 1;
            break;
        }
        __builtin_amdgcn_s_sleep(K1_POLL_SLEEP);
#pragma unroll
        for (int i = 0; i < N; i++)
            if ((miss >> i) & 1u) r[i] = xch_load(q[i]);
    }
#pragma unroll
    for (int i = 0; i < N; i++) o[i] = __builtin_bit_cast(float, (uint32_t)r[i]);
}

/* q_load with the block type chosen at run time (the type comes from the
 * layer descriptor, so the branch is wave-uniform). */
__device__ __forceinline__ QChunk q_load_t(int q6, const uint8_t *m, size_t row, int nb, int lb, int c)
{
    const int lbc = lb < nb ? lb : nb - 1;
    return q6 ? q_load<true>(m + (row * nb + lbc) * RQ6K_BYTES, c) : q_load<false>(m + (row * nb + lbc) * RQ4K_BYTES, c);
}

__device__ __forceinline__ int q_run_a_t(int q6, int c) { return q6 ? q_run_a<true>(c) : q_run_a<false>(c); }

/* silu(gate_j . x) * (up_j . x) from the lane's chunks of one gate/up row
 * pair, x and its run sums in LDS (gu_row's arithmetic for one token). */
__device__ __forceinline__ float k1_gu_pair(int g6, int u6, const QChunk2 &ch, const float *xn, const float *xsum,
                                            bool swz, int nb, int lane)
{
    const int c = lane & 7, lb = lane >> 3;
    float pg = 0.0f, pu = 0.0f;
    if (lb < nb) {
        const int ga = lb * RQK + q_run_a_t(g6, c), gb = ga + (g6 ? 64 : 32);
        const int ua = lb * RQK + q_run_a_t(u6, c), ub = ua + (u6 ? 64 : 32);
        float4 x0[4], x1[4];
        load_x16(xn, ga, x0, swz);
        load_x16(xn, gb, x1, swz);
        pg = g6 ? q_chunk_dot_r<true>(ch.g, c, x0, x1, xsum[ga >> 4], xsum[gb >> 4])
                : q_chunk_dot_r<false>(ch.g, c, x0, x1, xsum[ga >> 4], xsum[gb >> 4]);
        load_x16(xn, ua, x0, swz);
        load_x16(xn, ub, x1, swz);
        pu = u6 ? q_chunk_dot_r<true>(ch.u, c, x0, x1, xsum[ua >> 4], xsum[ub >> 4])
                : q_chunk_dot_r<false>(ch.u, c, x0, x1, xsum[ua >> 4], xsum[ub >> 4]);
    }
    pg = group_sum<64>(pg);
    pu = group_sum<64>(pu);
    return silu_mul(pg, pu);
}

/* One gate or up row's dot (k1_gu_pair's arithmetic for one of its rows). */
__device__ __forceinline__ float k1_q_row(int q6, const QChunk &ch, const float *xn, const float *xsum, bool swz, int nb,
                                          int lane)
{
    const int c = lane & 7, lb = lane >> 3;
    float p = 0.0f;
    if (lb < nb) {
        const int a = lb * RQK + q_run_a_t(q6, c), b = a + (q6 ? 64 : 32);
        float4 x0[4], x1[4];
        load_x16(xn, a, x0, swz);
        load_x16(xn, b, x1, swz);
        p = q6 ? q_chunk_dot_r<true>(ch, c, x0, x1, xsum[a >> 4], xsum[b >> 4])
               : q_chunk_dot_r<false>(ch, c, x0, x1, xsum[a >> 4], xsum[b >> 4]);
    }
    return group_sum<64>(p);
}

/* One down row's lane partial against a SiLU*up vector in LDS (plain layout)
 * and its run sums (down_one_token's arithmetic), reduced over the row's
 * lpr lanes. */
__device__ __forceinline__ float k1_down_row(int d6, const QChunk &ch, const float *eh, const float *ehs, bool live,
                                             int lpr, int lane)
{
    const int lr = lane % lpr, c = lr & 7, lb = lr >> 3;
    float part = 0.0f;
    if (live) {
        const int ca = lb * RQK + q_run_a_t(d6, c), cb = ca + (d6 ? 64 : 32);
        part = d6 ? q_chunk_dot<true>(ch, c, eh + ca, eh + cb, ehs[ca >> 4], ehs[cb >> 4])
                  : q_chunk_dot<false>(ch, c, eh + ca, eh + cb, ehs[ca >> 4], ehs[cb >> 4]);
    }
    return group_sum_w(part, lpr);
}

/* Router-row dot of one token (router_body's arithmetic): lane partials over
 * its 8 float4 of the row, then the wave sum. */
__device__ __forceinline__ float k1_row_dot(const float4 (&w)[8], const float4 *x4, int H, bool swz, int lane)
{
    float acc = 0.0f;
#pragma unroll
    for (int m = 0; m < 8; m++) {
        const int c0 = 4 * lane + 256 * m;
        if (c0 < H) {
            const float4 x = x4[xpos(c0 >> 2, swz)];
            acc = fmaf(w[m].x, x.x, acc);
            acc = fmaf(w[m].y, x.y, acc);
            acc = fmaf(w[m].z, x.z, acc);
            acc = fmaf(w[m].w, x.w, acc);
        }
    }
    return group_sum<64>(acc);
}

/* SiLU*up vectors of I values in this XCD's region are stored run-major:
 * value j (run j / 16, position j % 16) at slot (j % 16) * (I / 16) + j / 16,
 * so that the 16 polling loads of a gather each read one contiguous span of
 * I / 16 slots across the lanes (two cache lines for I = 512) instead of
 * one line per lane. */
__device__ __forceinline__ size_t k1_run_slot(int j, int I) { return (size_t)(j & 15) * (I >> 4) + (j >> 4); }

/* Run r (values 16r .. 16r + 15) of a run-major vector into dst, and their
 * sum in sum16's order. */
__device__ __forceinline__ float k1_gather_run(const uint64_t *base, int I, int r, uint32_t ep, int &dead,
                                               uint32_t spin, float *dst)
{
    float v[16];
    const uint64_t *q[16];
#pragma unroll
    for (int i = 0; i < 16; i++) q[i] = base + (size_t)i * (I >> 4) + r;
    xch_gather<16>(q, 0xFFFFu, ep, dead, spin, v);
#pragma unroll
    for (int i = 0; i < 16; i += 4) *(float4 *)(dst + i) = make_float4(v[i], v[i + 1], v[i + 2], v[i + 3]);
    return ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7])) +
           (((v[8] + v[9]) + (v[10] + v[11])) + ((v[12] + v[13]) + (v[14] + v[15])));
}

/* Wait until an LDS flag set by another wave of the workgroup reaches v
 * (acquire: that wave's LDS stores before the flag are then visible).  The
 * waves that set the flags reach them through bounded waits only. */
__device__ __forceinline__ void k1_flag_wait(int *flag, int v)
{
    while (__hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < v) __builtin_amdgcn_s_sleep(1);
}

#define K1_SYNC_DEAD()          \
    do {                        \
        if (dead) s_dead = 1;   \
        __syncthreads();        \
        dead = s_dead;          \
    } while (0)

/* The loads of layer l that depend on nothing computed in it, parked in LDS
 * (held in registers they would stay live across the whole layer loop) by
 * waves 1..7, so that wave 0, which combines and publishes h, never waits for
 * them: router row gw (wave K1_WR), the shared-gate vector (K1_WGI), the norm
 * weights (K1_WN), this workgroup's shared gate/up pairs (the last SP waves:
 * a SIMD's second wave is wave w + 4, and waves 1 and 0 on SIMDs 1 and 0 must
 * not share them with a pair's dot when they dot the router row and rank the
 * top 8) and shared down rows (the last nsd waves).  Each store waits for
 * its own loads; waves 1..7 have nothing else to do at that point of a layer.
 * (Every XCD computing all E logits itself would save the relay but read the
 * router 8 times: measured slower over 40 layers.) */
struct K1Pre {
    float4 (*rw)[64];           /* [m][lane] router row gw */
    float4 (*gin)[64];          /* [m][lane] shared-gate vector */
    float *nw;                  /* [H] norm weights */
    QChunk2 (*shc)[64];         /* [pair][lane] */
    QChunk (*sdc)[64];          /* [task][lane] */
};

template <int TY>
__device__ __forceinline__ void k1_prefetch(const DecArgs &A, const DecLayer &L, int l, const K1Pre &P, int wv,
                                            bool rrow, int SP, int sdt, int RO, int rpw, int lane)
{
    const int ws = K1_W - SP;                                /* first shared gate/up pair */
    const int sg6 = TY < 0 ? L.sq6[0] : (TY >> 3) & 1, su6 = TY < 0 ? L.sq6[1] : (TY >> 4) & 1;
    const int sd6 = TY < 0 ? L.sq6[2] : (TY >> 5) & 1;
    const int H = A.H, HU = H / 4, c = lane & 7, lb = lane >> 3;
    const int nbh = H / RQK, nbi = A.I / RQK, lpr = lanes_per_row(nbi), rw_ = lane / lpr, lr = lane % lpr;
    const int gw = blockIdx.x;
    if (wv == 0) return;
    float4 r1[8];
    QChunk2 shc;
    QChunk sdc;
    const float *nw = A.do_norm && A.norm_w ? A.norm_w + (size_t)(l - A.layer0) * H : NULL;
    if (wv == K1_WR && rrow) {
#pragma unroll
        for (int m = 0; m < 8; m++) r1[m] = gld_f4(L.router + (size_t)gw * H + min(4 * lane + 256 * m, H - 4));
    } else if (wv == K1_WGI) {
#pragma unroll
        for (int m = 0; m < 8; m++) r1[m] = gld_f4(L.gate_inp + min(4 * lane + 256 * m, H - 4));
    } else if (wv == K1_WN && nw) {
#pragma unroll
        for (int m = 0; m < 8; m++) r1[m] = ((const float4 *)nw)[min(lane + 64 * m, HU - 1)];
    }
    if (wv >= ws) {
        const size_t j = (size_t)gw * SP + (wv - ws);
        shc.g = q_load_t(sg6, L.sgate, j, nbh, lb, c);
        shc.u = q_load_t(su6, L.sup, j, nbh, lb, c);
    }
    if (sdt >= 0) sdc = q_load_t(sd6, L.sdown, (size_t)min(gw * RO + sdt * rpw + rw_, H - 1), nbi, lr >> 3, lr & 7);
    if (wv == K1_WR && rrow) {
#pragma unroll
        for (int m = 0; m < 8; m++) P.rw[m][lane] = r1[m];
    } else if (wv == K1_WGI) {
#pragma unroll
        for (int m = 0; m < 8; m++) P.gin[m][lane] = r1[m];
    } else if (wv == K1_WN && nw) {
#pragma unroll
        for (int m = 0; m < 8; m++)
            if (lane + 64 * m < HU) ((float4 *)P.nw)[lane + 64 * m] = r1[m];
    }
    if (wv >= ws) P.shc[wv - ws][lane] = shc;
    if (sdt >= 0) P.sdc[sdt][lane] = sdc;
}

/* Layer i of the call from its LDS copy, as wave-uniform (scalar) values. */
__device__ __forceinline__ DecLayer k1_layer(const DecLayer *Ls, int i)
{
    DecLayer L;
    const uint32_t *s = (const uint32_t *)(Ls + i);
    uint32_t *d = (uint32_t *)&L;
#pragma unroll
    for (int w = 0; w < (int)(sizeof(DecLayer) / 4); w++) d[w] = __builtin_amdgcn_readfirstlane(s[w]);
    return L;
}

/* End of a one-launch stack kernel.  A stack call (A.y NULL) stages its final
 * hidden state, nh epoch-tagged values at hst written by other workgroups,
 * instead of writing the caller's h.  Every workgroup reports a wait that gave
 * up (error bit 2) and then counts itself done on A.cnt (thread 0 waits for the
 * report to be performed before counting); the last of the K1_NWG, which then
 * sees every report, copies the staged state over A.h only when none gave up:
 * it first waits (bounded, like every exchange) until each staged value
 * carries the layer's epoch, then writes them all, so a call that failed
 * leaves h as it was.  The count stays a multiple of K1_NWG between launches
 * (layer-output calls, A.y set, only report).  Called by every thread;
 * dead_any workgroup-uniform; s_last is LDS. */
__device__ __forceinline__ void k1_finish(const DecArgs &A, bool dead_any, int *s_last, const uint64_t *hst, int nh,
                                          uint32_t epl)
{
    __syncthreads();
    if (A.y) {                           /* layer output written directly: nothing staged, no count */
        if (threadIdx.x == 0 && dead_any) atomicOr(A.err, 2);
        return;
    }
    if (threadIdx.x == 0) {
        /* The report is performed at the device-coherent point before this
         * workgroup counts itself, so the last to count reads every report.
         * No release fence: the staged values carry their epoch and are polled
         * for it, so their stores need no ordering (an agent-scope release
         * writes back the XCD's whole L2, ~7 us per launch). */
        if (dead_any) __hip_atomic_fetch_or(A.err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        const uint32_t old = __hip_atomic_fetch_add(A.cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        int sl = 0;
        if ((old + 1u) % (uint32_t)K1_NWG == 0u) {
            asm volatile("" ::: "memory");
            sl = (__hip_atomic_load(A.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & 2) ? 0 : 1;
        }
        *s_last = sl;
    }
    __syncthreads();
    if (!*s_last) return;                                     /* workgroup-uniform */
    int dead = 0;
    for (int r = threadIdx.x; r < nh; r += blockDim.x) (void)xch_get(hst + r, epl, dead, A.spin);
    if (dead) *s_last = 2;
    __syncthreads();
    if (*s_last == 2) {
        if (threadIdx.x == 0) atomicOr(A.err, 2);
        return;
    }
    for (int r = threadIdx.x; r < nh; r += blockDim.x) A.h[r] = __builtin_bit_cast(float, (uint32_t)xch_load(hst + r));
}

template <int NPG, int ND, int TY>
__device__ __forceinline__ void stack1_body(const DecArgs &A)
{
    __shared__ __align__(16) float xn[K1_MAXH];
    __shared__ float xsum[K1_MAXH / 16];
    __shared__ __align__(16) float hraw[K1_MAXH];           /* this layer's h (the owned rows' residual) */
    __shared__ __align__(16) float nw_s[K1_MAXH];
    __shared__ __align__(16) float ehk[K1_MAXI];
    __shared__ float ehks[K1_MAXI / 16];
    __shared__ __align__(16) float ehsh[K1_MAXI];
    __shared__ float ehshs[K1_MAXI / 16];
    __shared__ TopkScratch tks;
    __shared__ int ids_s[RTOPK];
    __shared__ float w_s[RTOPK + 1];
    __shared__ float red_s[4];
    __shared__ __align__(16) DecLayer Ls[K1_MAXL];
    __shared__ float4 rrow_s[8][64];                          /* router row gw */
    __shared__ float4 gin_s[8][64];
    __shared__ QChunk2 shc_s[K1_MAXI / 256][64];
    __shared__ QChunk sdc_s[4][64];
    __shared__ int s_dead, s_err;
    __shared__ int s_ids_ready, s_ehsh_ready;                  /* layer index + 1 once ids_s / ehsh are in */

    const int H = A.H, I = A.I, E = A.E, HU = H / 4, nbh = H / RQK, nbi = I / RQK;
    const int tid = threadIdx.x, lane = tid & 63, wv = wave_id();
    /* group = the XCD this workgroup runs on: the dispatcher deals the grid's
     * workgroups to the 8 XCDs in turn, starting at an XCD that varies from
     * launch to launch, so XCD(b) = (b + r) % 8 with one r per launch and
     * b / 8 numbers the 32 workgroups of each XCD (the library checks the
     * pattern once per process; without it groups are b % 8 and every slot
     * goes through memory) */
    unsigned xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    xcc &= 0xFu;
    const bool l2 = A.xl2 && xcc < (unsigned)K1_G;
    if (A.xl2 && !l2 && threadIdx.x == 0) atomicOr(A.err, 4);
    const int grp = l2 ? (int)xcc : (int)(blockIdx.x % K1_G), gi = blockIdx.x / K1_G, gw = blockIdx.x;
    const bool swz = A.xswz;
    uint64_t *xlg = A.xch + XCH_LG(E, H, I);                  /* across XCDs */
    uint64_t *xehs = A.xch + XCH_EHS(E, H, I);
    uint64_t *xdx = A.xch + XCH_DX(E, H, I);
    uint64_t *xdsh = A.xch + XCH_DSH(E, H, I);
    uint64_t *loc = A.xch + XCH_LOC0(E, H, I) + (size_t)grp * XCH_LOCN(E, H, I);   /* this XCD's */
    uint64_t *llg = loc + XCH_LLG(I), *lehs = loc + XCH_LEHS(I), *lehx = loc + XCH_LEHX(I), *lh = loc + XCH_LH(I);
    const int RO = H / 256;                                  /* shared down rows of this workgroup */
    const int SP = I / 256;                                  /* shared gate/up pairs of this workgroup */
    const int RD = H / K1_GW;                                /* routed down rows; rows combined */
    const int LPW = E / K1_GW, SPW = I / K1_GW;              /* logits, shared SiLU*up relayed into the XCD */
    const int lpr = lanes_per_row(nbi), rpw = 64 / lpr;
    const int nsd = (RO + rpw - 1) / rpw;                    /* shared down tasks */
    const int sdt = wv - (K1_W - nsd);
    const K1Pre P = {rrow_s, gin_s, nw_s, shc_s, sdc_s};
    const bool rrow = gw < E && !A.logits_in;                /* this workgroup dots router row gw */
    const int n = A.nlayers;
#ifdef ROASTER_PHASE_TS
    unsigned long long tsv[2][16] = {};
    int tsl = 0;
#define K1_TS(i) asm volatile("s_memrealtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(tsv[tsl][i]) : : "memory")
#else
#define K1_TS(i) ((void)0)
#endif
    if (tid == 0) {
        s_dead = 0;
        s_err = 0;
        s_ids_ready = 0;
        s_ehsh_ready = 0;
    }

    /* first layer: h (threads < 256: units t and t + 256), then the weights
     * of the layer */
    float4 hq[2];
#pragma unroll
    for (int k = 0; k < 2; k++) hq[k] = ((const float4 *)A.h)[min(tid + 256 * k, HU - 1)];
    /* error bit 2 from an earlier launch that gave up: wait for nothing */
    int dead = (gld_u32(A.err) & 2u) != 0;
    /* the call's layer descriptors into LDS (read there from the second layer
     * on: a scalar load in flight would hold every LDS wait) */
    constexpr int DQ = (int)(sizeof(DecLayer) / 16);
    const uint4 lq = ((const uint4 *)(A.layers + A.layer0))[min(tid, n * DQ - 1)];
    DecLayer L = A.layers[A.layer0];
    k1_prefetch<TY>(A, L, A.layer0, P, wv, rrow, SP, sdt, RO, rpw, lane);

    for (int li = 0; li < n; li++) {
        /* the thread index as a value opaque to the compiler, per layer: else
         * every lane-derived address is hoisted out of this loop and stays
         * live across it (spilling) */
        int tid_v = (int)threadIdx.x;
        asm volatile("" : "+v"(tid_v));
        const int tid = tid_v, lane = tid_v & 63, c = lane & 7, lb = lane >> 3;
        const int rw_ = lane / lpr, lr = lane % lpr, lbd = lr >> 3;
        const int l = A.layer0 + li;
        const uint32_t ep = A.epoch + (uint32_t)li;
        const bool last = li + 1 == n;
        const float *nwl = A.do_norm && A.norm_w ? nw_s : NULL;
        /* matrix types: from the descriptor, or fixed by TY (bit k: routed
         * gate, up, down, shared gate, up, down is Q6_K) so that every load of
         * a phase is straight-line code and each use waits for its own loads */
        const int g6 = TY < 0 ? L.q6[0] : (TY & 1), u6 = TY < 0 ? L.q6[1] : (TY >> 1) & 1;
        const int d6 = TY < 0 ? L.q6[2] : (TY >> 2) & 1, sg6 = TY < 0 ? L.sq6[0] : (TY >> 3) & 1;
        const int su6 = TY < 0 ? L.sq6[1] : (TY >> 4) & 1, sd6 = TY < 0 ? L.sq6[2] : (TY >> 5) & 1;
#ifdef ROASTER_PHASE_TS
        tsl = li + 1 == n ? 1 : 0;
#endif
        K1_TS(0);
        /* ---- 1. h (after the first layer: this XCD's copy), normalised ------ */
        if (li > 0 && tid < 256) {
            const uint64_t *q[8];
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; i++) q[i] = lh + (size_t)(i & 3) * HU + min(tid + 256 * (i >> 2), HU - 1);
            xch_gather<8>(q, (tid < HU ? 0x0Fu : 0u) | (tid + 256 < HU ? 0xF0u : 0u), ep - 1, dead, A.spin, v);
            hq[0] = make_float4(v[0], v[1], v[2], v[3]);
            hq[1] = make_float4(v[4], v[5], v[6], v[7]);
        }
        float4 *x4 = (float4 *)xn;
        if (li == 0 && n > 1 && tid < n * DQ) ((uint4 *)Ls)[tid] = lq;
        if (tid < 256) {
            float ss = 0.0f;
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const int u = tid + k * 256;
                if (u < HU) {
                    const float4 v = hq[k];
                    ss = fmaf(v.x, v.x, ss);
                    ss = fmaf(v.y, v.y, ss);
                    ss = fmaf(v.z, v.z, ss);
                    ss = fmaf(v.w, v.w, ss);
                    ((float4 *)hraw)[u] = v;
                }
            }
            ss = group_sum<64>(ss);
            if (lane == 0) red_s[wv] = ss;
        }
        K1_SYNC_DEAD();
        if (dead) break;                                  /* workgroup-uniform */
        K1_TS(1);
        /* the normalised input from the h still in registers (waves 0..3,
         * units tid and tid + 256), and the run sums: run r is units 4r ..
         * 4r + 3, i.e. the four lanes of a quad, added pairwise by DPP in
         * the order ((s0 + s1) + (s2 + s3)) */
        if (tid < 256) {
            float inv = 1.0f;
            if (A.do_norm) {
                float s2 = 0.0f;
#pragma unroll
                for (int w = 0; w < 4; w++) s2 += red_s[w];
                inv = 1.0f / sqrtf(s2 / (float)H + A.eps);
            }
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const int u = tid + k * 256;
                float4 v = hq[k];
                if (A.do_norm) {
                    v.x *= inv; v.y *= inv; v.z *= inv; v.w *= inv;
                    if (nwl) {
                        const float4 wq = ((const float4 *)nwl)[min(u, HU - 1)];
                        v.x *= wq.x; v.y *= wq.y; v.z *= wq.z; v.w *= wq.w;
                    }
                }
                float r = (v.x + v.y) + (v.z + v.w);
                r += dpp_f<DPP_XOR1>(r);
                r += dpp_f<DPP_XOR2>(r);
                if (u < HU) {
                    x4[xpos(u, swz)] = v;
                    if ((tid & 3) == 0) xsum[u >> 2] = r;
                }
            }
        }
        __syncthreads();
        K1_TS(2);

        /* ---- 2. router logit gw (wave K1_WR), the shared-gate logit (wave
         * K1_WGI), this workgroup's shared SiLU*up values (the last SP waves): the
         * logit and the shared values go to every XCD ------------------------ */
        if (wv == K1_WR && rrow) {
            float4 rw[8];
#pragma unroll
            for (int m = 0; m < 8; m++) rw[m] = rrow_s[m][lane];
            const float s = k1_row_dot(rw, x4, H, swz, lane);
            if (lane == 0) {
                xch_put(xlg + (size_t)gw * XCH_LN, s, ep);
                if (last) A.logits[gw] = s;
            }
        } else if (wv == K1_WGI) {
            float4 rw[8];
#pragma unroll
            for (int m = 0; m < 8; m++) rw[m] = gin_s[m][lane];
            const float s = k1_row_dot(rw, x4, H, swz, lane);
            if (lane == 0) w_s[RTOPK] = 1.0f / (1.0f + expf(-s));
        } else if (wv >= K1_W - SP) {
            const int pr = wv - (K1_W - SP);
            const float eh = k1_gu_pair(sg6, su6, shc_s[pr][lane], xn, xsum, swz, nbh, lane);
            if (lane == 0) xch_put(xehs + (size_t)gw * XCH_LN + pr, eh, ep);
        }
        K1_TS(3);
        /* ---- 3. wave 0 relays this workgroup's share of the logits (lanes <
         * LPW) into this XCD's region, gathers all E from there and ranks the
         * top 8; wave K1_WN relays its share of the shared SiLU*up values and
         * gathers them all.  The two relays are kept apart so that the logits
         * never wait for the later shared values. ---------------------------- */
        if (wv == 0) {
            if (lane < LPW && !A.logits_in) {
                const int j = gi * LPW + lane;
                const uint64_t *q[1] = {xlg + (size_t)j * XCH_LN};
                float v[1];
                xch_gather<1>(q, 1u, ep, dead, A.spin, v);
                xch_put_xcd(llg + j, v[0], ep, l2);
            }
            K1_TS(13);
            float v4[4];
            if (A.logits_in) {
#pragma unroll
                for (int i = 0; i < 4; i++) v4[i] = A.logits_in[min(lane + 64 * i, E - 1)];
            } else {
                const uint64_t *q[4];
#pragma unroll
                for (int i = 0; i < 4; i++) q[i] = llg + min(lane + 64 * i, E - 1);
                xch_gather<4>(q, 0xFu, ep, dead, A.spin, v4);
            }
            K1_TS(10);
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (lane + 64 * i >= E) v4[i] = -INFINITY;
            topk8_fast(v4, E, ids_s, w_s, &s_err, &tks, &s_ids_ready, li + 1);
            K1_TS(14);
        } else if (wv == K1_WN) {
            if (lane < SPW) {                       /* shared value j: slot j % SP of line j / SP */
                const int j = gi * SPW + lane;
                const uint64_t *q[1] = {xehs + (size_t)(j / SP) * XCH_LN + j % SP};
                float v[1];
                xch_gather<1>(q, 1u, ep, dead, A.spin, v);
                xch_put_xcd(lehs + k1_run_slot(j, I), v[0], ep, l2);
            }
            if (lane < I / 16) ehshs[lane] = k1_gather_run(lehs, I, lane, ep, dead, A.spin, ehsh + 16 * lane);
            if (lane == 0) __hip_atomic_store(&s_ehsh_ready, li + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        /* the other waves go on as soon as wave 0 has stored the ids (before
         * the softmax weights, which only wave 0 uses, in the combine) */
        if (wv == 0) {
            if (gw == 0) {
                if (lane < RTOPK) {
                    const size_t o = (size_t)li * RTOPK + lane;
                    if (A.ids_out) A.ids_out[o] = ids_s[lane];
                    if (A.w_out) A.w_out[o] = w_s[lane];
                }
                if (lane == 0 && s_err) atomicOr(A.err, 1);
            }
        } else {
            k1_flag_wait(&s_ids_ready, li + 1);
        }
        K1_TS(4);

        /* ---- 4. the slot's expert -------------------------------------------- */
        const int e = ids_s[grp];
        const bool live_slot = e >= 0;
        const size_t ee = live_slot ? (size_t)e : 0;          /* an unselected slot reads expert 0, unused */
        const uint8_t *ge = L.gate + ee * L.eb[0], *ue = L.up + ee * L.eb[1], *de = L.down + ee * L.eb[2];
        const int RGP = I / K1_GW, npg = NPG ? NPG : (RGP + K1_W - 1) / K1_W;
        const int ndt = (RD + rpw - 1) / rpw, nd = ND ? ND : (ndt + K1_W - 1) / K1_W;
        constexpr int MPG = NPG ? NPG : K1_MAXPG, MD = ND ? ND : K1_MAXD;
        QChunk2 gch[MPG];
        QChunk dch[MD];
#pragma unroll
        for (int f = 0; f < MPG; f++) {
            if (NPG || f < npg) {
                const size_t j = (size_t)gi * RGP + min(wv + f * K1_W, RGP - 1);
                gch[f].g = q_load_t(g6, ge, j, nbh, lb, c);
            }
        }
#pragma unroll
        for (int f = 0; f < MPG; f++) {
            if (NPG || f < npg) {
                const size_t j = (size_t)gi * RGP + min(wv + f * K1_W, RGP - 1);
                gch[f].u = q_load_t(u6, ue, j, nbh, lb, c);
            }
        }
        /* the shared expert's down rows [gw RO, (gw + 1) RO) while the routed
         * rows are in flight (its SiLU*up values came with the top-8): slot 8
         * of the down outputs */
        if (sdt >= 0) {
            if (wv != K1_WN) k1_flag_wait(&s_ehsh_ready, li + 1);
            const int rl = sdt * rpw + rw_;
            const bool live = rl < RO && lbd < nbi;
            const float part = k1_down_row(sd6, sdc_s[sdt][lane], ehsh, ehshs, live, lpr, lane);
            if (live && lr == 0) xch_put(xdsh + (size_t)gw * XCH_LN + rl, part, ep);
        }
        /* the gate rows were issued first: their dots run while the up rows
         * arrive (each waits for its own rows only: loads complete in order);
         * then the down rows are issued, behind the up rows (issued with the
         * gate rows they measured slower: a 64 KB burst per CU) */
        float pgs[MPG];
#pragma unroll
        for (int f = 0; f < MPG; f++) pgs[f] = (NPG || f < npg) ? k1_q_row(g6, gch[f].g, xn, xsum, swz, nbh, lane) : 0.0f;
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("; gate rows dotted" ::"v"(pgs[0]) : "memory");
#pragma unroll
        for (int f = 0; f < MD; f++) {
            if (ND || f < nd) {
                const int task = min(wv + f * K1_W, ndt - 1);
                dch[f] = q_load_t(d6, de, (size_t)min(gi * RD + task * rpw + rw_, H - 1), nbi, lbd, lr & 7);
            }
        }
        K1_TS(5);
#pragma unroll
        for (int f = 0; f < MPG; f++) {
            const int pj = wv + f * K1_W;
            if ((NPG || f < npg) && pj < RGP) {
                const float eh = silu_mul(pgs[f], k1_q_row(u6, gch[f].u, xn, xsum, swz, nbh, lane));
                if (lane == 0) xch_put_xcd(lehx + k1_run_slot(gi * RGP + pj, I), live_slot ? eh : 0.0f, ep, l2);
            }
        }
        K1_TS(6);
        if (wv == 0 && lane < I / 16) ehks[lane] = k1_gather_run(lehx, I, lane, ep, dead, A.spin, ehk + 16 * lane);
        K1_SYNC_DEAD();
        K1_TS(7);
#pragma unroll
        for (int f = 0; f < MD; f++) {
            const int task = wv + f * K1_W;
            if ((ND || f < nd) && task < ndt) {
                const int rl = task * rpw + rw_, row = gi * RD + rl;
                const bool live = rl < RD && lbd < nbi;
                const float part = k1_down_row(d6, dch[f], ehk, ehks, live, lpr, lane);
                if (live && lr == 0) xch_put(xdx + (size_t)grp * H + row, live_slot ? part : 0.0f, ep);
            }
        }
        K1_TS(8);

        /* ---- 5. the next layer's loads; this XCD's rows [gi RD, (gi + 1) RD)
         * of h: the nine slots' down outputs combined -------------------------- */
        if (!last) {
            L = k1_layer(Ls, li + 1);
            k1_prefetch<TY>(A, L, l + 1, P, wv, rrow, SP, sdt, RO, rpw, lane);
        }
        K1_TS(11);
        if (wv == 0) {
            const int row = gi * RD + min(lane, RD - 1);
            const uint64_t *q[RTOPK + 1];
            float d[RTOPK + 1];
#pragma unroll
            for (int k = 0; k < RTOPK; k++) q[k] = xdx + (size_t)k * H + row;
            q[RTOPK] = xdsh + (size_t)(row / RO) * XCH_LN + row % RO;
            xch_gather<RTOPK + 1>(q, lane < RD ? 0x1FFu : 0u, ep, dead, A.spin, d);
            K1_TS(12);
            if (lane < RD) {
                float y = 0.0f;
#pragma unroll
                for (int k = 0; k < RTOPK; k++) y = fmaf(w_s[k], d[k], y);
                y = fmaf(w_s[RTOPK], d[RTOPK], y);
                const float hn = hraw[row] + y;
                if (!last) xch_put_xcd(lh + (size_t)(row & 3) * (H / 4) + (row >> 2), hn, ep, l2);
                else if (grp == 0) {
                    if (A.y) A.y[row] = y;
                    else xch_put(A.xch + XCH_HST(E, H, I) + row, hn, ep);
                }
            }
        }
        K1_TS(9);
    }
    __shared__ int s_last;
    if (dead) s_dead = 1;
    __syncthreads();
    k1_finish(A, s_dead != 0, &s_last, A.xch + XCH_HST(E, H, I), H, A.epoch + (uint32_t)(n - 1));
#ifdef ROASTER_PHASE_TS
    if (threadIdx.x == 0 || threadIdx.x == 64 || threadIdx.x == 192)
        for (int k = 0; k < 2; k++)
            for (int i = 0; i < 16; i++) g_k1_ts[k][blockIdx.x][min((int)threadIdx.x >> 6, 2)][i] = tsv[k][i];
#endif
#undef K1_TS
}

extern "C" __global__ void __launch_bounds__(K1_T, 1) dec_stack1_kernel(DecArgs A) { stack1_body<0, 0, -1>(A); }
/* hidden 2048, inter 512: two gate/up pairs and two down tasks per wave;
 * gate/up Q4_K and down Q6_K, routed and shared (types 0b100100) */
extern "C" __global__ void __launch_bounds__(K1_T, 1) dec_stack1_2x2_kernel(DecArgs A) { stack1_body<2, 2, 0x24>(A); }

/* ---- one token, the router folded into the combine (dec_stack1r_kernel) ----
 * 256 experts, hidden 2048, inter 512, gate/up Q4_K and down Q6_K (routed and
 * shared).  Groups and slots as in dec_stack1_kernel (XCD k serves routed
 * slot k; workgroup gi of every XCD combines rows [64 gi, 64 gi + 64)), but
 * each layer's router logits come from the rows the workgroups have just
 * combined, by linearity of the norm once 1/rms is known:
 *   logit_e = inv_rms * sum_gi P[e][gi],   P[e][gi] = sum_{r in rows(gi)} W_r[e][r] (nw[r] h[r]),
 *   inv_rms = 1 / sqrt(sum_gi S[gi] / H + eps),  S[gi] = sum_{r in rows(gi)} h[r]^2.
 * XCD k's workgroup gi computes P for experts 32k .. 32k + 31 (its 8 KB slice
 * of the router, in LDS), so the chain from a combine to the next layer's top
 * 8 is: the partials (one wave: products, then a reduce-scatter over its
 * lanes) -> across XCDs -> each workgroup sums the partials of 8 experts ->
 * within the XCD -> top 8.  The hidden state's gather and normalisation,
 * which only the gate/up dots need, run beside that chain.  Per layer:
 *   wave 0: partials, row sum of squares and its 64 rows of h published; the
 *     logits of experts 8 gi .. 8 gi + 7 into the XCD's copy; all 256 logits
 *     gathered, the top 8 (ids flag); its share of the slot expert's rows; the
 *     XCD's SiLU*up gather; the combine of its 64 rows (h kept in registers);
 *   waves 1..4: this XCD's copy of h (first layer: the caller's h), 1/rms from
 *     the 32 row sums, the normalised input and its run sums (xn counter);
 *     wave 2 then the shared-gate logit, wave 3 the shared SiLU*up relay and
 *     gather;
 *   wave 5: the next layer's router slice and norm weights into LDS (two
 *     buffers by layer parity, a counter for wave 0), then its rows;
 *   waves 6, 7: the shared expert's gate/up pairs and down rows.
 * One workgroup barrier per layer (before the down dots).  The final hidden
 * state is staged in the exchange buffer; the last workgroup to finish copies
 * it over the caller's h only when no wait gave up anywhere, so a call that
 * reports ROASTER_EDEVICE leaves h as it was.  The dots, the routed and shared
 * SiLU*up values, the softmax and the combine are the three-kernel path's;
 * the logits and 1/rms differ from it in their summation order only. */
#define R1_H 2048
#define R1_I 512
#define R1_E 256
#define R1_RD (R1_H / K1_GW)        /* rows combined per workgroup */
#define R1_EX (R1_E / K1_G)         /* experts whose partials one XCD computes */
#define R1_RSP (R1_EX + 4)          /* LDS pitch (floats) of a router-slice row */
#define R1_WPF 5                    /* wave that prefetches the router slice and norm weights */

/* Sums over the 64 lanes of v[0..31]: lanes 2j and 2j + 1 receive value j's
 * sum.  A reduce-scatter: permlane32 / permlane16 swaps exchange halves of
 * the values, then row mirrors and quad swaps; the order is fixed, so the
 * sums are deterministic. */
__device__ __forceinline__ float wave_rs32(float (&v)[32])
{
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const auto p = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v[j]),
                                                        __builtin_bit_cast(uint32_t, v[j + 16]), false, false);
        v[j] = __builtin_bit_cast(float, (uint32_t)p[0]) + __builtin_bit_cast(float, (uint32_t)p[1]);
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const auto p = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v[j]),
                                                        __builtin_bit_cast(uint32_t, v[j + 8]), false, false);
        v[j] = __builtin_bit_cast(float, (uint32_t)p[0]) + __builtin_bit_cast(float, (uint32_t)p[1]);
    }
    const bool b3 = (lane & 8) != 0, b2 = (lane & 4) != 0, b1 = (lane & 2) != 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float keep = b3 ? v[j + 4] : v[j], send = b3 ? v[j] : v[j + 4];
        v[j] = keep + dpp_f<DPP_MIRROR>(send);
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const float keep = b2 ? v[j + 2] : v[j], send = b2 ? v[j] : v[j + 2];
        v[j] = keep + dpp_f<DPP_HALF_MIRROR>(send);
    }
    const float keep = b1 ? v[1] : v[0], send = b1 ? v[0] : v[1];
    const float s = keep + dpp_f<DPP_XOR2>(send);
    return s + dpp_f<DPP_XOR1>(s);
}

#define DPP_ROR8 0x128         /* row_ror:8 (lane i <- lane i ^ 8 within 16) */

/* LDS position of run r (values 16r .. 16r + 15) of a SiLU*up vector in the
 * folded-router kernel: run r moved up by ((r >> 3) & 3) 16-byte granules, so
 * that the 16 lanes of a down row (runs {0..3, 8..11} + 16 lb and those + 4)
 * read 16 different bank groups in each ds_read_b128 pass instead of four
 * lanes per group.  off is a multiple of 16; the vector needs 12 floats more. */
__device__ __forceinline__ int r1_ehpos(int off) { return off + 4 * ((off >> 7) & 3); }

/* k1_gather_run into the rotated layout (dst + r1_ehpos(16 r)). */
__device__ __forceinline__ float r1_gather_run(const uint64_t *base, int I, int r, uint32_t ep, int &dead,
                                               uint32_t spin, float *dst)
{
    return k1_gather_run(base, I, r, ep, dead, spin, dst + r1_ehpos(16 * r));
}

/* k1_down_row's arithmetic on a rotated SiLU*up vector. */
__device__ __forceinline__ float r1_down_row(const QChunk &ch, const float *eh, const float *ehs, bool live, int lane)
{
    const int lr = lane & 15, c = lr & 7, lb = lr >> 3;
    float part = 0.0f;
    if (live) {
        const int ca = lb * RQK + q_run_a<true>(c), cb = ca + 64;
        part = q_chunk_dot<true>(ch, c, eh + r1_ehpos(ca), eh + r1_ehpos(cb), ehs[ca >> 4], ehs[cb >> 4]);
    }
    return group_sum<16>(part);
}

/* The sum over the 8 lanes l, l ^ 8, ..., l ^ 56 (fixed order; the same value
 * in each of them). */
__device__ __forceinline__ float sum_over_l8(float s)
{
    s += dpp_f<DPP_ROR8>(s);
    auto p = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, s), __builtin_bit_cast(uint32_t, s), false, false);
    s = __builtin_bit_cast(float, (uint32_t)p[0]) + __builtin_bit_cast(float, (uint32_t)p[1]);
    p = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, s), __builtin_bit_cast(uint32_t, s), false, false);
    return __builtin_bit_cast(float, (uint32_t)p[0]) + __builtin_bit_cast(float, (uint32_t)p[1]);
}

/* 1/rms from the 32 row sums of squares of an XCD (lanes 0..31 hold them). */
__device__ __forceinline__ float r1_inv_rms(const DecArgs &A, float ssv)
{
    const int lane = threadIdx.x & 63;
    const float ss = group_sum<64>(lane < 32 ? ssv : 0.0f);
    return A.do_norm ? 1.0f / sqrtf(ss / (float)R1_H + A.eps) : 1.0f;
}

/* Layer l's router slice (experts 32 grp .., rows 64 gi ..; stored [row][expert]
 * with pitch R1_RSP) and norm weights into LDS buffer b (wave R1_WPF). */
__device__ __forceinline__ void r1_prefetch_rs(const DecArgs &A, const DecLayer &L, int l, int grp, int gi,
                                               float (*rsl)[R1_RD * R1_RSP], float (*nws)[R1_H], int b, bool router)
{
    const int lane = threadIdx.x & 63;
    float4 r[8], w[8];
    const float *nw = A.do_norm && A.norm_w ? A.norm_w + (size_t)(l - A.layer0) * R1_H : NULL;
    /* both loads unconditional (without norm weights the first 8 KB of the
     * router stand in, never stored): conditionally filled arrays are kept in
     * scratch memory by the compiler */
    const float *nwp = nw ? nw : L.router;
#pragma unroll
    for (int m = 0; m < 8; m++) {
        const int q = lane + 64 * m, e = q >> 4, c4 = q & 15;
        r[m] = gld_f4(L.router + (size_t)(R1_EX * grp + e) * R1_H + R1_RD * gi + 4 * c4);
    }
#pragma unroll
    for (int m = 0; m < 8; m++) w[m] = gld_f4(nwp + 4 * (lane + 64 * m));
    if (router) {
#pragma unroll
        for (int m = 0; m < 8; m++) {
            const int q = lane + 64 * m, e = q >> 4, c4 = q & 15;
            float *d = rsl[b] + (4 * c4) * R1_RSP + e;
            d[0] = r[m].x;
            d[R1_RSP] = r[m].y;
            d[2 * R1_RSP] = r[m].z;
            d[3 * R1_RSP] = r[m].w;
        }
    }
    if (nw) {
#pragma unroll
        for (int m = 0; m < 8; m++) ((float4 *)nws[b])[lane + 64 * m] = w[m];
    }
}

extern "C" __global__ void __launch_bounds__(K1_T, 1) dec_stack1r_kernel(DecArgs A)
{
    constexpr int H = R1_H, I = R1_I, E = R1_E, HU = H / 4, nbh = H / RQK, nbi = I / RQK;
    constexpr int RD = R1_RD, SP = I / 256, RO = H / 256, RGP = I / K1_GW;
    constexpr int lpr = 16, rpw = 64 / lpr, ndt = RD / rpw, nsd = (RO + rpw - 1) / rpw, SPW = I / K1_GW;
    static_assert(RGP == 2 * K1_W && ndt == 2 * K1_W && SP == 2 && nsd == 2, "two gate/up pairs and two down tasks per wave");
    __shared__ __align__(16) float xn[H];
    __shared__ float xsum[H / 16];
    __shared__ __align__(16) float nw_s[2][H];
    __shared__ __align__(16) float rsl_s[2][RD * R1_RSP];
    __shared__ __align__(16) float ehk[I + 16];
    __shared__ float ehks[I / 16];
    __shared__ __align__(16) float ehsh[I + 16];
    __shared__ float ehshs[I / 16];
    __shared__ TopkScratch tks;
    __shared__ int ids_s[RTOPK];
    __shared__ float w_s[RTOPK + 1];
    __shared__ __align__(16) DecLayer Ls[K1_MAXL];
    __shared__ float4 gin_s[8][64];
    __shared__ QChunk2 shc_s[SP][64];
    __shared__ QChunk sdc_s[nsd][64];
    __shared__ int s_dead, s_err, s_last;
    __shared__ int s_ids_ready, s_xn, s_pre;

    const int tid = threadIdx.x, wv = wave_id();
    unsigned xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    xcc &= 0xFu;
    const bool l2 = A.xl2 && xcc < (unsigned)K1_G;
    if (A.xl2 && !l2 && threadIdx.x == 0) atomicOr(A.err, 4);
    const int grp = l2 ? (int)xcc : (int)(blockIdx.x % K1_G), gi = blockIdx.x / K1_G, gw = blockIdx.x;
    const bool swz = A.xswz;
    uint64_t *xpl = A.xch + XR_PL(E, H, I);                   /* across XCDs */
    uint64_t *xehs = A.xch + XR_EHS(E, H, I);
    uint64_t *xdx = A.xch + XR_DX(E, H, I);
    uint64_t *xdsh = A.xch + XR_DSH(E, H, I);
    uint64_t *xhst = A.xch + XR_HST(E, H, I);
    uint64_t *loc = A.xch + XR_LOC0(E, H, I) + (size_t)grp * XR_LOCN(E, H, I);   /* this XCD's */
    uint64_t *llg = loc + XR_LLG(I), *lss = loc + XR_LSS(I), *lehs = loc + XR_LEHS(I), *lehx = loc + XR_LEHX(I),
             *lh = loc + XR_LH(I);
    const int n = A.nlayers;
    const bool given = A.logits_in != NULL;
    const bool stage = A.y == NULL;                          /* stack mode: h is updated in place */
#ifdef ROASTER_PHASE_TS
    unsigned long long tsv[2][16] = {};
    int tsl = 0;
#define R1_TS(i) asm volatile("s_memrealtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(tsv[tsl][i]) : : "memory")
#else
#define R1_TS(i) ((void)0)
#endif
#define R1_TSW(w, i)            \
    do {                        \
        if (wv == (w)) R1_TS(i); \
    } while (0)
    if (tid == 0) {
        s_dead = 0;
        s_err = 0;
        s_ids_ready = 0;
        s_xn = 0;
        s_pre = 1;                                           /* the first layer's slice: before the second barrier */
    }
    /* error bit 2 from an earlier launch that gave up: wait for nothing */
    int dead = (gld_u32(A.err) & 2u) != 0;
    constexpr int DQ = (int)(sizeof(DecLayer) / 16);
    if (tid < n * DQ) ((uint4 *)Ls)[tid] = ((const uint4 *)(A.layers + A.layer0))[tid];
    __syncthreads();
    DecLayer L = k1_layer(Ls, 0);
    /* the first layer's loads that depend on nothing computed */
    {
        const int lane = tid & 63, c = lane & 7, lb = lane >> 3, rw_ = lane / lpr, lr = lane % lpr;
        if (wv == R1_WPF) r1_prefetch_rs(A, L, A.layer0, grp, gi, rsl_s, nw_s, 0, !given);
        if (wv == K1_WGI) {
#pragma unroll
            for (int m = 0; m < 8; m++) gin_s[m][lane] = gld_f4(L.gate_inp + 4 * lane + 256 * m);
        }
        if (wv >= K1_W - SP) {
            const size_t j = (size_t)gw * SP + (wv - (K1_W - SP));
            QChunk2 ch;
            ch.g = q_load_t(0, L.sgate, j, nbh, lb, c);
            ch.u = q_load_t(0, L.sup, j, nbh, lb, c);
            shc_s[wv - (K1_W - SP)][lane] = ch;
            const int sdt = wv - (K1_W - nsd);
            sdc_s[sdt][lane] = q_load_t(1, L.sdown, (size_t)min(gw * RO + sdt * rpw + rw_, H - 1), nbi, lr >> 3, lr & 7);
        }
    }
    __syncthreads();
    float hcur = 0.0f;                                       /* wave 0, lane r: h of row 64 gi + r */
    if (wv == 0) hcur = A.h[RD * gi + (tid & 63)];

    for (int li = 0; li < n; li++) {
        int tid_v = (int)threadIdx.x;
        asm volatile("" : "+v"(tid_v));
        const int lane = tid_v & 63, c = lane & 7, lb = lane >> 3;
        const int rw_ = lane / lpr, lr = lane % lpr, lbd = lr >> 3;
        const int l = A.layer0 + li, par = li & 1;
        const uint32_t ep = A.epoch + (uint32_t)li;
        const bool last = li + 1 == n;
        const bool nwl = A.do_norm && A.norm_w;
        float4 *x4 = (float4 *)xn;
#ifdef ROASTER_PHASE_TS
        tsl = last ? 1 : 0;
#endif
        R1_TSW(6, 0);
        R1_TSW(3, 0);
        if (wv == 0) {
            R1_TS(0);
            /* ---- A. partials of XCD grp's experts over rows 64 gi .. ------------ */
            const int row = RD * gi + lane;
            const float ss = group_sum<64>(hcur * hcur);
            if (lane == 0) xch_put_xcd(lss + gi, ss, ep, l2);
            if (li > 0) xch_put_xcd(lh + (size_t)(row & 3) * HU + (row >> 2), hcur, ep, l2);
            if (li > 0) k1_flag_wait(&s_pre, li + 1);
            R1_TS(10);
            if (!given) {
                const float hn = nwl ? nw_s[par][row] * hcur : hcur;
                float v[32];
                const float4 *rs = (const float4 *)(rsl_s[par] + lane * R1_RSP);
#pragma unroll
                for (int m = 0; m < 8; m++) {
                    const float4 w = rs[m];
                    v[4 * m] = w.x * hn;
                    v[4 * m + 1] = w.y * hn;
                    v[4 * m + 2] = w.z * hn;
                    v[4 * m + 3] = w.w * hn;
                }
                const float p = wave_rs32(v);
                R1_TS(11);
                if ((lane & 1) == 0) xch_put(xpl + (size_t)(grp * K1_GW + gi) * R1_EX + (lane >> 1), p, ep);
            }
            R1_TS(1);
            /* ---- B. logits of experts 8 gi .. 8 gi + 7 ------------------------- */
            float lg4[4];
            if (!given) {
                const int kx = gi >> 2, ex = 8 * (gi & 3) + (lane & 7);
                const uint64_t *q[5];
#pragma unroll
                for (int i = 0; i < 4; i++) q[i] = xpl + (size_t)(kx * K1_GW + (lane >> 3) + 8 * i) * R1_EX + ex;
                q[4] = lss + (lane & 31);
                float v[5];
                xch_gather<5>(q, lane < 32 ? 0x1Fu : 0x0Fu, ep, dead, A.spin, v);
                const float s = sum_over_l8((v[0] + v[1]) + (v[2] + v[3]));
                const float lgt = s * r1_inv_rms(A, v[4]);
                if (lane < 8) {
                    xch_put_xcd(llg + 8 * gi + lane, lgt, ep, l2);
                    if (last && grp == 0) A.logits[8 * gi + lane] = lgt;
                }
                R1_TS(2);
                /* ---- C. the 256 logits from this XCD's copy, top 8 ------------- */
                const uint64_t *q4[4];
#pragma unroll
                for (int i = 0; i < 4; i++) q4[i] = llg + lane + 64 * i;
                xch_gather<4>(q4, 0xFu, ep, dead, A.spin, lg4);
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) lg4[i] = A.logits_in[lane + 64 * i];
            }
            R1_TS(3);
            topk8_fast(lg4, E, ids_s, w_s, &s_err, &tks, &s_ids_ready, li + 1);
            R1_TS(4);
            asm volatile("; R1MARK topk done" ::: "memory");
            if (gw == 0) {
                if (lane < RTOPK) {
                    const size_t o = (size_t)li * RTOPK + lane;
                    if (A.ids_out) A.ids_out[o] = ids_s[lane];
                    if (A.w_out) A.w_out[o] = w_s[lane];
                }
                if (lane == 0 && s_err) atomicOr(A.err, 1);
            }
        } else if (wv <= 4) {
            /* ---- h of the layer, 1/rms, the normalised input --------------------- */
            const int t = tid_v - 64;                        /* units t and t + 256 */
            float4 hq[2];
            float ssv;
            if (li == 0) {
                const uint64_t *q[1] = {lss + (lane & 31)};
                float v[1];
#pragma unroll
                for (int k = 0; k < 2; k++) hq[k] = ((const float4 *)A.h)[t + 256 * k];
                xch_gather<1>(q, lane < 32 ? 1u : 0u, ep, dead, A.spin, v);
                ssv = v[0];
            } else {
                /* the h units and (lanes < 32) the row sums in one gather */
                const uint64_t *q[9];
                float v[9];
#pragma unroll
                for (int i = 0; i < 8; i++) q[i] = lh + (size_t)(i & 3) * HU + t + 256 * (i >> 2);
                q[8] = lss + (lane & 31);
                xch_gather<9>(q, lane < 32 ? 0x1FFu : 0xFFu, ep, dead, A.spin, v);
                hq[0] = make_float4(v[0], v[1], v[2], v[3]);
                hq[1] = make_float4(v[4], v[5], v[6], v[7]);
                ssv = v[8];
            }
            R1_TSW(6, 1);
            R1_TSW(3, 1);
            const float inv = r1_inv_rms(A, ssv);
            if (li > 0 && nwl) k1_flag_wait(&s_pre, li + 1);    /* this layer's norm weights */
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const int u = t + k * 256;
                float4 v = hq[k];
                if (A.do_norm) {
                    v.x *= inv; v.y *= inv; v.z *= inv; v.w *= inv;
                    if (nwl) {
                        const float4 wq = ((const float4 *)nw_s[par])[u];
                        v.x *= wq.x; v.y *= wq.y; v.z *= wq.z; v.w *= wq.w;
                    }
                }
                float r = (v.x + v.y) + (v.z + v.w);
                r += dpp_f<DPP_XOR1>(r);
                r += dpp_f<DPP_XOR2>(r);
                x4[xpos(u, swz)] = v;
                if ((t & 3) == 0) xsum[u >> 2] = r;
            }
            if (lane == 0) __hip_atomic_fetch_add(&s_xn, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            R1_TSW(6, 2);
            R1_TSW(3, 2);
            if (wv == K1_WGI) {
                k1_flag_wait(&s_xn, 4 * (li + 1));
                float4 rw[8];
#pragma unroll
                for (int m = 0; m < 8; m++) rw[m] = gin_s[m][lane];
                const float s = k1_row_dot(rw, x4, H, swz, lane);
                if (lane == 0) w_s[RTOPK] = 1.0f / (1.0f + expf(-s));
            }
        } else if (wv == R1_WPF) {
            if (!last) {
                const DecLayer Ln = k1_layer(Ls, li + 1);
                r1_prefetch_rs(A, Ln, l + 1, grp, gi, rsl_s, nw_s, par ^ 1, !given);
                if (lane == 0) __hip_atomic_store(&s_pre, li + 2, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
        } else {
            /* ---- the shared expert's gate/up pairs of this workgroup ------------ */
            k1_flag_wait(&s_xn, 4 * (li + 1));
            R1_TSW(6, 1);
            const int pr = wv - (K1_W - SP);
            const float eh = k1_gu_pair(0, 0, shc_s[pr][lane], xn, xsum, swz, nbh, lane);
            if (lane == 0) xch_put(xehs + (size_t)gw * XCH_LN + pr, eh, ep);
            R1_TSW(6, 2);
        }
        if (wv != 0) k1_flag_wait(&s_ids_ready, li + 1);
        R1_TSW(6, 4);
        R1_TSW(3, 4);

        /* ---- D. the slot's expert ------------------------------------------------ */
        R1_TSW(0, 14);
        const int e = ids_s[grp];
        const bool live_slot = e >= 0;
        const size_t ee = live_slot ? (size_t)e : 0;          /* an unselected slot reads expert 0, unused */
        const uint8_t *ge = L.gate + ee * L.eb[0], *ue = L.up + ee * L.eb[1], *de = L.down + ee * L.eb[2];
        QChunk2 gch[2];
        QChunk dch[2];
        R1_TSW(0, 15);
#pragma unroll
        for (int f = 0; f < 2; f++) gch[f].g = q_load_t(0, ge, (size_t)gi * RGP + wv + f * K1_W, nbh, lb, c);
#pragma unroll
        for (int f = 0; f < 2; f++) gch[f].u = q_load_t(0, ue, (size_t)gi * RGP + wv + f * K1_W, nbh, lb, c);
        const int sdt = wv - (K1_W - nsd);
        asm volatile("; R1MARK before xn wait" ::: "memory");
        R1_TSW(0, 12);
        k1_flag_wait(&s_xn, 4 * (li + 1));
        R1_TS(5);
        float pgs[2];
#pragma unroll
        for (int f = 0; f < 2; f++) pgs[f] = k1_q_row(0, gch[f].g, xn, xsum, swz, nbh, lane);
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("; gate rows dotted" ::"v"(pgs[0]) : "memory");
        R1_TSW(0, 13);
#pragma unroll
        for (int f = 0; f < 2; f++)
            dch[f] = q_load_t(1, de, (size_t)(gi * RD + (wv + f * K1_W) * rpw + rw_), nbi, lbd, lr & 7);
#pragma unroll
        for (int f = 0; f < 2; f++) {
            const int pj = wv + f * K1_W;
            const float eh = silu_mul(pgs[f], k1_q_row(0, gch[f].u, xn, xsum, swz, nbh, lane));
            if (lane == 0) xch_put_xcd(lehx + k1_run_slot(gi * RGP + pj, I), live_slot ? eh : 0.0f, ep, l2);
        }
        R1_TSW(6, 6);
        R1_TSW(3, 6);
        if (wv == K1_WN) {
            /* the shared SiLU*up values: this workgroup's share relayed from the
             * producing workgroups (published before the top 8) into the XCD's
             * copy, then all of them from there (the shared down rows use them
             * after the barrier) */
            if (lane < SPW) {                                /* shared value j: slot j % SP of line j / SP */
                const int j = gi * SPW + lane;
                const uint64_t *q[1] = {xehs + (size_t)(j / SP) * XCH_LN + j % SP};
                float v[1];
                xch_gather<1>(q, 1u, ep, dead, A.spin, v);
                xch_put_xcd(lehs + k1_run_slot(j, I), v[0], ep, l2);
            }
            R1_TS(8);
            if (lane < I / 16) ehshs[lane] = r1_gather_run(lehs, I, lane, ep, dead, A.spin, ehsh);
            R1_TS(3);
        }
        if (wv == 0) {
            R1_TS(6);
            if (lane < I / 16) ehks[lane] = r1_gather_run(lehx, I, lane, ep, dead, A.spin, ehk);
        }
        K1_SYNC_DEAD();
        if (dead) break;                                      /* workgroup-uniform */
        R1_TS(7);
        if (sdt >= 0) {
            /* the shared expert's down rows [gw RO, (gw + 1) RO): slot 8 of the
             * down outputs (their SiLU*up values came in before the barrier) */
            const int rl = sdt * rpw + rw_;
            const bool live = rl < RO && lbd < nbi;
            const float part = r1_down_row(sdc_s[sdt][lane], ehsh, ehshs, live, lane);
            if (live && lr == 0) xch_put(xdsh + (size_t)gw * XCH_LN + rl, part, ep);
        }
#pragma unroll
        for (int f = 0; f < 2; f++) {
            const int rl = (wv + f * K1_W) * rpw + rw_, row = gi * RD + rl;
            const float part = r1_down_row(dch[f], ehk, ehks, true, lane);
            if (lr == 0) xch_put(xdx + (size_t)grp * H + row, live_slot ? part : 0.0f, ep);
        }

        /* ---- E. the next layer's loads; the combine of rows 64 gi .. ------------ */
        if (!last) {
            L = k1_layer(Ls, li + 1);
            if (wv == K1_WGI) {
                float4 r1[8];
#pragma unroll
                for (int m = 0; m < 8; m++) r1[m] = gld_f4(L.gate_inp + 4 * lane + 256 * m);
#pragma unroll
                for (int m = 0; m < 8; m++) gin_s[m][lane] = r1[m];
            } else if (wv >= K1_W - SP) {
                const size_t j = (size_t)gw * SP + (wv - (K1_W - SP));
                QChunk2 ch;
                ch.g = q_load_t(0, L.sgate, j, nbh, lb, c);
                ch.u = q_load_t(0, L.sup, j, nbh, lb, c);
                const QChunk sd = q_load_t(1, L.sdown, (size_t)min(gw * RO + sdt * rpw + rw_, H - 1), nbi, lbd, lr & 7);
                shc_s[wv - (K1_W - SP)][lane] = ch;
                sdc_s[sdt][lane] = sd;
            }
        }
        if (wv == 0) {
            R1_TS(8);
            const int row = gi * RD + lane;
            const uint64_t *q[RTOPK + 1];
            float d[RTOPK + 1];
#pragma unroll
            for (int k = 0; k < RTOPK; k++) q[k] = xdx + (size_t)k * H + row;
            q[RTOPK] = xdsh + (size_t)(row / RO) * XCH_LN + row % RO;
            xch_gather<RTOPK + 1>(q, 0x1FFu, ep, dead, A.spin, d);
            R1_TS(9);
            float y = 0.0f;
#pragma unroll
            for (int k = 0; k < RTOPK; k++) y = fmaf(w_s[k], d[k], y);
            y = fmaf(w_s[RTOPK], d[RTOPK], y);
            hcur += y;
            if (last && grp == 0) {
                if (!stage) A.y[row] = y;
                else xch_put(xhst + row, hcur, ep);
            }
        }
    }
    /* the staged h over the caller's only when no wait gave up anywhere */
    if (dead) s_dead = 1;
    __syncthreads();
    k1_finish(A, s_dead != 0, &s_last, xhst, H, A.epoch + (uint32_t)(n - 1));
#ifdef ROASTER_PHASE_TS
    if (threadIdx.x == 0 || threadIdx.x == 192 || threadIdx.x == 384)
        for (int k = 0; k < 2; k++)
            for (int i = 0; i < 16; i++) g_k1_ts[k][blockIdx.x][threadIdx.x == 0 ? 0 : threadIdx.x == 192 ? 1 : 2][i] = tsv[k][i];
#endif
#undef R1_TS
#undef R1_TSW
}

/* ---- the batched one-launch stack: 2..8 tokens --------------------------------
 * The one-token stack's groups and exchanges with a token index: group k (an
 * XCD) serves slot k of every token (the token's k-th expert), so the chain
 * of exchanges per layer is the one-token chain carrying B values where it
 * carried one, and the expert rows of the B tokens are streamed back to back.
 * Per layer:
 *   1. every thread u < H/4: unit u of each token's h (this XCD's copy, or the
 *      caller's h in the first layer) into LDS; the sums of squares in the
 *      one-token order (lane t: units t and t + 256, waves 0..3, the wave sums
 *      in wave order), 1/rms per token, the normalised inputs and their run
 *      sums, the owned rows' residuals;
 *   2. router row gw for token b on wave b; the shared expert's SiLU*up pairs
 *      of this workgroup on waves 1..7;
 *   3. wave 0 relays the logits, wave K1_WN the shared values, into the XCD's
 *      region; wave b ranks token b's top 8 and raises token b's ids flag;
 *   4. the slot experts' gate/up rows token after token, each token's once its
 *      ids flag is up (the next token's rows in flight while the current one's
 *      are dotted; a wave's four rows share one read of the token's
 *      activations), SiLU*up within the XCD; wave b takes token b's
 *      shared-gate logit while its first rows arrive, gathers token b's shared
 *      and slot SiLU*up values and raises its flag; the shared expert's down
 *      rows, then the slot experts' down rows token after token, each token's
 *      once its flag is up;
 *   5. wave b combines token b's owned rows (model.c:1139-1144 order) and
 *      publishes them within the XCD.
 * The workgroup barriers are those of step 1; later handoffs are LDS flags,
 * and the one LDS buffer a wave may rewrite for the next layer before another
 * wave has read it for this one (the shared down rows) is double-buffered by
 * layer parity.
 * Every dot, sum, softmax and combine is the one-token kernel's, in its order,
 * so each token's results equal its one-token results bit for bit.  Shapes:
 * inter 512, hidden 512..2048 in whole 256-row blocks, at most 256 experts;
 * gate/up Q4_K and down Q6_K, routed and shared (dec_layerB_ok and the launch
 * check the rest). */
template <int NB>
__device__ __forceinline__ void k1b_gather_h(const uint64_t *lh, int H, int HU, int u, int b0, int B, uint32_t ep,
                                             int &dead, uint32_t spin, float (*xn)[K1_MAXH])
{
    uint64_t r[NB][4];
    const int uc = min(u, HU - 1);
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int i = 0; i < 4; i++) r[b][i] = xch_load(lh + (size_t)(b0 + b) * H + (size_t)i * HU + uc);
    unsigned it = 0;
    for (;;) {
        unsigned miss = 0;
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                miss |= b0 + b < B && u < HU && (uint32_t)(r[b][i] >> 32) != ep ? 1u << (4 * b + i) : 0u;
        if (!miss || dead) break;
        if (++it > spin) {
            dead = 1;
            break;
        }
        __builtin_amdgcn_s_sleep(K1_POLL_SLEEP);
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                if ((miss >> (4 * b + i)) & 1u) r[b][i] = xch_load(lh + (size_t)(b0 + b) * H + (size_t)i * HU + uc);
    }
    if (u < HU) {
#pragma unroll
        for (int b = 0; b < NB; b++)
            if (b0 + b < B)
                ((float4 *)xn[b0 + b])[u] =
                    make_float4(__builtin_bit_cast(float, (uint32_t)r[b][0]), __builtin_bit_cast(float, (uint32_t)r[b][1]),
                                __builtin_bit_cast(float, (uint32_t)r[b][2]), __builtin_bit_cast(float, (uint32_t)r[b][3]));
    }
}

template <int NB>
__device__ __forceinline__ void stackB_body(const DecArgs &A)
{
    __shared__ __align__(16) float xn[NB][K1_MAXH];
    __shared__ float xsum[NB][K1_MAXH / 16];
    __shared__ float hown[NB][64];                           /* the owned rows' residual */
    __shared__ __align__(16) float ehk[NB][512];
    __shared__ float ehks[NB][512 / 16];
    __shared__ __align__(16) float ehsh[NB][512];
    __shared__ float ehshs[NB][512 / 16];
    __shared__ TopkScratch tks[NB];
    __shared__ int ids_s[NB][RTOPK];
    __shared__ float w_s[NB][RTOPK + 1];
    __shared__ float red_s[K1_W][NB];
    __shared__ __align__(16) DecLayer Ls[K1_MAXL];
    __shared__ float4 rrow_s[8][64];                          /* router row gw */
    __shared__ float4 gin_s[8][64];                           /* shared-gate vector */
    __shared__ QChunk2 shc_s[2][64];                          /* this workgroup's shared gate/up pairs */
    /* its shared down rows (H <= 2048: 2 tasks), by layer parity: a wave
     * parks the next layer's once its own h units are in, which need not be
     * after every other wave's reads of this layer's */
    __shared__ QChunk sdc_s[2][2][64];
    __shared__ int s_dead, s_err;
    __shared__ int s_ids_rdy[NB];                             /* layer index + 1 once token b's ids are in */
    __shared__ int s_eh_rdy[NB];                              /* ... once its SiLU*up vectors are in */

    constexpr int I = 512, nbi = 2, SP = 2, RGP = I / K1_GW;
    const int H = A.H, E = A.E, B = A.B, HU = H / 4, nbh = H / RQK;
    const int tid = threadIdx.x, wv = wave_id();
    unsigned xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    xcc &= 0xFu;
    const bool l2 = A.xl2 && xcc < (unsigned)K1_G;
    if (A.xl2 && !l2 && threadIdx.x == 0) atomicOr(A.err, 4);
    const int grp = l2 ? (int)xcc : (int)(blockIdx.x % K1_G), gi = blockIdx.x / K1_G, gw = blockIdx.x;
    const bool swz = A.xswz;
    uint64_t *xlg = A.xch + XCHB_LG(NB, E, H, I), *xehs = A.xch + XCHB_EHS(NB, E, H, I);
    uint64_t *xdx = A.xch + XCHB_DX(NB, E, H, I), *xdsh = A.xch + XCHB_DSH(NB, E, H, I);
    uint64_t *loc = A.xch + XCHB_LOC0(NB, E, H, I) + (size_t)grp * XCHB_LOCN(NB, E, H, I);
    uint64_t *llg = loc + XCHB_LLG(NB, I), *lehs = loc + XCHB_LEHS(NB, I), *lehx = loc + XCHB_LEHX(NB, I);
    uint64_t *lh = loc + XCHB_LH(NB, I);
    const int RO = H / 256, RD = H / K1_GW;
    const int LPW = E / K1_GW, SPW = I / K1_GW;
    const int lpr = lanes_per_row(nbi), rpw = 64 / lpr;
    const int nsd = (RO + rpw - 1) / rpw, sdt = wv - (K1_W - nsd);
    const int ndt = (RD + rpw - 1) / rpw;
    const bool rrow = gw < E && !A.logits_in;
    const int n = A.nlayers;
#ifdef ROASTER_PHASE_TS
    unsigned long long tsv[2][16] = {};
    int tsl = 0;
#define K1_TS(i) asm volatile("s_memrealtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(tsv[tsl][i]) : : "memory")
#else
#define K1_TS(i) ((void)0)
#endif
    if (tid == 0) {
        s_dead = 0;
        s_err = 0;
    }
    if (tid < NB) {
        s_ids_rdy[tid] = 0;
        s_eh_rdy[tid] = 0;
    }
    int dead = (gld_u32(A.err) & 2u) != 0;
    constexpr int DQ = (int)(sizeof(DecLayer) / 16);
    if (tid < n * DQ) ((uint4 *)Ls)[tid] = ((const uint4 *)(A.layers + A.layer0))[tid];
    __syncthreads();

    /* each layer's router row, shared-gate vector and shared expert rows:
     * with 2 token slots waves 4..7 combine nothing and load the next layer's
     * at the end of a layer (so no wave's h gather queues behind them); with
     * 4 or 8 (measured slower that way: registers), the waves K1_WR, K1_WGI
     * and the last ones load them at the start of the layer */
    float4 rw[8];
    QChunk2 shc;
    QChunk sdc;
    constexpr bool EARLY = NB == 2;
    const int wR = EARLY ? 4 : K1_WR, wG = EARLY ? 5 : K1_WGI;
    for (int li = 0; li < n; li++) {
        int tid_v = (int)threadIdx.x;
        asm volatile("" : "+v"(tid_v));
        const int tid = tid_v, lane = tid_v & 63, c = lane & 7, lb = lane >> 3;
        const int rw_ = lane / lpr, lr = lane % lpr, lbd = lr >> 3;
        const int l = A.layer0 + li;
        const uint32_t ep = A.epoch + (uint32_t)li;
        const bool last = li + 1 == n;
        const DecLayer L = k1_layer(Ls, li);
#ifdef ROASTER_PHASE_TS
        tsl = li + 1 == n ? 1 : 0;
#endif
        K1_TS(0);
        const float *nwg = A.do_norm && A.norm_w ? A.norm_w + (size_t)(l - A.layer0) * H : NULL;

        /* ---- 1. this layer's own weights first (they do not depend on h),
         * then h, normalised per token ---------------------------------------- */
        auto wload = [&](const DecLayer &Lx) {
            if ((wv == wR && rrow) || wv == wG) {
                const float *row = wv == wR ? Lx.router + (size_t)gw * H : Lx.gate_inp;
#pragma unroll
                for (int m = 0; m < 8; m++) rw[m] = gld_f4(row + min(4 * lane + 256 * m, H - 4));
            }
            if (wv >= K1_W - SP) {
                const size_t j = (size_t)gw * SP + (wv - (K1_W - SP));
                shc.g = q_load_t(0, Lx.sgate, j, nbh, lb, c);
                shc.u = q_load_t(0, Lx.sup, j, nbh, lb, c);
            }
            if (sdt >= 0) sdc = q_load_t(1, Lx.sdown, (size_t)min(gw * RO + sdt * rpw + rw_, H - 1), nbi, lr >> 3, lr & 7);
        };
        if (!EARLY || li == 0) wload(L);
        const int u = tid;
        const float4 nwv = nwg ? ((const float4 *)nwg)[min(u, HU - 1)] : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
        /* h, raw, into xn (unit order) */
        if (li == 0) {
            if (u < HU)
                for (int b = 0; b < B; b++) ((float4 *)xn[b])[u] = ((const float4 *)A.h)[(size_t)b * HU + u];
        } else {
            constexpr int NG = NB < 4 ? NB : 4;           /* tokens per polling round (registers) */
#pragma unroll
            for (int b0 = 0; b0 < NB; b0 += NG)
                if (b0 < B) k1b_gather_h<NG>(lh, H, HU, u, b0, B, ep - 1, dead, A.spin, xn);
        }
        K1_TS(1);
        /* parked for the per-token dots of phase 2 (their loads were issued
         * before the gather's and have completed with it) */
        if ((wv == wR && rrow) || wv == wG) {
            float4 (*dst)[64] = wv == wR ? rrow_s : gin_s;
#pragma unroll
            for (int m = 0; m < 8; m++) dst[m][lane] = rw[m];
        }
        if (wv >= K1_W - SP) shc_s[wv - (K1_W - SP)][lane] = shc;
        if (sdt >= 0) sdc_s[li & 1][sdt][lane] = sdc;
        K1_SYNC_DEAD();
        if (dead) break;                                  /* workgroup-uniform */
        /* the owned rows' residual (rows gi RD .. + RD), each unit's own h */
        if (tid < RD) {
            for (int b = 0; b < B; b++) hown[b][tid] = xn[b][gi * RD + tid];
        }
        float4 hv[NB];
#pragma unroll
        for (int b = 0; b < NB; b++)
            hv[b] = b < B ? ((const float4 *)xn[b])[min(u, HU - 1)] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        /* sums of squares in the one-token order: lane t adds units t and
         * t + 256, waves 0..3, the four wave sums in wave order */
        if (A.do_norm && tid < 256) {
            for (int b = 0; b < B; b++) {
                float ss = 0.0f;
#pragma unroll
                for (int k = 0; k < 2; k++) {
                    const int uu = tid + 256 * k;
                    if (uu < HU) {
                        const float4 v = ((const float4 *)xn[b])[uu];
                        ss = fmaf(v.x, v.x, ss);
                        ss = fmaf(v.y, v.y, ss);
                        ss = fmaf(v.z, v.z, ss);
                        ss = fmaf(v.w, v.w, ss);
                    }
                }
                ss = group_sum<64>(ss);
                if (lane == 0) red_s[wv][b] = ss;
            }
        }
        __syncthreads();
        /* 1 / rms of token b in lane b of every wave, then broadcast */
        float inv_l = 1.0f;
        if (A.do_norm && lane < B) {
            float s2 = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; w++) s2 += red_s[w][lane];
            inv_l = 1.0f / sqrtf(s2 / (float)H + A.eps);
        }
#pragma unroll
        for (int b = 0; b < NB; b++) {
            if (b >= B) break;
            float4 v = hv[b];
            if (A.do_norm) {
                const float inv = lane_f(inv_l, b);
                v.x *= inv; v.y *= inv; v.z *= inv; v.w *= inv;
                if (nwg) { v.x *= nwv.x; v.y *= nwv.y; v.z *= nwv.z; v.w *= nwv.w; }
            }
            float r = (v.x + v.y) + (v.z + v.w);
            r += dpp_f<DPP_XOR1>(r);
            r += dpp_f<DPP_XOR2>(r);
            if (u < HU) {
                ((float4 *)xn[b])[xpos(u, swz)] = v;
                if ((u & 3) == 0) xsum[b][u >> 2] = r;
            }
        }
        __syncthreads();

        K1_TS(2);
        /* ---- 2. per token b, on wave b: router logit gw; the 2 B shared
         * SiLU*up values (pair t % SP of token t / SP) dealt to waves 1..7 in
         * turn (wave 0 goes on to relay the logits) --------------------------- */
        for (int b = wv; b < B; b += K1_W) {
            float4 r4[8];
            if (rrow) {
#pragma unroll
                for (int m = 0; m < 8; m++) r4[m] = rrow_s[m][lane];
                const float s = k1_row_dot(r4, (const float4 *)xn[b], H, swz, lane);
                if (lane == 0) {
                    xch_put(xlg + ((size_t)b * 256 + gw) * XCH_LN, s, ep);
                    if (last) A.logits[(size_t)b * E + gw] = s;
                }
            }
        }
        for (int t = wv - 1; wv > 0 && t < SP * B; t += K1_W - 1) {
            const int pr = t % SP, b = t / SP;
            const float eh = k1_gu_pair(0, 0, shc_s[pr][lane], xn[b], xsum[b], swz, nbh, lane);
            if (lane == 0) xch_put(xehs + ((size_t)b * 256 + gw) * XCH_LN + pr, eh, ep);
        }

        K1_TS(3);
        /* ---- 3. relays into the XCD's region; token b's top 8 (wave b) and its
         * shared SiLU*up values -------------------------------------------------- */
        if (wv == 0 && !A.logits_in && lane < B * LPW) {
            const int b = lane / LPW, j = gi * LPW + lane % LPW;
            const uint64_t *q[1] = {xlg + ((size_t)b * 256 + j) * XCH_LN};
            float v[1];
            xch_gather<1>(q, 1u, ep, dead, A.spin, v);
            xch_put_xcd(llg + (size_t)b * 256 + j, v[0], ep, l2);
        } else if (wv == K1_WN) {
            for (int idx = lane; idx < B * SPW; idx += 64) {
                const int b = idx / SPW, j = gi * SPW + idx % SPW;
                const uint64_t *q[1] = {xehs + ((size_t)b * 256 + j / SP) * XCH_LN + j % SP};
                float v[1];
                xch_gather<1>(q, 1u, ep, dead, A.spin, v);
                xch_put_xcd(lehs + (size_t)b * I + k1_run_slot(j, I), v[0], ep, l2);
            }
        }
        if (wv < B) {
            const int b = wv;
            float v4[4];
            if (A.logits_in) {
#pragma unroll
                for (int i = 0; i < 4; i++) v4[i] = A.logits_in[(size_t)b * E + min(lane + 64 * i, E - 1)];
            } else {
                const uint64_t *q[4];
#pragma unroll
                for (int i = 0; i < 4; i++) q[i] = llg + (size_t)b * 256 + min(lane + 64 * i, E - 1);
                xch_gather<4>(q, 0xFu, ep, dead, A.spin, v4);
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (lane + 64 * i >= E) v4[i] = -INFINITY;
            topk8_fast<true>(v4, E, ids_s[b], w_s[b], &s_err, &tks[b], &s_ids_rdy[b], li + 1);
            if (gw == 0) {
                if (lane < RTOPK) {
                    const size_t o = ((size_t)li * B + b) * RTOPK + lane;
                    if (A.ids_out) A.ids_out[o] = ids_s[b][lane];
                    if (A.w_out) A.w_out[o] = w_s[b][lane];
                }
                if (lane == 0 && s_err) atomicOr(A.err, 1);
            }
        }
        K1_TS(13);
        K1_TS(4);
        /* no barrier: each wave takes token b's rows as soon as wave b has
         * stored its ids (an LDS flag set before the softmax weights) */

        /* ---- 4. the slot experts of the B tokens -------------------------- */
        float sg = 0.0f;
        {
            constexpr int DG = 2;                            /* tokens' gate/up rows in flight */
            QChunk2 st[DG][2];
            auto gu_load = [&](int b, QChunk2 (&ch)[2]) {
                k1_flag_wait(&s_ids_rdy[min(b, B - 1)], li + 1);
                const int e = __builtin_amdgcn_readfirstlane(ids_s[min(b, B - 1)][grp]);   /* wave-uniform */
                const size_t ee = e >= 0 ? (size_t)e : 0;
                const uint8_t *ge = L.gate + ee * L.eb[0], *ue = L.up + ee * L.eb[1];
#pragma unroll
                for (int f = 0; f < 2; f++) ch[f].g = q_load_t(0, ge, (size_t)gi * RGP + wv + f * K1_W, nbh, lb, c);
#pragma unroll
                for (int f = 0; f < 2; f++) ch[f].u = q_load_t(0, ue, (size_t)gi * RGP + wv + f * K1_W, nbh, lb, c);
            };
#pragma unroll
            for (int b = 0; b < DG - 1; b++) gu_load(b, st[b]);
            /* wave b: token b's shared-gate logit while the first rows arrive
             * (kept in a register for the combine; xn[b] is read here, before
             * this wave's gate/up outputs, which every next-layer h value
             * waits for) */
            if (wv < B) {
                float4 r4[8];
#pragma unroll
                for (int m = 0; m < 8; m++) r4[m] = gin_s[m][lane];
                sg = 1.0f / (1.0f + expf(-k1_row_dot(r4, (const float4 *)xn[wv], H, swz, lane)));
                asm volatile("" ::"v"(sg) : "memory");    /* computed here, before the wave's stores */
            }
#pragma unroll
            for (int b = 0; b < NB; b++) {
                if (b >= B) break;
                const bool live_slot = ids_s[b][grp] >= 0;
                if (b + DG - 1 < NB) gu_load(b + DG - 1, st[(b + DG - 1) % DG]);   /* past the last token: unused */
                QChunk2 (&cur)[2] = st[b % DG];
                /* the wave's four rows share one read of the token's x
                 * (k1_q_row's arithmetic per row) */
                float pg[2] = {0.0f, 0.0f}, pu[2] = {0.0f, 0.0f};
                if (lb < nbh) {
                    const int xa = lb * RQK + q_run_a_t(0, c), xb = xa + 32;
                    float4 x0[4], x1[4];
                    load_x16(xn[b], xa, x0, swz);
                    load_x16(xn[b], xb, x1, swz);
                    const float sa = xsum[b][xa >> 4], sb = xsum[b][xb >> 4];
#pragma unroll
                    for (int f = 0; f < 2; f++) {
                        pg[f] = q_chunk_dot_r<false>(cur[f].g, c, x0, x1, sa, sb);
                        pu[f] = q_chunk_dot_r<false>(cur[f].u, c, x0, x1, sa, sb);
                    }
                }
                if constexpr (NB <= 4) {
                    /* both rows' SiLU*up in one pass: lane 0 row wv, lane 1 row
                     * wv + 8 (with 8 slots measured slower) */
                    const float g0 = group_sum<64>(pg[0]), u0 = group_sum<64>(pu[0]);
                    const float g1 = group_sum<64>(pg[1]), u1 = group_sum<64>(pu[1]);
                    const int f = lane & 1;
                    const float eh = silu_mul(f ? g1 : g0, f ? u1 : u0);
                    if (lane < 2)
                        xch_put_xcd(lehx + (size_t)b * I + k1_run_slot(gi * RGP + wv + f * K1_W, I), live_slot ? eh : 0.0f,
                                    ep, l2);
                } else {
#pragma unroll
                    for (int f = 0; f < 2; f++) {
                        const int pj = wv + f * K1_W;
                        const float eh = silu_mul(group_sum<64>(pg[f]), group_sum<64>(pu[f]));
                        if (lane == 0)
                            xch_put_xcd(lehx + (size_t)b * I + k1_run_slot(gi * RGP + pj, I), live_slot ? eh : 0.0f, ep, l2);
                    }
                }
            }
        }
        K1_TS(5);
        {
            constexpr int DD = 2;                            /* tokens' down rows in flight */
            QChunk st[DD][2];
            auto dn_load = [&](int b, QChunk (&ch)[2]) {
                const int e = __builtin_amdgcn_readfirstlane(ids_s[min(b, B - 1)][grp]);   /* wave-uniform */
                const size_t ee = e >= 0 ? (size_t)e : 0;
                const uint8_t *de = L.down + ee * L.eb[2];
#pragma unroll
                for (int f = 0; f < 2; f++) {
                    const int task = min(wv + f * K1_W, ndt - 1);
                    ch[f] = q_load_t(1, de, (size_t)min(gi * RD + task * rpw + rw_, H - 1), nbi, lbd, lr & 7);
                }
            };
            /* 2 slots: the first token's down rows in flight through the
             * gathers (with more tokens the gathers' polls, queued behind
             * them, measured slower) */
            if constexpr (NB == 2) {
#pragma unroll
                for (int b = 0; b < DD - 1; b++) dn_load(b, st[b]);
            }
            K1_TS(6);
            /* wave b: token b's shared SiLU*up values (relayed during the top
             * 8) and its slot expert's */
            if (wv < B && lane < I / 16) {
                ehshs[wv][lane] = k1_gather_run(lehs + (size_t)wv * I, I, lane, ep, dead, A.spin, ehsh[wv] + 16 * lane);
                ehks[wv][lane] = k1_gather_run(lehx + (size_t)wv * I, I, lane, ep, dead, A.spin, ehk[wv] + 16 * lane);
            }
            /* no barrier: a token's down rows wait for its own flag */
            if (wv < B && lane == 0) __hip_atomic_store(&s_eh_rdy[wv], li + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            K1_TS(10);
            K1_TS(7);
            if constexpr (NB != 2) {
#pragma unroll
                for (int b = 0; b < DD - 1; b++) dn_load(b, st[b]);
            }
            /* the shared expert's down rows [gw RO, (gw + 1) RO) for every
             * token while the first routed rows arrive: task t (rows of chunk
             * t % nsd, token t / nsd) on wave t % 8 */
            for (int t = wv; t < nsd * B; t += K1_W) {
                const int k = t % nsd, b = t / nsd;
                const int rl = k * rpw + rw_;
                const bool live = rl < RO && lbd < nbi;
                k1_flag_wait(&s_eh_rdy[b], li + 1);
                const float part = k1_down_row(1, sdc_s[li & 1][k][lane], ehsh[b], ehshs[b], live, lpr, lane);
                if (live && lr == 0) xch_put(xdsh + ((size_t)b * 256 + gw) * XCH_LN + rl, part, ep);
            }
#pragma unroll
            for (int b = 0; b < NB; b++) {
                if (b >= B) break;
                const bool live_slot = ids_s[b][grp] >= 0;
                if (b + DD - 1 < NB) dn_load(b + DD - 1, st[(b + DD - 1) % DD]);
                QChunk (&cur)[2] = st[b % DD];
                k1_flag_wait(&s_eh_rdy[b], li + 1);
#pragma unroll
                for (int f = 0; f < 2; f++) {
                    const int task = wv + f * K1_W;
                    if (task < ndt) {
                        const int rl = task * rpw + rw_, row = gi * RD + rl;
                        const bool live = rl < RD && lbd < nbi;
                        const float part = k1_down_row(1, cur[f], ehk[b], ehks[b], live, lpr, lane);
                        if (live && lr == 0) xch_put(xdx + ((size_t)b * 8 + grp) * H + row, live_slot ? part : 0.0f, ep);
                    }
                }
            }
        }

        if constexpr (EARLY) {
            if (!last) wload(k1_layer(Ls, li + 1));
        }
        K1_TS(8);
        /* ---- 5. wave b: token b's owned rows combined (model.c:1139-1144) --- */
        if (wv < B) {
            const int b = wv;
            const int row = gi * RD + min(lane, RD - 1);
            const uint64_t *q[RTOPK + 1];
            float d[RTOPK + 1];
#pragma unroll
            for (int k = 0; k < RTOPK; k++) q[k] = xdx + ((size_t)b * 8 + k) * H + row;
            q[RTOPK] = xdsh + ((size_t)b * 256 + row / RO) * XCH_LN + row % RO;
            xch_gather<RTOPK + 1>(q, lane < RD ? 0x1FFu : 0u, ep, dead, A.spin, d);
            if (lane < RD) {
                float y = 0.0f;
#pragma unroll
                for (int k = 0; k < RTOPK; k++) y = fmaf(w_s[b][k], d[k], y);
                y = fmaf(sg, d[RTOPK], y);
                const float hn = hown[b][lane] + y;
                if (!last) xch_put_xcd(lh + (size_t)b * H + (size_t)(row & 3) * HU + (row >> 2), hn, ep, l2);
                else if (grp == 0) {
                    if (A.y) A.y[(size_t)b * H + row] = y;
                    else xch_put(A.xch + XCHB_HST(NB, E, H, I) + (size_t)b * H + row, hn, ep);
                }
            }
        }
        K1_TS(9);
    }
    /* a wait that gave up after the layer's last barrier is known only to
     * its own thread: every such thread reports it */
    __shared__ int s_last;
    if (dead) s_dead = 1;
    __syncthreads();
    k1_finish(A, s_dead != 0, &s_last, A.xch + XCHB_HST(NB, E, H, I), B * H, A.epoch + (uint32_t)(n - 1));
#ifdef ROASTER_PHASE_TS
    if (threadIdx.x == 0 || threadIdx.x == 64 || threadIdx.x == 448)
        for (int k = 0; k < 2; k++)
            for (int i = 0; i < 16; i++) g_k1_ts[k][blockIdx.x][min((int)threadIdx.x >> 6, 2)][i] = tsv[k][i];
#endif
#undef K1_TS
}

extern "C" __global__ void __launch_bounds__(K1_T, 1) dec_stackB2_kernel(DecArgs A) { stackB_body<2>(A); }
extern "C" __global__ void __launch_bounds__(K1_T, 1) dec_stackB4_kernel(DecArgs A) { stackB_body<4>(A); }
extern "C" __global__ void __launch_bounds__(K1_T, 1) dec_stackB8_kernel(DecArgs A) { stackB_body<8>(A); }

/* Every workgroup's XCC_ID, in a grid of the stack kernel's shape. */
extern "C" __global__ void __launch_bounds__(K1_T, 1) dec_xcd_probe_kernel(unsigned *out)
{
    unsigned xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    if (threadIdx.x == 0) out[blockIdx.x] = xcc & 0xFu;
}

/* Clears an exchange buffer (before epochs start again at 1). */
extern "C" __global__ void dec_xch_clear_kernel(uint64_t *p, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0ull;
}

/* ---- host side ------------------------------------------------------------ */
static size_t norm_lds(int B, int H) { return (size_t)B * H * 4 + (size_t)B * (H / 16) * 4; }

static int launch_layer(const DecArgs &A0, int l, bool with_router)
{
    RtState &R = rt();
    DecArgs A = A0;
    /* one-token down path (down_one_token): one down type for all 9 slots and
     * every task within D_PF per wave */
    const DecLayer *Lh = A.layers_h ? A.layers_h + l : nullptr;
    const int rpw1 = 64 / lanes_per_row(A.I / RQK);
    A.d1 = 0;
    if (A.B == 1 && !A.ffn_out && Lh && Lh->q6[2] == Lh->sq6[2] && 9 * ((D_ROWS + rpw1 - 1) / rpw1) <= DW * D_PF &&
        9 * A.I / 4 <= 5 * DT)
        A.d1 = Lh->q6[2] ? 2 : 1;
    const size_t lds = norm_lds(A.B, A.H);
    if (with_router) {
        const int ntask = (A.logits_in ? 0 : A.E) + 1 + A.I;
        if (A.B == 1) hipLaunchKernelGGL(dec_router1_kernel, dim3((ntask + DW - 1) / DW), dim3(DT), lds, R.stream, A, l);
        else hipLaunchKernelGGL(dec_router_kernel, dim3((ntask + DW - 1) / DW), dim3(DT), lds, R.stream, A, l);
        if (rt_check(hipGetLastError(), "router launch")) return ROASTER_EDEVICE;
    }
    if (A.B == 1 && !A.ffn_out) hipLaunchKernelGGL(dec_gu1_kernel, dim3(2 * R.n_cu), dim3(DT), lds, R.stream, A, l);
    else hipLaunchKernelGGL(dec_gu_kernel, dim3(2 * R.n_cu), dim3(DT), lds, R.stream, A, l);
    if (rt_check(hipGetLastError(), "gate/up launch")) return ROASTER_EDEVICE;
    const int nslot = A.ffn_out ? A.ffn_n : 9, dr = A.B > 1 ? D_ROWS_B : D_ROWS;
    const size_t dlds = (size_t)nslot * A.I * 4 + (size_t)nslot * (A.I / 16) * 4;
    const int nrb = (A.H + dr - 1) / dr;
    hipLaunchKernelGGL(dec_down_kernel, dim3(nrb * (A.ffn_out ? 1 : A.B)), dim3(DT), dlds, R.stream, A, l, dr);
    return rt_check(hipGetLastError(), "down launch") ? ROASTER_EDEVICE : 0;
}

static int g_layer1 = 1;            /* roaster_decode_fused_layer */
static int g_coop = 0;              /* roaster_decode_cooperative_launch */

extern "C" int roaster_decode_cooperative_launch(int enable)
{
    std::lock_guard<std::recursive_mutex> g(rt_lock());
    if (enable == 0 || enable == 1) g_coop = enable;
    return g_coop;
}

/* Whether every one-launch stack kernel fits one workgroup per CU on at least
 * K1_NWG CUs (registers and LDS as compiled), checked once per process: else
 * their grids could never be resident at once and the three-kernel path runs. */
static int g_k1_fits = -1;

static bool k1_fits()
{
    if (g_k1_fits >= 0) return g_k1_fits == 1;
    const void *fns[] = {(const void *)dec_stack1_kernel, (const void *)dec_stack1_2x2_kernel,
                         (const void *)dec_stack1r_kernel, (const void *)dec_stackB2_kernel,
                         (const void *)dec_stackB4_kernel, (const void *)dec_stackB8_kernel};
    bool ok = rt().n_cu >= K1_NWG;
    for (const void *f : fns) {
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, f, K1_T, 0) != hipSuccess) {
            (void)hipGetLastError();
            nb = 0;
        }
        ok = ok && nb >= 1;
    }
    g_k1_fits = ok ? 1 : 0;
    return ok;
}

/* A one-launch stack kernel on the library stream.  Its 256 workgroups wait
 * on each other, so all of them must be resident at once: a cooperative
 * launch makes the runtime guarantee that (or refuse the launch, reported as
 * ROASTER_EDEVICE) instead of leaving the waits to give up when other work
 * holds some of the CUs. */
static int launch_k1(const void *fn, DecArgs &A)
{
    if (g_coop) {
        void *args[] = {&A};
        return rt_check(hipLaunchCooperativeKernel(fn, dim3(K1_NWG), dim3(K1_T), args, 0, rt().stream),
                        "stack launch (cooperative)") ? ROASTER_EDEVICE : 0;
    }
    hipLaunchKernel(fn, dim3(K1_NWG), dim3(K1_T), (void **)(void *[]){&A}, 0, rt().stream);
    return rt_check(hipGetLastError(), "stack launch") ? ROASTER_EDEVICE : 0;
}
static uint32_t g_spin = K1_SPIN;   /* roaster_decode_spin_limit */

extern "C" unsigned roaster_decode_spin_limit(unsigned polls)
{
    std::lock_guard<std::recursive_mutex> g(rt_lock());
    if (polls) g_spin = polls;
    return g_spin;
}

extern "C" int roaster_decode_fused_layer(int enable)
{
    std::lock_guard<std::recursive_mutex> g(rt_lock());
    if (enable >= 0 && enable <= 2) g_layer1 = enable;
    return g_layer1;
}

/* The router-folded one-token kernel's shapes (dec_stack1r_kernel); the
 * matrix types are checked per launch. */
static bool dec_r1_shape(int E, int H, int I) { return g_layer1 == 1 && E == R1_E && H == R1_H && I == R1_I; }

size_t dec_xch_need1(int E, int H, int I)
{
    return std::max((size_t)XCH_U64(E, H, I), dec_r1_shape(E, H, I) ? (size_t)XR_U64(E, H, I) : (size_t)0);
}

bool dec_layer1_ok(int E, int H, int I, int B)
{
    return g_layer1 && B == 1 && k1_fits() && E >= RTOPK && E <= 256 && E % K1_GW == 0 && H % RQK == 0 &&
           H <= K1_MAXH && I % RQK == 0 && I <= K1_MAXI;
}

/* The batched kernel's shapes: inter 512 (two gate/up rows and two down
 * tasks per wave), hidden 512..2048 in whole 256-row blocks, at most 256
 * experts (one logit per lane of a wave's 64 for 8 tokens). */
bool dec_layerB_ok(int E, int H, int I, int B)
{
    return g_layer1 && B >= 2 && B <= K1B_MAXB && k1_fits() && E >= RTOPK && E <= 256 && E % K1_GW == 0 &&
           I == 512 && H % 256 == 0 && H >= 512 && H <= K1_MAXH;
}

static DecXch g_xch;

void dec_release()
{
    if (g_xch.p) (void)hipFree(g_xch.p);
    g_xch.p = NULL;
    g_xch.n = 0;
    g_xch.epoch = 0;
}

int dec_xch_clear(DecXch &X)
{
    hipLaunchKernelGGL(dec_xch_clear_kernel, dim3(64), dim3(256), 0, rt().stream, X.p, X.n);
    if (rt_check(hipGetLastError(), "exchange buffer clear")) return ROASTER_EDEVICE;
    X.epoch = 0;
    return 0;
}

DecXch *dec_xch_default(int E, int H, int I)
{
    const size_t n = std::max(dec_xch_need1(E, H, I), (size_t)XCHB_U64(K1B_MAXB, E, H, I));
    if (g_xch.p && g_xch.n >= n) return &g_xch;
    if (g_xch.p) {
        (void)hipStreamSynchronize(rt().stream);
        (void)hipFree(g_xch.p);
        g_xch.p = NULL;
        g_xch.n = 0;
    }
    if (rt_check(hipMalloc((void **)&g_xch.p, n * 8), "exchange buffer hipMalloc")) {
        g_xch.p = NULL;
        return NULL;
    }
    hipLaunchKernelGGL(dec_xch_clear_kernel, dim3(64), dim3(256), 0, rt().stream, g_xch.p, n);
    if (rt_check(hipGetLastError(), "exchange buffer clear")) return NULL;
    g_xch.n = n;
    g_xch.epoch = 0;
    return &g_xch;
}

/* Whether the dispatcher deals the stack kernel's grid to the XCDs in turn,
 * XCC_ID(b) = (b + r) % 8 (then a group is an XCD and its SiLU*up slots stay
 * in its L2): -1 = not probed yet. */
static int g_xl2 = -1;

int dec_probe_placement()
{
    g_xl2 = 0;
    unsigned *d = NULL;
    if (rt().n_cu < K1_NWG) return 0;
    if (rt_check(hipMalloc((void **)&d, K1_NWG * sizeof(unsigned)), "placement probe hipMalloc")) return ROASTER_EDEVICE;
    unsigned h[K1_NWG];
    hipLaunchKernelGGL(dec_xcd_probe_kernel, dim3(K1_NWG), dim3(K1_T), 0, rt().stream, d);
    int rc = rt_check(hipGetLastError(), "placement probe launch");
    if (!rc) rc = rt_check(hipMemcpyAsync(h, d, sizeof(h), hipMemcpyDeviceToHost, rt().stream), "placement probe copy");
    if (!rc) rc = rt_check(hipStreamSynchronize(rt().stream), "placement probe sync");
    (void)hipFree(d);
    if (rc) return ROASTER_EDEVICE;
    /* one rotation r for the whole grid: XCC_ID(b) = (b + r) % 8 */
    int ok = h[0] < (unsigned)K1_G;
    for (int b = 0; b < K1_NWG; b++) ok &= h[b] < (unsigned)K1_G && ((h[b] - b) & 7u) == ((h[0] - 0u) & 7u);
    g_xl2 = ok;
    return 0;
}

void dec_placement_failed() { g_xl2 = 0; }

/* Which one-token kernel runs layers [c0, c0 + cn) of A on an exchange
 * buffer of xn slots: 0 dec_stack1r_kernel, 1 dec_stack1_2x2_kernel, 2
 * dec_stack1_kernel. */
static int stack1_choice(const DecArgs &A, int c0, int cn, size_t xn)
{
    const int nbi = A.I / RQK, rpw = 64 / lanes_per_row(nbi);
    const int npg = (A.I / K1_GW + K1_W - 1) / K1_W, nd = ((A.H / K1_GW + rpw - 1) / rpw + K1_W - 1) / K1_W;
    bool ty = A.layers_h != nullptr;
    for (int l = c0; ty && l < c0 + cn; l++) {
        const DecLayer *Lh = A.layers_h + l;
        ty = !Lh->q6[0] && !Lh->q6[1] && Lh->q6[2] && !Lh->sq6[0] && !Lh->sq6[1] && Lh->sq6[2];
    }
    if (ty && A.cnt && dec_r1_shape(A.E, A.H, A.I) && xn >= (size_t)XR_U64(A.E, A.H, A.I)) return 0;
    return npg == 2 && nd == 2 && ty ? 1 : 2;
}

/* One launch per run of up to K1_MAXL layers (dec_stack1_kernel) on the
 * exchange buffer A.xbuf. */
static int launch_stack1(DecArgs &A0)
{
    DecXch &X = *A0.xbuf;
    for (int c0 = A0.layer0; c0 < A0.layer0 + A0.nlayers; c0 += K1_MAXL) {
        const int cn = min(K1_MAXL, A0.layer0 + A0.nlayers - c0), off = c0 - A0.layer0;
        DecArgs A = A0;
        A.xch = X.p;
        A.layer0 = c0;
        A.nlayers = cn;
        if (A.ids_out) A.ids_out += (size_t)off * RTOPK;
        if (A.w_out) A.w_out += (size_t)off * RTOPK;
        if (A.norm_w) A.norm_w += (size_t)off * A.H;
        if (X.epoch > 0xFFFFFFFFu - (uint32_t)cn - 1u) {  /* epochs start again on cleared slots */
            hipLaunchKernelGGL(dec_xch_clear_kernel, dim3(64), dim3(256), 0, rt().stream, X.p, X.n);
            if (rt_check(hipGetLastError(), "exchange buffer clear")) return ROASTER_EDEVICE;
            X.epoch = 0;
        }
        A.epoch = X.epoch + 1;
        X.epoch += (uint32_t)cn;
        A.spin = g_spin;
        A.xl2 = g_xl2 == 1;
        const int ch = stack1_choice(A, c0, cn, X.n);
        const void *fn = ch == 0 ? (const void *)dec_stack1r_kernel
                         : ch == 1 ? (const void *)dec_stack1_2x2_kernel : (const void *)dec_stack1_kernel;
        if (int rc = launch_k1(fn, A)) return rc;
    }
    return 0;
}

/* One launch per run of up to K1_MAXL layers of B = 2..8 tokens
 * (dec_stackB*_kernel, the smallest of 2, 4, 8 slots that holds B), when
 * every layer has Q4_K gate/up and Q6_K down matrices, routed and shared;
 * else 1 (the caller runs the three-kernel path). */
static int launch_stackB(DecArgs &A0)
{
    if (!A0.layers_h) return 1;
    for (int l = A0.layer0; l < A0.layer0 + A0.nlayers; l++) {
        const DecLayer *Lh = A0.layers_h + l;
        if (Lh->q6[0] || Lh->q6[1] || !Lh->q6[2] || Lh->sq6[0] || Lh->sq6[1] || !Lh->sq6[2]) return 1;
    }
    DecXch &X = *A0.xbuf;
    if (X.n < (size_t)XCHB_U64(K1B_MAXB, A0.E, A0.H, A0.I)) return 1;
    for (int c0 = A0.layer0; c0 < A0.layer0 + A0.nlayers; c0 += K1_MAXL) {
        const int cn = min(K1_MAXL, A0.layer0 + A0.nlayers - c0), off = c0 - A0.layer0;
        DecArgs A = A0;
        A.xch = X.p;
        A.layer0 = c0;
        A.nlayers = cn;
        if (A.ids_out) A.ids_out += (size_t)off * A.B * RTOPK;
        if (A.w_out) A.w_out += (size_t)off * A.B * RTOPK;
        if (A.norm_w) A.norm_w += (size_t)off * A.H;
        if (X.epoch > 0xFFFFFFFFu - (uint32_t)cn - 1u) {  /* epochs start again on cleared slots */
            hipLaunchKernelGGL(dec_xch_clear_kernel, dim3(64), dim3(256), 0, rt().stream, X.p, X.n);
            if (rt_check(hipGetLastError(), "exchange buffer clear")) return ROASTER_EDEVICE;
            X.epoch = 0;
        }
        A.epoch = X.epoch + 1;
        X.epoch += (uint32_t)cn;
        A.spin = g_spin;
        A.xl2 = g_xl2 == 1;
        const void *fn = A.B <= 2 ? (const void *)dec_stackB2_kernel
                         : A.B <= 4 ? (const void *)dec_stackB4_kernel : (const void *)dec_stackB8_kernel;
        if (int rc = launch_k1(fn, A)) return rc;
    }
    return 0;
}

/* The kernels a decode call of A (table fields, B, layers, y) would launch,
 * on the library's own exchange buffer. */
const char *dec_kernel_names(const DecArgs &A)
{
    if (dec_layer1_ok(A.E, A.H, A.I, A.B)) {
        DecArgs C = A;
        if (!C.cnt) C.cnt = (uint32_t *)&C;               /* only its presence matters here */
        const int ch = stack1_choice(C, A.layer0, std::min(A.nlayers, K1_MAXL), dec_xch_need1(A.E, A.H, A.I));
        return ch == 0 ? "dec_stack1r_kernel" : ch == 1 ? "dec_stack1_2x2_kernel" : "dec_stack1_kernel";
    }
    bool tyB = A.layers_h != nullptr;
    for (int l = A.layer0; tyB && l < A.layer0 + A.nlayers; l++) {
        const DecLayer *Lh = A.layers_h + l;
        tyB = !Lh->q6[0] && !Lh->q6[1] && Lh->q6[2] && !Lh->sq6[0] && !Lh->sq6[1] && Lh->sq6[2];
    }
    if (tyB && dec_layerB_ok(A.E, A.H, A.I, A.B))
        return A.B <= 2 ? "dec_stackB2_kernel" : A.B <= 4 ? "dec_stackB4_kernel" : "dec_stackB8_kernel";
    return A.B == 1 ? "dec_router1_kernel + dec_gu1_kernel + dec_down_kernel per layer"
                    : "dec_router_kernel + dec_gu_kernel + dec_down_kernel per layer";
}

int dec_launch(DecArgs &A)
{
    A.xswz = A.H % 512 == 0;
    if (A.E > 256) return rt_fail(ROASTER_EINVAL, "decode supports at most 256 routed experts");
    if (!A.plan_g || !A.err) {          /* caller-provided plan and error word, or the library's own */
        unsigned *ctrl = rt_ctrl();
        A.plan_g = (DecPlan *)rt_scratch(SCR_C, sizeof(DecPlan));
        if (!ctrl || !A.plan_g) return ROASTER_ENOMEM;
        A.err = (int *)(ctrl + 16);
        A.cnt = ctrl + 32;
    }
    if (!A.cnt) {                       /* the one-launch kernels' completion counter */
        unsigned *ctrl = rt_ctrl();
        if (!ctrl) return ROASTER_ENOMEM;
        A.cnt = ctrl + 32;
    }
    if (A.xbuf && !A.ffn_out && dec_layer1_ok(A.E, A.H, A.I, A.B)) return launch_stack1(A);
    if (A.xbuf && !A.ffn_out && dec_layerB_ok(A.E, A.H, A.I, A.B))
        if (int rc = launch_stackB(A); rc <= 0) return rc;
    for (int l = A.layer0; l < A.layer0 + A.nlayers; l++)
        if (int rc = launch_layer(A, l, true)) return rc;
    return 0;
}

int dec_ffn_launch(DecArgs &A)
{
    A.xswz = A.H % 512 == 0;
    unsigned *ctrl = rt_ctrl();
    A.plan_g = (DecPlan *)rt_scratch(SCR_C, sizeof(DecPlan));
    if (!ctrl || !A.plan_g) return ROASTER_ENOMEM;
    A.err = (int *)(ctrl + 16);
    return launch_layer(A, 0, false);
}
