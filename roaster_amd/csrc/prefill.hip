/*
 * prefill.hip -- the MoE block over T tokens (model.c:1671-1791) on the GPU.
 *
 *   pf_router_mfma_kernel  logits = X . W_r^T in f32 on v_mfma_f32_32x32x2_f32,
 *                      split over K into 8 partial sums added in fixed order
 *                      by the token kernel (model.c:1679)
 *   pf_token_kernel    one wave per token: logits (+ bias), top-8 and
 *                      renormalised weights (model.c:1681-1692), the shared
 *                      expert's sigmoid gate (model.c:1707-1708), the row
 *                      scale of X for the fp16 GEMM operands
 *   pf_bucket_kernel   one workgroup per expert: that expert's token list in
 *                      token order, i.e. the stable counting sort over (t, k)
 *                      of model.c:1713-1731
 *   pf_plan_kernel     offsets (prefix sums of the counts), groups and the
 *                      tile list; the shared expert is one more group over
 *                      all T tokens (model.c:1694-1711)
 *   grouped GEMMs      gate/up with the SiLU(gate) * up epilogue, then down
 *                      (pf_gemm.hip)
 *   pf_combine_kernel  Y[t] = sigmoid(s_t) * shared(t), then += w * expert
 *                      output in ascending expert id (model.c:1709-1711,
 *                      1776-1788), one fused multiply-add per term
 *
 * Slots: routed pair (t, k) with expert e owns slot off[e] + rank, where rank
 * is t's position in e's list; token t's shared-expert row owns slot 8T + t.
 */
#include "internal.h"
#include "gemm.h"
#include "prefill.h"
#include "table.h"
#include "topk.h"

#include <string.h>

#define PF_MAX_T (1 << 16)
#define RT_KSPLIT 8               /* router K split */

/* Natural position p (multiple of 4) inside a super-block -> the slot of its
 * first element in the fp16 GEMM's permuted K order (pf_gemm.hip). */
__device__ __forceinline__ int pf_perm_slot4(int p)
{
    const int h = p >> 7, q = p & 127, hi = q >> 6, r = q & 63;
    const int l0 = r < 32 ? r : r - 32, i0 = r < 32 ? 0 : 4;
    return (8 * hi + (l0 >> 2)) * 16 + 8 * h + i0;
}

/* Exclusive prefix sum over a 256-thread workgroup; *total gets the sum. */
__device__ int block_scan_256(int v, int *lds, int *total)
{
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int inc = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int o = __shfl_up(inc, d);
        if (lane >= d) inc += o;
    }
    if (lane == 63) lds[w] = inc;
    __syncthreads();
    int before = 0, all = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int c = lds[i];
        before += i < w ? c : 0;
        all += c;
    }
    __syncthreads();
    *total = all;
    return before + inc - v;
}

/* ---- router on MFMA: part[s][t][e] = sum over k in split s of X[t][k] W[e][k]
 * A workgroup (4 waves) takes 32 tokens x 128 experts of K split s; wave w
 * owns experts e0 + 32 w .. + 31 in one v_mfma_f32_32x32x2_f32 accumulator
 * (A = X rows, B = W rows, fp32 products and sums).  The tokens' K slice is
 * staged once in LDS (row stride klen + 4 floats: the 16 rows a ds_read_b128
 * pass reads fall in 16 different bank groups); each wave reads its weight
 * rows straight from global memory, one 32-wide K chunk ahead.  In a chunk,
 * lane half h supplies k = 16 h + j to MFMA j (j = 0..15), so 16 MFMAs cover
 * the chunk and every lane reads 16 consecutive floats of X and of W. */
#define RM_E 128                  /* experts per workgroup */
#define RM_T 32                   /* tokens per workgroup */

extern "C" __global__ void __launch_bounds__(256, 2) pf_router_mfma_kernel(const float *X, const float *W, float *part,
                                                                           int T, int E, int H)
{
    extern __shared__ __align__(16) float xs[];         /* [RM_T][klen + 4] */
    const int tid = threadIdx.x, l = tid & 63, h = l >> 5, n = l & 31;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t0 = blockIdx.x * RM_T, e0 = blockIdx.y * RM_E + 32 * w, s = blockIdx.z;
    const int klen = H / RT_KSPLIT, kbeg = s * klen, ld = klen + 4;
    /* stage X[t0 .. t0 + 31][kbeg .. kbeg + klen) (klen <= 512: at most 16
     * float4 per thread, all loaded before the first store; rows past T read
     * row T - 1, pieces past the slice repeat its last one) */
    const int q4 = klen / 4, nq = RM_T * q4;           /* float4 per row, in the slice */
    float4 v[16];
#pragma unroll
    for (int k = 0; k < 16; k++) {
        const int i = min(tid + 256 * k, nq - 1), r = i / q4, c = i - r * q4;
        v[k] = *(const float4 *)(X + (size_t)min(t0 + r, T - 1) * H + kbeg + 4 * c);
    }
#pragma unroll
    for (int k = 0; k < 16; k++) {
        const int i = min(tid + 256 * k, nq - 1), r = i / q4, c = i - r * q4;
        *(float4 *)(xs + r * ld + 4 * c) = v[k];
    }
    __syncthreads();
    /* this lane's weight row (clamped past E; those columns are not stored) */
    const float *wr = W + (size_t)min(e0 + n, E - 1) * H + kbeg + 16 * h;
    const float *xr = xs + n * ld + 16 * h;
    f32x16 acc = (f32x16){};
    /* weights in batches of RM_B chunks, the next batch loaded during the
     * current one (chunk indices clamped; chunks past nch are not used) */
    constexpr int RM_B = 4;
    const int nch = klen / 32;
    float4 wb[2][RM_B][4];
    auto w_batch = [&](float4 (&dst)[RM_B][4], int c0) {
#pragma unroll
        for (int j = 0; j < RM_B; j++)
#pragma unroll
            for (int q = 0; q < 4; q++) dst[j][q] = *(const float4 *)(wr + 32 * min(c0 + j, nch - 1) + 4 * q);
    };
    auto compute = [&](const float4 (&src)[RM_B][4], int c0) {
#pragma unroll
        for (int j = 0; j < RM_B; j++) {
            if (c0 + j >= nch) break;
            float4 xa[4];
#pragma unroll
            for (int q = 0; q < 4; q++) xa[q] = *(const float4 *)(xr + 32 * (c0 + j) + 4 * q);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[q].x, src[j][q].x, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[q].y, src[j][q].y, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[q].z, src[j][q].z, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[q].w, src[j][q].w, acc, 0, 0, 0);
            }
        }
    };
    w_batch(wb[0], 0);
    for (int c = 0; c < nch; c += 2 * RM_B) {
        w_batch(wb[1], c + RM_B);
        compute(wb[0], c);
        if (c + RM_B >= nch) break;
        w_batch(wb[0], c + 2 * RM_B);
        compute(wb[1], c + RM_B);
    }
    /* D item i: token t0 + 8 (i / 4) + 4 h + i % 4, expert e0 + n */
    if (e0 + n < E) {
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int m = t0 + 8 * (i >> 2) + 4 * h + (i & 3);
            if (m < T) part[((size_t)s * T + m) * E + e0 + n] = acc[i];
        }
    }
}


/* ---- per token: logits, top-8, shared gate, X row scale ------------------ */
struct PfTokArgs {
    const float *X;
    const float *gate_inp;
    const float *part;          /* router partial sums [KSPLIT][T][E], or NULL */
    const float *logits_in;     /* [T x E] or NULL */
    const float *bias;          /* [E] or NULL */
    float *logits_out;          /* [T x E] or NULL */
    int *ids;                   /* [T x 8] */
    float *w;                   /* [T x 8] */
    int *ids_out;
    float *w_out;
    float *sg;                  /* [T] */
    float *xinv, *xfwd;         /* [T] (fp16 mode) or NULL */
    uint16_t *x16;              /* [T x H] fp16 X * xinv in the GEMM's permuted K order, or NULL */
    int *err;
    int T, E, H;
};

extern "C" __global__ void __launch_bounds__(256) pf_token_kernel(PfTokArgs A)
{
    __shared__ int bad[4];
    __shared__ TopkScratch ts[4];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int t = blockIdx.x * 4 + wv;
    if (t >= A.T) return;
    /* The token's logits (or router partial sums) and biases are loaded
     * first, then its X row (H <= 2048: at most 8 float4 per lane) and the
     * gate vector, indices clamped.  A wave's loads complete in order, so
     * the top 8 runs on the logits while the X row is still arriving; the
     * row then stays in registers for the fp16 conversion. */
    float v4[4], b4[4] = { 0.0f, 0.0f, 0.0f, 0.0f };
    /* the router's 4 x RT_KSPLIT partial sums (or the 4 logits) in one
     * batch, summed in split order once the X row is on its way */
    const size_t TE = (size_t)A.T * A.E;
    float p[4][RT_KSPLIT];
    if (A.logits_in) {
#pragma unroll
        for (int i = 0; i < 4; i++) v4[i] = A.logits_in[(size_t)t * A.E + min(lane + 64 * i, A.E - 1)];
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int s = 0; s < RT_KSPLIT; s++) p[i][s] = A.part[s * TE + (size_t)t * A.E + min(lane + 64 * i, A.E - 1)];
    }
    if (A.bias) {
#pragma unroll
        for (int i = 0; i < 4; i++) b4[i] = A.bias[min(lane + 64 * i, A.E - 1)];
    }
    const float *x = A.X + (size_t)t * A.H;
    float4 xv[8], gv[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int k = min(4 * lane + 256 * i, A.H - 4);
        xv[i] = *(const float4 *)(x + k);
        gv[i] = *(const float4 *)(A.gate_inp + k);
    }
    if (!A.logits_in) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float sum = p[i][0];
#pragma unroll
            for (int s = 1; s < RT_KSPLIT; s++) sum += p[i][s];
            v4[i] = sum;
        }
    }
    /* logits (+ bias) and the top 8 */
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int e = lane + 64 * i;
        float l = -INFINITY;
        if (e < A.E) {
            l = v4[i];
            if (A.bias) l = l + b4[i];
            if (A.logits_out) A.logits_out[(size_t)t * A.E + e] = l;
        }
        v4[i] = l;
    }
    if (lane == 0) bad[wv] = 0;
    __builtin_amdgcn_wave_barrier();
    topk8_fast(v4, A.E, A.ids + (size_t)t * 8, A.w + (size_t)t * 8, &bad[wv], &ts[wv]);
    /* X row: max |x|, the shared-expert gate dot, the fp16 copy */
    float mx = 0.0f, dot = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        if (4 * lane + 256 * i < A.H) {
            const float4 v = xv[i], g = gv[i];
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
            dot = fmaf(v.x, g.x, dot); dot = fmaf(v.y, g.y, dot);
            dot = fmaf(v.z, g.z, dot); dot = fmaf(v.w, g.w, dot);
        }
    }
    dot = group_sum<64>(dot);
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) mx = fmaxf(mx, __shfl_xor(mx, d));
    if (A.xinv) {
        float inv, fwd;
        row_scale(mx, inv, fwd);
        if (lane == 0) {
            A.xinv[t] = inv;
            A.xfwd[t] = fwd;
        }
        if (A.x16) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int k = 4 * lane + 256 * i;
                if (k < A.H) {
                    const float4 v = xv[i];
                    const f32x8 e = { v.x * inv, v.y * inv, v.z * inv, v.w * inv, 0.f, 0.f, 0.f, 0.f };
                    const uint4 c = __builtin_bit_cast(uint4, __builtin_convertvector(e, f16x8));
                    *(uint2 *)(A.x16 + (size_t)t * A.H + (k & ~255) + pf_perm_slot4(k & 255)) = make_uint2(c.x, c.y);
                }
            }
        }
    }
    if (lane == 0) A.sg[t] = 1.0f / (1.0f + expf(-dot));
    if (lane < 8) {
        if (A.ids_out) A.ids_out[(size_t)t * 8 + lane] = A.ids[(size_t)t * 8 + lane];
        if (A.w_out) A.w_out[(size_t)t * 8 + lane] = A.w[(size_t)t * 8 + lane];
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    if (lane == 0 && bad[wv]) atomicOr(A.err, 1);
}

/* ---- bucketing: list[e][r] = r-th token (ascending) that selected e ------- */
extern "C" __global__ void __launch_bounds__(256) pf_bucket_kernel(const int *ids, int T, int *list, int *rank,
                                                                   int *cnt)
{
    __shared__ int wsum[4];
    const int e = blockIdx.x;
    int base = 0;
    /* 2048 tokens per round: thread i takes tokens 8i .. 8i + 7 of the round
     * (their ids loaded at once, indices clamped), counts its matches, and one
     * block scan gives its first rank, so the ranks follow token order */
    for (int c0 = 0; c0 < T; c0 += 8 * 256) {
        int4 a[8], b[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int t = min(c0 + 8 * (int)threadIdx.x + j, T - 1);
            a[j] = *(const int4 *)(ids + (size_t)t * 8);
            b[j] = *(const int4 *)(ids + (size_t)t * 8 + 4);
        }
        int k[8], n = 0;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int t = c0 + 8 * (int)threadIdx.x + j;
            k[j] = -1;
            if (t < T)
                k[j] = a[j].x == e ? 0 : a[j].y == e ? 1 : a[j].z == e ? 2 : a[j].w == e ? 3
                     : b[j].x == e ? 4 : b[j].y == e ? 5 : b[j].z == e ? 6 : b[j].w == e ? 7 : -1;
            n += k[j] >= 0 ? 1 : 0;
        }
        int total;
        int r = base + block_scan_256(n, wsum, &total);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            if (k[j] >= 0) {
                const int t = c0 + 8 * (int)threadIdx.x + j;
                list[(size_t)e * T + r] = t;
                rank[(size_t)t * 8 + k[j]] = r;
                r++;
            }
        }
        base += total;
    }
    if (threadIdx.x == 0) cnt[e] = base;
}

/* ---- plan: offsets, groups, tiles ----------------------------------------- */
struct PfPlanArgs {
    DecLayer L;
    TileLayer TL;
    size_t eb_g, eb_u, eb_d;    /* per-expert matrix bytes */
    size_t teb_g, teb_u, teb_d; /* per-expert tile-layout bytes */
    int q6g, q6u, q6d, sq6g, sq6u, sq6d;
    const int *cnt;
    const int *list;
    int *off;                   /* [E] */
    int *counts_out;            /* [E] or NULL */
    PfGroup *groups;            /* [E + 1] */
    const float *dbound;        /* [E + 1] down-row L1 bounds of the layer */
    PfTile *tiles;
    int *ntiles;
    int *gu_ctr;                /* [8] zeroed for the persistent gate/up GEMM */
    int *dn_bnd;                /* [n_wg + 1] the balanced down GEMM's split, or NULL */
    PfDnTile *dn_tiles;         /* the tile list as down records (with dn_bnd) */
    int *fx;                    /* fused GEMMs: [0, 9) XCD tile bounds, [16, 24) down chunk
                                   counters, [32, 32 + max tiles) tile counters; or NULL */
    int n_wg;                   /* its workgroups */
    int nt_out;                 /* its units per tile: H / PF_DN_ROWS */
    int T, E;
    int chunk;                  /* rows per tile */
};

/* Cost of the down-GEMM units of a group of c rows cut into tiles of chunk
 * rows (the start of each tile counted as a range start). */
__device__ __forceinline__ int pf_dn_tile_cost(int rows, int nt_out)
{
    return PF_DN_CP + nt_out * (PF_DN_CA + PF_DN_CB * ((rows + 31) >> 5));
}
__device__ __forceinline__ int pf_dn_group_cost(int c, int chunk, int nt_out)
{
    if (c <= 0) return 0;
    const int nt = (c + chunk - 1) / chunk;
    return (nt - 1) * pf_dn_tile_cost(chunk, nt_out) + pf_dn_tile_cost(c - (nt - 1) * chunk, nt_out);
}

/* Three exclusive prefix sums over a 256-thread workgroup in one pass (one
 * LDS exchange); *total gets the sums. */
__device__ int3 block_scan3_256(int3 v, int *lds, int3 *total)
{
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int3 inc = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int ox = __shfl_up(inc.x, d), oy = __shfl_up(inc.y, d), oz = __shfl_up(inc.z, d);
        if (lane >= d) { inc.x += ox; inc.y += oy; inc.z += oz; }
    }
    if (lane == 63) { lds[w] = inc.x; lds[4 + w] = inc.y; lds[8 + w] = inc.z; }
    __syncthreads();
    int3 before = make_int3(0, 0, 0), all = make_int3(0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int cx = lds[i], cy = lds[4 + i], cz = lds[8 + i];
        if (i < w) { before.x += cx; before.y += cy; before.z += cz; }
        all.x += cx; all.y += cy; all.z += cz;
    }
    __syncthreads();
    *total = all;
    return make_int3(before.x + inc.x - v.x, before.y + inc.y - v.y, before.z + inc.z - v.z);
}

extern "C" __global__ void __launch_bounds__(256) pf_plan_kernel(PfPlanArgs A)
{
    __shared__ int wsum[12];
    __shared__ int s_gc[258], s_toff[257], s_c[257];
    const int e = threadIdx.x;
    if (e < 8) A.gu_ctr[e] = 0;
    /* every global read first (their latencies overlap) */
    const int c = e < A.E ? A.cnt[e] : 0;
    const float dbnd = e < A.E ? A.dbound[e] : 0.0f, sdbnd = A.dbound[A.E];
    const int nt = (c + A.chunk - 1) / A.chunk;
    const int cost = A.dn_bnd && e < A.E ? pf_dn_group_cost(c, A.chunk, A.nt_out) : 0;
    int3 tot;
    const int3 pre = block_scan3_256(make_int3(c, nt, cost), wsum, &tot);
    const int off = pre.x, toff = pre.y, tot_tiles = tot.y;
    const int nsh = (A.T + A.chunk - 1) / A.chunk;
    /* per group: tile offset and rows (group E: the shared expert); with the
     * balanced down GEMM, its cost prefix (each tile a range start plus its
     * units) */
    if (e < A.E) { s_toff[e] = toff; s_c[e] = c; }
    if (e == 0) { s_toff[A.E] = tot_tiles; s_c[A.E] = A.T; }
    if (A.dn_bnd) {
        if (e < A.E) s_gc[e] = pre.z;
        if (e == 0) {
            s_gc[A.E] = tot.z;
            s_gc[A.E + 1] = tot.z + pf_dn_group_cost(A.T, A.chunk, A.nt_out);
        }
    }
    if (e < A.E) {
        A.off[e] = off;
        if (A.counts_out) A.counts_out[e] = c;
        PfGroup G;
        G.g = A.L.gate + (size_t)e * A.eb_g;
        G.u = A.L.up + (size_t)e * A.eb_u;
        G.d = A.L.down + (size_t)e * A.eb_d;
        G.tg = A.TL.gate + (size_t)e * A.teb_g;
        G.tu = A.TL.up + (size_t)e * A.teb_u;
        G.td = A.TL.down + (size_t)e * A.teb_d;
        G.gq6 = A.q6g; G.uq6 = A.q6u; G.dq6 = A.q6d;
        G.n = c;
        G.slot0 = off;
        G.tok0 = 0;
        G.tok = A.list + (size_t)e * A.T;
        G.dbnd = dbnd;
        A.groups[e] = G;
        for (int i = 0; i < nt; i++) A.tiles[toff + i] = PfTile{ e, i * A.chunk };
        if (A.dn_bnd)
            for (int i = 0; i < nt; i++)
                A.dn_tiles[toff + i] = PfDnTile{ G.td, off + i * A.chunk, min(A.chunk, c - i * A.chunk), G.dq6, dbnd, { 0, 0 } };
    }
    if (e == 0) {
        PfGroup G;
        G.g = A.L.sgate; G.u = A.L.sup; G.d = A.L.sdown;
        G.tg = A.TL.sgate; G.tu = A.TL.sup; G.td = A.TL.sdown;
        G.gq6 = A.sq6g; G.uq6 = A.sq6u; G.dq6 = A.sq6d;
        G.n = A.T;
        G.slot0 = 8 * A.T;
        G.tok0 = 0;
        G.tok = nullptr;
        G.dbnd = sdbnd;
        A.groups[A.E] = G;
        *A.ntiles = tot_tiles + nsh;
    }
    for (int i = e; i < nsh; i += 256) {
        A.tiles[tot_tiles + i] = PfTile{ A.E, i * A.chunk };
        if (A.dn_bnd)
            A.dn_tiles[tot_tiles + i] = PfDnTile{ A.TL.sdown, 8 * A.T + i * A.chunk, min(A.chunk, A.T - i * A.chunk),
                                                  A.sq6d, sdbnd, { 0, 0 } };
    }
    if (A.fx) {
        /* the fused GEMMs: counters zeroed, and the tiles split over the 8
         * XCDs by a prefix of tile weights (routed groups, then the shared
         * one), each bound rounded to a tile */
        const int ntot = tot_tiles + nsh;
        for (int i = e; i < ntot; i += 256) A.fx[32 + i] = 0;
        if (e < 8) A.fx[16 + e] = 0;
        auto tw = [&](int rows) { return PF_FX_CA + PF_FX_CB * ((rows + 31) >> 5); };
        auto gw = [&](int cnt) {
            if (cnt <= 0) return 0;
            const int ntg = (cnt + A.chunk - 1) / A.chunk;
            return (ntg - 1) * tw(A.chunk) + tw(cnt - (ntg - 1) * A.chunk);
        };
        __shared__ int s_fw[258];
        int wall;
        const int wpre = block_scan_256(e < A.E ? gw(c) : 0, wsum, &wall);
        if (e < A.E) s_fw[e] = wpre;
        if (e == 0) { s_fw[A.E] = wall; s_fw[A.E + 1] = wall + gw(A.T); }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (e <= 8) {
            int tb = e == 0 ? 0 : ntot;
            if (e > 0 && e < 8) {
                const int target = (int)((long long)e * s_fw[A.E + 1] / 8);
                int lo = 0, hi = A.E;              /* the last group g <= E with s_fw[g] <= target */
                while (lo < hi) {
                    const int mid = (lo + hi + 1) >> 1;
                    if (s_fw[mid] <= target) lo = mid; else hi = mid - 1;
                }
                const int g = lo, cg = s_c[g];
                const int ntg = (cg + A.chunk - 1) / A.chunk, off = target - s_fw[g];
                const int i = min((off + tw(A.chunk) / 2) / tw(A.chunk), ntg);
                tb = s_toff[g] + i;
            }
            A.fx[e] = tb;
        }
    }
    if (A.dn_bnd) {
        /* the balanced down GEMM's split: workgroup b starts at the unit
         * where the cost prefix reaches b / n_wg of the total; the bounds are
         * non-decreasing in b, so the ranges cover every unit once */
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");   /* LDS only: the stores stay in flight */
        const int ctot = s_gc[A.E + 1];
        const bool narrow = (unsigned long long)ctot * (unsigned)A.n_wg < (1ull << 32);
        const int full = pf_dn_tile_cost(A.chunk, A.nt_out);
        for (int b = e; b <= A.n_wg; b += 256) {
            int u = (tot_tiles + nsh) * A.nt_out;
            if (b < A.n_wg) {
                const int cpos = narrow ? (int)((unsigned)b * (unsigned)ctot / (unsigned)A.n_wg)
                                        : (int)((long long)b * ctot / A.n_wg);
                int lo = 0, hi = A.E;              /* the last group g <= E with s_gc[g] <= cpos */
                while (lo < hi) {
                    const int mid = (lo + hi + 1) >> 1;
                    if (s_gc[mid] <= cpos) lo = mid; else hi = mid - 1;
                }
                const int g = lo, cg = s_c[g], ntg = (cg + A.chunk - 1) / A.chunk, go = cpos - s_gc[g];
                const int i = min(go / full, ntg - 1);
                const int rows = i < ntg - 1 ? A.chunk : cg - i * A.chunk;
                const int uc = PF_DN_CA + PF_DN_CB * ((rows + 31) >> 5), rem = go - i * full - PF_DN_CP;
                u = (s_toff[g] + i) * A.nt_out + (rem <= 0 ? 0 : min(A.nt_out, (rem + uc - 1) / uc));
            }
            A.dn_bnd[b] = u;
        }
    }
}

/* ---- combine -------------------------------------------------------------- */
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

/* Token t's routed slots and weights in ascending expert id (sl = -1 for an
 * unrouted pick).  Lane k of each wave (k < 8) holds pick k: its id, weight
 * and slot (off[id] + its rank, rank indexed by (t, k)); its place in the
 * ascending order of (id, k) — ids of one token are distinct, -1 marks an
 * unrouted pick — is the count of picks before it, and entry p is read out
 * of the lane whose place is p.  All loads are issued unconditionally, in
 * two round trips (picks, then offsets). */
__device__ __forceinline__ void pf_token_slots(const int *ids, const float *w, const int *rank, const int *off, int t,
                                               int (&sl)[8], float (&wt)[8])
{
    const int lane = (int)threadIdx.x & 63, k = lane & 7;
    const int id = ids[(size_t)t * 8 + k];
    const float wk = w[(size_t)t * 8 + k];
    const int rk = rank[(size_t)t * 8 + k];
    const int of = off[id >= 0 ? id : 0];
    const int s = id >= 0 ? of + rk : -1;
    int pos = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int ij = __builtin_amdgcn_readlane(id, j);
        pos += ij < id || (ij == id && j < k) ? 1 : 0;
    }
#pragma unroll
    for (int p = 0; p < 8; p++) {
        const unsigned long long m = __ballot(pos == p && lane < 8);
        const int src = (int)__builtin_ctzll(m);
        sl[p] = __builtin_amdgcn_readlane(s, src);
        wt[p] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wk), src));
    }
}

/* Y[t] = g_t * shared row + sum over the routed rows in ascending expert id of
 * w * row (f32 rows), one fused multiply-add per term. */
extern "C" __global__ void __launch_bounds__(256) pf_combine_kernel(const float *ed, const int *ids, const float *w,
                                                                    const int *rank, const int *off, const float *sg,
                                                                    float *Y, int T, int H)
{
    const int t = blockIdx.x;
    int sl[8];
    float wt[8];
    pf_token_slots(ids, w, rank, off, t, sl, wt);
    const float g = sg[t];
    const float *sh = ed + ((size_t)8 * T + t) * H;
    /* H <= 2048: two float4 columns per thread, all 18 row loads issued
     * before the first use (columns clamped, unrouted slots read the shared
     * row; neither is used) */
    float4 s4[2], d4[2][8];
#pragma unroll
    for (int c = 0; c < 2; c++) {
        const int i = min((int)threadIdx.x * 4 + 1024 * c, H - 4);
        s4[c] = *(const float4 *)(sh + i);
#pragma unroll
        for (int k = 0; k < 8; k++)
            d4[c][k] = *(const float4 *)((sl[k] >= 0 ? ed + (size_t)sl[k] * H : sh) + i);
    }
#pragma unroll
    for (int c = 0; c < 2; c++) {
        const int i = threadIdx.x * 4 + 1024 * c;
        if (i >= H) break;
        float4 y = make_float4(g * s4[c].x, g * s4[c].y, g * s4[c].z, g * s4[c].w);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            if (sl[k] < 0) continue;
            const float4 d = d4[c][k];
            y.x = fmaf(wt[k], d.x, y.x);
            y.y = fmaf(wt[k], d.y, y.y);
            y.z = fmaf(wt[k], d.z, y.z);
            y.w = fmaf(wt[k], d.w, y.w);
        }
        *(float4 *)(Y + (size_t)t * H + i) = y;
    }
}

/* The combine on fp16 rows (fp16 mode), row s holding product * 2^-oexp[s]:
 * each term multiplies by w * 2^oexp[s] instead (exact: a power-of-two
 * scaling of the weight), so every fused multiply-add equals the f32
 * combine's on the fp16-rounded product.  8 columns (16 bytes) per thread,
 * all 9 row loads issued before the first use. */
extern "C" __global__ void __launch_bounds__(256) pf_combine16_kernel(const uint16_t *ed, const int8_t *oexp,
                                                                      const int *ids, const float *w, const int *rank,
                                                                      const int *off, const float *sg, float *Y, int T,
                                                                      int H)
{
    const int t = blockIdx.x;
    int sl[8];
    float wt[8];
    pf_token_slots(ids, w, rank, off, t, sl, wt);
    const size_t shrow = (size_t)8 * T + t;
    /* the rows' scale exponents and the rows themselves in one round trip
     * (unrouted picks read the shared row, unused) */
    int ex[8];
#pragma unroll
    for (int k = 0; k < 8; k++) ex[k] = oexp[sl[k] >= 0 ? (size_t)sl[k] : shrow];
    const int exs = oexp[shrow];
    const int i = min((int)threadIdx.x * 8, H - 8);
    const uint4 s8 = *(const uint4 *)(ed + shrow * H + i);
    uint4 d8[8];
#pragma unroll
    for (int k = 0; k < 8; k++) d8[k] = *(const uint4 *)(ed + (sl[k] >= 0 ? (size_t)sl[k] : shrow) * H + i);
    const float g = __builtin_ldexpf(sg[t], exs);
#pragma unroll
    for (int k = 0; k < 8; k++)
        if (sl[k] >= 0) wt[k] = __builtin_ldexpf(wt[k], ex[k]);
    if ((int)threadIdx.x * 8 >= H) return;
    const f16x8_t sh = __builtin_bit_cast(f16x8_t, s8);
    float y[8];
#pragma unroll
    for (int c = 0; c < 8; c++) y[c] = g * (float)sh[c];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        if (sl[k] < 0) continue;
        const f16x8_t d = __builtin_bit_cast(f16x8_t, d8[k]);
#pragma unroll
        for (int c = 0; c < 8; c++) y[c] = fmaf(wt[k], (float)d[c], y[c]);
    }
    float4 *yo = (float4 *)(Y + (size_t)t * H + i);
    yo[0] = make_float4(y[0], y[1], y[2], y[3]);
    yo[1] = make_float4(y[4], y[5], y[6], y[7]);
}

/* ---- host ---------------------------------------------------------------- */
static inline size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

extern "C" int roaster_moe_prefill(RoasterTable *t, int layer, const float *X, int T, float *Y,
                                   const RoasterPrefillOpts *o)
{
    std::lock_guard<std::recursive_mutex> lk(rt_lock());
    if (rt_init_locked()) return ROASTER_EDEVICE;
    RoasterPrefillOpts opt;
    memset(&opt, 0, sizeof(opt));
    if (o) opt = *o;
    if (!t || layer < 0 || layer >= t->d.n_layers || !X || !Y || T < 1 || T > PF_MAX_T)
        return rt_fail(ROASTER_EINVAL, "roaster_moe_prefill: bad arguments (T must be 1..%d)", PF_MAX_T);
    if (opt.precision != ROASTER_PREC_F16 && opt.precision != ROASTER_PREC_SPLIT && opt.precision != ROASTER_PREC_BF16)
        return rt_fail(ROASTER_EINVAL, "roaster_moe_prefill: unknown precision %d", opt.precision);
    const int E = t->d.n_experts, H = (int)t->d.hidden, I = (int)t->d.inter;
    if (E > 256) return rt_fail(ROASTER_EINVAL, "roaster_moe_prefill: at most 256 routed experts");
    const int op = opt.precision == ROASTER_PREC_F16 ? PF_F16 : opt.precision == ROASTER_PREC_SPLIT ? PF_SPLIT : PF_BF16;
    const size_t TT = (size_t)T, slots = 9 * TT;
    const LayerGeo &LG = t->geo[layer];
    const int chunk = pf_gemm_chunk(op, LG.q6[0] != LG.q6[1] || LG.sh_q6[0] != LG.sh_q6[1]);
    const int max_tiles = (int)((8 * TT + chunk - 1) / chunk + E + (TT + chunk - 1) / chunk);

    /* workspace */
    size_t sz = 0;
    auto take = [&](size_t n) { const size_t at = sz; sz += align256(n); return at; };
    const size_t o_part = opt.logits_in ? 0 : take((size_t)RT_KSPLIT * TT * E * 4);
    const size_t o_ids = take(TT * 8 * 4), o_w = take(TT * 8 * 4), o_rank = take(TT * 8 * 4);
    const size_t o_sg = take(TT * 4), o_xinv = take(TT * 4), o_xfwd = take(TT * 4);
    const size_t o_x16 = op == PF_F16 ? take(TT * H * 2) : 0;
    const size_t o_cnt = take((size_t)E * 4), o_off = take((size_t)E * 4), o_list = take((size_t)E * TT * 4);
    const size_t o_grp = take(sizeof(PfGroup) * (E + 1)), o_tiles = take(sizeof(PfTile) * max_tiles);
    const size_t o_nt = take(4), o_pmax = take(slots * (size_t)(I / 16) * 4);
    const size_t o_act = take(slots * I * 4), o_ed = take((slots + 1) * H * (op == PF_F16 ? 2 : 4));
    const size_t o_oexp = op == PF_F16 ? take(slots) : 0;
    RtState &R = rt();
    const size_t o_bnd = op == PF_F16 ? take((size_t)(R.n_cu + 1) * 4) : 0;
    const size_t o_dnt = op == PF_F16 ? take(sizeof(PfDnTile) * max_tiles) : 0;
    const size_t o_fx = op == PF_F16 ? take((size_t)(32 + max_tiles) * 4) : 0;
    uint8_t *ws = (uint8_t *)rt_scratch(SCR_PF, sz);
    unsigned *ctrl = rt_ctrl();
    if (!ws || !ctrl) return ROASTER_ENOMEM;
    const DecLayer &L = t->layers_h[layer];

    if (!opt.logits_in) {
        dim3 g((T + RM_T - 1) / RM_T, (E + RM_E - 1) / RM_E, RT_KSPLIT);
        const size_t xlds = (size_t)RM_T * (H / RT_KSPLIT + 4) * 4;
        hipLaunchKernelGGL(pf_router_mfma_kernel, g, dim3(256), xlds, R.stream, X, L.router, (float *)(ws + o_part), T,
                           E, H);
        if (rt_check(hipGetLastError(), "prefill router launch")) return ROASTER_EDEVICE;
    }
    PfTokArgs ta;
    ta.X = X;
    ta.gate_inp = L.gate_inp;
    ta.part = opt.logits_in ? nullptr : (const float *)(ws + o_part);
    ta.logits_in = opt.logits_in;
    ta.bias = opt.logit_bias;
    ta.logits_out = opt.logits_out;
    ta.ids = (int *)(ws + o_ids);
    ta.w = (float *)(ws + o_w);
    ta.ids_out = opt.ids_out;
    ta.w_out = opt.w_out;
    ta.sg = (float *)(ws + o_sg);
    ta.xinv = op == PF_F16 ? (float *)(ws + o_xinv) : nullptr;
    ta.xfwd = op == PF_F16 ? (float *)(ws + o_xfwd) : nullptr;
    ta.x16 = op == PF_F16 ? (uint16_t *)(ws + o_x16) : nullptr;
    ta.err = (int *)(ctrl + 16);
    ta.T = T; ta.E = E; ta.H = H;
    hipLaunchKernelGGL(pf_token_kernel, dim3((T + 3) / 4), dim3(256), 0, R.stream, ta);
    if (rt_check(hipGetLastError(), "prefill token launch")) return ROASTER_EDEVICE;

    hipLaunchKernelGGL(pf_bucket_kernel, dim3(E), dim3(256), 0, R.stream, (const int *)(ws + o_ids), T,
                       (int *)(ws + o_list), (int *)(ws + o_rank), (int *)(ws + o_cnt));
    if (rt_check(hipGetLastError(), "prefill bucket launch")) return ROASTER_EDEVICE;

    PfPlanArgs pa;
    pa.L = L;
    pa.TL = t->tlayers_h[layer];
    pa.eb_g = LG.eb[0]; pa.eb_u = LG.eb[1]; pa.eb_d = LG.eb[2];
    pa.teb_g = LG.teb[0]; pa.teb_u = LG.teb[1]; pa.teb_d = LG.teb[2];
    pa.q6g = LG.q6[0]; pa.q6u = LG.q6[1]; pa.q6d = LG.q6[2];
    pa.sq6g = LG.sh_q6[0]; pa.sq6u = LG.sh_q6[1]; pa.sq6d = LG.sh_q6[2];
    pa.cnt = (const int *)(ws + o_cnt);
    pa.list = (const int *)(ws + o_list);
    pa.off = (int *)(ws + o_off);
    pa.counts_out = opt.counts_out;
    pa.groups = (PfGroup *)(ws + o_grp);
    pa.dbound = t->dbound + (size_t)layer * (E + 1);
    pa.tiles = (PfTile *)(ws + o_tiles);
    pa.ntiles = (int *)(ws + o_nt);
    pa.gu_ctr = (int *)(ws + o_nt) + 32;            /* its own cache line of the 256-byte slot */
    pa.dn_bnd = op == PF_F16 ? (int *)(ws + o_bnd) : nullptr;
    pa.dn_tiles = op == PF_F16 ? (PfDnTile *)(ws + o_dnt) : nullptr;
    /* both GEMMs in one persistent kernel: fp16 mode on the persistent gate/up
     * grid and the balanced down GEMM, 8 XCDs of equal CU counts */
    const int q6 = LG.q6[0];
    const bool gu_one = LG.q6[1] == q6 && LG.sh_q6[0] == q6 && LG.sh_q6[1] == q6;
    const int gu_pers = op == PF_F16 && gu_one && (H / 256) % 2 == 0 && H / 256 >= 8 ? 1 + q6 : 0;
    const bool fused = gu_pers && I <= 2 * GK && R.n_xcd == 8 && R.n_cu % 8 == 0 && pf_fused_enabled();
    pa.fx = fused ? (int *)(ws + o_fx) : nullptr;
    pa.n_wg = R.n_cu;
    pa.nt_out = H / PF_DN_ROWS;
    pa.T = T; pa.E = E;
    pa.chunk = chunk;
    hipLaunchKernelGGL(pf_plan_kernel, dim3(1), dim3(256), 0, R.stream, pa);
    if (rt_check(hipGetLastError(), "prefill plan launch")) return ROASTER_EDEVICE;

    PfGemmArgs ga;
    ga.groups = pa.groups;
    ga.tiles = pa.tiles;
    ga.ntiles = pa.ntiles;
    ga.X = X;
    ga.X16 = ta.x16;
    ga.xinv = ta.xinv;
    ga.xfwd = ta.xfwd;
    ga.act = (float *)(ws + o_act);
    ga.act16 = (uint16_t *)(ws + o_act);
    ga.pmax = op == PF_F16 ? (float *)(ws + o_pmax) : nullptr;
    /* fp16 mode: per-(token, expert) products in fp16, each row scaled by a
     * power of two of its bound (half the bytes of f32 rows, written by the
     * down GEMM and read back by the combine) */
    ga.out = op == PF_F16 ? nullptr : (float *)(ws + o_ed);
    ga.out16 = op == PF_F16 ? (uint16_t *)(ws + o_ed) : nullptr;
    ga.oexp = op == PF_F16 ? (int8_t *)(ws + o_oexp) : nullptr;
    ga.H = H; ga.I = I;
    ga.chunk = chunk;
    ga.dn_nt = 0;
    ga.dn_bnd = pa.dn_bnd;
    ga.dn_tiles = pa.dn_tiles;
    ga.dn_spare = (int)slots;                    /* o_ed holds one row past the slots */
    /* the persistent gate/up grid takes layers whose routed and shared gate
     * and up matrices share one type and whose K loop has an even number
     * (>= 8) of super-block steps */
    ga.gu_pers = gu_pers;
    ga.gu_ctr = pa.gu_ctr;
    ga.fused = fused ? 1 : 0;
    ga.xcd_tb = fused ? pa.fx : nullptr;
    ga.dn_ctr = fused ? pa.fx + 16 : nullptr;
    ga.tile_done = fused ? pa.fx + 32 : nullptr;
    ga.err = (int *)(ctrl + 16);
    if (int rc = pf_gemm_launch(ga, max_tiles, op)) return rc;

    if (op == PF_F16)
        hipLaunchKernelGGL(pf_combine16_kernel, dim3(T), dim3(256), 0, R.stream, (const uint16_t *)ga.out16,
                           (const int8_t *)ga.oexp, (const int *)ta.ids, (const float *)ta.w, (const int *)(ws + o_rank),
                           (const int *)pa.off, (const float *)ta.sg, Y, T, H);
    else
        hipLaunchKernelGGL(pf_combine_kernel, dim3(T), dim3(256), 0, R.stream, (const float *)ga.out,
                           (const int *)ta.ids, (const float *)ta.w, (const int *)(ws + o_rank), (const int *)pa.off,
                           (const float *)ta.sg, Y, T, H);
    return rt_check(hipGetLastError(), "prefill combine launch") ? ROASTER_EDEVICE : 0;
}
