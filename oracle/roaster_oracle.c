/*
 * roaster_oracle.c -- CPU restatement of the reference's MoE-FFN CPU path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product): loaded by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg, nothing else.
 *
 * The reference computes its dots with 8-lane AVX2 vectors.  This file keeps
 * the same arithmetic as plain scalar code over an explicit 8-lane array: every
 * lane does the same multiply / fused multiply-add sequence, and horizontal sums
 * follow the reference's shuffle order.  Build with -ffp-contract=off so the
 * compiler fuses nothing beyond the explicit fmaf() calls; the fmaf() calls sit
 * exactly where gcc -O3 -mfma fuses the reference's expressions.
 */
#include "roaster_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define L8 8

/* kernels.c:56-96.  F16C conversion is exact; so is this bit-level one
 * (subnormals are mantissa * 2^-24, which is exact in f32). */
float orc_fp16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t ex = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (ex == 0) {
        float v = (float)man * 0x1p-24f;
        return sign ? -v : v;
    } else if (ex == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((ex + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* kernels.c:154-173: six-bit scale / min unpack of the 12 packed bytes at +4. */
void orc_q4k_scales(const uint8_t *blk, int sc[8], int mn[8])
{
    const uint8_t *s = blk + 4;
    for (int j = 0; j < 4; j++) {
        sc[j] = s[j] & 63;
        mn[j] = s[j + 4] & 63;
    }
    for (int j = 4; j < 8; j++) {
        sc[j] = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        mn[j] = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* hsum256 (kernels.c:224-232): ((v0+v4)+(v2+v6)) + ((v1+v5)+(v3+v7)). */
static float hsum8(const float v[L8])
{
    float a0 = v[0] + v[4], a1 = v[1] + v[5], a2 = v[2] + v[6], a3 = v[3] + v[7];
    float b0 = a0 + a2, b1 = a1 + a3;
    return b0 + b1;
}

/* kernels.c:102-129: two 8-lane FMA accumulators over 16-float steps, lane-wise
 * add, horizontal sum, then a scalar fused tail. */
float orc_dot_f32(const float *a, const float *b, size_t n)
{
    float s0[L8] = {0}, s1[L8] = {0};
    size_t i = 0;
    for (; i + 16 <= n; i += 16)
        for (int l = 0; l < L8; l++) {
            s0[l] = fmaf(a[i + l], b[i + l], s0[l]);
            s1[l] = fmaf(a[i + 8 + l], b[i + 8 + l], s1[l]);
        }
    for (int l = 0; l < L8; l++) s0[l] = s0[l] + s1[l];
    float sum = hsum8(s0);
    for (; i < n; i++) sum = fmaf(a[i], b[i], sum);
    return sum;
}

/* kernels.c:131-148 */
void orc_matvec_f32(const float *W, const float *x, float *y, size_t rows, size_t cols)
{
    for (size_t r = 0; r < rows; r++) y[r] = orc_dot_f32(W + r * cols, x, cols);
}

/* kernels.c:246-288: folded Q4_K row dot,
 *   total += d*sc * sum(q*x) - dmin*m * sum(x)   per 32-weight sub-block,
 * where lane l of the 8-lane vectors covers columns l, l+8, l+16, l+24. */
static float dot_q4k_row(const uint8_t *blocks, const float *x, size_t nb)
{
    float total[L8] = {0};
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = blocks + b * ORC_Q4K_BYTES;
        const uint8_t *qs = blk + 16;
        const float *xb = x + b * ORC_QK;
        float d = orc_fp16_to_f32(rd16(blk)), dmin = orc_fp16_to_f32(rd16(blk + 2));
        int sc[8], mn[8];
        orc_q4k_scales(blk, sc, mn);
        for (int g = 0; g < 4; g++) {
            const uint8_t *q = qs + 32 * g;
            const float *xl = xb + 64 * g, *xh = xl + 32;
            float sql[L8], sqh[L8], sxl[L8], sxh[L8];
            for (int l = 0; l < L8; l++) {
                float v = (float)(q[l] & 15) * xl[l];
                v = fmaf((float)(q[8 + l] & 15), xl[8 + l], v);
                v = fmaf((float)(q[16 + l] & 15), xl[16 + l], v);
                v = fmaf((float)(q[24 + l] & 15), xl[24 + l], v);
                sql[l] = v;
                float h = (float)(q[l] >> 4) * xh[l];
                h = fmaf((float)(q[8 + l] >> 4), xh[8 + l], h);
                h = fmaf((float)(q[16 + l] >> 4), xh[16 + l], h);
                h = fmaf((float)(q[24 + l] >> 4), xh[24 + l], h);
                sqh[l] = h;
                sxl[l] = (xl[l] + xl[8 + l]) + (xl[16 + l] + xl[24 + l]);
                sxh[l] = (xh[l] + xh[8 + l]) + (xh[16 + l] + xh[24 + l]);
            }
            float ds0 = d * (float)sc[2 * g], dm0 = dmin * (float)mn[2 * g];
            float ds1 = d * (float)sc[2 * g + 1], dm1 = dmin * (float)mn[2 * g + 1];
            for (int l = 0; l < L8; l++) {
                float t = fmaf(ds0, sql[l], total[l]);
                t = fmaf(-dm0, sxl[l], t);
                t = fmaf(ds1, sqh[l], t);
                total[l] = fmaf(-dm1, sxh[l], t);
            }
        }
    }
    return hsum8(total);
}

/* kernels.c:290-342: Q6_K row dot.  For half n, q1..q4 are the 32-byte vectors
 * (ql[l] lo | qh[l] bits 0-1), (ql[l+32] lo | bits 2-3), (ql[l] hi | bits 4-5),
 * (ql[l+32] hi | bits 6-7), each minus 32; q6_accum splits each into two 16-wide
 * halves with their own int8 scale. */
static void q6_half(float total[L8], const int8_t q[32], const float *xp, float d, int s0, int s1)
{
    float v0[L8], v1[L8];
    for (int l = 0; l < L8; l++) {
        v0[l] = fmaf((float)q[8 + l], xp[8 + l], (float)q[l] * xp[l]);
        v1[l] = fmaf((float)q[24 + l], xp[24 + l], (float)q[16 + l] * xp[16 + l]);
    }
    float a = d * (float)s0, c = d * (float)s1;
    for (int l = 0; l < L8; l++) {
        float t = fmaf(a, v0[l], total[l]);
        total[l] = fmaf(c, v1[l], t);
    }
}

static float dot_q6k_row(const uint8_t *blocks, const float *x, size_t nb)
{
    float total[L8] = {0};
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = blocks + b * ORC_Q6K_BYTES;
        const uint8_t *ql = blk, *qh = blk + 128;
        const int8_t *sc = (const int8_t *)(blk + 192);
        const float d = orc_fp16_to_f32(rd16(blk + 208));
        const float *xb = x + b * ORC_QK;
        for (int n = 0; n < 2; n++) {
            int8_t q1[32], q2[32], q3[32], q4[32];
            for (int l = 0; l < 32; l++) {
                q1[l] = (int8_t)(((ql[l] & 15) | ((qh[l] & 3) << 4)) - 32);
                q2[l] = (int8_t)(((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32);
                q3[l] = (int8_t)(((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
                q4[l] = (int8_t)(((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
            }
            const float *xs = xb + n * 128;
            q6_half(total, q1, xs, d, sc[0], sc[1]);
            q6_half(total, q2, xs + 32, d, sc[2], sc[3]);
            q6_half(total, q3, xs + 64, d, sc[4], sc[5]);
            q6_half(total, q4, xs + 96, d, sc[6], sc[7]);
            ql += 64; qh += 32; sc += 8;
        }
    }
    return hsum8(total);
}

float orc_dot_q4k(const void *row, const float *x, size_t n)
{
    if (n % ORC_QK) return NAN;   /* partial blocks: not on the path (rejected) */
    return dot_q4k_row((const uint8_t *)row, x, n / ORC_QK);
}

float orc_dot_q6k(const void *row, const float *x, size_t n)
{
    if (n % ORC_QK) return NAN;
    return dot_q6k_row((const uint8_t *)row, x, n / ORC_QK);
}

/* kernels.c:407-432, 553-578 */
void orc_matvec_q4k(const void *W, const float *x, float *y, size_t rows, size_t cols)
{
    const size_t rb = cols / ORC_QK * ORC_Q4K_BYTES;
    for (size_t r = 0; r < rows; r++) y[r] = orc_dot_q4k((const uint8_t *)W + r * rb, x, cols);
}

void orc_matvec_q6k(const void *W, const float *x, float *y, size_t rows, size_t cols)
{
    const size_t rb = cols / ORC_QK * ORC_Q6K_BYTES;
    for (size_t r = 0; r < rows; r++) y[r] = orc_dot_q6k((const uint8_t *)W + r * rb, x, cols);
}

void orc_matvec_quant(int q6, const void *W, const float *x, float *y, size_t rows, size_t cols)
{
    if (q6) orc_matvec_q6k(W, x, y, rows, cols);
    else    orc_matvec_q4k(W, x, y, rows, cols);
}

/* kernels.c:1839-1853: w = (d*sc)*q - dmin*m, fused as one multiply-subtract. */
void orc_dequant_q4k_block(const void *blk_, float *o)
{
    const uint8_t *blk = (const uint8_t *)blk_;
    float d = orc_fp16_to_f32(rd16(blk)), dmin = orc_fp16_to_f32(rd16(blk + 2));
    int sc[8], mn[8];
    orc_q4k_scales(blk, sc, mn);
    for (int g = 0; g < 4; g++) {
        const uint8_t *q = blk + 16 + 32 * g;
        float s0 = d * (float)sc[2 * g], m0 = dmin * (float)mn[2 * g];
        float s1 = d * (float)sc[2 * g + 1], m1 = dmin * (float)mn[2 * g + 1];
        for (int i = 0; i < 32; i++) {
            o[64 * g + i] = fmaf(s0, (float)(q[i] & 15), -m0);
            o[64 * g + 32 + i] = fmaf(s1, (float)(q[i] >> 4), -m1);
        }
    }
}

/* kernels.c:1855-1874: w = (d*sc)*q, two roundings. */
void orc_dequant_q6k_block(const void *blk_, float *o)
{
    const uint8_t *blk = (const uint8_t *)blk_;
    const float d = orc_fp16_to_f32(rd16(blk + 208));
    const uint8_t *ql = blk, *qh = blk + 128;
    const int8_t *sc = (const int8_t *)(blk + 192);
    for (int n = 0; n < ORC_QK; n += 128) {
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = ((ql[l] & 15) | ((qh[l] & 3) << 4)) - 32;
            int q2 = ((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32;
            int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            o[n + l] = d * (float)sc[is] * (float)q1;
            o[n + l + 32] = d * (float)sc[is + 2] * (float)q2;
            o[n + l + 64] = d * (float)sc[is + 4] * (float)q3;
            o[n + l + 96] = d * (float)sc[is + 6] * (float)q4;
        }
        ql += 64; qh += 32; sc += 8;
    }
}

/* kernels.c:1876-1914: per (row, token) the block-by-block sum of 256-wide
 * f32 dots of the dequantised block against the token's slice. */
void orc_matmul_quant(int q6, const void *W, const float *X, float *Y,
                      size_t rows, size_t cols, size_t T)
{
    const size_t bpr = cols / ORC_QK, bs = q6 ? ORC_Q6K_BYTES : ORC_Q4K_BYTES;
    float w[ORC_QK];
    float *acc = (float *)calloc(T ? T : 1, sizeof(float));
    if (!acc) return;
    for (size_t r = 0; r < rows; r++) {
        memset(acc, 0, T * sizeof(float));
        for (size_t b = 0; b < bpr; b++) {
            const uint8_t *blk = (const uint8_t *)W + (r * bpr + b) * bs;
            if (q6) orc_dequant_q6k_block(blk, w);
            else    orc_dequant_q4k_block(blk, w);
            for (size_t t = 0; t < T; t++)
                acc[t] = acc[t] + orc_dot_f32(w, X + t * cols + b * ORC_QK, ORC_QK);
        }
        for (size_t t = 0; t < T; t++) Y[t * rows + r] = acc[t];
    }
    free(acc);
}

/* kernels.c:584-605: serial fused sum of squares, then x * inv_rms * w. */
void orc_rmsnorm(float *out, const float *in, const float *w, size_t n, float eps)
{
    float ss = 0.0f;
    for (size_t i = 0; i < n; i++) ss = fmaf(in[i], in[i], ss);
    float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (size_t i = 0; i < n; i++) out[i] = in[i] * inv * w[i];
}

/* model.c:869-897: insertion into a descending top-8 with strict '>' (the
 * earlier, lower index wins ties; NaN never enters), then softmax over the
 * eight selected logits. */
void orc_select_top8(const float *logits, int n, int ids[8], float w[8])
{
    for (int i = 0; i < ORC_TOPK; i++) { ids[i] = -1; w[i] = -INFINITY; }
    for (int e = 0; e < n; e++) {
        float v = logits[e];
        int p = ORC_TOPK;
        for (int i = 0; i < ORC_TOPK; i++)
            if (v > w[i]) { p = i; break; }
        if (p == ORC_TOPK) continue;
        for (int j = ORC_TOPK - 1; j > p; j--) { w[j] = w[j - 1]; ids[j] = ids[j - 1]; }
        w[p] = v;
        ids[p] = e;
    }
    float mx = w[0], sum = 0.0f;
    for (int i = 0; i < ORC_TOPK; i++) { w[i] = expf(w[i] - mx); sum = sum + w[i]; }
    float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    for (int i = 0; i < ORC_TOPK; i++) w[i] = w[i] * inv;
}

static float silu_mul(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

/* model.c:1108-1133 */
void orc_expert_decode(const OrcExpert *e, const float *x, size_t inter, size_t hidden, float *out)
{
    float *g = (float *)malloc(2 * inter * sizeof(float));
    if (!g) return;
    float *u = g + inter;
    orc_matvec_quant(e->gate_q6, e->gate, x, g, inter, hidden);
    orc_matvec_quant(e->up_q6, e->up, x, u, inter, hidden);
    for (size_t i = 0; i < inter; i++) g[i] = silu_mul(g[i], u[i]);
    orc_matvec_quant(e->down_q6, e->down, g, out, hidden, inter);
    free(g);
}

/* model.c:1059-1146 */
int orc_moe_decode(const OrcLayer *L, const float *x, const float *logits_in,
                   float *y, float *logits, int ids_out[8], float w_out[8])
{
    const size_t H = L->hidden, I = L->inter;
    const int E = L->n_experts;
    float *lg = (float *)malloc((size_t)E * sizeof(float));
    float *d = (float *)malloc((ORC_TOPK + 1) * H * sizeof(float));
    int ids[8];
    float w[8];
    int rc = -1;
    if (!lg || !d) goto out;
    if (logits_in) memcpy(lg, logits_in, (size_t)E * sizeof(float));
    else orc_matvec_f32(L->router, x, lg, (size_t)E, H);
    if (logits) memcpy(logits, lg, (size_t)E * sizeof(float));
    orc_select_top8(lg, E, ids, w);
    if (ids_out) memcpy(ids_out, ids, sizeof(ids));
    if (w_out) memcpy(w_out, w, sizeof(w));
    for (int k = 0; k < ORC_TOPK; k++)
        if (ids[k] < 0 || ids[k] >= E) goto out;
    for (int k = 0; k < ORC_TOPK; k++) orc_expert_decode(&L->experts[ids[k]], x, I, H, d + k * H);
    orc_expert_decode(&L->shared, x, I, H, d + ORC_TOPK * H);
    float raw = orc_dot_f32(L->shexp_gate_inp, x, H);
    float sg = 1.0f / (1.0f + expf(-raw));
    for (size_t i = 0; i < H; i++) y[i] = 0.0f;
    for (int k = 0; k < ORC_TOPK; k++)
        for (size_t i = 0; i < H; i++) y[i] = fmaf(w[k], d[k * H + i], y[i]);
    for (size_t i = 0; i < H; i++) y[i] = fmaf(sg, d[ORC_TOPK * H + i], y[i]);
    rc = 0;
out:
    free(lg);
    free(d);
    return rc;
}

/* kernels.c:2176-2196 */
void orc_moe_groups(const OrcMoeGroup *ex, int count, const float *X, float *D,
                    size_t inter, size_t hidden)
{
    size_t maxn = 0;
    for (int i = 0; i < count; i++) if (ex[i].n > maxn) maxn = ex[i].n;
    float *g = (float *)malloc(2 * (maxn ? maxn : 1) * inter * sizeof(float));
    if (!g) return;
    float *u = g + maxn * inter;
    size_t row = 0;
    for (int i = 0; i < count; i++) {
        size_t n = ex[i].n;
        if (!n) continue;
        orc_matmul_quant(ex[i].gate_q6, ex[i].gate, X + row * hidden, g, inter, hidden, n);
        orc_matmul_quant(ex[i].up_q6, ex[i].up, X + row * hidden, u, inter, hidden, n);
        for (size_t k = 0; k < n * inter; k++) g[k] = silu_mul(g[k], u[k]);
        orc_matmul_quant(ex[i].down_q6, ex[i].down, g, D + row * hidden, hidden, inter, n);
        row += n;
    }
    free(g);
}

/* model.c:1713-1731 */
void orc_bucket(const int *ids, int T, int E, int *cnt, int *off, int *lt, int *lk)
{
    for (int e = 0; e < E; e++) cnt[e] = 0;
    for (int i = 0; i < T * ORC_TOPK; i++) cnt[ids[i]]++;
    off[0] = 0;
    for (int e = 0; e < E; e++) off[e + 1] = off[e] + cnt[e];
    int *fill = (int *)malloc((size_t)E * sizeof(int));
    if (!fill) return;
    for (int e = 0; e < E; e++) fill[e] = off[e];
    for (int t = 0; t < T; t++)
        for (int k = 0; k < ORC_TOPK; k++) {
            int e = ids[t * ORC_TOPK + k], pos = fill[e]++;
            lt[pos] = t;
            lk[pos] = k;
        }
    free(fill);
}

/* model.c:1671-1791 (expert batching does not change any value: each expert's
 * rows are computed independently and scattered in expert-ascending order). */
int orc_moe_prefill(const OrcLayer *L, const float *X, int T, const float *logits_in,
                    const float *logit_bias, float *Y, int *ids_out, float *w_out, float *logits_out)
{
    const size_t H = L->hidden, I = L->inter;
    const int E = L->n_experts;
    int rc = -1;
    float *rl = (float *)malloc((size_t)T * E * sizeof(float));
    int *ids = (int *)malloc((size_t)T * ORC_TOPK * sizeof(int));
    float *wts = (float *)malloc((size_t)T * ORC_TOPK * sizeof(float));
    float *sg = (float *)malloc((size_t)T * I * sizeof(float));
    float *su = (float *)malloc((size_t)T * I * sizeof(float));
    float *sd = (float *)malloc((size_t)T * H * sizeof(float));
    int *cnt = (int *)malloc((size_t)E * sizeof(int));
    int *off = (int *)malloc(((size_t)E + 1) * sizeof(int));
    int *lt = (int *)malloc((size_t)T * ORC_TOPK * sizeof(int));
    int *lk = (int *)malloc((size_t)T * ORC_TOPK * sizeof(int));
    float *xg = NULL, *ed = NULL;
    if (!rl || !ids || !wts || !sg || !su || !sd || !cnt || !off || !lt || !lk) goto out;

    for (int t = 0; t < T; t++) {
        float *l = rl + (size_t)t * E;
        if (logits_in) memcpy(l, logits_in + (size_t)t * E, (size_t)E * sizeof(float));
        else orc_matvec_f32(L->router, X + (size_t)t * H, l, (size_t)E, H);
        if (logit_bias)
            for (int e = 0; e < E; e++) l[e] = l[e] + logit_bias[e];
        orc_select_top8(l, E, ids + t * ORC_TOPK, wts + t * ORC_TOPK);
        for (int k = 0; k < ORC_TOPK; k++)
            if (ids[t * ORC_TOPK + k] < 0 || ids[t * ORC_TOPK + k] >= E) goto out;
    }
    if (logits_out) memcpy(logits_out, rl, (size_t)T * E * sizeof(float));
    if (ids_out) memcpy(ids_out, ids, (size_t)T * ORC_TOPK * sizeof(int));
    if (w_out) memcpy(w_out, wts, (size_t)T * ORC_TOPK * sizeof(float));

    /* shared expert for all tokens (model.c:1694-1711) */
    orc_matmul_quant(L->shared.gate_q6, L->shared.gate, X, sg, I, H, (size_t)T);
    orc_matmul_quant(L->shared.up_q6, L->shared.up, X, su, I, H, (size_t)T);
    for (size_t i = 0; i < (size_t)T * I; i++) sg[i] = silu_mul(sg[i], su[i]);
    orc_matmul_quant(L->shared.down_q6, L->shared.down, sg, sd, H, I, (size_t)T);
    for (int t = 0; t < T; t++) {
        float raw = orc_dot_f32(L->shexp_gate_inp, X + (size_t)t * H, H);
        float g = 1.0f / (1.0f + expf(-raw));
        for (size_t i = 0; i < H; i++) Y[(size_t)t * H + i] = g * sd[(size_t)t * H + i];
    }

    orc_bucket(ids, T, E, cnt, off, lt, lk);
    size_t maxn = 0;
    for (int e = 0; e < E; e++) if ((size_t)cnt[e] > maxn) maxn = (size_t)cnt[e];
    xg = (float *)malloc((maxn ? maxn : 1) * H * sizeof(float));
    ed = (float *)malloc((maxn ? maxn : 1) * H * sizeof(float));
    if (!xg || !ed) goto out;
    for (int e = 0; e < E; e++) {
        const int n = cnt[e];
        if (!n) continue;
        for (int a = 0; a < n; a++)
            memcpy(xg + (size_t)a * H, X + (size_t)lt[off[e] + a] * H, H * sizeof(float));
        const OrcExpert *ex = &L->experts[e];
        OrcMoeGroup grp = { ex->gate, ex->up, ex->down, ex->gate_q6, ex->up_q6, ex->down_q6, (size_t)n };
        orc_moe_groups(&grp, 1, xg, ed, I, H);
        for (int a = 0; a < n; a++) {
            const int t = lt[off[e] + a], k = lk[off[e] + a];
            const float wt = wts[t * ORC_TOPK + k];
            float *dst = Y + (size_t)t * H;
            const float *src = ed + (size_t)a * H;
            for (size_t i = 0; i < H; i++) dst[i] = fmaf(wt, src[i], dst[i]);
        }
    }
    rc = 0;
out:
    free(rl); free(ids); free(wts); free(sg); free(su); free(sd);
    free(cnt); free(off); free(lt); free(lk); free(xg); free(ed);
    return rc;
}
