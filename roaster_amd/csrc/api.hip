/*
 * api.hip -- the C-ABI: kernels.h entry points on host buffers and the
 * table-based decode entry points of roaster_moe.h.
 *
 * Host-buffer entry points follow the reference's contract (kernels.c): they
 * are synchronous, the caller owns every buffer, and weight pointers are
 * translated to their HBM copy.  Unlike the reference there is no CPU
 * fallback: a device failure is printed and reported through the return value
 * (or NaN outputs for signatures without one).
 */
#include "internal.h"
#include "decode.h"
#include "matvec.h"
#include "prefill.h"
#include "table.h"

#define PF_SPLIT_OP 1           /* gemm.h PF_SPLIT: bf16 hi + lo operands, 3 MFMAs, fp32 accumulation */
#define GEMM_ROWS 64            /* gemm.h GM / GN: rows per tile, output rows per block */
#define MM_MFMA_MIN_T 16        /* kernel_matmul_quant_batch jobs with at least this many tokens use MFMA */

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <vector>

typedef std::lock_guard<std::recursive_mutex> Guard;

static void fill_nan(float *p, size_t n)
{
    for (size_t i = 0; i < n; i++) p[i] = NAN;
}

/* ---- quantised matvec batch (split-phase) ---------------------------------- */
struct Pending {
    int open;
    const KernelMatvecJob *jobs;
    int n;
    std::vector<size_t> out_off;
    float *stage;            /* pinned copy of all outputs */
    int failed;
};
static Pending g_pend;

static int mv_upload_and_launch(const KernelMatvecJob *jobs, int n)
{
    RtState &R = rt();
    /* device layout: [vectors (deduplicated by pointer+cols)] [outputs] */
    std::vector<size_t> voff(n), ooff(n);
    std::vector<int> owner(n);
    size_t vtot = 0, otot = 0;
    for (int i = 0; i < n; i++) {
        const KernelMatvecJob &j = jobs[i];
        if (!j.matrix || !j.vector || !j.output || !j.rows || !j.cols || j.cols % RQK || j.rows > 0x7FFFFFFF)
            return rt_fail(ROASTER_EINVAL, "kernel_matvec_quant: invalid job %d (cols must be a multiple of 256)", i);
        owner[i] = i;
        for (int p = 0; p < i; p++)
            if (owner[p] == p && jobs[p].vector == j.vector && jobs[p].cols == j.cols) { owner[i] = p; break; }
        if (owner[i] == i) { voff[i] = vtot; vtot += (j.cols * 4 + 255) & ~(size_t)255; }
        else voff[i] = voff[owner[i]];
        ooff[i] = otot;
        otot += (j.rows * 4 + 255) & ~(size_t)255;
    }
    uint8_t *dv = (uint8_t *)rt_scratch(SCR_IN, vtot);
    uint8_t *dout = (uint8_t *)rt_scratch(SCR_OUT, otot);
    MvJob *djobs = (MvJob *)rt_scratch(SCR_A, sizeof(MvJob) * n);
    uint8_t *pin = (uint8_t *)rt_pinned(0, vtot + sizeof(MvJob) * n);
    float *stage = (float *)rt_pinned(1, otot);
    if (!dv || !dout || !djobs || !pin || !stage) return ROASTER_ENOMEM;
    std::vector<MvJob> hj(n);
    int tasks = 0;
    for (int i = 0; i < n; i++) {
        const KernelMatvecJob &j = jobs[i];
        const size_t bytes = rq_mat_bytes(j.is_q6, j.rows, j.cols);
        const uint8_t *W = (const uint8_t *)rt_weight_dev(j.matrix, bytes);
        if (!W) return ROASTER_EDEVICE;
        if (owner[i] == i) memcpy(pin + voff[i], j.vector, j.cols * 4);
        hj[i].W = W;
        hj[i].X = (const float *)(dv + voff[i]);
        hj[i].Y = (float *)(dout + ooff[i]);
        hj[i].rows = (int)j.rows;
        hj[i].cols = (int)j.cols;
        hj[i].T = 1;
        hj[i].q6 = j.is_q6 ? 1 : 0;
        hj[i].task0 = tasks;
        tasks += mv_tasks_for((int)j.rows, j.cols);
    }
    memcpy(pin + vtot, hj.data(), sizeof(MvJob) * n);
    if (rt_check(hipMemcpyAsync(dv, pin, vtot, hipMemcpyHostToDevice, R.stream), "vector upload") ||
        rt_check(hipMemcpyAsync(djobs, pin + vtot, sizeof(MvJob) * n, hipMemcpyHostToDevice, R.stream), "job upload"))
        return ROASTER_EDEVICE;
    int rc = mv_launch(djobs, n, tasks);
    if (rc) return rc;
    if (rt_check(hipMemcpyAsync(stage, dout, otot, hipMemcpyDeviceToHost, R.stream), "output download"))
        return ROASTER_EDEVICE;
    g_pend.out_off = ooff;
    g_pend.stage = stage;
    return 0;
}

extern "C" void kernel_matvec_quant_end(void)
{
    Guard g(rt_lock());
    if (!g_pend.open) return;
    g_pend.open = 0;
    int rc = g_pend.failed ? ROASTER_EDEVICE : rt_check(hipStreamSynchronize(rt().stream), "matvec sync");
    for (int i = 0; i < g_pend.n; i++) {
        const KernelMatvecJob &j = g_pend.jobs[i];
        if (rc) fill_nan(j.output, j.rows);
        else memcpy(j.output, (const uint8_t *)g_pend.stage + g_pend.out_off[i], j.rows * 4);
    }
}

extern "C" int kernel_matvec_quant_begin(const KernelMatvecJob *jobs, int n)
{
    Guard g(rt_lock());
    if (n <= 0 || !jobs) return 0;
    kernel_matvec_quant_end();
    if (rt_init_locked()) {
        for (int i = 0; i < n; i++) if (jobs[i].output) fill_nan(jobs[i].output, jobs[i].rows);
        return 0;
    }
    int rc = mv_upload_and_launch(jobs, n);
    g_pend.open = 1;
    g_pend.jobs = jobs;
    g_pend.n = n;
    g_pend.failed = rc != 0;
    return rc == 0;
}

extern "C" void kernel_matvec_quant_batch(const KernelMatvecJob *jobs, int n)
{
    Guard g(rt_lock());
    if (n <= 0) return;
    kernel_matvec_quant_begin(jobs, n);
    kernel_matvec_quant_end();
}

extern "C" void kernel_matvec_q4_k(const void *matrix, const float *vector, float *output, size_t rows, size_t cols)
{
    KernelMatvecJob j = { 0, matrix, vector, output, rows, cols };
    kernel_matvec_quant_batch(&j, 1);
}

extern "C" void kernel_matvec_q6_k(const void *matrix, const float *vector, float *output, size_t rows, size_t cols)
{
    KernelMatvecJob j = { 1, matrix, vector, output, rows, cols };
    kernel_matvec_quant_batch(&j, 1);
}

static float dot_quant(int q6, const void *w, const float *x, size_t n)
{
    if (n == 0) return 0.0f;
    if (n % RQK) {
        rt_fail(ROASTER_EINVAL, "kernel_dot_q%d_k: n = %zu is not a multiple of 256", q6 ? 6 : 4, n);
        return NAN;
    }
    float y = NAN;
    KernelMatvecJob j = { q6, w, x, &y, 1, n };
    kernel_matvec_quant_batch(&j, 1);
    return y;
}

extern "C" float kernel_dot_q4_k(const void *weights, const float *x, size_t n) { return dot_quant(0, weights, x, n); }
extern "C" float kernel_dot_q6_k(const void *weights, const float *x, size_t n) { return dot_quant(1, weights, x, n); }

/* ---- grouped GEMMs on MFMA for the host-buffer entry points ------------------
 * Tile lists and group tables for pf_gemm (prefill.h) built on the host and
 * uploaded through pinned staging: one group per expert (or per matmul job),
 * its rows consecutive in X, D and the intermediate buffer. */
struct GemmWs { PfGroup *groups; PfTile *tiles; int *ntiles; int nt; };

static int gemm_ws(const std::vector<PfGroup> &hg, GemmWs &W)
{
    std::vector<PfTile> ht;
    for (int i = 0; i < (int)hg.size(); i++)
        for (int m0 = 0; m0 < hg[i].n; m0 += GEMM_ROWS) ht.push_back(PfTile{ i, m0 });
    W.nt = (int)ht.size();
    const size_t gb = (sizeof(PfGroup) * hg.size() + 255) & ~(size_t)255, tb = (sizeof(PfTile) * ht.size() + 255) & ~(size_t)255;
    uint8_t *dev = (uint8_t *)rt_scratch(SCR_E, gb + tb + 256);
    uint8_t *pin = (uint8_t *)rt_pinned(2, gb + tb + 256);
    if (!dev || !pin) return ROASTER_ENOMEM;
    if (rt_check(hipStreamSynchronize(rt().stream), "staging wait")) return ROASTER_EDEVICE;   /* pin is reused */
    memcpy(pin, hg.data(), sizeof(PfGroup) * hg.size());
    memcpy(pin + gb, ht.data(), sizeof(PfTile) * ht.size());
    memcpy(pin + gb + tb, &W.nt, sizeof(int));
    if (rt_check(hipMemcpyAsync(dev, pin, gb + tb + 256, hipMemcpyHostToDevice, rt().stream), "tile list upload"))
        return ROASTER_EDEVICE;
    W.groups = (PfGroup *)dev;
    W.tiles = (PfTile *)(dev + gb);
    W.ntiles = (int *)(dev + gb + tb);
    return 0;
}

/* Y[t * rows + r] = W[r] . X[t] on device buffers (rows a multiple of 64). */
int matmul_mfma(const uint8_t *W, int q6, const float *X, float *Y, size_t rows, size_t cols, size_t T)
{
    std::vector<PfGroup> hg(1);
    memset(hg.data(), 0, sizeof(PfGroup));
    hg[0].d = W;
    hg[0].dq6 = q6;
    hg[0].n = (int)T;
    GemmWs ws;
    if (int rc = gemm_ws(hg, ws)) return rc;
    PfGemmArgs ga;
    memset(&ga, 0, sizeof(ga));
    ga.groups = ws.groups;
    ga.tiles = ws.tiles;
    ga.ntiles = ws.ntiles;
    ga.act = (float *)X;
    ga.out = Y;
    ga.H = (int)rows;
    ga.I = (int)cols;
    ga.chunk = GEMM_ROWS;
    return pf_matmul_launch(ga, ws.nt);
}

/* ---- multi-token matmul ---------------------------------------------------- */
static int mm_valid(const KernelMatmulJob *j)
{
    return j->matrix && j->X && j->Y && j->rows && j->cols && j->T && (j->cols % RQK) == 0 &&
           j->rows <= 0x7FFFFFFF && j->cols <= 0x7FFFFFFF && j->T <= 0x7FFFFFFF;
}

extern "C" int kernel_matmul_quant_batch(const KernelMatmulJob *jobs, int n)
{
    Guard g(rt_lock());
    if (!jobs || n < 0) return -1;
    for (int i = 0; i < n; i++)
        if (!mm_valid(&jobs[i])) return -1;
    if (n == 0) return 0;
    kernel_matvec_quant_end();
    if (rt_init_locked()) return -1;
    RtState &R = rt();
    std::vector<size_t> xoff(n), yoff(n);
    std::vector<int> owner(n);
    size_t xt = 0, yt = 0;
    for (int i = 0; i < n; i++) {
        const KernelMatmulJob &j = jobs[i];
        owner[i] = i;
        for (int p = 0; p < i; p++)
            if (owner[p] == p && jobs[p].X == j.X && jobs[p].cols == j.cols && jobs[p].T == j.T) { owner[i] = p; break; }
        if (owner[i] == i) { xoff[i] = xt; xt += (j.T * j.cols * 4 + 255) & ~(size_t)255; }
        else xoff[i] = xoff[owner[i]];
        yoff[i] = yt;
        yt += (j.T * j.rows * 4 + 255) & ~(size_t)255;
    }
    uint8_t *dx = (uint8_t *)rt_scratch(SCR_IN, xt);
    uint8_t *dy = (uint8_t *)rt_scratch(SCR_OUT, yt);
    MvJob *dj = (MvJob *)rt_scratch(SCR_A, sizeof(MvJob) * n);
    if (!dx || !dy || !dj) return -1;
    std::vector<MvJob> hj(n);
    int tasks = 0;
    for (int i = 0; i < n; i++) {
        const KernelMatmulJob &j = jobs[i];
        const uint8_t *W = (const uint8_t *)rt_weight_dev(j.matrix, rq_mat_bytes(j.is_q6, j.rows, j.cols));
        if (!W) return -1;
        if (owner[i] == i &&
            rt_check(hipMemcpyAsync(dx + xoff[i], j.X, j.T * j.cols * 4, hipMemcpyHostToDevice, R.stream), "X upload"))
            return -1;
        const bool big = j.T >= MM_MFMA_MIN_T && j.rows % GEMM_ROWS == 0;
        if (!big && (int)j.T >= dense_mfma_min_tokens() && j.cols <= 4096) {
            /* a few tokens: the quants-on-MFMA product, eight tokens per launch */
            for (size_t t0 = 0; t0 < j.T; t0 += 8)
                if (dense_mm8_launch(W, j.is_q6 ? 1 : 0, (const float *)(dx + xoff[i]) + t0 * j.cols,
                                     (float *)(dy + yoff[i]) + t0 * j.rows, j.rows, j.cols,
                                     (int)(j.T - t0 < 8 ? j.T - t0 : 8)))
                    return -1;
            hj[i] = MvJob{ W, (const float *)(dx + xoff[i]), (float *)(dy + yoff[i]), 0, (int)j.cols, 0, j.is_q6 ? 1 : 0,
                           tasks };
            continue;
        }
        if (big) {
            /* split-operand MFMA GEMM (the down GEMM of the prefill path as a
             * plain product); the job keeps a zero-task slot in the matvec launch */
            if (matmul_mfma(W, j.is_q6 ? 1 : 0, (const float *)(dx + xoff[i]), (float *)(dy + yoff[i]), j.rows, j.cols,
                            j.T))
                return -1;
            hj[i] = MvJob{ W, (const float *)(dx + xoff[i]), (float *)(dy + yoff[i]), 0, (int)j.cols, 0, j.is_q6 ? 1 : 0,
                           tasks };
            continue;
        }
        hj[i] = MvJob{ W, (const float *)(dx + xoff[i]), (float *)(dy + yoff[i]), (int)j.rows, (int)j.cols, (int)j.T,
                       j.is_q6 ? 1 : 0, tasks };
        tasks += mv_tasks_for((int)j.rows, j.cols);
    }
    if (rt_check(hipMemcpyAsync(dj, hj.data(), sizeof(MvJob) * n, hipMemcpyHostToDevice, R.stream), "job upload"))
        return -1;
    if (tasks && mv_launch(dj, n, tasks)) return -1;
    for (int i = 0; i < n; i++)
        if (rt_check(hipMemcpyAsync(jobs[i].Y, dy + yoff[i], jobs[i].T * jobs[i].rows * 4, hipMemcpyDeviceToHost,
                                    R.stream), "Y download"))
            return -1;
    return rt_check(hipStreamSynchronize(R.stream), "matmul sync") ? -1 : 0;
}

/* ---- prefill MoE on host buffers (kernels.c:2198-2214) --------------------
 * The expert row groups as the prefill path's grouped GEMMs on MFMA: gate/up
 * with the SiLU*up epilogue, then down, in split mode (bf16 hi + lo operands,
 * three MFMAs per product block, fp32 accumulation: about 5e-6 of max|D|,
 * inside the 2e-4 of the reference's own test, test_kernels.c:31), reading
 * the weights' HBM copies in their GGML layout. */
static int moe_groups_mfma(const KernelMoeExpert *ex, int na, const float *dx, float *dd, size_t inter, size_t hidden,
                           size_t total)
{
    std::vector<PfGroup> hg(na);
    size_t row = 0;
    for (int i = 0; i < na; i++) {
        const KernelMoeExpert &e = ex[i];
        PfGroup &G = hg[i];
        memset(&G, 0, sizeof(G));
        G.g = (const uint8_t *)rt_weight_dev(e.gate, rq_mat_bytes(e.gate_q6, inter, hidden));
        G.u = (const uint8_t *)rt_weight_dev(e.up, rq_mat_bytes(e.up_q6, inter, hidden));
        G.d = (const uint8_t *)rt_weight_dev(e.down, rq_mat_bytes(e.down_q6, hidden, inter));
        if (!G.g || !G.u || !G.d) return ROASTER_EDEVICE;
        G.gq6 = e.gate_q6 ? 1 : 0;
        G.uq6 = e.up_q6 ? 1 : 0;
        G.dq6 = e.down_q6 ? 1 : 0;
        G.n = (int)e.n;
        G.slot0 = (int)row;
        G.tok0 = (int)row;
        row += e.n;
    }
    float *act = (float *)rt_scratch(SCR_B, total * inter * 4);
    if (!act) return ROASTER_ENOMEM;
    GemmWs ws;
    if (int rc = gemm_ws(hg, ws)) return rc;
    PfGemmArgs ga;
    memset(&ga, 0, sizeof(ga));
    ga.groups = ws.groups;
    ga.tiles = ws.tiles;
    ga.ntiles = ws.ntiles;
    ga.X = dx;
    ga.act = act;
    ga.out = dd;
    ga.H = (int)hidden;
    ga.I = (int)inter;
    ga.chunk = GEMM_ROWS;
    return pf_gemm_launch(ga, ws.nt, PF_SPLIT_OP);
}

int prefill_groups_device(const KernelMoeExpert *ex, int na, const float *X, float *D, size_t inter, size_t hidden,
                          size_t total);

extern "C" int kernel_moe_prefill(const KernelMoeExpert *ex, int count, const float *X, float *D, size_t inter,
                                  size_t hidden)
{
    Guard g(rt_lock());
    if (!ex || count < 0 || !X || !D || !inter || !hidden || (inter % RQK) || (hidden % RQK)) return -1;
    std::vector<KernelMoeExpert> act;
    size_t total = 0;
    for (int i = 0; i < count; i++) {
        if (!ex[i].gate || !ex[i].up || !ex[i].down) return -1;
        if (ex[i].n) { act.push_back(ex[i]); total += ex[i].n; }
    }
    if (!total) return 0;
    kernel_matvec_quant_end();
    if (rt_init_locked()) return -1;
    RtState &R = rt();
    float *dx = (float *)rt_scratch(SCR_IN, total * hidden * 4);
    float *dd = (float *)rt_scratch(SCR_OUT, total * hidden * 4);
    if (!dx || !dd) return -1;
    if (rt_check(hipMemcpyAsync(dx, X, total * hidden * 4, hipMemcpyHostToDevice, R.stream), "X upload")) return -1;
    if (moe_groups_mfma(act.data(), (int)act.size(), dx, dd, inter, hidden, total)) return -1;
    if (rt_check(hipMemcpyAsync(D, dd, total * hidden * 4, hipMemcpyDeviceToHost, R.stream), "D download")) return -1;
    return rt_check(hipStreamSynchronize(R.stream), "prefill sync") ? -1 : 0;
}

/* Expert row groups on device buffers with the matvec kernel: gate and up of
 * every group in one launch, SiLU*up, then every down in one launch. */
int prefill_groups_device(const KernelMoeExpert *ex, int na, const float *dx, float *dd, size_t inter, size_t hidden,
                          size_t total)
{
    RtState &R = rt();
    float *gu = (float *)rt_scratch(SCR_B, 2 * total * inter * 4);
    MvJob *dj = (MvJob *)rt_scratch(SCR_A, sizeof(MvJob) * 2 * na);
    if (!gu || !dj) return ROASTER_ENOMEM;
    float *G = gu, *U = gu + total * inter;
    std::vector<MvJob> hj;
    int tasks = 0;
    size_t row = 0;
    for (int i = 0; i < na; i++) {
        const KernelMoeExpert &e = ex[i];
        const uint8_t *gw = (const uint8_t *)rt_weight_dev(e.gate, rq_mat_bytes(e.gate_q6, inter, hidden));
        const uint8_t *uw = (const uint8_t *)rt_weight_dev(e.up, rq_mat_bytes(e.up_q6, inter, hidden));
        if (!gw || !uw) return ROASTER_EDEVICE;
        hj.push_back(MvJob{ gw, dx + row * hidden, G + row * inter, (int)inter, (int)hidden, (int)e.n, e.gate_q6 ? 1 : 0, tasks });
        tasks += mv_tasks_for((int)inter, hidden);
        hj.push_back(MvJob{ uw, dx + row * hidden, U + row * inter, (int)inter, (int)hidden, (int)e.n, e.up_q6 ? 1 : 0, tasks });
        tasks += mv_tasks_for((int)inter, hidden);
        row += e.n;
    }
    std::vector<MvJob> hd;
    int dtasks = 0;
    row = 0;
    for (int i = 0; i < na; i++) {
        const KernelMoeExpert &e = ex[i];
        const uint8_t *dw = (const uint8_t *)rt_weight_dev(e.down, rq_mat_bytes(e.down_q6, hidden, inter));
        if (!dw) return ROASTER_EDEVICE;
        hd.push_back(MvJob{ dw, G + row * inter, dd + row * hidden, (int)hidden, (int)inter, (int)e.n, e.down_q6 ? 1 : 0, dtasks });
        dtasks += mv_tasks_for((int)hidden, inter);
        row += e.n;
    }
    MvJob *djd = (MvJob *)rt_scratch(SCR_C, sizeof(MvJob) * na);
    if (!djd) return ROASTER_ENOMEM;
    if (rt_check(hipMemcpyAsync(dj, hj.data(), sizeof(MvJob) * hj.size(), hipMemcpyHostToDevice, R.stream), "jobs") ||
        rt_check(hipMemcpyAsync(djd, hd.data(), sizeof(MvJob) * hd.size(), hipMemcpyHostToDevice, R.stream), "jobs"))
        return ROASTER_EDEVICE;
    int rc = mv_launch(dj, (int)hj.size(), tasks);
    if (!rc) rc = silu_mul_launch(G, U, total * inter);
    if (!rc) rc = mv_launch(djd, (int)hd.size(), dtasks);
    if (!rc) rc = rt_check(hipStreamSynchronize(R.stream), "groups sync");   /* host job vectors go out of scope */
    return rc;
}

/* ---- fused decode experts (kernels.c:1703-1830) ---------------------------- */
extern "C" int kernel_ffn_fused(const KernelFfnExpert *ex, int n, const float *x, size_t inter, size_t hidden)
{
    Guard g(rt_lock());
    if (!ex || !x || n <= 0 || n > 9) return 0;
    if (!inter || !hidden || (inter & 255u) || (hidden & 255u)) return 0;
    if (inter > 2048 || hidden > 2048) return 0;     /* one wave pass per row: <= 8 super-blocks */
    kernel_matvec_quant_end();
    if (rt_init_locked()) return 0;
    RtState &R = rt();
    DecActive hx[9];
    memset(hx, 0, sizeof(hx));
    for (int i = 0; i < n; i++) {
        if (!ex[i].gate || !ex[i].up || !ex[i].down || !ex[i].out) return 0;
        hx[i].g = (const uint8_t *)rt_weight_dev(ex[i].gate, rq_mat_bytes(ex[i].gate_q6, inter, hidden));
        hx[i].u = (const uint8_t *)rt_weight_dev(ex[i].up, rq_mat_bytes(ex[i].up_q6, inter, hidden));
        hx[i].d = (const uint8_t *)rt_weight_dev(ex[i].down, rq_mat_bytes(ex[i].down_q6, hidden, inter));
        if (!hx[i].g || !hx[i].u || !hx[i].d) return 0;
        hx[i].gq6 = ex[i].gate_q6 ? 1 : 0;
        hx[i].uq6 = ex[i].up_q6 ? 1 : 0;
        hx[i].dq6 = ex[i].down_q6 ? 1 : 0;
    }
    float *dx = (float *)rt_scratch(SCR_IN, hidden * 4);
    float *dout = (float *)rt_scratch(SCR_OUT, (size_t)n * hidden * 4);
    float *eh = (float *)rt_scratch(SCR_B, 9 * inter * 4);
    DecActive *dex = (DecActive *)rt_scratch(SCR_A, sizeof(hx));
    /* pinned staging: x then the expert table (one upload), then the outputs
     * (one download); pageable copies cost a bounce each */
    const size_t xo = (hidden * 4 + 255) & ~(size_t)255, oo = xo + ((sizeof(hx) + 255) & ~(size_t)255);
    uint8_t *pin = (uint8_t *)rt_pinned(3, oo + (size_t)n * hidden * 4);
    if (!dx || !dout || !eh || !dex || !pin) return 0;
    memcpy(pin, x, hidden * 4);
    memcpy(pin + xo, hx, sizeof(hx));
    if (rt_check(hipMemcpyAsync(dx, pin, hidden * 4, hipMemcpyHostToDevice, R.stream), "x upload") ||
        rt_check(hipMemcpyAsync(dex, pin + xo, sizeof(hx), hipMemcpyHostToDevice, R.stream), "expert upload"))
        return 0;
    DecArgs A;
    memset(&A, 0, sizeof(A));
    A.H = (int)hidden;
    A.I = (int)inter;
    A.B = 1;
    A.nlayers = 1;
    A.h = dx;
    A.eh = eh;
    A.ffn_ex = dex;
    A.ffn_n = n;
    A.ffn_out = dout;
    if (dec_ffn_launch(A)) return 0;
    if (rt_check(hipMemcpyAsync(pin + oo, dout, (size_t)n * hidden * 4, hipMemcpyDeviceToHost, R.stream), "out download"))
        return 0;
    if (rt_take_err()) return 0;     /* synchronises the stream */
    for (int i = 0; i < n; i++) memcpy(ex[i].out, pin + oo + (size_t)i * hidden * 4, hidden * 4);
    return 1;
}

/* ---- table-based decode ---------------------------------------------------- */
static void fill_table_args(DecArgs &A, const RoasterTable *t)
{
    memset(&A, 0, sizeof(A));
    A.layers = t->layers_d;
    A.layers_h = t->layers_h.data();
    A.E = t->d.n_experts;
    A.H = (int)t->d.hidden;
    A.I = (int)t->d.inter;
}

static int dec_scratch(DecArgs &A)
{
    const size_t E = (size_t)A.E, B = (size_t)A.B;
    A.logits = (float *)rt_scratch(SCR_D, B * E * 4);
    A.sgate_raw = (float *)rt_scratch(SCR_E, B * 4);
    A.eh = (float *)rt_scratch(SCR_F, B * 9 * (size_t)A.I * 4);
    A.xn_g = (float *)rt_scratch(SCR_B, B * ((size_t)A.H + A.H / 16) * 4);
    if ((dec_layer1_ok(A.E, A.H, A.I, A.B) || dec_layerB_ok(A.E, A.H, A.I, A.B)) && !(A.xbuf = dec_xch_default(A.E, A.H, A.I))) return ROASTER_ENOMEM;
    return A.logits && A.sgate_raw && A.eh && A.xn_g ? 0 : ROASTER_ENOMEM;
}

extern "C" int roaster_moe_decode(RoasterTable *t, int layer, const float *x, int B, float *y,
                                  const RoasterDecodeIO *io)
{
    Guard g(rt_lock());
    if (rt_init_locked()) return ROASTER_EDEVICE;
    if (!t || !x || !y || B < 1 || B > RMAX_B || layer < 0 || layer >= t->d.n_layers)
        return rt_fail(ROASTER_EINVAL, "roaster_moe_decode: bad arguments");
    DecArgs A;
    fill_table_args(A, t);
    A.layer0 = layer;
    A.nlayers = 1;
    A.B = B;
    A.h = (float *)x;
    A.y = y;
    A.do_norm = 0;
    if (io) {
        A.logits_in = io->logits_in;
        A.ids_out = io->ids_out;
        A.w_out = io->w_out;
    }
    if (dec_scratch(A)) return ROASTER_ENOMEM;
    int rc = dec_launch(A);
    if (rc) return rc;
    if (io && io->logits_out) {
        const float *src = A.logits_in ? A.logits_in : A.logits;
        if (rt_check(hipMemcpyAsync(io->logits_out, src, (size_t)B * A.E * 4, hipMemcpyDeviceToDevice, rt().stream),
                     "logits copy"))
            return ROASTER_EDEVICE;
    }
    return 0;
}

extern "C" int roaster_moe_decode_stack(RoasterTable *t, float *h, int B, int layer0, int n_layers,
                                        const float *norm_w, float eps, int *ids_out, float *w_out)
{
    Guard g(rt_lock());
    if (rt_init_locked()) return ROASTER_EDEVICE;
    if (!t || !h || B < 1 || B > RMAX_B || layer0 < 0 || n_layers < 1 || layer0 + n_layers > t->d.n_layers)
        return rt_fail(ROASTER_EINVAL, "roaster_moe_decode_stack: bad arguments");
    DecArgs A;
    fill_table_args(A, t);
    A.layer0 = layer0;
    A.nlayers = n_layers;
    A.B = B;
    A.h = h;
    A.y = NULL;
    A.norm_w = norm_w;
    A.eps = eps;
    A.do_norm = 1;
    A.ids_out = ids_out;
    A.w_out = w_out;
    if (dec_scratch(A)) return ROASTER_ENOMEM;
    return dec_launch(A);
}

extern "C" const char *roaster_decode_stack_kernel(RoasterTable *t, int B, int layer0, int n_layers)
{
    Guard g(rt_lock());
    if (rt_init_locked()) return "";
    if (!t || B < 1 || B > RMAX_B || layer0 < 0 || n_layers < 1 || layer0 + n_layers > t->d.n_layers) return "";
    DecArgs A;
    fill_table_args(A, t);
    A.layer0 = layer0;
    A.nlayers = n_layers;
    A.B = B;
    return dec_kernel_names(A);
}

/* ---- the layer stack without allocation -------------------------------------
 * roaster_moe_decode_stack_noalloc runs the kernels of roaster_moe_decode_stack
 * with every intermediate (error word, plan, logits, shared-gate logits,
 * SiLU*up rows, normalised input) in one file-scope device array instead of
 * the library's grow-only scratch, so that a caller that cannot allocate
 * device memory can call it.  In host code `scratch` names a host-side
 * stand-in, not the device array: its device address is looked up once per
 * device at initialisation (noalloc_setup) and only that address is used. */
#define NOALLOC_BYTES (576u << 10)
static __device__ __align__(256) uint8_t scratch[NOALLOC_BYTES];

#define NOALLOC_MAX_DEV 64
static uint8_t *g_noalloc[NOALLOC_MAX_DEV];      /* device address of `scratch` per device */

int noalloc_setup(int dev)
{
    if (dev < 0 || dev >= NOALLOC_MAX_DEV) return rt_fail(ROASTER_EDEVICE, "device index %d out of range", dev);
    if (g_noalloc[dev]) return 0;
    void *p = NULL;
    if (rt_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)")) return ROASTER_EDEVICE;
    g_noalloc[dev] = (uint8_t *)p;
    rt_set_aux_err((int *)p);        /* the error word is the array's first int */
    return 0;
}

static size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }

extern "C" int roaster_moe_decode_stack_noalloc(RoasterTable *t, float *h, int B, int layer0, int n_layers,
                                                const float *norm_w, float eps, int *ids_out, float *w_out)
{
    Guard g(rt_lock());
    if (rt_init_locked()) return ROASTER_EDEVICE;
    if (!t || !h || B < 1 || B > RMAX_B || layer0 < 0 || n_layers < 1 || layer0 + n_layers > t->d.n_layers)
        return rt_fail(ROASTER_EINVAL, "roaster_moe_decode_stack_noalloc: bad arguments");
    uint8_t *base = g_noalloc[rt().device];
    if (!base) return rt_fail(ROASTER_EDEVICE, "roaster_moe_decode_stack_noalloc: scratch address not set up");
    DecArgs A;
    fill_table_args(A, t);
    const size_t E = (size_t)A.E, Bz = (size_t)B, H = (size_t)A.H, I = (size_t)A.I;
    const size_t o_plan = 256, o_log = o_plan + al256(sizeof(DecPlan)), o_sg = o_log + al256(Bz * E * 4),
                 o_eh = o_sg + al256(Bz * 4), o_xn = o_eh + al256(Bz * 9 * I * 4), o_x = o_xn + al256(Bz * (H + H / 16) * 4);
    /* one token runs the one-launch kernel when its exchange slots fit behind
     * the intermediates, else three kernels per layer */
    const bool one = dec_layer1_ok(A.E, A.H, A.I, B) && o_x + al256(dec_xch_need1(A.E, A.H, A.I) * 8) <= NOALLOC_BYTES;
    const size_t end = o_x + (one ? al256(dec_xch_need1(A.E, A.H, A.I) * 8) : 0);
    if (end > NOALLOC_BYTES)
        return rt_fail(ROASTER_EINVAL,
                       "roaster_moe_decode_stack_noalloc: %d tokens x hidden %zu x inter %zu x %zu experts need %zu "
                       "scratch bytes, above the %u-byte maximum",
                       B, H, I, E, end, NOALLOC_BYTES);
    A.layer0 = layer0;
    A.nlayers = n_layers;
    A.B = B;
    A.h = h;
    A.y = NULL;
    A.norm_w = norm_w;
    A.eps = eps;
    A.do_norm = 1;
    A.ids_out = ids_out;
    A.w_out = w_out;
    A.err = (int *)base;
    A.cnt = (uint32_t *)(base + 64);     /* the one-token kernel's completion counter */
    rt_aux_err_used();
    A.plan_g = (DecPlan *)(base + o_plan);
    A.logits = (float *)(base + o_log);
    A.sgate_raw = (float *)(base + o_sg);
    A.eh = (float *)(base + o_eh);
    A.xn_g = (float *)(base + o_xn);
    /* The exchange slots keep their own epoch counter; the array was
     * zero-filled at load.  Its bytes past o_x are the exchange of the shape
     * that last ran the one-launch kernel; any other call (another shape, or
     * the three-kernel path of 2-8 tokens) may store plain intermediates there,
     * whose bits could later match an epoch: then the region is cleared by a
     * fill kernel (no allocation) and epochs start again. */
    static DecXch xb[NOALLOC_MAX_DEV];
    static uint64_t xkey[NOALLOC_MAX_DEV];   /* shape of the last call that ran the one-launch kernel; 0: none or dirty */
    DecXch &X = xb[rt().device];
    const uint64_t key = one ? (E << 44) ^ (H << 24) ^ (I << 4) ^ 1u : 0u;
    if (one) {
        X.p = (uint64_t *)(base + o_x);
        X.n = dec_xch_need1(A.E, A.H, A.I);
        if (xkey[rt().device] != key && dec_xch_clear(X)) return ROASTER_EDEVICE;
        A.xbuf = &X;
    }
    xkey[rt().device] = key;
    return dec_launch(A);
}

/* ---- f32 router matvec (kernels.c:131-148) -------------------------------- */
static int up(void *d, const void *s, size_t n)
{
    return rt_check(hipMemcpyAsync(d, s, n, hipMemcpyHostToDevice, rt().stream), "upload");
}

static int down_sync(void *d, const void *s, size_t n)
{
    if (rt_check(hipMemcpyAsync(d, s, n, hipMemcpyDeviceToHost, rt().stream), "download")) return -1;
    return rt_check(hipStreamSynchronize(rt().stream), "sync");
}

extern "C" void kernel_matvec_f32(const float *matrix, const float *vector, float *output, size_t rows, size_t cols)
{
    Guard g(rt_lock());
    if (!rows) return;
    kernel_matvec_quant_end();
    const float *W = rt_init_locked() ? NULL : (const float *)rt_weight_dev(matrix, rows * cols * 4);
    float *dx = (float *)rt_scratch(SCR_IN, cols * 4 + 16);
    float *dy = (float *)rt_scratch(SCR_OUT, rows * 4 + 16);
    if (!W || !dx || !dy || up(dx, vector, cols * 4) || matvec_f32_launch(W, dx, dy, rows, cols) ||
        down_sync(output, dy, rows * 4))
        fill_nan(output, rows);
}

/* ---- per-call helpers that stay on the host --------------------------------
 * The reference runs these on the CPU (kernels.c:102-129, 584-720): each call
 * touches a few kilobytes (one attention head, one conv state, one embedding
 * row), less than one PCIe round trip would cost, and model.c calls some of
 * them per head and per KV position (model.c:838, 1580).  They are plain host
 * code of this library; nothing of the MoE path runs here. */
extern "C" float kernel_dot_f32(const float *a, const float *b, size_t n)
{
    float acc[16] = { 0 };
    size_t i = 0;
    for (; i + 16 <= n; i += 16)
        for (int l = 0; l < 16; l++) acc[l] = fmaf(a[i + l], b[i + l], acc[l]);
    for (int w = 8; w >= 1; w >>= 1)
        for (int l = 0; l < w; l++) acc[l] += acc[l + w];
    float s = acc[0];
    for (; i < n; i++) s = fmaf(a[i], b[i], s);
    return s;
}

static float sum_squares(const float *x, size_t n)
{
    float acc[16] = { 0 };
    size_t i = 0;
    for (; i + 16 <= n; i += 16)
        for (int l = 0; l < 16; l++) acc[l] = fmaf(x[i + l], x[i + l], acc[l]);
    for (int w = 8; w >= 1; w >>= 1)
        for (int l = 0; l < w; l++) acc[l] += acc[l + w];
    float s = acc[0];
    for (; i < n; i++) s = fmaf(x[i], x[i], s);
    return s;
}

/* y = x * (1 / sqrt(mean(x^2) + eps)) * w   (kernels.c:584-605) */
extern "C" void kernel_rmsnorm(float *output, const float *input, const float *weight, size_t n, float epsilon)
{
    if (!n) return;
    const float inv = 1.0f / sqrtf(sum_squares(input, n) / (float)n + epsilon);
    for (size_t i = 0; i < n; i++) output[i] = input[i] * inv * weight[i];
}

/* y = x / sqrt(sum(x^2) + eps)   (kernels.c:607-622) */
extern "C" void kernel_l2norm(float *output, const float *input, size_t n, float epsilon)
{
    if (!n) return;
    const float inv = 1.0f / sqrtf(sum_squares(input, n) + epsilon);
    for (size_t i = 0; i < n; i++) output[i] = input[i] * inv;
}

/* Scalar activations with the reference's two-branch sigmoid (kernels.c:628-642). */
extern "C" float kernel_sigmoid(float x)
{
    if (x >= 0.0f) { float z = expf(-x); return 1.0f / (1.0f + z); }
    float z = expf(x);
    return z / (1.0f + z);
}

extern "C" float kernel_silu(float x) { return x * kernel_sigmoid(x); }

extern "C" void kernel_silu_array(float *x, size_t n)
{
    for (size_t i = 0; i < n; i++) x[i] = kernel_silu(x[i]);
}

static float h2f(uint16_t h)
{
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
    uint32_t b;
    if (e == 0) {
        if (!m) b = s;
        else {                                           /* subnormal: m * 2^-24 */
            float f = ldexpf((float)m, -24);
            memcpy(&b, &f, 4);
            b |= s;
        }
    } else if (e == 31) b = s | 0x7F800000u | (m << 13);
    else b = s | ((e + 112) << 23) | (m << 13);
    float f;
    memcpy(&f, &b, 4);
    return f;
}

/* One token row of a Q4_K table dequantised (kernels.c:660-690): sub-block j
 * of a super-block has scale d*sc_j and offset dmin*m_j, the 6-bit sc / m
 * unpacked from the 12 scale bytes (kernels.c:154-173). */
extern "C" void kernel_embedding_row_q4_k(const void *weights, size_t token_id, float *output, size_t hidden_size)
{
    if (!hidden_size) return;
    if (hidden_size % RQK) {
        rt_fail(ROASTER_EINVAL, "embedding row: hidden not a multiple of 256");
        fill_nan(output, hidden_size);
        return;
    }
    const size_t nb = hidden_size / RQK;
    const uint8_t *row = (const uint8_t *)weights + token_id * nb * RQ4K_BYTES;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = row + b * RQ4K_BYTES;
        uint16_t hd, hm;
        memcpy(&hd, blk, 2);
        memcpy(&hm, blk + 2, 2);
        const float d = h2f(hd), dmin = h2f(hm);
        const uint8_t *sb = blk + 4, *qs = blk + 16;
        float *o = output + b * RQK;
        for (int j = 0; j < 8; j++) {
            int sc, mn;
            if (j < 4) { sc = sb[j] & 63; mn = sb[j + 4] & 63; }
            else { sc = (sb[j + 4] & 15) | ((sb[j - 4] >> 6) << 4); mn = (sb[j + 4] >> 4) | ((sb[j] >> 6) << 4); }
            const float s = d * (float)sc, m = dmin * (float)mn;
            const uint8_t *q = qs + 32 * (j / 2);
            const int sh = (j & 1) * 4;
            for (int i = 0; i < 32; i++) o[32 * j + i] = s * (float)((q[i] >> sh) & 15) - m;
        }
    }
}

/* out[c] = sum_k history[k][c] * kernel[c][k] + input[c] * kernel[c][K-1]
 * (kernels.c:693-720): one causal step of a depthwise convolution. */
extern "C" void kernel_conv1d_causal_f32(const float *input, const float *history, const float *kernel, float *output,
                                         size_t channels, size_t kernel_size)
{
    if (!kernel_size) return;
    const size_t K = kernel_size;
    for (size_t c = 0; c < channels; c++) {
        float s = 0.0f;
        for (size_t k = 0; k + 1 < K; k++) s += history[k * channels + c] * kernel[c * K + k];
        s += input[c] * kernel[c * K + K - 1];
        output[c] = s;
    }
}
