/*
 * matvec.hip -- multi-job quantised matvec / small-T matmul and the small
 * vector kernels behind kernels.h.
 *
 * Reference: kernel_matvec_quant_batch (kernels.c:1582-1646: all jobs of a call
 * in one submit), kernel_matmul_quant_batch (kernels.c:1916-2069,
 * Y[t*rows + r] = dot(W[r], X[t])), and the CPU vector kernels
 * (kernels.c:102-148, 584-719).
 *
 * One wave serves a task = (job, group of rows).  Lane layout per row:
 * lpr = lanes_per_row(blocks) lanes (qdot.h), 8 per 256-weight super-block
 * (qdot.h); each lane's quant chunk is loaded once and applied to all T tokens.
 */
#include "internal.h"
#include "qdot.h"
#include "matvec.h"

#define MV_THREADS 256

template <bool Q6>
__device__ __forceinline__ void matvec_task(const MvJob &J, int task, int lane)
{
    const int nb = J.cols / RQK;
    const int lpr = lanes_per_row(nb), rpw = 64 / lpr;
    const int rw = lane / lpr, lr = lane % lpr, c = lr & 7, lb = lr >> 3;
    const int row = (task - J.task0) * rpw + rw;
    const bool live = row < J.rows;
    const size_t bs = Q6 ? RQ6K_BYTES : RQ4K_BYTES;
    const uint8_t *wrow = J.W + (size_t)(live ? row : 0) * nb * bs;
    for (int t = 0; t < J.T; t++) {
        const float *x = J.X + (size_t)t * J.cols;
        float part = 0.0f;
        for (int b = lb; live && b < nb; b += 8) {
            QChunk ch = q_load<Q6>(wrow + (size_t)b * bs, c);
            const int ca = b * RQK + q_run_a<Q6>(c), cb = ca + q_run_b_off<Q6>();
            part += q_chunk_dot<Q6>(ch, c, x + ca, x + cb, sum16(x + ca), sum16(x + cb));
        }
        part = group_sum_w(part, lpr);
        if (live && lr == 0) J.Y[(size_t)t * J.rows + row] = part;
    }
}

__global__ void __launch_bounds__(MV_THREADS) matvec_jobs_kernel(const MvJob *jobs, int njobs, int ntasks)
{
    const int lane = threadIdx.x & 63;
    const int gw = blockIdx.x * (MV_THREADS / 64) + (threadIdx.x >> 6), nw = gridDim.x * (MV_THREADS / 64);
    for (int task = gw; task < ntasks; task += nw) {
        int j = 0;
        while (j + 1 < njobs && jobs[j + 1].task0 <= task) j++;
        const MvJob J = jobs[j];
        if (J.q6) matvec_task<true>(J, task, lane);
        else matvec_task<false>(J, task, lane);
    }
}

/* ---- dense projections on device buffers ---------------------------------
 * y[t][r] = W[r] . x[t] for a [rows x cols] Q4_K / Q6_K matrix and T <= 8
 * tokens: the dense projections around the MoE block and the LM head
 * (model.c:795-800, 1284-1290, 1344-1347, 1368-1370; the same products
 * tensor_matvec_f32_or_quant, model.c:113-121, sends to kernel_matvec_q*_k).
 * cols <= 2048, so one lane group covers a whole row (8 lanes per
 * super-block, lanes_per_row(blocks) lanes per row, 64 / lpr rows per wave pass).
 * Each lane's activation runs are fixed for every row it serves: with one
 * token they sit in registers for the whole kernel, with more in LDS.  Every
 * wave keeps DMV_PF row passes' loads in flight before it computes them. */
#ifndef DMV_PF
#define DMV_PF 2                           /* row passes in flight per wave */
#endif
#ifndef DMV_GRID
#define DMV_GRID 8                         /* workgroups per CU at most */
#endif

static int g_dense_mfma_t = 9;             /* no call reaches it until measured to pay off */
int matmul_mfma(const uint8_t *W, int q6, const float *X, float *Y, size_t rows, size_t cols, size_t T);   /* api.hip */

template <bool Q6, bool ONE, int KB>
__global__ void __launch_bounds__(MV_THREADS) dense_mv_kernel(const uint8_t *W, const float *X, float *Y, int rows,
                                                              int cols, int T)
{
    extern __shared__ __align__(16) float xs[];            /* [T][cols] + run sums [T][cols / 16] (T > 1) */
    const int lane = threadIdx.x & 63;
    const int nb = cols / RQK, lpr = lanes_per_row(nb), rpw = 64 / lpr;
    const int rw = lane / lpr, lr = lane % lpr, c = lr & 7, lb = lr >> 3;
    const size_t bs = Q6 ? RQ6K_BYTES : RQ4K_BYTES, row_bytes = (size_t)nb * bs;
    /* KB super-blocks per lane: lb, lb + 8 (rows of more than 8 blocks) */
    bool blk_live[KB];
    int ca[KB], cb[KB];
#pragma unroll
    for (int k = 0; k < KB; k++) {
        blk_live[k] = lb + 8 * k < nb;
        ca[k] = (lb + 8 * k) * RQK + q_run_a<Q6>(c);
        cb[k] = ca[k] + q_run_b_off<Q6>();
    }
    float4 xa[KB][4], xb[KB][4];
    float sxa[KB], sxb[KB];
    float *xsum = xs + (size_t)T * cols;
    if (ONE) {
#pragma unroll
        for (int k = 0; k < KB; k++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                xa[k][i] = blk_live[k] ? gld_f4(X + ca[k] + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
                xb[k][i] = blk_live[k] ? gld_f4(X + cb[k] + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
            sxa[k] = ((xa[k][0].x + xa[k][0].y) + (xa[k][0].z + xa[k][0].w)) + ((xa[k][1].x + xa[k][1].y) + (xa[k][1].z + xa[k][1].w)) +
                     (((xa[k][2].x + xa[k][2].y) + (xa[k][2].z + xa[k][2].w)) + ((xa[k][3].x + xa[k][3].y) + (xa[k][3].z + xa[k][3].w)));
            sxb[k] = ((xb[k][0].x + xb[k][0].y) + (xb[k][0].z + xb[k][0].w)) + ((xb[k][1].x + xb[k][1].y) + (xb[k][1].z + xb[k][1].w)) +
                     (((xb[k][2].x + xb[k][2].y) + (xb[k][2].z + xb[k][2].w)) + ((xb[k][3].x + xb[k][3].y) + (xb[k][3].z + xb[k][3].w)));
        }
    } else {
        for (int i = threadIdx.x; i < T * cols / 4; i += MV_THREADS) ((float4 *)xs)[i] = gld_f4(X + 4 * i);
        __syncthreads();
        for (int i = threadIdx.x; i < T * cols / 16; i += MV_THREADS) xsum[i] = sum16(xs + 16 * i);
        __syncthreads();
    }
    const int gw = blockIdx.x * (MV_THREADS / 64) + (threadIdx.x >> 6), nw = gridDim.x * (MV_THREADS / 64);
    const int npass = (rows + rpw - 1) / rpw;
    for (int p0 = gw; p0 < npass; p0 += nw * DMV_PF) {
        QChunk ch[DMV_PF][KB];
#pragma unroll
        for (int f = 0; f < DMV_PF; f++) {
            const int row = (p0 + f * nw) * rpw + rw;
#pragma unroll
            for (int k = 0; k < KB; k++)
                if (blk_live[k] && row < rows)
                    ch[f][k] = q_load<Q6>(W + (size_t)row * row_bytes + (size_t)(lb + 8 * k) * bs, c);
        }
#pragma unroll
        for (int f = 0; f < DMV_PF; f++) {
            const int pass = p0 + f * nw;
            if (pass >= npass) break;
            const int row = pass * rpw + rw;
            const bool live = row < rows;
            for (int t = 0; t < (ONE ? 1 : T); t++) {
                float part = 0.0f;
#pragma unroll
                for (int k = 0; k < KB; k++) {
                    if (live && blk_live[k]) {
                        if (ONE) {
                            part += q_chunk_dot_r<Q6>(ch[f][k], c, xa[k], xb[k], sxa[k], sxb[k]);
                        } else {
                            const float *x = xs + (size_t)t * cols, *sx = xsum + (size_t)t * (cols / 16);
                            part += q_chunk_dot<Q6>(ch[f][k], c, x + ca[k], x + cb[k], sx[ca[k] >> 4], sx[cb[k] >> 4]);
                        }
                    }
                }
                part = group_sum_w(part, lpr);
                if (live && lr == 0) Y[(size_t)t * rows + row] = part;
            }
        }
    }
}

/* eh = (g / (1 + exp(-g))) * u over n elements (kernels.c:2191, model.c:1124). */
__global__ void silu_mul_kernel(float *g, const float *u, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const float a = g[i];
        g[i] = (a / (1.0f + expf(-a))) * u[i];
    }
}

/* f32 matvec rows (kernel_matvec_f32 / kernel_dot_f32): one wave per row. */
__global__ void __launch_bounds__(MV_THREADS) matvec_f32_kernel(const float *W, const float *x, float *y, size_t rows,
                                                                size_t cols)
{
    const int lane = threadIdx.x & 63;
    const size_t gw = (size_t)blockIdx.x * (MV_THREADS / 64) + (threadIdx.x >> 6);
    const size_t nw = (size_t)gridDim.x * (MV_THREADS / 64);
    for (size_t r = gw; r < rows; r += nw) {
        const float *row = W + r * cols;
        float acc = 0.0f;
        for (size_t i = lane; i < cols; i += 64) acc = fmaf(row[i], x[i], acc);
        acc = group_sum<64>(acc);
        if (lane == 0) y[r] = acc;
    }
}

/* ---- host launchers ------------------------------------------------------- */
int mv_launch(const MvJob *jobs_dev, int njobs, int ntasks)
{
    if (ntasks <= 0) return 0;
    const int wpb = MV_THREADS / 64;
    int blocks = (ntasks + wpb - 1) / wpb;
    if (blocks > 8 * rt().n_cu) blocks = 8 * rt().n_cu;
    hipLaunchKernelGGL(matvec_jobs_kernel, dim3(blocks), dim3(MV_THREADS), 0, rt().stream, jobs_dev, njobs, ntasks);
    return rt_check(hipGetLastError(), "matvec launch") ? ROASTER_EDEVICE : 0;
}

int mv_tasks_for(int rows, size_t cols)
{
    const int nb = (int)(cols / RQK);
    const int lpr = lanes_per_row(nb);
    const int rpw = 64 / lpr;
    return (rows + rpw - 1) / rpw;
}

extern "C" int roaster_matvec_q(const void *W, int q6, const float *X, float *Y, size_t rows, size_t cols, int T)
{
    std::lock_guard<std::recursive_mutex> g(rt_lock());
    if (rt_init_locked()) return ROASTER_EDEVICE;
    if (!W || !X || !Y || !rows || !cols || cols % RQK || cols > 4096 || T < 1 || T > 8 || rows > (size_t)INT32_MAX)
        return rt_fail(ROASTER_EINVAL, "roaster_matvec_q: need cols a multiple of 256 and <= 4096, 1 <= T <= 8");
    if (T >= g_dense_mfma_t && rows % 64 == 0)           /* several tokens: the split-operand MFMA GEMM */
        return matmul_mfma((const uint8_t *)W, q6 ? 1 : 0, X, Y, rows, cols, (size_t)T);
    const int nb = (int)(cols / RQK), rpw = 64 / lanes_per_row(nb);
    const size_t npass = (rows + rpw - 1) / rpw;
    size_t blocks = (npass + 3) / 4;
    if (blocks > (size_t)DMV_GRID * rt().n_cu) blocks = (size_t)DMV_GRID * rt().n_cu;
    const size_t lds = T > 1 ? (size_t)T * cols * 4 + (size_t)T * (cols / 16) * 4 : 0;
    const dim3 gd((unsigned)blocks), bd(MV_THREADS);
    const uint8_t *w = (const uint8_t *)W;
    const int r = (int)rows, cc = (int)cols;
#define DMV(Q6_, ONE_, KB_) hipLaunchKernelGGL((dense_mv_kernel<Q6_, ONE_, KB_>), gd, bd, ONE_ ? 0 : lds, rt().stream, w, X, Y, r, cc, T)
    if (nb <= 8) {
        if (q6 && T == 1) DMV(true, true, 1);
        else if (q6) DMV(true, false, 1);
        else if (T == 1) DMV(false, true, 1);
        else DMV(false, false, 1);
    } else {
        if (q6 && T == 1) DMV(true, true, 2);
        else if (q6) DMV(true, false, 2);
        else if (T == 1) DMV(false, true, 2);
        else DMV(false, false, 2);
    }
#undef DMV
    return rt_check(hipGetLastError(), "dense matvec launch") ? ROASTER_EDEVICE : 0;
}

/* roaster_dense_mfma_min_tokens: calls with at least this many tokens (and
 * rows a multiple of 64) run as the split-operand MFMA GEMM; 0 = query. */
extern "C" int roaster_dense_mfma_min_tokens(int t)
{
    std::lock_guard<std::recursive_mutex> g(rt_lock());
    if (t > 0) g_dense_mfma_t = t;
    return g_dense_mfma_t;
}

int silu_mul_launch(float *g, const float *u, size_t n)
{
    int blocks = (int)((n + 255) / 256);
    if (blocks > 4096) blocks = 4096;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(silu_mul_kernel, dim3(blocks), dim3(256), 0, rt().stream, g, u, n);
    return rt_check(hipGetLastError(), "silu launch") ? ROASTER_EDEVICE : 0;
}

int matvec_f32_launch(const float *W, const float *x, float *y, size_t rows, size_t cols)
{
    size_t blocks = (rows + 3) / 4;
    if (blocks > 4096) blocks = 4096;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(matvec_f32_kernel, dim3((unsigned)blocks), dim3(MV_THREADS), 0, rt().stream, W, x, y, rows,
                       cols);
    return rt_check(hipGetLastError(), "matvec_f32 launch") ? ROASTER_EDEVICE : 0;
}
