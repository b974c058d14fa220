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

template <bool Q6, bool ONE>
__global__ void __launch_bounds__(MV_THREADS) dense_mv_kernel(const uint8_t *W, const float *X, float *Y, int rows,
                                                              int cols, int T)
{
    extern __shared__ __align__(16) float xs[];            /* [T][cols] + run sums [T][cols / 16] (T > 1) */
    const int lane = threadIdx.x & 63;
    const int nb = cols / RQK, lpr = lanes_per_row(nb), rpw = 64 / lpr;
    const int rw = lane / lpr, lr = lane % lpr, c = lr & 7, lb = lr >> 3;
    const bool lane_live = lb < nb;
    const size_t bs = Q6 ? RQ6K_BYTES : RQ4K_BYTES, row_bytes = (size_t)nb * bs;
    const int ca = lb * RQK + q_run_a<Q6>(c), cb = ca + q_run_b_off<Q6>();
    float4 xa[4], xb[4];
    float sxa = 0.0f, sxb = 0.0f;
    float *xsum = xs + (size_t)T * cols;
    if (ONE) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            xa[i] = lane_live ? gld_f4(X + ca + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
            xb[i] = lane_live ? gld_f4(X + cb + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        sxa = ((xa[0].x + xa[0].y) + (xa[0].z + xa[0].w)) + ((xa[1].x + xa[1].y) + (xa[1].z + xa[1].w)) +
              (((xa[2].x + xa[2].y) + (xa[2].z + xa[2].w)) + ((xa[3].x + xa[3].y) + (xa[3].z + xa[3].w)));
        sxb = ((xb[0].x + xb[0].y) + (xb[0].z + xb[0].w)) + ((xb[1].x + xb[1].y) + (xb[1].z + xb[1].w)) +
              (((xb[2].x + xb[2].y) + (xb[2].z + xb[2].w)) + ((xb[3].x + xb[3].y) + (xb[3].z + xb[3].w)));
    } else {
        for (int i = threadIdx.x; i < T * cols / 4; i += MV_THREADS) ((float4 *)xs)[i] = gld_f4(X + 4 * i);
        __syncthreads();
        for (int i = threadIdx.x; i < T * cols / 16; i += MV_THREADS) xsum[i] = sum16(xs + 16 * i);
        __syncthreads();
    }
    const int gw = blockIdx.x * (MV_THREADS / 64) + (threadIdx.x >> 6), nw = gridDim.x * (MV_THREADS / 64);
    const int npass = (rows + rpw - 1) / rpw;
    for (int p0 = gw; p0 < npass; p0 += nw * DMV_PF) {
        QChunk ch[DMV_PF];
#pragma unroll
        for (int f = 0; f < DMV_PF; f++) {
            const int row = (p0 + f * nw) * rpw + rw;
            if (lane_live && row < rows) ch[f] = q_load<Q6>(W + (size_t)row * row_bytes + (size_t)lb * bs, c);
        }
#pragma unroll
        for (int f = 0; f < DMV_PF; f++) {
            const int pass = p0 + f * nw;
            if (pass >= npass) break;
            const int row = pass * rpw + rw;
            const bool live = lane_live && row < rows;
            for (int t = 0; t < (ONE ? 1 : T); t++) {
                float part = 0.0f;
                if (live) {
                    if (ONE) {
                        part = q_chunk_dot_r<Q6>(ch[f], c, xa, xb, sxa, sxb);
                    } else {
                        const float *x = xs + (size_t)t * cols, *sx = xsum + (size_t)t * (cols / 16);
                        part = q_chunk_dot<Q6>(ch[f], c, x + ca, x + cb, sx[ca >> 4], sx[cb >> 4]);
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
    if (!W || !X || !Y || !rows || !cols || cols % RQK || cols > 2048 || T < 1 || T > 8 || rows > (size_t)INT32_MAX)
        return rt_fail(ROASTER_EINVAL, "roaster_matvec_q: need cols a multiple of 256 and <= 2048, 1 <= T <= 8");
    const int nb = (int)(cols / RQK), rpw = 64 / lanes_per_row(nb);
    const size_t npass = (rows + rpw - 1) / rpw;
    size_t blocks = (npass + 3) / 4;
    if (blocks > (size_t)DMV_GRID * rt().n_cu) blocks = (size_t)DMV_GRID * rt().n_cu;
    const size_t lds = T > 1 ? (size_t)T * cols * 4 + (size_t)T * (cols / 16) * 4 : 0;
    const dim3 gd((unsigned)blocks), bd(MV_THREADS);
    if (q6 && T == 1) hipLaunchKernelGGL((dense_mv_kernel<true, true>), gd, bd, 0, rt().stream, (const uint8_t *)W, X, Y, (int)rows, (int)cols, T);
    else if (q6) hipLaunchKernelGGL((dense_mv_kernel<true, false>), gd, bd, lds, rt().stream, (const uint8_t *)W, X, Y, (int)rows, (int)cols, T);
    else if (T == 1) hipLaunchKernelGGL((dense_mv_kernel<false, true>), gd, bd, 0, rt().stream, (const uint8_t *)W, X, Y, (int)rows, (int)cols, T);
    else hipLaunchKernelGGL((dense_mv_kernel<false, false>), gd, bd, lds, rt().stream, (const uint8_t *)W, X, Y, (int)rows, (int)cols, T);
    return rt_check(hipGetLastError(), "dense matvec launch") ? ROASTER_EDEVICE : 0;
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
