/*
 * matvec.h -- job descriptor and launchers of matvec.hip.
 */
#ifndef ROASTER_MATVEC_H
#define ROASTER_MATVEC_H

#include <stdint.h>
#include <stddef.h>

/* One quantised matvec / small-T matmul: Y[t*rows + r] = dot(W[r], X[t]). */
struct MvJob {
    const uint8_t *W;   /* device, rows x cols quantised */
    const float *X;     /* device, T x cols */
    float *Y;           /* device, T x rows */
    int rows, cols, T, q6;
    int task0;          /* first task index of this job (prefix over jobs) */
};

int mv_tasks_for(int rows, size_t cols);
int mv_launch(const MvJob *jobs_dev, int njobs, int ntasks);
int silu_mul_launch(float *g, const float *u, size_t n);
int matvec_f32_launch(const float *W, const float *x, float *y, size_t rows, size_t cols);
/* Y[t * rows + r] = W[r] . X[t] for 1 <= T <= 8 and cols <= 4096 with the
 * quants as MFMA operands (dense_mm8_kernel), device buffers. */
int dense_mm8_launch(const uint8_t *W, int q6, const float *X, float *Y, size_t rows, size_t cols, int T);
/* Token count from which multi-token products take dense_mm8_launch. */
int dense_mfma_min_tokens();

#endif
