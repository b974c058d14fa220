/*
 * kernels.h -- the reference's kernel C API, served by libroaster_moe.so on one
 * MI355X (gfx950).  Every declaration keeps the reference's name, argument
 * meaning, struct layout and return convention (src/kernels.h:1-106 of the
 * reference), so model.c and weights.c link against this library unchanged.
 *
 * What differs underneath:
 *   - All array work runs as HIP kernels on the GPU.  There is no CPU
 *     fallback: a device failure is reported (stderr + return code where the
 *     signature has one, NaN for float-returning dots) instead of silently
 *     recomputing on the host.
 *   - Weight pointers may be (a) host addresses inside kernel_vk_alloc_weights
 *     memory or a kernel_vk_register_region region, uploaded to HBM on first use;
 *     (b) any other host address, uploaded and cached per (pointer, size) until
 *     kernel_vk_release_host_ptr; or (c) device addresses handed out by the
 *     expert table (roaster_moe.h), used in place.
 *   - cols / inter / hidden must be multiples of 256 (whole super-blocks), as
 *     every GPU path of the reference requires (kernels.c:1247, 1918, 2201).
 */
#ifndef KERNELS_H
#define KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Float kernels -- reference kernels.h:8-9 (kernels.c:102-148). */
float kernel_dot_f32(const float *a, const float *b, size_t n);
void  kernel_matvec_f32(const float *matrix, const float *vector, float *output, size_t rows, size_t cols);

/* Quantised dot products / matvecs -- reference kernels.h:12-15 (kernels.c:345-578, 1648-1658). */
float kernel_dot_q4_k(const void *weights, const float *x, size_t n);
float kernel_dot_q6_k(const void *weights, const float *x, size_t n);
void  kernel_matvec_q4_k(const void *matrix, const float *vector, float *output, size_t rows, size_t cols);
void  kernel_matvec_q6_k(const void *matrix, const float *vector, float *output, size_t rows, size_t cols);

/* Normalisation and activations -- reference kernels.h:18-22 (kernels.c:584-652). */
void  kernel_rmsnorm(float *output, const float *input, const float *weight, size_t n, float epsilon);
void  kernel_l2norm(float *output, const float *input, size_t n, float epsilon);
float kernel_sigmoid(float x);
float kernel_silu(float x);
void  kernel_silu_array(float *x, size_t n);

/* Embedding row (Q4_K) and causal convolution -- reference kernels.h:25-27 (kernels.c:660-719). */
void kernel_embedding_row_q4_k(const void *weights, size_t token_id, float *output, size_t hidden_size);
void kernel_conv1d_causal_f32(const float *input, const float *history, const float *kernel,
                              float *output, size_t channels, size_t kernel_size);

/* Batched quantised matvec -- reference kernels.h:34-49 (kernels.c:1582-1646).
 * Jobs are independent; all jobs of a call run in one stream submission; jobs
 * sharing `vector` (and cols) upload it once. */
typedef struct {
    int is_q6;             /* 0 = Q4_K, 1 = Q6_K */
    const void *matrix;
    const float *vector;
    float *output;
    size_t rows;
    size_t cols;
} KernelMatvecJob;

void kernel_matvec_quant_batch(const KernelMatvecJob *jobs, int n);
/* Split-phase: begin() launches and returns 1 while the batch is in flight;
 * end() is mandatory and copies the outputs back.  `jobs` must stay valid until
 * end() -- reference kernels.h:45-49. */
int  kernel_matvec_quant_begin(const KernelMatvecJob *jobs, int n);
void kernel_matvec_quant_end(void);

/* Multi-token matmul Y[t*rows + r] = dot(W[r], X[t]) -- reference kernels.h:51-64
 * (kernels.c:1916-2069).  Returns 0, or -1 for invalid arguments. */
typedef struct {
    int is_q6;             /* 0 = Q4_K, 1 = Q6_K */
    const void *matrix;    /* rows x cols quantised */
    const float *X;        /* T x cols */
    float *Y;              /* T x rows */
    size_t rows, cols, T;
} KernelMatmulJob;
int kernel_matmul_quant_batch(const KernelMatmulJob *jobs, int n);

/* Prefill MoE FFN over experts' row groups, D_e = down(silu(gate X_e) * (up X_e))
 * -- reference kernels.h:66-80 (kernels.c:2071-2214).  X and D hold the groups
 * back to back.  Returns 0, or -1 for invalid arguments or a device failure. */
typedef struct {
    const void *gate, *up, *down;
    int gate_q6, up_q6, down_q6;
    size_t n;              /* tokens routed to this expert */
} KernelMoeExpert;
int kernel_moe_prefill(const KernelMoeExpert *experts, int count, const float *X, float *D,
                       size_t inter, size_t hidden);

/* One expert FFN sharing the input x -- reference kernels.h:82-92 (kernels.c:1661-1830). */
typedef struct {
    const void *gate, *up, *down;
    int gate_q6, up_q6, down_q6;     /* 0 = Q4_K, 1 = Q6_K */
    float *out;                      /* `hidden` floats */
} KernelFfnExpert;

/* Runs n experts (n <= 9) gate/up -> SiLU*up -> down.  Returns 1 on success,
 * 0 when unavailable (the caller then uses the generic path). */
int kernel_ffn_fused(const KernelFfnExpert *experts, int n, const float *x, size_t inter, size_t hidden);

/* Backend lifecycle and weight memory -- reference kernels.h:94-105 (kernels.c:1400-1573).
 * The names are kept as the allocation ABI; memory is HBM behind a host address. */
void   kernel_vk_trim_scratch(void);
void   kernel_vk_shutdown(void);
void   kernel_vk_release_host_ptr(const void *ptr);
int    kernel_vk_register_region(const void *ptr, size_t size);
void  *kernel_vk_alloc_weights(size_t size, size_t *granted);
int    kernel_vk_owns_weights(const void *ptr);
int    kernel_vk_free_weights(void *ptr);

#ifdef __cplusplus
}
#endif
#endif
