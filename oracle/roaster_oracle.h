/*
 * roaster_oracle.h -- CPU restatement of the reference's MoE-FFN CPU path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker, never the product:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  The product path (libroaster_moe.so) never links or calls it.
 *
 * Every function restates one reference function and reproduces its fp32
 * operation order exactly (8-lane AVX2 accumulation order, FMA contraction as
 * gcc -O3 -mfma emits it, glibc expf), so that outputs are bit-identical to the
 * reference built with -O3 -mavx2 -mfma -mf16c.  Cited lines are in
 * src/kernels.c and src/model.c of the reference.
 *
 * Layout: Q4_K super-block = 144 B (d f16, dmin f16, scales[12], qs[128]),
 *         Q6_K super-block = 210 B (ql[128], qh[64], scales int8[16], d f16),
 *         256 weights per block, matrix rows = cols/256 consecutive blocks.
 */
#ifndef ROASTER_ORACLE_H
#define ROASTER_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QK 256
#define ORC_Q4K_BYTES 144
#define ORC_Q6K_BYTES 210
#define ORC_TOPK 8

/* kernels.c:56-96 */
float orc_fp16_to_f32(uint16_t h);
/* kernels.c:154-173 */
void  orc_q4k_scales(const uint8_t *blk, int sc[8], int mn[8]);
/* kernels.c:102-129 (AVX2 branch) */
float orc_dot_f32(const float *a, const float *b, size_t n);
/* kernels.c:131-148 */
void  orc_matvec_f32(const float *W, const float *x, float *y, size_t rows, size_t cols);
/* kernels.c:345-356 -> 246-288 (n % 256 == 0); returns NaN otherwise */
float orc_dot_q4k(const void *row, const float *x, size_t n);
/* kernels.c:490-501 -> 304-342 (n % 256 == 0); returns NaN otherwise */
float orc_dot_q6k(const void *row, const float *x, size_t n);
/* kernels.c:407-432 / 553-578 */
void  orc_matvec_q4k(const void *W, const float *x, float *y, size_t rows, size_t cols);
void  orc_matvec_q6k(const void *W, const float *x, float *y, size_t rows, size_t cols);
void  orc_matvec_quant(int q6, const void *W, const float *x, float *y, size_t rows, size_t cols);
/* kernels.c:1839-1874 */
void  orc_dequant_q4k_block(const void *blk, float out[256]);
void  orc_dequant_q6k_block(const void *blk, float out[256]);
/* kernels.c:1876-1914: Y[t*rows + r] = dot(W[r], X[t]) */
void  orc_matmul_quant(int q6, const void *W, const float *X, float *Y,
                       size_t rows, size_t cols, size_t T);
/* kernels.c:584-605 */
void  orc_rmsnorm(float *out, const float *in, const float *w, size_t n, float eps);
/* model.c:869-897 for n experts (the reference fixes n = 256) */
void  orc_select_top8(const float *logits, int n, int ids[8], float w[8]);

/* One expert's three quantised matrices (KernelFfnExpert / KernelMoeExpert). */
typedef struct {
    const void *gate, *up, *down;
    int gate_q6, up_q6, down_q6;
} OrcExpert;

/* One MoE layer: n_experts routed experts + 1 shared expert. */
typedef struct {
    int n_experts;                /* 256 */
    size_t hidden, inter;         /* 2048, 512 */
    const float *router;          /* [n_experts x hidden] f32 row-major */
    const float *shexp_gate_inp;  /* [hidden] f32: shared-expert gate vector */
    const OrcExpert *experts;     /* [n_experts] */
    OrcExpert shared;
} OrcLayer;

/* One expert, decode form (folded dots): out = down(silu(gate x) * (up x)).
 * model.c:1108-1133 (generic path: matvecs + CPU SiLU). */
void orc_expert_decode(const OrcExpert *e, const float *x, size_t inter, size_t hidden,
                       float *out);

/* Decode MoE block for one token, model.c:1059-1146 (router -> top-8 -> experts ->
 * combine k = 0..7 then shared).  If `logits_in` is non-NULL it replaces the
 * router matvec (the caller supplies identical logits).  Outputs: y[hidden],
 * and optionally logits[n_experts], ids[8], w[8].  Returns 0, or -1 when fewer
 * than 8 finite logits exist (model.c:1074-1075). */
int  orc_moe_decode(const OrcLayer *L, const float *x, const float *logits_in,
                    float *y, float *logits, int ids[8], float w[8]);

/* kernels.c:2176-2196 (moe_cpu): D_e = down(silu(gate X_e) * (up X_e)) per row group. */
typedef struct {
    const void *gate, *up, *down;
    int gate_q6, up_q6, down_q6;
    size_t n;
} OrcMoeGroup;
void orc_moe_groups(const OrcMoeGroup *g, int count, const float *X, float *D,
                    size_t inter, size_t hidden);

/* model.c:1713-1731: stable counting sort of the (t, k) pairs by expert.
 * cnt[E], off[E+1], lt[T*8], lk[T*8]. */
void orc_bucket(const int *ids, int T, int n_experts, int *cnt, int *off, int *lt, int *lk);

/* Prefill MoE block, model.c:1671-1791 for T tokens.  Router logits are
 * computed per token with the F32 matvec unless `logits_in` ([T x n_experts])
 * is given; `logit_bias` ([n_experts], may be NULL) is added to each token's
 * logits before top-8.  Y[T x hidden] = sigmoid(gate_inp . x) * shared(x),
 * then += w * expert(x) in expert-ascending order.  Optional outputs: ids/w
 * [T x 8] and logits [T x n_experts].  Returns 0 or -1. */
int  orc_moe_prefill(const OrcLayer *L, const float *X, int T, const float *logits_in,
                     const float *logit_bias, float *Y, int *ids, float *w, float *logits);

#ifdef __cplusplus
}
#endif
#endif
