/*
 * roaster_moe.h -- MI355X-native entry points of the MoE-FFN hot path that have
 * no one-to-one counterpart in the reference's kernels.h.  They replace the
 * reference's per-layer host loop around the kernels (model.c:1059-1146 decode,
 * model.c:1671-1791 prefill) and its SSD expert cache (weights.c:420-652,
 * 952-1112) with an HBM-resident expert table and whole-layer GPU launches.
 *
 * Conventions: all tensors are row-major f32 unless stated; every pointer
 * argument of the decode / prefill calls is a DEVICE pointer (allocate with
 * roaster_dev_alloc, or pass any HIP device allocation); calls are ordered on
 * the library's stream (roaster_stream) and return after launch, except where
 * noted.  Return codes: ROASTER_OK or a negative ROASTER_E* (message in
 * roaster_last_error()).  Calls that overlap from several host threads are
 * serialised by an internal lock.
 */
#ifndef ROASTER_MOE_H
#define ROASTER_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ROASTER_OK        0
#define ROASTER_EINVAL   (-1)   /* bad argument / shape */
#define ROASTER_EDEVICE  (-2)   /* HIP runtime or launch failure */
#define ROASTER_EROUTE   (-3)   /* fewer than 8 finite router logits (model.c:1074-1075, 1688) */
#define ROASTER_ENOMEM   (-4)

/* Matrix kinds of an expert. */
#define ROASTER_GATE 0
#define ROASTER_UP   1
#define ROASTER_DOWN 2

/* Prefill arithmetic. */
/* Prefill GEMM operand precision (fp32 accumulation in every mode). */
#define ROASTER_PREC_F16   0   /* fp16 operands, activations scaled per row by a power of two; the
                                  per-(token, expert) down rows kept in fp16 until the combine (default) */
#define ROASTER_PREC_SPLIT 1   /* bf16 hi+lo split of both operands, 3 MFMAs per product block */
#define ROASTER_PREC_BF16  2   /* bf16 operands: fastest to convert, about 8 significant bits */

/* ---- runtime ------------------------------------------------------------ */
const char *roaster_last_error(void);
int   roaster_init(void);               /* idempotent; every entry point calls it */
void *roaster_stream(void);             /* the hipStream_t all launches use */
int   roaster_sync(void);               /* wait for the stream; reports kernel-side errors */
int   roaster_device_info(int *n_cu, int *n_xcd, size_t *hbm_bytes);
void *roaster_dev_alloc(size_t bytes);
void  roaster_dev_free(void *p);
int   roaster_h2d(void *dst, const void *src, size_t bytes);   /* synchronous */
int   roaster_d2h(void *dst, const void *src, size_t bytes);   /* synchronous */
int   roaster_memset(void *dst, int value, size_t bytes);      /* stream-ordered */

/* Host weight memory behind kernels.h (kernel_vk_alloc_weights, registered
 * regions, other host pointers) is served from HBM copies that each call
 * brings up to date with the host bytes: written pages are found by
 * userfaultfd write tracking where the kernel offers it (asynchronous write
 * protection and PAGEMAP_SCAN, Linux 6.7+), else every used range is copied
 * on each use.  ROASTER_WEIGHT_SYNC=copy in the environment forces copying.
 * roaster_weight_tracking: enable 1 = track (where available), 0 = copy every
 * used range on each use (memory that a device writes by DMA after pinning
 * it), -1 = query.  Returns 1 when writes are tracked.  Needs no GPU. */
int roaster_weight_tracking(int enable);
int roaster_weight_sync_stats(unsigned long long *bytes_copied, int *tracking);

/* ---- HBM-resident expert table (replaces weights.c's per-layer LRU cache) -- */
typedef struct {
    int    n_layers;      /* 40 */
    int    n_experts;     /* routed experts per layer, 256 */
    size_t hidden;        /* 2048, multiple of 256 */
    size_t inter;         /* 512, multiple of 256 */
    int    q6[3];         /* routed gate / up / down type: 0 = Q4_K, 1 = Q6_K */
    int    sh_q6[3];      /* shared expert gate / up / down type */
} RoasterTableDesc;

typedef struct RoasterTable RoasterTable;

RoasterTable *roaster_table_create(const RoasterTableDesc *desc);
/* The same with per-layer matrix types, as quantised GGUF files mix them:
 * types[6 * layer + k] for k = routed gate, up, down, shared gate, up, down
 * (0 = Q4_K, 1 = Q6_K); NULL = desc's types in every layer. */
RoasterTable *roaster_table_create_layers(const RoasterTableDesc *desc, const int *types);
void   roaster_table_destroy(RoasterTable *t);
size_t roaster_table_bytes(const RoasterTable *t);
/* Upload one expert's three matrices from host memory (expert == n_experts is
 * the shared expert).  Synchronous.  weights.c:380-419 slices the same bytes
 * out of the GGUF *_exps tensors. */
int roaster_table_set_expert(RoasterTable *t, int layer, int expert,
                             const void *gate, const void *up, const void *down);
/* Upload one whole [n_experts][rows][row_bytes] GGUF tensor of `kind`. */
int roaster_table_set_exps(RoasterTable *t, int layer, int kind, const void *data, size_t bytes);
/* Router [n_experts x hidden] and shared-expert gate vector [hidden], host f32. */
int roaster_table_set_router(RoasterTable *t, int layer, const float *router, const float *shexp_gate_inp);
/* Device addresses of an expert's matrices (usable as kernels.h weight pointers). */
int roaster_table_expert_ptrs(const RoasterTable *t, int layer, int expert,
                              const void **gate, const void **up, const void **down);

/* ---- GGUF v3 model files (weights.c:657-922 parsing rules) -------------- */
typedef struct {
    int      version;         /* 3 */
    uint64_t n_tensors;
    uint64_t alignment;       /* general.alignment, default 32 */
    uint64_t data_offset;     /* file offset of the tensor data section */
    int      n_layers;        /* layers 0 .. n_layers-1, each with the eight MoE tensors */
    int      n_experts;       /* dims[2] of the *_exps tensors */
    size_t   hidden, inter;
    int      q6[3], sh_q6[3]; /* layer 0's types (0 = Q4_K, 1 = Q6_K) */
    int      mixed_types;     /* 1 if some layer's types differ from layer 0's */
    int      router_type;     /* GGML type of blk.0.ffn_gate_inp.weight: 0 F32, 1 F16, 12 Q4_K, 14 Q6_K */
} RoasterGgufInfo;

/* Parse the header, metadata and tensor table and check the MoE tensors of
 * every layer: blk.L.ffn_{gate,up,down}_exps.weight (3-D [hidden, inter, E] /
 * [inter, hidden, E], Q4_K or Q6_K), ffn_gate_inp.weight (router [hidden, E]:
 * F32, F16, Q4_K or Q6_K), ffn_gate_inp_shexp.weight ([hidden], F32 or F16),
 * ffn_{gate,up,down}_shexp.weight (2-D, Q4_K or Q6_K).  Host only (no GPU
 * call).  ROASTER_EINVAL with the reason in roaster_last_error(). */
int roaster_gguf_scan(const char *path, RoasterGgufInfo *info);
/* Create an expert table from the file and upload every MoE tensor once:
 * *_exps tensors whole (the table's routed regions are those tensors byte for
 * byte), the router and gate vector converted to f32, the shared expert as it
 * is.  info may be NULL.  NULL on error. */
RoasterTable *roaster_table_load_gguf(const char *path, RoasterGgufInfo *info);

/* ---- synthetic inputs (deterministic; identical on host and device) ------ */
typedef struct {
    float q4k_lo, q4k_hi;     /* Q4_K d and dmin ~ f16(U(lo, hi)); default 1e-3, 2e-2 */
    float q6k_lo, q6k_hi;     /* Q6_K d ~ f16(U(lo, hi)); default 1e-3, 1e-2 */
    float router_sigma;       /* router ~ N(0, sigma^2); default 0.02 */
    float gate_inp_sigma;     /* shared gate vector ~ N(0, sigma^2); default 0.02 */
} RoasterSynthSpec;

/* Stream id of (layer, expert, kind); kind 0..2 = matrices, 3 = router, 4 = gate vector. */
uint64_t roaster_synth_stream(int layer, int expert, int kind);
void roaster_synth_q4k(uint64_t seed, uint64_t stream, size_t nblocks, float lo, float hi, void *out);
void roaster_synth_q6k(uint64_t seed, uint64_t stream, size_t nblocks, float lo, float hi, void *out);
void roaster_synth_normal(uint64_t seed, uint64_t stream, size_t n, float sigma, float *out);
/* Fill every matrix of the table on the device and upload host-generated
 * routers / gate vectors.  spec may be NULL (defaults).  Synchronous. */
int roaster_table_synth(RoasterTable *t, uint64_t seed, const RoasterSynthSpec *spec);

/* ---- decode: one launch per call ---------------------------------------- */
typedef struct {
    const float *logits_in;   /* [B x E]: replaces the router matvec, or NULL */
    float *logits_out;        /* [B x E] or NULL */
    int   *ids_out;           /* [B x 8] selected experts, descending logit, or NULL */
    float *w_out;             /* [B x 8] renormalised weights, or NULL */
} RoasterDecodeIO;

/* y[b] = sum_k w[b,k] * expert_{id[b,k]}(x[b]) + sigmoid(gate_inp . x[b]) * shared(x[b])
 * for B (1..8) independent tokens: model.c:1059-1146 per token. */
int roaster_moe_decode(RoasterTable *t, int layer, const float *x, int B, float *y,
                       const RoasterDecodeIO *io);

/* The layer stack with the hidden state on the GPU:
 *   for l in [layer0, layer0 + n_layers): h += MoE_l(RMSNorm(h; norm_w[l - layer0], eps))
 * (model.c:1352-1358 without the mixer).  norm_w is [n_layers x hidden] or NULL
 * (all ones).  ids_out / w_out: [n_layers x B x 8] or NULL.  One launch. */
int roaster_moe_decode_stack(RoasterTable *t, float *h, int B, int layer0, int n_layers,
                             const float *norm_w, float eps, int *ids_out, float *w_out);

/* Decode runs a call's layers as one launch (router, top-8, experts and
 * combine in 256 workgroups that exchange values through memory) wherever the
 * shapes allow it: a device with at least 256 CUs on which each one-launch
 * kernel fits one workgroup per CU, experts a multiple of 32 up to 256; for
 * one token hidden up to 2048 and inter up to 1024; for 2..8 tokens inter 512,
 * hidden 512..2048 in multiples of 256, and gate/up Q4_K and down Q6_K in
 * every layer of the call.  Otherwise each layer runs as three launches.
 * One token at 256 experts, hidden 2048, inter 512 with gate/up Q4_K and down
 * Q6_K folds the router into the previous layer's combine: its logits and
 * 1/rms are sums of per-workgroup partials, equal to the three-kernel path's
 * up to fp32 summation order, and its ids equal given identical logits.
 * Every other one-launch case gives results bit-identical to the three-kernel
 * path, each token's equal to its one-token result.
 * roaster_decode_fused_layer: 1 = one launch where possible (default), 2 = the
 * same but one token always with the three-kernel path's arithmetic (no folded
 * router), 0 = always three, -1 = query; returns the mode in force. */
int roaster_decode_fused_layer(int enable);
/* Polls a one-launch layer's wait makes before it gives up (sets error bit 2,
 * reported by roaster_sync as ROASTER_EDEVICE, and the launch ends with
 * unusable outputs; the folded-router kernel leaves a stack call's h as it
 * was); 0 = query.  Default 2^20 (about a second); tests set it tiny to
 * exercise that path. */
unsigned roaster_decode_spin_limit(unsigned polls);
/* The one-launch kernels' 256 workgroups wait on each other, so they must all
 * be resident at once.  1: launch them cooperatively, so that the runtime
 * guarantees it or refuses the launch (ROASTER_EDEVICE) -- for a GPU shared
 * with other work; it measured 0.5 us per layer slower on an idle MI355X.
 * 0 (default): ordinary launches, whose waits give up after the spin limit if
 * other work holds CUs.  -1 = query; returns the mode in force. */
int roaster_decode_cooperative_launch(int enable);
/* The kernel(s) roaster_moe_decode_stack(t, ., B, layer0, n_layers, ...) would
 * launch in the current modes, as a static string ("" for bad arguments). */
const char *roaster_decode_stack_kernel(RoasterTable *t, int B, int layer0, int n_layers);

/* No counterpart in the reference: roaster_moe_decode_stack for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments and results (one
 * token: the same one-launch kernel; 2..8 tokens: three launches per layer);
 * every intermediate lives in a fixed 576 KiB device array that the
 * library sets up in roaster_init (call it first) and keeps until the process
 * ends, so the call itself makes no allocation.  Calls whose three-kernel
 * intermediates exceed it -- about 8 tokens x hidden 2048 x inter 2048 or
 * more -- return ROASTER_EINVAL before anything runs; one token whose
 * one-launch exchange slots do not fit beside them runs three kernels per
 * layer instead (same results).  Every call on a device shares that device's array and
 * leaves its contents behind: calls on the library stream run one after the
 * other, but two processes' or streams' calls that overlapped would race. */
int roaster_moe_decode_stack_noalloc(RoasterTable *t, float *h, int B, int layer0, int n_layers,
                                     const float *norm_w, float eps, int *ids_out, float *w_out);

/* ---- dense projections ---------------------------------------------------- */
/* Y[t * rows + r] = W[r] . X[t * cols ..] for t < T (1..8): a quantised
 * [rows x cols] matrix on the device (q6: 0 = Q4_K, 1 = Q6_K, cols a multiple
 * of 256, at most 4096) -- the projections on either side of the MoE block
 * (the attention output and DeltaNet ssm_out projections have 4096 columns,
 * model.c:862, 1344-1347) and the LM head (model.c:795-800, 1284-1290,
 * 1368-1370), the products kernel_matvec_q4_k / _q6_k compute from host
 * buffers.  Device pointers; ordered on the library stream. */
int roaster_matvec_q(const void *W, int q6, const float *X, float *Y, size_t rows, size_t cols, int T);
/* Calls of roaster_matvec_q with at least t tokens (default 2) run with the
 * quants as MFMA operands instead of the dequantising matvec (t = 9: never);
 * t = 0 queries.  Returns the threshold in force. */
int roaster_dense_mfma_min_tokens(int t);

/* ---- prefill ------------------------------------------------------------ */
typedef struct {
    int precision;             /* ROASTER_PREC_F16 (default), _SPLIT or _BF16 */
    const float *logits_in;    /* [T x E] replaces the router matmul, or NULL */
    const float *logit_bias;   /* [E] added to every token's logits, or NULL */
    float *logits_out;         /* [T x E] or NULL */
    int   *ids_out;            /* [T x 8] or NULL */
    float *w_out;              /* [T x 8] or NULL */
    int   *counts_out;         /* [E] tokens per expert, or NULL */
} RoasterPrefillOpts;

/* Y[t] = sigmoid(gate_inp . X[t]) * shared(X[t]) + sum over t's experts in
 * ascending id of w * expert(X[t]) -- model.c:1671-1791.  X, Y: [T x hidden]. */
int roaster_moe_prefill(RoasterTable *t, int layer, const float *X, int T, float *Y,
                        const RoasterPrefillOpts *opts);
/* The fp16-mode down GEMM (inter <= 512) as one workgroup per CU over an even
 * split of its output tiles (1, default) or one workgroup per four output
 * tiles (0); -1 queries.  Both give bit-identical results.  Returns the mode
 * in force. */
int roaster_prefill_balanced_down(int enable);
/* The fp16-mode gate/up GEMM on a persistent grid, one workgroup per CU taking
 * (tile, 128-column) units from work counters and preparing the next unit
 * while one runs (1, default; layers whose routed and shared gate and up
 * matrices share one type and whose hidden size is a multiple of 512, at
 * least 2048), or one workgroup per unit (0); -1 queries.  Both give
 * bit-identical results.  Returns the mode in force. */
int roaster_prefill_persistent_gate_up(int enable);
/* Both fp16-mode GEMMs in one persistent kernel (1, where the persistent
 * gate/up grid and the balanced down GEMM both apply and the GPU has 8
 * XCDs): each XCD's workgroups take its share of the tiles' gate/up units,
 * then their down chunks once a chunk's tile is complete, so the down work
 * fills the gate/up tail; or two kernels (0, default: the one kernel
 * measured 1-3% faster, within the spread between boxes); -1 queries.  Both
 * give bit-identical results.  Returns the mode in force. */
int roaster_prefill_fused_gemm(int enable);

#ifdef __cplusplus
}
#endif
#endif
