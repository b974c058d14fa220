/*
 * decode.h -- argument structures of the decode kernel (decode.hip), shared
 * with the host code that fills them (api.hip).
 */
#ifndef ROASTER_DECODE_H
#define ROASTER_DECODE_H

#include <stdint.h>
#include <stddef.h>

#define RMAX_ACT (8 * 8 + 1)        /* distinct routed experts of 8 tokens + shared */

/* Device addresses of one layer's tensors in the expert table, with the
 * layer's matrix types (a GGUF file may quantise layers differently). */
struct DecLayer {
    const uint8_t *gate, *up, *down;      /* [E][rows][row_bytes], GGUF *_exps layout */
    const uint8_t *sgate, *sup, *sdown;   /* shared expert */
    const float *router;                  /* [E x H] */
    const float *gate_inp;                /* [H] */
    size_t eb[3];                         /* bytes of one routed expert's gate / up / down */
    int q6[3];                            /* routed gate / up / down: 0 = Q4_K, 1 = Q6_K */
    int sq6[3];                           /* shared expert gate / up / down */
};
static_assert(sizeof(DecLayer) % 16 == 0, "DecLayer is copied in 16-byte units");

/* One active expert of a decode plan: its matrices and the (token, slot)
 * pairs that use it (pair p = t*9 + k, k = 8 for the shared expert). */
struct DecActive {
    const uint8_t *g, *u, *d;
    int gq6, uq6, dq6;
    int ntok;
    int tk[8];
};

struct DecPlan {
    int nact;               /* active experts: [0, nroute) routed, then the shared expert */
    int nroute;
    int err;
    int pad0;
    DecActive a[RMAX_ACT];
    int ids[8][8];
    float w[8][9];          /* routing weights, [8] = sigmoid(shared gate logit) */
    int pad1[2];
    const uint8_t *dsl[8][9];   /* down matrix of token t's slot k (8 = shared), NULL when unselected */
    int dq6k[9];                /* type of slot k's down matrix (the same for every token) */
    int pad2[3];
};
static_assert(sizeof(DecPlan) % 16 == 0, "DecPlan is copied in 16-byte units");

struct DecArgs {
    const DecLayer *layers;     /* device array indexed by layer */
    int layer0, nlayers;
    int E, H, I, B;
    float *h;                   /* [B x H]: stack state (in/out), or the layer input */
    float *y;                   /* [B x H] layer output, or NULL in stack mode */
    const float *norm_w;        /* [nlayers x H] or NULL */
    float eps;
    int do_norm;
    int xswz;                   /* activations in LDS stored swizzled (H % 512 == 0: whole 128-unit blocks per row) */
    const float *logits_in;     /* [B x E] or NULL */
    float *logits;              /* [B x E] */
    float *sgate_raw;           /* [B] */
    float *eh;                  /* [B*9 x I] */
    float *xn_g;                /* [B x H] normalised input + [B x H/16] run sums, published by R */
    int *ids_out;               /* [nlayers x B x 8] or NULL */
    float *w_out;
    DecPlan *plan_g;            /* plan written by the gate/up kernel, read by the down kernel */
    int *err;
    const DecLayer *layers_h;   /* host copy of layers (read by the launch code only) or NULL */
    int d1;                     /* per launch: one-token down path, 0 off, 1 Q4_K, 2 Q6_K down matrices */
    /* kernel_ffn_fused mode */
    const DecActive *ffn_ex;    /* [n] device */
    int ffn_n;
    float *ffn_out;             /* [n x H] or NULL */
    /* one-launch stack (dec_stack1_kernel): exchange slots, u64 = (epoch << 32) | f32 bits */
    uint64_t *xch;              /* [XCH_U64(E, H, I)] or NULL (then the three-kernel path runs) */
    uint32_t epoch;             /* epoch of the launch's first layer (layer i: epoch + i) */
    uint32_t spin;              /* polls before a wait gives up (set by the launch code) */
    int xl2;                    /* 1: slots read only within the writer's XCD stay in its L2 */
    struct DecXch *xbuf;        /* host side: the buffer behind xch and its epoch counter, or NULL */
    uint32_t *cnt;              /* dec_stack1r_kernel: completion counter (a multiple of 256 between launches), or NULL */
};

/* Exchange regions of the one-launch stack, in u64 slots; every region
 * starts on a 128-byte line.  Read across XCDs, each value by one workgroup
 * per XCD, and each line written by one workgroup (lines shared by writers on
 * different XCDs are slow to propagate): router logit b [256][16], workgroup
 * b's shared-expert SiLU*up values [256][16], the 8 routed slots' down
 * outputs [8][H] and the shared expert's, H/256 rows per workgroup,
 * [256][16].  Then one region per XCD, written and read within it: its copy
 * of the logits [256] and of the shared SiLU*up values [I], its group's
 * routed SiLU*up [I] and its copy of the next layer's hidden state [H].  The
 * per-XCD vectors are stored so that a gather's lanes read contiguous slots:
 * SiLU*up value j at (j % 16) (I / 16) + j / 16 (a lane reads one 16-value
 * run), hidden row r at (r % 4) (H / 4) + r / 4 (a lane reads one float4). */
#define XCH_LN 16                                   /* slots per line */
#define XCH_LG(E, H, I) ((size_t)0)
#define XCH_EHS(E, H, I) ((size_t)256 * XCH_LN)
#define XCH_DX(E, H, I) ((size_t)512 * XCH_LN)
#define XCH_DSH(E, H, I) (XCH_DX(E, H, I) + 8 * (size_t)(H))
#define XCH_LOC0(E, H, I) (XCH_DSH(E, H, I) + (size_t)256 * XCH_LN)
#define XCH_LOCN(E, H, I) ((size_t)256 + 2 * (size_t)(I) + (size_t)(H))
#define XCH_LLG(I) ((size_t)0)
#define XCH_LEHS(I) ((size_t)256)
#define XCH_LEHX(I) ((size_t)256 + (size_t)(I))
#define XCH_LH(I) ((size_t)256 + 2 * (size_t)(I))
/* then the staged final hidden state [H] (a stack call's h is written only
 * when no wait gave up) */
#define XCH_HST(E, H, I) (XCH_LOC0(E, H, I) + 8 * XCH_LOCN(E, H, I))
#define XCH_U64(E, H, I) (XCH_HST(E, H, I) + (size_t)(H))

/* The same regions for the batched one-launch stack (2..8 tokens, sized for
 * NB >= B tokens), each with a token index outermost: logits [NB][256][16],
 * shared SiLU*up [NB][256][16], routed down outputs [NB][8][H], shared down
 * outputs [NB][256][16]; per XCD: logits [NB][256], shared SiLU*up [NB][I],
 * routed SiLU*up [NB][I], next hidden state [NB][H] (the per-token vectors in
 * the run-major layouts above). */
#define XCHB_LG(NB, E, H, I) ((size_t)0)
#define XCHB_EHS(NB, E, H, I) ((size_t)(NB) * 256 * XCH_LN)
#define XCHB_DX(NB, E, H, I) (XCHB_EHS(NB, E, H, I) + (size_t)(NB) * 256 * XCH_LN)
#define XCHB_DSH(NB, E, H, I) (XCHB_DX(NB, E, H, I) + (size_t)(NB) * 8 * (size_t)(H))
#define XCHB_LOC0(NB, E, H, I) (XCHB_DSH(NB, E, H, I) + (size_t)(NB) * 256 * XCH_LN)
#define XCHB_LOCN(NB, E, H, I) ((size_t)(NB) * ((size_t)256 + 2 * (size_t)(I) + (size_t)(H)))
#define XCHB_LLG(NB, I) ((size_t)0)
#define XCHB_LEHS(NB, I) ((size_t)(NB) * 256)
#define XCHB_LEHX(NB, I) ((size_t)(NB) * ((size_t)256 + (size_t)(I)))
#define XCHB_LH(NB, I) ((size_t)(NB) * ((size_t)256 + 2 * (size_t)(I)))
#define XCHB_HST(NB, E, H, I) (XCHB_LOC0(NB, E, H, I) + 8 * XCHB_LOCN(NB, E, H, I))   /* staged h [NB][H] */
#define XCHB_U64(NB, E, H, I) (XCHB_HST(NB, E, H, I) + (size_t)(NB) * (H))
#define K1B_MAXB 8                                  /* tokens of the batched one-launch stack */

/* Regions of the one-token stack whose router is folded into the combine
 * (dec_stack1r_kernel: 256 experts, hidden 2048, inter 512).  Read across
 * XCDs: the router partials [8][32][32] (XCD k's workgroup gi writes the 32
 * partial logits of experts 32k..32k+31 over its 64 combined rows, two lines
 * of its own), workgroup b's shared SiLU*up values [256][16], the routed
 * down outputs [8][H], the shared down outputs [256][16] and the staged
 * final hidden state [H].  Then one region
 * per XCD: its logits [256], the row sums of squares of its 32 workgroups
 * [32], its copies of the shared and routed SiLU*up values [I] each, and its
 * copy of the hidden state [H] (SiLU*up and hidden rows in the run-major
 * layouts above). */
#define XR_PL(E, H, I) ((size_t)0)
#define XR_EHS(E, H, I) ((size_t)8 * 32 * 32)
#define XR_DX(E, H, I) (XR_EHS(E, H, I) + (size_t)256 * XCH_LN)
#define XR_DSH(E, H, I) (XR_DX(E, H, I) + 8 * (size_t)(H))
#define XR_HST(E, H, I) (XR_DSH(E, H, I) + (size_t)256 * XCH_LN)
#define XR_LOC0(E, H, I) (XR_HST(E, H, I) + (size_t)(H))
#define XR_LOCN(E, H, I) ((size_t)256 + 32 + 2 * (size_t)(I) + (size_t)(H))
#define XR_LLG(I) ((size_t)0)
#define XR_LSS(I) ((size_t)256)
#define XR_LEHS(I) ((size_t)256 + 32)
#define XR_LEHX(I) ((size_t)256 + 32 + (size_t)(I))
#define XR_LH(I) ((size_t)256 + 32 + 2 * (size_t)(I))
#define XR_U64(E, H, I) (XR_LOC0(E, H, I) + 8 * XR_LOCN(E, H, I))

/* Exchange buffer of the one-launch stack: the slots and the last epoch
 * written into them.  Epochs grow by one per layer; before the 32-bit epoch
 * would wrap, the slots are cleared (by a fill kernel) and epochs start
 * again at 1, so a slot never holds a later layer's epoch. */
struct DecXch { uint64_t *p; size_t n; uint32_t epoch; };

/* All layers of A: 3 kernels per layer.  A.plan_g and A.err may be set by the
 * caller (device memory of sizeof(DecPlan) and one int); when either is NULL
 * the library's own scratch and control words are used. */
int dec_launch(DecArgs &A);
int dec_ffn_launch(DecArgs &A);      /* kernel_ffn_fused: gate/up + down kernels */
/* Whether one token's layers can run as one launch (dec_stack1_kernel) for
 * these shapes on this device. */
bool dec_layer1_ok(int E, int H, int I, int B);
/* The kernels a decode call of A would launch (a static string). */
const char *dec_kernel_names(const DecArgs &A);
/* The exchange slots a one-token launch of these shapes uses (0: none). */
size_t dec_xch_need1(int E, int H, int I);
/* Whether B = 2..8 tokens' layers can run as one launch (dec_stackB_kernel)
 * for these shapes on this device (the matrix types are checked per launch). */
bool dec_layerB_ok(int E, int H, int I, int B);
/* Clears X's slots on the library stream (a fill kernel) and restarts its epochs. */
int dec_xch_clear(DecXch &X);
/* The library's exchange buffer (allocated and cleared on first use). */
DecXch *dec_xch_default(int E, int H, int I);

#endif
