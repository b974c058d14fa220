/*
 * prefill.h -- grouped expert GEMMs (prefill.hip), shared with the kernels.h
 * implementation of kernel_moe_prefill (api.hip).
 *
 * A group is one expert's row list: n rows, row a reads activation row
 * tok[a] (or tok0 + a) of X and owns slot slot0 + a of the intermediate and
 * output buffers.  A tile is 64 consecutive rows of one group.
 */
#ifndef ROASTER_PREFILL_H
#define ROASTER_PREFILL_H

#include <stdint.h>
#include <stddef.h>

struct PfGroup {
    const uint8_t *g, *u, *d;      /* gate [I x H], up [I x H], down [H x I] */
    const uint8_t *tg, *tu, *td;   /* the same matrices in the MFMA tile layout (tile.h) */
    int gq6, uq6, dq6;
    int n;                          /* rows */
    int slot0;                      /* first slot */
    int tok0;                       /* rows read X[tok0 + a] when tok is NULL */
    const int *tok;                 /* [n] activation rows, or NULL */
    float dbnd;                     /* bound on the L1 norm of any row of d (fp16 products), or 0 */
};

struct PfTile {
    int grp, m0;
};

/* A tile as the balanced down GEMM reads it (one record, no group lookup). */
struct PfDnTile {
    const uint8_t *td;              /* the group's down matrix in the tile layout */
    int slot;                       /* slot of the tile's first row */
    int mlen;                       /* rows */
    int dq6;                        /* down type Q6_K */
    float dbnd;                     /* the group's dbnd */
    int pad[2];
};

struct PfGemmArgs {
    const PfGroup *groups;
    const PfTile *tiles;
    const int *ntiles;              /* device count of valid tiles */
    const float *X;                 /* [* x H] activations (f32, natural order) */
    const uint16_t *X16;            /* [* x H] fp16 activations, scaled, permuted (v2), or NULL */
    const float *xinv, *xfwd;       /* per X row power-of-two scales (fp16 mode), or NULL */
    float *act;                     /* [slots x I]: silu(gate) * up (f32 operand modes) */
    uint16_t *act16;                /* [slots x I]: the same in fp16, each 16-column part scaled by the
                                       power of two of its pmax entry (fp16 mode) */
    float *pmax;                    /* [slots][inter / 16] partial max |act| (fp16 mode) */
    float *out;                     /* [slots x H]: down products (f32), when out16 is NULL */
    uint16_t *out16;                /* [slots x H]: the same in fp16, row s scaled by 2^-oexp[s], or NULL */
    int8_t *oexp;                   /* [slots] scale exponents of out16's rows */
    int H, I;
    int chunk;                      /* rows per tile of the tile list (pf_gemm_chunk) */
    int dn_nt;                      /* down GEMM: output tiles per workgroup (set by the launcher) */
    int gu_pers;                    /* fp16 gate/up on the persistent grid: 0 no, 1 every unit Q4_K,
                                       2 every unit Q6_K (one type for all, H / 256 even and >= 8) */
    int *gu_ctr;                    /* [8] its work counters, zeroed by the plan kernel */
    const int *dn_bnd;              /* [n_cu + 1] first unit of each workgroup of the balanced down
                                       GEMM, written by the plan kernel (with dn_tiles), or NULL */
    const PfDnTile *dn_tiles;       /* [max_tiles] the tile list as down records, or NULL */
    int dn_spare;                   /* with dn_tiles: a slot past the last, which takes the balanced down
                                       GEMM's products of rows past a tile's end (never read) */
    /* both GEMMs in one persistent kernel (with gu_pers and dn_tiles): each
     * XCD owns tiles [xcd_tb[x], xcd_tb[x + 1]) for both, its workgroups
     * taking gate/up units, then down chunks whose tile's gate/up units are
     * done (tile_done[tile] == inter / 128); the plan kernel writes the
     * bounds and zeroes the counters */
    int fused;
    const int *xcd_tb;              /* [9] */
    int *dn_ctr;                    /* [8] down chunks taken, per XCD */
    int *tile_done;                 /* [max_tiles] gate/up units done, per tile */
    int *err;                       /* device error word: bit 8 = a tile wait gave up */
};

/* Tile weight of the fused kernel's split of the tiles over the XCDs (both
 * GEMMs' cost of a tile of ms 32-row blocks, in relative units). */
#define PF_FX_CA 10
#define PF_FX_CB 3

/* The balanced down GEMM's units are (tile, PF_DN_ROWS output rows); the plan
 * kernel splits them over the workgroups by a cost model measured on the
 * all-Q6_K and Zipf 2048-wide layers (units of about 0.25 us): a unit of a
 * tile with ms 32-row blocks costs PF_DN_CA + PF_DN_CB * ms, a tile range's
 * start (row scales and activation staging) PF_DN_CP more.  PF_DN_CP is below
 * the measured ~10 us per range start: a range that starts on a tile's first
 * unit is charged its own start, the others are not, and the lower charge
 * measured fastest (kernel trace, 8 / 5 / 28 against 8 / 5 / 40 and 4 / 3 / 16
 * in these units: -1.6 and -2.9 us on the two layers). */
#define PF_DN_ROWS 256
#define PF_DN_CA 8
#define PF_DN_CB 5
#define PF_DN_CP 28

/* Whether prefill runs both fp16 GEMMs as one persistent kernel where it can
 * (roaster_prefill_fused_gemm). */
bool pf_fused_enabled();

/* Rows per tile the GEMMs of operand mode op expect in the tile list;
 * mixed_gate_up: the gate and up matrices of some group differ in type. */
int pf_gemm_chunk(int op, bool mixed_gate_up);

/* Launch the gate/up and down GEMMs over up to max_tiles tiles.  op: PF_F16,
 * PF_SPLIT or PF_BF16 (gemm.h).  0 or ROASTER_EDEVICE. */
int pf_gemm_launch(const PfGemmArgs &A, int max_tiles, int op);

/* The down GEMM alone in split mode as a plain product: out[slot][r] =
 * act[slot] . W[r] over A.I columns for A.H (a multiple of 64) rows of each
 * group's d matrix.  0 or ROASTER_EDEVICE. */
int pf_matmul_launch(const PfGemmArgs &A, int max_tiles);

#endif
