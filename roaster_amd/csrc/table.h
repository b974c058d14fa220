/*
 * table.h -- internal layout of the HBM expert table (table.hip).
 */
#ifndef ROASTER_TABLE_H
#define ROASTER_TABLE_H

#include <vector>
#include "decode.h"

/* Device addresses of one layer's matrices in the MFMA tile layout (tile.h). */
struct TileLayer {
    const uint8_t *gate, *up, *down;      /* [E] consecutive matrices */
    const uint8_t *sgate, *sup, *sdown;
};

/* Types, sizes and offsets of one layer's matrices (types may differ by layer). */
struct LayerGeo {
    int q6[3], sh_q6[3];                  /* 0 = Q4_K, 1 = Q6_K */
    size_t eb[3], sb[3];                  /* GGML bytes: one routed expert's matrix / the shared one's */
    size_t off_exps[3], off_sh[3];        /* offsets inside the layer's GGML region */
    size_t teb[3], tsb[3];                /* the same in the tile layout */
    size_t toff_exps[3], toff_sh[3];
    size_t base, tbase;                   /* the layer's offsets in qmem / tmem */
};

struct RoasterTable {
    RoasterTableDesc d;
    std::vector<LayerGeo> geo;
    size_t qbytes, tbytes, fbytes;
    uint8_t *qmem = nullptr; /* quantised matrices (GGML layout), all layers */
    uint8_t *tmem = nullptr; /* the same matrices in the MFMA tile layout (prefill GEMM operands) */
    float *fmem = nullptr;   /* routers and gate vectors */
    std::vector<DecLayer> layers_h;
    DecLayer *layers_d = nullptr;
    std::vector<TileLayer> tlayers_h;
    float *dbound = nullptr; /* [n_layers][E + 1]: bound on the L1 norm of any row of each down matrix */
};

#endif
