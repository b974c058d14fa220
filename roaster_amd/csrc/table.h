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

struct RoasterTable {
    RoasterTableDesc d;
    size_t eb[3];            /* bytes of one routed expert's gate / up / down */
    size_t sb[3];            /* bytes of the shared expert's gate / up / down */
    size_t off_exps[3];      /* offsets inside a layer */
    size_t off_sh[3];
    size_t layer_bytes;
    size_t qbytes, fbytes;
    uint8_t *qmem = nullptr; /* quantised matrices, all layers */
    float *fmem = nullptr;   /* routers and gate vectors */
    std::vector<DecLayer> layers_h;
    DecLayer *layers_d = nullptr;
    /* the same matrices in the MFMA tile layout (prefill GEMM operands) */
    size_t teb[3], tsb[3], toff_exps[3], toff_sh[3];
    size_t tlayer_bytes, tbytes;
    uint8_t *tmem = nullptr;
    std::vector<TileLayer> tlayers_h;
};

#endif
