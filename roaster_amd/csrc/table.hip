/*
 * table.hip -- the HBM-resident expert table and synthetic inputs.
 *
 * Replaces the reference's per-layer LRU expert cache (weights.c:420-652,
 * 952-1112): every expert of every layer is uploaded once.  Per layer the
 * routed experts of one matrix kind are contiguous, [E][rows][row_bytes], which
 * is exactly the GGUF 3-D *_exps tensor (weights.c:380-419 slices expert e at
 * e * size / E), followed by the shared expert's three matrices.  Routers
 * ([E x H] f32) and shared-gate vectors ([H] f32) sit in a second allocation.
 * A third allocation holds every matrix again in the MFMA tile layout of
 * tile.h (same order), rebuilt on the device after every upload; the prefill
 * GEMMs read only that copy, decode only the GGML copy.
 */
#include "internal.h"
#include "decode.h"
#include "table.h"
#include "synth.h"
#include "tile.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <vector>

static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

/* types: [n_layers][6] = routed gate, up, down, shared gate, up, down (0 = Q4_K,
 * 1 = Q6_K), or NULL for the description's types in every layer. */
extern "C" RoasterTable *roaster_table_create_layers(const RoasterTableDesc *d, const int *types)
{
    std::lock_guard<std::recursive_mutex> g(rt_lock());
    if (rt_init_locked()) return NULL;
    if (!d || d->n_layers <= 0 || d->n_experts < RTOPK || d->n_experts > 4096 || !d->hidden || !d->inter ||
        d->hidden % RQK || d->inter % RQK || d->hidden > 2048 || d->inter > 2048) {
        rt_fail(ROASTER_EINVAL, "invalid table description");
        return NULL;
    }
    for (int i = 0; types && i < 6 * d->n_layers; i++)
        if (types[i] != 0 && types[i] != 1) {
            rt_fail(ROASTER_EINVAL, "invalid matrix type %d (0 = Q4_K, 1 = Q6_K)", types[i]);
            return NULL;
        }
    RoasterTable *t = new RoasterTable();
    t->d = *d;
    const size_t H = d->hidden, I = d->inter, E = (size_t)d->n_experts;
    t->geo.resize(d->n_layers);
    size_t qoff = 0, toff = 0;
    for (int l = 0; l < d->n_layers; l++) {
        LayerGeo &G = t->geo[l];
        for (int k = 0; k < 3; k++) {
            G.q6[k] = types ? types[6 * l + k] : (d->q6[k] ? 1 : 0);
            G.sh_q6[k] = types ? types[6 * l + 3 + k] : (d->sh_q6[k] ? 1 : 0);
            const size_t rows = k == 2 ? H : I, cols = k == 2 ? I : H;
            G.eb[k] = rq_mat_bytes(G.q6[k], rows, cols);
            G.sb[k] = rq_mat_bytes(G.sh_q6[k], rows, cols);
            G.teb[k] = tl_mat_bytes(G.q6[k], rows, cols);
            G.tsb[k] = tl_mat_bytes(G.sh_q6[k], rows, cols);
        }
        size_t off = 0, tof = 0;
        for (int k = 0; k < 3; k++) {
            G.off_exps[k] = off; off += align256(E * G.eb[k]);
            G.toff_exps[k] = tof; tof += align256(E * G.teb[k]);
        }
        for (int k = 0; k < 3; k++) {
            G.off_sh[k] = off; off += align256(G.sb[k]);
            G.toff_sh[k] = tof; tof += align256(G.tsb[k]);
        }
        G.base = qoff; qoff += off;
        G.tbase = toff; toff += tof;
    }
    t->qbytes = qoff;
    t->tbytes = toff;
    t->fbytes = (size_t)d->n_layers * (E * H + H) * sizeof(float);
    if (hipMalloc((void **)&t->qmem, t->qbytes + RT_TAIL_PAD) != hipSuccess ||
        hipMalloc((void **)&t->tmem, t->tbytes + RT_TAIL_PAD) != hipSuccess ||
        hipMalloc((void **)&t->fmem, t->fbytes) != hipSuccess ||
        hipMalloc((void **)&t->layers_d, sizeof(DecLayer) * d->n_layers) != hipSuccess ||
        hipMalloc((void **)&t->dbound, sizeof(float) * d->n_layers * (E + 1)) != hipSuccess ||
        hipMemset(t->dbound, 0, sizeof(float) * d->n_layers * (E + 1)) != hipSuccess) {
        (void)hipGetLastError();
        rt_fail(ROASTER_ENOMEM, "expert table of %zu bytes does not fit in HBM", t->qbytes + t->tbytes + t->fbytes);
        if (t->qmem) (void)hipFree(t->qmem);
        if (t->tmem) (void)hipFree(t->tmem);
        if (t->fmem) (void)hipFree(t->fmem);
        if (t->layers_d) (void)hipFree(t->layers_d);
        if (t->dbound) (void)hipFree(t->dbound);
        delete t;
        return NULL;
    }
    rt_register_device_range(t->qmem, t->qbytes);
    rt_register_device_range(t->fmem, t->fbytes);
    t->layers_h.resize(d->n_layers);
    t->tlayers_h.resize(d->n_layers);
    for (int l = 0; l < d->n_layers; l++) {
        const LayerGeo &G = t->geo[l];
        DecLayer &L = t->layers_h[l];
        uint8_t *base = t->qmem + G.base;
        L.gate = base + G.off_exps[0];
        L.up = base + G.off_exps[1];
        L.down = base + G.off_exps[2];
        L.sgate = base + G.off_sh[0];
        L.sup = base + G.off_sh[1];
        L.sdown = base + G.off_sh[2];
        L.router = t->fmem + (size_t)l * (E * H + H);
        L.gate_inp = L.router + E * H;
        for (int k = 0; k < 3; k++) {
            L.eb[k] = G.eb[k];
            L.q6[k] = G.q6[k];
            L.sq6[k] = G.sh_q6[k];
        }
        TileLayer &TL = t->tlayers_h[l];
        uint8_t *tbase = t->tmem + G.tbase;
        TL.gate = tbase + G.toff_exps[0];
        TL.up = tbase + G.toff_exps[1];
        TL.down = tbase + G.toff_exps[2];
        TL.sgate = tbase + G.toff_sh[0];
        TL.sup = tbase + G.toff_sh[1];
        TL.sdown = tbase + G.toff_sh[2];
    }
    if (rt_check(hipMemcpy(t->layers_d, t->layers_h.data(), sizeof(DecLayer) * d->n_layers, hipMemcpyHostToDevice),
                 "layer table upload")) {
        roaster_table_destroy(t);
        return NULL;
    }
    return t;
}

extern "C" RoasterTable *roaster_table_create(const RoasterTableDesc *d) { return roaster_table_create_layers(d, NULL); }

extern "C" void roaster_table_destroy(RoasterTable *t)
{
    std::lock_guard<std::recursive_mutex> g(rt_lock());
    if (!t) return;
    (void)hipStreamSynchronize(rt().stream);
    rt_unregister_device_range(t->qmem);
    rt_unregister_device_range(t->fmem);
    (void)hipFree(t->qmem);
    (void)hipFree(t->tmem);
    (void)hipFree(t->fmem);
    (void)hipFree(t->layers_d);
    (void)hipFree(t->dbound);
    delete t;
}

extern "C" size_t roaster_table_bytes(const RoasterTable *t) { return t ? t->qbytes + t->tbytes + t->fbytes : 0; }

static uint8_t *mat_ptr(const RoasterTable *t, int layer, int expert, int kind)
{
    const LayerGeo &G = t->geo[layer];
    uint8_t *base = t->qmem + G.base;
    if (expert == t->d.n_experts) return base + G.off_sh[kind];
    return base + G.off_exps[kind] + (size_t)expert * G.eb[kind];
}

static size_t mat_bytes(const RoasterTable *t, int layer, int expert, int kind)
{
    const LayerGeo &G = t->geo[layer];
    return expert == t->d.n_experts ? G.sb[kind] : G.eb[kind];
}

/* ---- MFMA tile layout ------------------------------------------------------ */
__device__ __forceinline__ uint32_t rd32(const uint8_t *p)
{
    return p[0] | (p[1] << 8) | (p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* One thread per lane record of nmat consecutive [rows x cols] matrices
 * (tile.h): record (m, tile g * nkb + kb, lane n + 32 h) from GGML block
 * (row 32 g + n, kb) of matrix m. */
__global__ void tile_repack_kernel(const uint8_t *src, uint8_t *dst, size_t src_mat, size_t dst_mat, int rows,
                                   int cols, int nmat, int q6)
{
    const int nkb = cols / RQK;
    const size_t per_mat = (size_t)(rows / TL_ROWS) * nkb * 64, total = per_mat * (size_t)nmat;
    const size_t bb = q6 ? RQ6K_BYTES : RQ4K_BYTES;
    for (size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x; gid < total;
         gid += (size_t)gridDim.x * blockDim.x) {
        const size_t m = gid / per_mat, rem = gid % per_mat, tt = rem / 64;
        const int l = (int)(rem % 64), n = l & 31, h = l >> 5;
        const int kb = (int)(tt % nkb), g = (int)(tt / nkb);
        const uint8_t *blk = src + m * src_mat + ((size_t)(TL_ROWS * g + n) * nkb + kb) * bb;
        uint8_t *tile = dst + m * dst_mat + tt * TL_BYTES(q6);
        uint32_t rec[28];
        if (q6) {
            for (int i = 0; i < 16; i++) rec[i] = rd32(blk + 4 * (16 * h + i));
            for (int i = 0; i < 8; i++) rec[16 + i] = rd32(blk + 128 + 4 * (8 * h + i));
            rec[24] = rd32(blk + 192 + 8 * h);
            rec[25] = rd32(blk + 196 + 8 * h);
            rec[26] = blk[208] | (blk[209] << 8);
            rec[27] = 0;
        } else {
            for (int i = 0; i < 4; i++) rec[i] = rd32(blk + 4 * i);
            for (int i = 0; i < 16; i++) rec[4 + i] = rd32(blk + 16 + 4 * (16 * h + i));
        }
        const int nq = 4 * TL_SLICES(q6);
        for (int q = 0; q < nq; q++) *(uint32_t *)(tile + 1024 * (q / 4) + 16 * l + 4 * (q % 4)) = rec[q];
    }
}

static uint8_t *tmat_ptr(const RoasterTable *t, int layer, int expert, int kind)
{
    const LayerGeo &G = t->geo[layer];
    uint8_t *base = t->tmem + G.tbase;
    if (expert == t->d.n_experts) return base + G.toff_sh[kind];
    return base + G.toff_exps[kind] + (size_t)expert * G.teb[kind];
}

/* Bound on the L1 norm of every row of nmat consecutive [rows x cols] down
 * matrices (one workgroup per matrix), from the block headers alone: a Q6_K
 * weight is d sc (q - 32) with |q - 32| <= 32, so a 16-weight sub-block sums
 * to at most 16 * 32 |d| |sc|; a Q4_K weight is d sc q - dmin m with q <= 15,
 * so a 32-weight sub-block sums to at most 32 (15 |d| sc + |dmin| m).  The
 * prefill stores its per-row down products in fp16 scaled by this bound times
 * the row's largest activation, which no product can exceed. */
__global__ void __launch_bounds__(256) dbound_kernel(const uint8_t *src, size_t src_mat, int rows, int cols, int q6,
                                                     float *dst)
{
    __shared__ float wmax[4];
    const uint8_t *mat = src + (size_t)blockIdx.x * src_mat;
    const int nkb = cols / RQK;
    const size_t bb = q6 ? RQ6K_BYTES : RQ4K_BYTES;
    float mx = 0.0f;
    for (int r = threadIdx.x; r < rows; r += blockDim.x) {
        float s = 0.0f;
        for (int kb = 0; kb < nkb; kb++) {
            const uint8_t *blk = mat + ((size_t)r * nkb + kb) * bb;
            if (q6) {
                const float d = fabsf((float)__builtin_bit_cast(_Float16, (uint16_t)(blk[208] | (blk[209] << 8))));
                int sc = 0;
                for (int j = 0; j < 16; j++) sc += abs((int)(int8_t)blk[192 + j]);
                s += 512.0f * d * (float)sc;
            } else {
                const float d = fabsf((float)__builtin_bit_cast(_Float16, (uint16_t)(blk[0] | (blk[1] << 8))));
                const float dm = fabsf((float)__builtin_bit_cast(_Float16, (uint16_t)(blk[2] | (blk[3] << 8))));
                const uint8_t *q = blk + 4;
                int sc = 0, mn = 0;
                for (int j = 0; j < 8; j++) {
                    if (j < 4) {
                        sc += q[j] & 63;
                        mn += q[j + 4] & 63;
                    } else {
                        sc += (q[j + 4] & 15) | ((q[j - 4] >> 6) << 4);
                        mn += (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
                    }
                }
                s += 32.0f * (15.0f * d * (float)sc + dm * (float)mn);
            }
        }
        mx = fmaxf(mx, s);
    }
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = mx;
    __syncthreads();
    if (threadIdx.x == 0) dst[blockIdx.x] = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
}

/* Rebuild the tile copy of nmat consecutive matrices of one kind (routed
 * experts e0 .. e0 + nmat - 1, or the shared expert when e0 == E), and for
 * down matrices their row bounds. */
static int tile_repack(const RoasterTable *t, int layer, int e0, int nmat, int kind)
{
    const RoasterTableDesc &d = t->d;
    const LayerGeo &G = t->geo[layer];
    const bool sh = e0 == d.n_experts;
    const int q6 = sh ? G.sh_q6[kind] : G.q6[kind];
    const int rows = kind == 2 ? d.hidden : d.inter, cols = kind == 2 ? d.inter : d.hidden;
    const size_t total = (size_t)(rows / TL_ROWS) * (cols / RQK) * 64 * (size_t)nmat;
    const int blocks = (int)((total + 255) / 256 < 65536 ? (total + 255) / 256 : 65536);
    hipLaunchKernelGGL(tile_repack_kernel, dim3(blocks), dim3(256), 0, rt().stream, mat_ptr(t, layer, e0, kind),
                       tmat_ptr(t, layer, e0, kind), mat_bytes(t, layer, e0, kind), sh ? G.tsb[kind] : G.teb[kind], rows,
                       cols, nmat, q6);
    if (rt_check(hipGetLastError(), "tile repack launch")) return ROASTER_EDEVICE;
    if (kind == 2) {
        hipLaunchKernelGGL(dbound_kernel, dim3(nmat), dim3(256), 0, rt().stream, mat_ptr(t, layer, e0, kind),
                           mat_bytes(t, layer, e0, kind), rows, cols, q6,
                           t->dbound + (size_t)layer * (d.n_experts + 1) + e0);
        if (rt_check(hipGetLastError(), "down bound launch")) return ROASTER_EDEVICE;
    }
    return 0;
}

extern "C" int roaster_table_set_expert(RoasterTable *t, int layer, int expert, const void *gate, const void *up,
                                        const void *down)
{
    std::lock_guard<std::recursive_mutex> g(rt_lock());
    if (!t || layer < 0 || layer >= t->d.n_layers || expert < 0 || expert > t->d.n_experts || !gate || !up || !down)
        return rt_fail(ROASTER_EINVAL, "roaster_table_set_expert: bad arguments");
    const void *src[3] = { gate, up, down };
    for (int k = 0; k < 3; k++) {
        if (rt_check(hipMemcpy(mat_ptr(t, layer, expert, k), src[k], mat_bytes(t, layer, expert, k), hipMemcpyHostToDevice),
                     "expert upload"))
            return ROASTER_EDEVICE;
        if (int rc = tile_repack(t, layer, expert, 1, k)) return rc;
    }
    return rt_check(hipStreamSynchronize(rt().stream), "tile repack") ? ROASTER_EDEVICE : 0;
}

extern "C" int roaster_table_set_exps(RoasterTable *t, int layer, int kind, const void *data, size_t bytes)
{
    std::lock_guard<std::recursive_mutex> g(rt_lock());
    if (!t || layer < 0 || layer >= t->d.n_layers || kind < 0 || kind > 2 || !data)
        return rt_fail(ROASTER_EINVAL, "roaster_table_set_exps: bad arguments");
    if (bytes != (size_t)t->d.n_experts * t->geo[layer].eb[kind])
        return rt_fail(ROASTER_EINVAL, "roaster_table_set_exps: expected %zu bytes, got %zu",
                       (size_t)t->d.n_experts * t->geo[layer].eb[kind], bytes);
    if (rt_check(hipMemcpy(mat_ptr(t, layer, 0, kind), data, bytes, hipMemcpyHostToDevice), "exps upload"))
        return ROASTER_EDEVICE;
    if (int rc = tile_repack(t, layer, 0, t->d.n_experts, kind)) return rc;
    return rt_check(hipStreamSynchronize(rt().stream), "tile repack") ? ROASTER_EDEVICE : 0;
}

extern "C" int roaster_table_set_router(RoasterTable *t, int layer, const float *router, const float *gate_inp)
{
    std::lock_guard<std::recursive_mutex> g(rt_lock());
    if (!t || layer < 0 || layer >= t->d.n_layers || !router || !gate_inp)
        return rt_fail(ROASTER_EINVAL, "roaster_table_set_router: bad arguments");
    const DecLayer &L = t->layers_h[layer];
    const size_t EH = (size_t)t->d.n_experts * t->d.hidden;
    if (rt_check(hipMemcpy((void *)L.router, router, EH * 4, hipMemcpyHostToDevice), "router upload") ||
        rt_check(hipMemcpy((void *)L.gate_inp, gate_inp, t->d.hidden * 4, hipMemcpyHostToDevice), "gate upload"))
        return ROASTER_EDEVICE;
    return 0;
}

extern "C" int roaster_table_expert_ptrs(const RoasterTable *t, int layer, int expert, const void **gate,
                                         const void **up, const void **down)
{
    if (!t || layer < 0 || layer >= t->d.n_layers || expert < 0 || expert > t->d.n_experts)
        return rt_fail(ROASTER_EINVAL, "roaster_table_expert_ptrs: bad arguments");
    if (gate) *gate = mat_ptr(t, layer, expert, 0);
    if (up) *up = mat_ptr(t, layer, expert, 1);
    if (down) *down = mat_ptr(t, layer, expert, 2);
    return 0;
}

/* ---- synthetic inputs ----------------------------------------------------- */
extern "C" uint64_t roaster_synth_stream(int layer, int expert, int kind) { return rs_stream(layer, expert, kind); }

extern "C" void roaster_synth_q4k(uint64_t seed, uint64_t stream, size_t nblocks, float lo, float hi, void *out)
{
    const uint64_t key = rs_key(seed, stream);
    for (size_t b = 0; b < nblocks; b++) rs_q4k_block(key, b, lo, hi, (uint8_t *)out + b * RQ4K_BYTES);
}

extern "C" void roaster_synth_q6k(uint64_t seed, uint64_t stream, size_t nblocks, float lo, float hi, void *out)
{
    const uint64_t key = rs_key(seed, stream);
    for (size_t b = 0; b < nblocks; b++) rs_q6k_block(key, b, lo, hi, (uint8_t *)out + b * RQ6K_BYTES);
}

/* Box-Muller, one normal per counter pair, computed in double. */
extern "C" void roaster_synth_normal(uint64_t seed, uint64_t stream, size_t n, float sigma, float *out)
{
    const uint64_t key = rs_key(seed, stream);
    for (size_t i = 0; i < n; i++) {
        const uint64_t r1 = rs_at(key, 2 * i), r2 = rs_at(key, 2 * i + 1);
        const double u1 = ((double)(r1 >> 11) + 1.0) * 0x1p-53;
        const double u2 = (double)(r2 >> 11) * 0x1p-53;
        const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        out[i] = (float)(z * (double)sigma);
    }
}

/* One thread per super-block of a set of consecutive matrices (one kind of
 * one layer: E routed experts, matrix m at dst + m * mat_bytes). */
__global__ void synth_blocks_kernel(uint8_t *dst, size_t mat_bytes, size_t blocks_per_mat, int nmat,
                                    uint64_t seed, int layer, int expert0, int kind, int q6, float lo, float hi)
{
    const size_t total = blocks_per_mat * (size_t)nmat;
    for (size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x; gid < total;
         gid += (size_t)gridDim.x * blockDim.x) {
        const int m = (int)(gid / blocks_per_mat);
        const size_t b = gid % blocks_per_mat;
        const uint64_t key = rs_key(seed, rs_stream(layer, expert0 + m, kind));
        uint8_t *o = dst + (size_t)m * mat_bytes;
        if (!q6) {
            uint8_t blk[RQ4K_BYTES];
            rs_q4k_block(key, b, lo, hi, blk);
            uint32_t *w = (uint32_t *)(o + b * RQ4K_BYTES);
            for (int i = 0; i < RQ4K_BYTES / 4; i++)
                w[i] = blk[4 * i] | (blk[4 * i + 1] << 8) | (blk[4 * i + 2] << 16) | ((uint32_t)blk[4 * i + 3] << 24);
        } else {
            uint8_t blk[RQ6K_BYTES];
            rs_q6k_block(key, b, lo, hi, blk);
            uint16_t *w = (uint16_t *)(o + b * RQ6K_BYTES);
            for (int i = 0; i < RQ6K_BYTES / 2; i++) w[i] = (uint16_t)(blk[2 * i] | (blk[2 * i + 1] << 8));
        }
    }
}

extern "C" int roaster_table_synth(RoasterTable *t, uint64_t seed, const RoasterSynthSpec *spec)
{
    std::lock_guard<std::recursive_mutex> g(rt_lock());
    if (!t) return rt_fail(ROASTER_EINVAL, "roaster_table_synth: NULL table");
    RoasterSynthSpec s = { 1e-3f, 2e-2f, 1e-3f, 1e-2f, 0.02f, 0.02f };
    if (spec) s = *spec;
    const RoasterTableDesc &d = t->d;
    const size_t H = d.hidden, I = d.inter, E = (size_t)d.n_experts;
    hipStream_t st = rt().stream;
    for (int l = 0; l < d.n_layers; l++) {
        for (int k = 0; k < 3; k++) {
            const size_t rows = k == 2 ? H : I, cols = k == 2 ? I : H;
            const size_t bpm = rows * (cols / RQK);
            for (int shared = 0; shared < 2; shared++) {
                const int q6 = shared ? t->geo[l].sh_q6[k] : t->geo[l].q6[k];
                const int nmat = shared ? 1 : (int)E;
                const int e0 = shared ? (int)E : 0;
                uint8_t *dst = mat_ptr(t, l, e0, k);
                const size_t mb = mat_bytes(t, l, e0, k);
                const float lo = q6 ? s.q6k_lo : s.q4k_lo, hi = q6 ? s.q6k_hi : s.q4k_hi;
                const size_t total = bpm * (size_t)nmat;
                const int blocks = (int)((total + 255) / 256 < 65536 ? (total + 255) / 256 : 65536);
                hipLaunchKernelGGL(synth_blocks_kernel, dim3(blocks), dim3(256), 0, st, dst, mb, bpm, nmat, seed, l,
                                   e0, k, q6, lo, hi);
                if (rt_check(hipGetLastError(), "synth launch")) return ROASTER_EDEVICE;
                if (int rc = tile_repack(t, l, e0, nmat, k)) return rc;
            }
        }
    }
    std::vector<float> router(E * H), gi(H);
    for (int l = 0; l < d.n_layers; l++) {
        roaster_synth_normal(seed, roaster_synth_stream(l, 0, 3), E * H, s.router_sigma, router.data());
        roaster_synth_normal(seed, roaster_synth_stream(l, 0, 4), H, s.gate_inp_sigma, gi.data());
        const DecLayer &L = t->layers_h[l];
        if (rt_check(hipMemcpyAsync((void *)L.router, router.data(), E * H * 4, hipMemcpyHostToDevice, st), "router") ||
            rt_check(hipMemcpyAsync((void *)L.gate_inp, gi.data(), H * 4, hipMemcpyHostToDevice, st), "gate_inp") ||
            rt_check(hipStreamSynchronize(st), "synth sync"))
            return ROASTER_EDEVICE;
    }
    return 0;
}
