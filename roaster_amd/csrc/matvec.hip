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

#include <type_traits>

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

static int g_dense_mfma_t = 2;             /* tokens from which dense_mm8_kernel serves a call */

template <bool Q6, bool ONE, int KB>
__global__ void __launch_bounds__(MV_THREADS) dense_mv_kernel(const uint8_t *W, const float *X, float *Y, int rows,
                                                              int cols, int T)
{
    extern __shared__ __align__(16) float xs[];            /* [T][cols] + run sums [T][cols / 16] (T > 1) */
    const int lane = threadIdx.x & 63;
    const int nb = cols / RQK, lpr = lanes_per_row(nb), rpw = 64 / lpr;
    const int rw = lane / lpr, lr = lane % lpr, c = lr & 7, lb = lr >> 3;
    const size_t bs = Q6 ? RQ6K_BYTES : RQ4K_BYTES, row_bytes = (size_t)nb * bs;
    /* KB super-blocks per lane: lb, lb + 8 (rows of more than 8 blocks) */
    bool blk_live[KB];
    int ca[KB], cb[KB];
#pragma unroll
    for (int k = 0; k < KB; k++) {
        blk_live[k] = lb + 8 * k < nb;
        ca[k] = (lb + 8 * k) * RQK + q_run_a<Q6>(c);
        cb[k] = ca[k] + q_run_b_off<Q6>();
    }
    float4 xa[KB][4], xb[KB][4];
    float sxa[KB], sxb[KB];
    float *xsum = xs + (size_t)T * cols;
    if (ONE) {
#pragma unroll
        for (int k = 0; k < KB; k++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                xa[k][i] = blk_live[k] ? gld_f4(X + ca[k] + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
                xb[k][i] = blk_live[k] ? gld_f4(X + cb[k] + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
            sxa[k] = ((xa[k][0].x + xa[k][0].y) + (xa[k][0].z + xa[k][0].w)) + ((xa[k][1].x + xa[k][1].y) + (xa[k][1].z + xa[k][1].w)) +
                     (((xa[k][2].x + xa[k][2].y) + (xa[k][2].z + xa[k][2].w)) + ((xa[k][3].x + xa[k][3].y) + (xa[k][3].z + xa[k][3].w)));
            sxb[k] = ((xb[k][0].x + xb[k][0].y) + (xb[k][0].z + xb[k][0].w)) + ((xb[k][1].x + xb[k][1].y) + (xb[k][1].z + xb[k][1].w)) +
                     (((xb[k][2].x + xb[k][2].y) + (xb[k][2].z + xb[k][2].w)) + ((xb[k][3].x + xb[k][3].y) + (xb[k][3].z + xb[k][3].w)));
        }
    } else {
        for (int i = threadIdx.x; i < T * cols / 4; i += MV_THREADS) ((float4 *)xs)[i] = gld_f4(X + 4 * i);
        __syncthreads();
        for (int i = threadIdx.x; i < T * cols / 16; i += MV_THREADS) xsum[i] = sum16(xs + 16 * i);
        __syncthreads();
    }
    const int gw = blockIdx.x * (MV_THREADS / 64) + (threadIdx.x >> 6), nw = gridDim.x * (MV_THREADS / 64);
    const int npass = (rows + rpw - 1) / rpw;
    for (int p0 = gw; p0 < npass; p0 += nw * DMV_PF) {
        QChunk ch[DMV_PF][KB];
#pragma unroll
        for (int f = 0; f < DMV_PF; f++) {
            const int row = (p0 + f * nw) * rpw + rw;
#pragma unroll
            for (int k = 0; k < KB; k++)
                if (blk_live[k] && row < rows)
                    ch[f][k] = q_load<Q6>(W + (size_t)row * row_bytes + (size_t)(lb + 8 * k) * bs, c);
        }
#pragma unroll
        for (int f = 0; f < DMV_PF; f++) {
            const int pass = p0 + f * nw;
            if (pass >= npass) break;
            const int row = pass * rpw + rw;
            const bool live = row < rows;
            for (int t = 0; t < (ONE ? 1 : T); t++) {
                float part = 0.0f;
#pragma unroll
                for (int k = 0; k < KB; k++) {
                    if (live && blk_live[k]) {
                        if (ONE) {
                            part += q_chunk_dot_r<Q6>(ch[f][k], c, xa[k], xb[k], sxa[k], sxb[k]);
                        } else {
                            const float *x = xs + (size_t)t * cols, *sx = xsum + (size_t)t * (cols / 16);
                            part += q_chunk_dot<Q6>(ch[f][k], c, x + ca[k], x + cb[k], sx[ca[k] >> 4], sx[cb[k] >> 4]);
                        }
                    }
                }
                part = group_sum_w(part, lpr);
                if (live && lr == 0) Y[(size_t)t * rows + row] = part;
            }
        }
    }
}

/* ---- 2..8 tokens on MFMA -----------------------------------------------------
 * y[t][r] = W[r] . x[t] with the quants as MFMA operands and the block scales
 * applied in f32 per scale sub-block (the reference's fold, kernels.c:
 * 1844-1874: d sc sum(q x) - dmin m sum(x) for Q4_K, d sc sum(q x) -
 * 32 d sc sum(x) for Q6_K):
 *   B = 16 weight rows x one scale sub-block (Q4_K: 32 weights on
 *       v_mfma_f32_16x16x32_f16, Q6_K: 16 on v_mfma_f32_16x16x16f16); each
 *       quant q enters as the fp16 bit pattern q, i.e. q * 2^-24 (a
 *       denormal, exact), one mask per pair;
 *   A = the tokens' activations of the super-block, scaled per (token,
 *       super-block) by a power of two (max |x| in [2^14, 2^15)) and split
 *       into fp16 hi + lo, row m = 2t + (lo);
 *   C = per-sub-block sums p: lane l holds weight row l % 16 and tokens
 *       2(l / 16), 2(l / 16) + 1 (hi and lo rows) and accumulates
 *       z += (2^24 d sc)(p_hi + p_lo) - (dmin m) X_s over the super-block's
 *       sub-blocks (X_s: the sub-block's scaled activation sum, f32), then
 *       y += 2^-e z.
 * x = hi + lo keeps 22 of the 24 bits of an f32 activation; products and
 * sums are f32.  mm8_prep_kernel builds the A operands once per call, in
 * fragment order (lane l's 8 / 4 halves contiguous; inside a sub-block the
 * K order follows the quant pairs the masks produce, bytes 0, 2, 1, 3 of each
 * dword); every workgroup of dense_mm8_kernel copies them into LDS, and each
 * wave streams 16-row groups, the next super-block's raw quants in flight
 * while the current one computes. */
#define MM8_T 512
#define MM8_W (MM8_T / 64)

typedef _Float16 mm_f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 mm_f16x4 __attribute__((ext_vector_type(4)));
typedef float mm_f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t gld_u32a2(const void *p)
{
    typedef uint32_t __attribute__((aligned(2))) u32_a2;
    return *(const GAS u32_a2 *)p;
}

/* Operand buffer of one call: A fragments [cols / SB][64 lanes] (cols * 32
 * bytes), sub-block sums xs [cols / SB][8 tokens], super-block scales
 * ge [cols / 256][8 tokens] (2^-e). */
__host__ __device__ static inline size_t mm8_frag_bytes(size_t cols) { return cols * 32; }
__host__ __device__ static inline size_t mm8_xs_bytes(size_t cols, int q6) { return cols / (q6 ? 16 : 32) * 8 * 4; }
__host__ __device__ static inline size_t mm8_buf_bytes(size_t cols, int q6) { return mm8_frag_bytes(cols) + mm8_xs_bytes(cols, q6) + cols / RQK * 8 * 4; }

/* Workgroup kb (256 threads): thread (t = tid / 32, c = tid % 32) holds
 * columns 256 kb + 8c .. + 7 of token t; it writes both halves (hi, lo) of
 * every fragment slot those columns fill, and sub-block sums are reduced
 * over the 4 (Q4_K) or 2 (Q6_K) threads of a sub-block. */
template <bool Q6>
__global__ void __launch_bounds__(256) mm8_prep_kernel(const float *X, int cols, int T, uint8_t *buf)
{
    constexpr int SB = Q6 ? 16 : 32, FB = Q6 ? 512 : 1024;
    const int kb = blockIdx.x, tid = threadIdx.x, t = tid >> 5, c = tid & 31;
    const int ns = cols / SB;
    uint8_t *frag = buf;
    float *xs = (float *)(buf + mm8_frag_bytes(cols));
    float *ge = xs + (size_t)ns * 8;
    float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0;
    if (t < T) {
        const float *xp = X + (size_t)t * cols + RQK * kb + 8 * c;
        v0 = gld_f4(xp);
        v1 = gld_f4(xp + 4);
    }
    float mx = fmaxf(fmaxf(fmaxf(fabsf(v0.x), fabsf(v0.y)), fmaxf(fabsf(v0.z), fabsf(v0.w))),
                     fmaxf(fmaxf(fabsf(v1.x), fabsf(v1.y)), fmaxf(fabsf(v1.z), fabsf(v1.w))));
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 32));
    int e = 0;
    if (mx > 0.0f && mx <= 3.0e38f) {
        int E;
        (void)frexpf(mx, &E);
        e = min(max(15 - E, -100), 100);
    }
    if (c == 0) ge[kb * 8 + t] = ldexpf(1.0f, -e);
    const float w8[8] = {ldexpf(v0.x, e), ldexpf(v0.y, e), ldexpf(v0.z, e), ldexpf(v0.w, e),
                         ldexpf(v1.x, e), ldexpf(v1.y, e), ldexpf(v1.z, e), ldexpf(v1.w, e)};
    _Float16 hi[8], lo[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        hi[i] = (_Float16)w8[i];
        lo[i] = (_Float16)(w8[i] - (float)hi[i]);
    }
    float sum = ((w8[0] + w8[1]) + (w8[2] + w8[3])) + ((w8[4] + w8[5]) + (w8[6] + w8[7]));
    if (!Q6) {
        /* sub-block s = c / 4 of this super-block, lane group j = c % 4: slots
         * 0..7 = columns 0, 2, 1, 3, 4, 6, 5, 7 */
        const int f = kb * 8 + (c >> 2), j = c & 3;
        const mm_f16x8 h8 = {hi[0], hi[2], hi[1], hi[3], hi[4], hi[6], hi[5], hi[7]};
        const mm_f16x8 l8 = {lo[0], lo[2], lo[1], lo[3], lo[4], lo[6], lo[5], lo[7]};
        if (t < 8) {
            *(mm_f16x8 *)(frag + (size_t)f * FB + (16 * j + 2 * t) * 16) = h8;
            *(mm_f16x8 *)(frag + (size_t)f * FB + (16 * j + 2 * t + 1) * 16) = l8;
        }
        sum += __shfl_xor(sum, 1, 32);
        sum += __shfl_xor(sum, 2, 32);
        if (j == 0) xs[f * 8 + t] = sum;
    } else {
        /* sub-block s = c / 2, lane groups j = 2 (c % 2) and + 1, 4 columns
         * each: slots 0..3 = columns 0, 2, 1, 3 */
        const int f = kb * 16 + (c >> 1), j0 = 2 * (c & 1);
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const mm_f16x4 h4 = {hi[4 * u], hi[4 * u + 2], hi[4 * u + 1], hi[4 * u + 3]};
            const mm_f16x4 l4 = {lo[4 * u], lo[4 * u + 2], lo[4 * u + 1], lo[4 * u + 3]};
            *(mm_f16x4 *)(frag + (size_t)f * FB + (16 * (j0 + u) + 2 * t) * 8) = h4;
            *(mm_f16x4 *)(frag + (size_t)f * FB + (16 * (j0 + u) + 2 * t + 1) * 8) = l4;
        }
        sum += __shfl_xor(sum, 1, 32);
        if ((c & 1) == 0) xs[f * 8 + t] = sum;
    }
}

struct Mm8Q4 { uint4 hd; uint2 p[4]; };              /* header; qs bytes 32g + 8j .. + 7 */
struct Mm8Q6 { uint32_t L[8], Hq[4]; uint4 sc; uint32_t d; };

__device__ __forceinline__ void mm8_load(Mm8Q4 &r, const uint8_t *blk, int j)
{
    r.hd = gld_u4(blk);
#pragma unroll
    for (int g = 0; g < 4; g++) r.p[g] = gld_u2(blk + 16 + 32 * g + 8 * j);
}

/* Q6_K sub-block s (weights 16 s .. 16 s + 15; n = s / 8, q = (s % 8) / 2,
 * hb = s % 2, kernels.c:449-468): lane j's 4 quants are the nibble q / 2 of
 * ql dword L[4 n + 2 (q % 2) + hb] (bytes 64 n + 32 (q % 2) + 16 hb + 4 j ..)
 * with bits 2 q of qh dword Hq[2 n + hb] (bytes 128 + 32 n + 16 hb + 4 j ..). */
__device__ __forceinline__ void mm8_load(Mm8Q6 &r, const uint8_t *blk, int j)
{
#pragma unroll
    for (int n = 0; n < 2; n++)
#pragma unroll
        for (int q = 0; q < 2; q++)
#pragma unroll
            for (int hb = 0; hb < 2; hb++) r.L[4 * n + 2 * q + hb] = gld_u32a2(blk + 64 * n + 32 * q + 16 * hb + 4 * j);
#pragma unroll
    for (int n = 0; n < 2; n++)
#pragma unroll
        for (int hb = 0; hb < 2; hb++) r.Hq[2 * n + hb] = gld_u32a2(blk + 128 + 32 * n + 16 * hb + 4 * j);
    r.sc = gld_u4a2(blk + 192);
    r.d = gld_u16(blk + 208);
}

/* Super-block kb of one 16-row group: 8 (Q4_K) or 16 (Q6_K) MFMAs; z0 / z1
 * accumulate tokens 2 (l / 16) and + 1 of row l % 16.  frag: this
 * super-block's A fragments, xs: its sub-block sums [sub][8 tokens]. */
__device__ __forceinline__ void mm8_block(const Mm8Q4 &r, const uint8_t *frag, const float *xs, int lane, float &z0,
                                          float &z1)
{
    const float d = f16_bits_to_f32(r.hd.x & 0xFFFFu) * 16777216.0f, dmin = f16_bits_to_f32(r.hd.x >> 16);
    const uint32_t s03 = r.hd.y, s47 = r.hd.z, s811 = r.hd.w;
    const int t0 = 2 * (lane >> 4);
#pragma unroll
    for (int s = 0; s < 8; s++) {
        const int g = s >> 1, hi = s & 1;
        int sc, m;
        if (s < 4) {
            sc = byte_of(s03, s) & 63;
            m = byte_of(s47, s) & 63;
        } else {
            sc = (byte_of(s811, s - 4) & 15) | ((byte_of(s03, s - 4) >> 6) << 4);
            m = (byte_of(s811, s - 4) >> 4) | ((byte_of(s47, s - 4) >> 6) << 4);
        }
        const uint32_t x = r.p[g].x >> (4 * hi), y = r.p[g].y >> (4 * hi);
        const uint4 bq = make_uint4(x & 0x000F000Fu, (x >> 8) & 0x000F000Fu, y & 0x000F000Fu, (y >> 8) & 0x000F000Fu);
        const mm_f16x8 b = __builtin_bit_cast(mm_f16x8, bq);
        const mm_f16x8 a = *(const mm_f16x8 *)(frag + s * 1024 + lane * 16);
        const mm_f32x4 cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, (mm_f32x4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        const float2 xm = *(const float2 *)(xs + s * 8 + t0);
        const float sa = d * (float)sc, ma = dmin * (float)m;
        z0 = fmaf(sa, cc[0] + cc[1], z0);
        z0 = fmaf(-ma, xm.x, z0);
        z1 = fmaf(sa, cc[2] + cc[3], z1);
        z1 = fmaf(-ma, xm.y, z1);
    }
}

__device__ __forceinline__ void mm8_block(const Mm8Q6 &r, const uint8_t *frag, const float *xs, int lane, float &z0,
                                          float &z1)
{
    const float d = f16_bits_to_f32(r.d) * 16777216.0f;
    const int t0 = 2 * (lane >> 4);
#pragma unroll
    for (int s = 0; s < 16; s++) {
        const int n = s >> 3, q = (s & 7) >> 1, hb = s & 1;
        const uint32_t lw = r.L[4 * n + 2 * (q & 1) + hb], hw = r.Hq[2 * n + hb];
        const uint32_t v = ((lw >> (4 * (q >> 1))) & 0x0F0F0F0Fu) | (((hw >> (2 * q)) & 0x03030303u) << 4);
        const uint2 bq = make_uint2(v & 0x00FF00FFu, (v >> 8) & 0x00FF00FFu);
        const mm_f16x4 b = __builtin_bit_cast(mm_f16x4, bq);
        const mm_f16x4 a = *(const mm_f16x4 *)(frag + s * 512 + lane * 8);
        const mm_f32x4 cc = __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, (mm_f32x4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        const float2 xm = *(const float2 *)(xs + s * 8 + t0);
        const uint32_t sw = s < 4 ? r.sc.x : s < 8 ? r.sc.y : s < 12 ? r.sc.z : r.sc.w;
        /* sa carries the quants' 2^24; the 32 d sc of the offset does not */
        const float sa = d * (float)(int)(int8_t)byte_of(sw, s & 3), ma = sa * 1.9073486328125e-06f;
        z0 = fmaf(sa, cc[0] + cc[1], z0);
        z0 = fmaf(-ma, xm.x, z0);
        z1 = fmaf(sa, cc[2] + cc[3], z1);
        z1 = fmaf(-ma, xm.y, z1);
    }
}

template <bool Q6>
__global__ void __launch_bounds__(MM8_T) dense_mm8_kernel(const uint8_t *W, const uint8_t *buf, float *Y, int rows,
                                                          int cols, int T, int ksplit)
{
    extern __shared__ __align__(16) uint8_t mm8_lds[];
    constexpr int SB = Q6 ? 16 : 32;                  /* weights per scale sub-block */
    constexpr int FB = Q6 ? 512 : 1024;               /* bytes per A fragment (64 lanes) */
    constexpr size_t BS = Q6 ? RQ6K_BYTES : RQ4K_BYTES;
    typedef typename std::conditional<Q6, Mm8Q6, Mm8Q4>::type Raw;
    const int ns = cols / SB, nb = cols / RQK;
    /* the call's operands: fragments, sub-block sums and super-block scales */
    const int n16 = (int)(mm8_buf_bytes(cols, Q6) / 16);
    for (int i = threadIdx.x; i < n16; i += MM8_T) ((uint4 *)mm8_lds)[i] = gld_u4(buf + 16 * (size_t)i);
    const uint8_t *frag = mm8_lds;
    const float *xs = (const float *)(mm8_lds + mm8_frag_bytes(cols));
    const float *ge = xs + (size_t)ns * 8;
    __syncthreads();
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int ngroups = (rows + 15) >> 4;
    if (ksplit) {
        /* few groups (nb <= 16): a workgroup per group, wave w takes super-
         * blocks w and w + 8, the 8 partial sums added by wave 0 in wave order */
        __shared__ float2 red[MM8_W][64];
        const int j = lane >> 4, t0 = 2 * j;
        for (int g = blockIdx.x; g < ngroups; g += gridDim.x) {
            const int r = min(16 * g + (lane & 15), rows - 1);
            const uint8_t *wr = W + (size_t)r * nb * BS;
            Raw r0, r1;
            const int k0 = min(wv, nb - 1), k1 = min(wv + MM8_W, nb - 1);
            mm8_load(r0, wr + (size_t)k0 * BS, j);
            mm8_load(r1, wr + (size_t)k1 * BS, j);
            float y0 = 0.0f, y1 = 0.0f;
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int kb = wv + u * MM8_W;
                if (kb < nb) {
                    float z0 = 0.0f, z1 = 0.0f;
                    mm8_block(u ? r1 : r0, frag + (size_t)kb * (RQK / SB) * FB, xs + (size_t)kb * (RQK / SB) * 8, lane,
                              z0, z1);
                    const float2 g2 = *(const float2 *)(ge + kb * 8 + t0);
                    y0 = fmaf(z0, g2.x, y0);
                    y1 = fmaf(z1, g2.y, y1);
                }
            }
            red[wv][lane] = make_float2(y0, y1);
            __syncthreads();
            if (wv == 0) {
                float2 a = red[0][lane];
#pragma unroll
                for (int w = 1; w < MM8_W; w++) {
                    const float2 b = red[w][lane];
                    a.x += b.x;
                    a.y += b.y;
                }
                const int rr = 16 * g + (lane & 15);
                if (rr < rows) {
                    if (t0 < T) Y[(size_t)t0 * rows + rr] = a.x;
                    if (t0 + 1 < T) Y[(size_t)(t0 + 1) * rows + rr] = a.y;
                }
            }
            __syncthreads();
        }
        return;
    }
    /* many groups: 16-row groups, wave-strided; items (group, kb) with the
     * next item's raw quants loaded while the current computes */
    const int gw = blockIdx.x * MM8_W + wv, nw = gridDim.x * MM8_W;
    const int mine = gw < ngroups ? (ngroups - 1 - gw) / nw + 1 : 0;
    const int total = mine * nb;
    if (total == 0) return;
    const int j = lane >> 4, t0 = 2 * j;
    auto blk = [&](int item) {
        const int g = gw + (item / nb) * nw, kb = item % nb;
        const int r = min(16 * g + (lane & 15), rows - 1);
        return W + ((size_t)r * nb + kb) * BS;
    };
    float y0 = 0.0f, y1 = 0.0f;
    auto compute = [&](const Raw &raw, int item) {
        const int kb = item % nb;
        float z0 = 0.0f, z1 = 0.0f;
        mm8_block(raw, frag + (size_t)kb * (RQK / SB) * FB, xs + (size_t)kb * (RQK / SB) * 8, lane, z0, z1);
        const float2 g2 = *(const float2 *)(ge + kb * 8 + t0);
        y0 = fmaf(z0, g2.x, y0);
        y1 = fmaf(z1, g2.y, y1);
        if (kb == nb - 1) {
            const int g = gw + (item / nb) * nw, r = 16 * g + (lane & 15);
            if (r < rows) {
                if (t0 < T) Y[(size_t)t0 * rows + r] = y0;
                if (t0 + 1 < T) Y[(size_t)(t0 + 1) * rows + r] = y1;
            }
            y0 = y1 = 0.0f;
        }
    };
    /* the loads are unconditional (past the last item: the last item again),
     * so that the wait before a computation counts only its own loads, not
     * the next item's behind them */
    Raw ra, rb;
    mm8_load(ra, blk(0), j);
    for (int it = 0;; it += 2) {
        mm8_load(rb, blk(min(it + 1, total - 1)), j);
        compute(ra, it);
        if (it + 1 >= total) break;
        mm8_load(ra, blk(min(it + 2, total - 1)), j);
        compute(rb, it + 1);
        if (it + 2 >= total) break;
    }
}

int dense_mfma_min_tokens() { return g_dense_mfma_t; }

int dense_mm8_launch(const uint8_t *W, int q6, const float *X, float *Y, size_t rows, size_t cols, int T)
{
    const size_t bytes = mm8_buf_bytes(cols, q6);
    uint8_t *buf = (uint8_t *)rt_scratch(SCR_MM, bytes);
    if (!buf) return ROASTER_EDEVICE;
    const size_t ng = (rows + 15) / 16;
    const size_t cap = (size_t)(bytes <= 80 * 1024 ? 2 : 1) * rt().n_cu;
    const int nb = (int)(cols / RQK);
    /* fewer groups than waves in a full grid (and at most 16 super-blocks):
     * the super-blocks of a group split over a workgroup's waves */
    const int ksplit = ng < MM8_W * cap && nb <= 2 * MM8_W;
    size_t blocks = ksplit ? ng : (ng + MM8_W - 1) / MM8_W;
    if (blocks > cap) blocks = cap;
    if (q6) {
        hipLaunchKernelGGL(mm8_prep_kernel<true>, dim3(nb), dim3(256), 0, rt().stream, X, (int)cols, T, buf);
        hipLaunchKernelGGL(dense_mm8_kernel<true>, dim3((unsigned)blocks), dim3(MM8_T), bytes, rt().stream, W, buf, Y,
                           (int)rows, (int)cols, T, ksplit);
    } else {
        hipLaunchKernelGGL(mm8_prep_kernel<false>, dim3(nb), dim3(256), 0, rt().stream, X, (int)cols, T, buf);
        hipLaunchKernelGGL(dense_mm8_kernel<false>, dim3((unsigned)blocks), dim3(MM8_T), bytes, rt().stream, W, buf, Y,
                           (int)rows, (int)cols, T, ksplit);
    }
    return rt_check(hipGetLastError(), "dense MFMA launch") ? ROASTER_EDEVICE : 0;
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
    if (!W || !X || !Y || !rows || !cols || cols % RQK || cols > 4096 || T < 1 || T > 8 || rows > (size_t)INT32_MAX)
        return rt_fail(ROASTER_EINVAL, "roaster_matvec_q: need cols a multiple of 256 and <= 4096, 1 <= T <= 8");
    if (T >= g_dense_mfma_t)                           /* several tokens: quants on MFMA */
        return dense_mm8_launch((const uint8_t *)W, q6, X, Y, rows, cols, T);
    const int nb = (int)(cols / RQK), rpw = 64 / lanes_per_row(nb);
    const size_t npass = (rows + rpw - 1) / rpw;
    size_t blocks = (npass + 3) / 4;
    if (blocks > (size_t)DMV_GRID * rt().n_cu) blocks = (size_t)DMV_GRID * rt().n_cu;
    const size_t lds = T > 1 ? (size_t)T * cols * 4 + (size_t)T * (cols / 16) * 4 : 0;
    const dim3 gd((unsigned)blocks), bd(MV_THREADS);
    const uint8_t *w = (const uint8_t *)W;
    const int r = (int)rows, cc = (int)cols;
#define DMV(Q6_, ONE_, KB_) hipLaunchKernelGGL((dense_mv_kernel<Q6_, ONE_, KB_>), gd, bd, ONE_ ? 0 : lds, rt().stream, w, X, Y, r, cc, T)
    if (nb <= 8) {
        if (q6 && T == 1) DMV(true, true, 1);
        else if (q6) DMV(true, false, 1);
        else if (T == 1) DMV(false, true, 1);
        else DMV(false, false, 1);
    } else {
        if (q6 && T == 1) DMV(true, true, 2);
        else if (q6) DMV(true, false, 2);
        else if (T == 1) DMV(false, true, 2);
        else DMV(false, false, 2);
    }
#undef DMV
    return rt_check(hipGetLastError(), "dense matvec launch") ? ROASTER_EDEVICE : 0;
}

/* roaster_dense_mfma_min_tokens: calls with at least this many tokens run
 * on dense_mm8_kernel; 0 = query. */
extern "C" int roaster_dense_mfma_min_tokens(int t)
{
    std::lock_guard<std::recursive_mutex> g(rt_lock());
    if (t > 0) g_dense_mfma_t = t;
    return g_dense_mfma_t;
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
