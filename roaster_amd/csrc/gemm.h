/*
 * gemm.h -- Q4_K / Q6_K dequantising MFMA tiles for gfx950 (prefill GEMMs).
 *
 * A workgroup of 256 threads (4 waves) computes a 64 x 64 output tile, one
 * 32 x 32 block per wave, with v_mfma_f32_32x32x16_{f16,bf16}.  The K loop
 * walks one 256-column super-block at a time: the tile's 64 weight rows are
 * dequantised in f32 exactly as kernels.c:1839-1874 does (Q4_K: d*sc*q - dmin*m
 * with one fused multiply-add, Q6_K: (d*sc)*(q-32)) and stored to LDS as 16-bit
 * MFMA operands; the 64 activation rows are scaled and converted alongside.
 *
 * Operand modes (fp32 accumulation in all of them):
 *   PF_F16   fp16 operands; activations carry a per-row power-of-two scale so
 *            that the row maximum lands in [2^14, 2^15) (exact, undone in f32
 *            after the product).  About 11 significant bits per operand.
 *   PF_BF16  bf16 operands, no scaling.  About 8 significant bits.
 *   PF_SPLIT each operand as a bf16 hi/lo pair; hi*hi + hi*lo + lo*hi (three
 *            MFMAs), about 16 significant bits per product.
 *
 * MFMA 32x32x16 16-bit operand lane layout (checked on the device):
 *   A[m][k]: lane l holds m = l%32, k = 8*(l/32) + i, i = 0..7
 *   B[k][n]: lane l holds k = 8*(l/32) + i, n = l%32
 *   D[m][n]: lane l holds m = 8*(i/4) + 4*(l/32) + i%4, n = l%32, i = 0..15
 */
#ifndef ROASTER_GEMM_H
#define ROASTER_GEMM_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qdot.h"

#define PF_F16 0
#define PF_SPLIT 1
#define PF_BF16 2

typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

#define GT 256                    /* threads per GEMM workgroup */
#define GM 64                     /* tile rows (token rows) */
#define GN 64                     /* tile columns (weight rows) */
#define GK 256                    /* K step: one super-block */
#define GLD (GK + 8)              /* LDS row stride in 16-bit elements */
#define G_TILE_ELEMS (GM * GLD)   /* one 64 x 256 operand tile */

/* LDS bytes of the two operand tiles (x2 for the lo halves in SPLIT mode). */
__host__ __device__ constexpr size_t gemm_lds_bytes(int op)
{
    return (size_t)(op == PF_SPLIT ? 4 : 2) * G_TILE_ELEMS * 2;
}

/* 8 f32 values -> 16-bit operands at hi[off..off+8) (and lo[...] in SPLIT). */
template <int OP>
__device__ __forceinline__ void store8(uint16_t *hi, uint16_t *lo, int off, f32x8 v)
{
    if (OP == PF_F16) {
        *(f16x8 *)(hi + off) = __builtin_convertvector(v, f16x8);
    } else {
        const bf16x8 h = __builtin_convertvector(v, bf16x8);
        *(bf16x8 *)(hi + off) = h;
        if (OP == PF_SPLIT) *(bf16x8 *)(lo + off) = __builtin_convertvector(v - __builtin_convertvector(h, f32x8), bf16x8);
    }
}

/* The 64 weights of quarter qd (columns 64*qd .. 64*qd+63) of one super-block. */
template <bool Q6>
__device__ __forceinline__ void dequant_quarter(const uint8_t *blk, int qd, float (&v)[64])
{
    if (!Q6) {
        /* quarter qd = group g (kernels.c:1844-1852): qs[32g .. 32g+32) low
         * nibbles use sub-block 2g, high nibbles 2g+1 */
        const uint4 hd = gld_u4(blk);
        const float d = f16_bits_to_f32(hd.x & 0xFFFFu), dmin = f16_bits_to_f32(hd.x >> 16);
        const int j0 = 2 * qd, j1 = j0 + 1;
        const uint32_t s03 = hd.y, s47 = hd.z, s811 = hd.w;
        int sc0, m0, sc1, m1;
        if (qd < 2) {
            sc0 = byte_of(s03, j0) & 63; m0 = byte_of(s47, j0) & 63;
            sc1 = byte_of(s03, j1) & 63; m1 = byte_of(s47, j1) & 63;
        } else {
            const int i0 = j0 - 4, i1 = j1 - 4;
            sc0 = (byte_of(s811, i0) & 15) | ((byte_of(s03, i0) >> 6) << 4);
            m0 = (byte_of(s811, i0) >> 4) | ((byte_of(s47, i0) >> 6) << 4);
            sc1 = (byte_of(s811, i1) & 15) | ((byte_of(s03, i1) >> 6) << 4);
            m1 = (byte_of(s811, i1) >> 4) | ((byte_of(s47, i1) >> 6) << 4);
        }
        const float s0 = d * (float)sc0, mm0 = dmin * (float)m0;
        const float s1 = d * (float)sc1, mm1 = dmin * (float)m1;
        const uint4 qa = gld_u4(blk + 16 + 32 * qd);
        const uint4 qb = gld_u4(blk + 32 + 32 * qd);
        const uint32_t w8[8] = { qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w };
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const uint32_t byte = (w8[i] >> (8 * b)) & 0xFFu;
                v[4 * i + b] = fmaf(s0, (float)(byte & 15u), -mm0);
                v[32 + 4 * i + b] = fmaf(s1, (float)(byte >> 4), -mm1);
            }
    } else {
        /* half n = qd/2 (kernels.c:1855-1874); even quarter: w[128n+l] from
         * ql[l] low nibble | qh bits 0-1 and w[128n+32+l] from ql[32+l] low |
         * qh bits 2-3; odd quarter: high nibbles with qh bits 4-5 / 6-7 */
        const int n = qd >> 1, hiq = qd & 1;
        const uint8_t *ql = blk + 64 * n, *qh = blk + 128 + 32 * n;
        const uint2 scw = gld_u2a2(blk + 192 + 8 * n);
        const uint32_t scl = hiq ? scw.y : scw.x;
        const float d = f16_bits_to_f32(gld_u16(blk + 208));
        const uint4 l0 = gld_u4a2(ql), l1 = gld_u4a2(ql + 16);
        const uint4 l2 = gld_u4a2(ql + 32), l3 = gld_u4a2(ql + 48);
        const uint4 h0 = gld_u4a2(qh), h1 = gld_u4a2(qh + 16);
        const uint32_t L[16] = { l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w,
                                 l2.x, l2.y, l2.z, l2.w, l3.x, l3.y, l3.z, l3.w };
        const uint32_t Hh[8] = { h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w };
        const float dA0 = d * (float)(int8_t)byte_of(scl, 0), dA1 = d * (float)(int8_t)byte_of(scl, 1);
        const float dB0 = d * (float)(int8_t)byte_of(scl, 2), dB1 = d * (float)(int8_t)byte_of(scl, 3);
        const int shl = hiq ? 4 : 0, shA = hiq ? 4 : 0, shB = hiq ? 6 : 2;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t qa = ((L[i] >> shl) & 0x0F0F0F0Fu) | (((Hh[i] >> shA) & 0x03030303u) << 4);
            const uint32_t qb = ((L[8 + i] >> shl) & 0x0F0F0F0Fu) | (((Hh[i] >> shB) & 0x03030303u) << 4);
            const float da = i < 4 ? dA0 : dA1, db = i < 4 ? dB0 : dB1;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                v[4 * i + b] = da * (float)((int)((qa >> (8 * b)) & 0xFFu) - 32);
                v[32 + 4 * i + b] = db * (float)((int)((qb >> (8 * b)) & 0xFFu) - 32);
            }
        }
    }
}

/* Dequantise one super-block column of the tile's weight rows into Wh/Wl.
 * Thread t owns row t/4 (blk: that row's block, or NULL for a zero row),
 * columns 64*(t%4) .. +64.  q6 must be uniform across each wave. */
template <int OP>
__device__ __forceinline__ void load_w_tile(const uint8_t *blk, bool q6, uint16_t *Wh, uint16_t *Wl)
{
    const int t = threadIdx.x, qd = t & 3;
    const int off = (t >> 2) * GLD + 64 * qd;
    float v[64];
    if (blk) {
        if (q6) dequant_quarter<true>(blk, qd, v);
        else dequant_quarter<false>(blk, qd, v);
    } else {
#pragma unroll
        for (int i = 0; i < 64; i++) v[i] = 0.0f;
    }
#pragma unroll
    for (int c = 0; c < 8; c++) {
        const f32x8 e = { v[8 * c], v[8 * c + 1], v[8 * c + 2], v[8 * c + 3],
                          v[8 * c + 4], v[8 * c + 5], v[8 * c + 6], v[8 * c + 7] };
        store8<OP>(Wh, Wl, off + 8 * c, e);
    }
}

/* Activations: thread t converts row t/4 (src: that row at the K step's first
 * column, or NULL for a zero row), columns 64*(t%4) .. +64, times scale. */
template <int OP>
__device__ __forceinline__ void load_x_tile(const float *src, float scale, uint16_t *Xh, uint16_t *Xl)
{
    const int t = threadIdx.x, qd = t & 3;
    const int off = (t >> 2) * GLD + 64 * qd;
    float4 v[16];
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = src ? gld_f4(src + 64 * qd + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int c = 0; c < 8; c++) {
        f32x8 e = { v[2 * c].x, v[2 * c].y, v[2 * c].z, v[2 * c].w,
                    v[2 * c + 1].x, v[2 * c + 1].y, v[2 * c + 1].z, v[2 * c + 1].w };
        if (OP == PF_F16) e = e * scale;
        store8<OP>(Xh, Xl, off + 8 * c, e);
    }
}

/* acc += X[32*wm .. +32][:] . W[32*wn .. +32][:]^T over one K step. */
template <int OP>
__device__ __forceinline__ void mfma_tile(f32x16 &acc, const uint16_t *Xh, const uint16_t *Xl, const uint16_t *Wh,
                                          const uint16_t *Wl, int wm, int wn)
{
    const int l = threadIdx.x & 63;
    const int ra = (32 * wm + (l & 31)) * GLD + 8 * (l >> 5);
    const int rb = (32 * wn + (l & 31)) * GLD + 8 * (l >> 5);
#pragma unroll 4
    for (int kk = 0; kk < GK / 16; kk++) {
        if (OP == PF_F16) {
            const f16x8 a = *(const f16x8 *)(Xh + ra + 16 * kk);
            const f16x8 b = *(const f16x8 *)(Wh + rb + 16 * kk);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
        } else {
            const bf16x8 a = *(const bf16x8 *)(Xh + ra + 16 * kk);
            const bf16x8 b = *(const bf16x8 *)(Wh + rb + 16 * kk);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
            if (OP == PF_SPLIT) {
                const bf16x8 al = *(const bf16x8 *)(Xl + ra + 16 * kk);
                const bf16x8 bl = *(const bf16x8 *)(Wl + rb + 16 * kk);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bl, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, b, acc, 0, 0, 0);
            }
        }
    }
}

/* Power-of-two scale pair for a row whose largest magnitude is amax: inv puts
 * the maximum in [2^14, 2^15), fwd = 1/inv (both exact). */
__device__ __forceinline__ void row_scale(float amax, float &inv, float &fwd)
{
    const int e = (int)((__builtin_bit_cast(uint32_t, amax) >> 23) & 255u) - 127;
    int s = e - 14;
    s = s < -100 ? -100 : (s > 100 ? 100 : s);
    inv = __builtin_bit_cast(float, (uint32_t)(127 - s) << 23);
    fwd = __builtin_bit_cast(float, (uint32_t)(127 + s) << 23);
}

#endif
