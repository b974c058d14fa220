/*
 * qdot.h -- device helpers: Q4_K / Q6_K super-block chunks for wave-wide
 * dequantising dot products (decode / matvec kernels).
 *
 * One 256-weight super-block is served by 8 lanes.  Lane chunk c (0..7) owns
 * 32 weights in two runs of 16 consecutive columns, A and B, and the 16 quant
 * bytes at block offset 16*c (+16 for Q4_K's header):
 *
 *   Q4_K (144 B: d, dmin, scales[12], qs[128]; kernels.c:29-34, 1839-1853):
 *     g = c/2; run A = 64g + 16(c&1) (low nibbles, sub-block 2g),
 *              run B = A + 32        (high nibbles, sub-block 2g+1).
 *     w = d*sc*q - dmin*m.
 *   Q6_K (210 B: ql[128], qh[64], scales[16], d; kernels.c:35-40, 1855-1874):
 *     n = c/4, p = c&3; run A = 128n + 32(p>>1) + 16(p&1) (low nibbles of ql,
 *     qh bits 2(p>>1)..+1), run B = A + 64 (high nibbles, qh bits 4+2(p>>1)..+1).
 *     w = d*sc*(q - 32), q unsigned 6-bit.
 *
 * Folded dot for a lane (kernels.c:242-245 uses the same identity):
 *   sum_i w_i x_i = sA * sum(qA x) - mA * sum(xA) + sB * sum(qB x) - mB * sum(xB)
 * with mA = dmin*m (Q4_K) or 32*d*sc (Q6_K).  Quant bytes are unpacked four at
 * a time in 32-bit registers and converted with the byte-select f32 converts.
 */
#ifndef ROASTER_QDOT_H
#define ROASTER_QDOT_H

#include <hip/hip_runtime.h>
#include <stdint.h>

struct __attribute__((packed, aligned(2))) u32x4_a2 { uint32_t x, y, z, w; };
struct __attribute__((packed, aligned(2))) u32x2_a2 { uint32_t x, y; };

/* Global-memory loads.  Weight pointers read out of device-side tables have no
 * provable address space, so plain dereferences compile to flat loads, and a
 * flat load also holds the LDS wait counter: every later LDS wait would then
 * wait for the weight fetch too.  These helpers load through address space 1
 * (global) explicitly; the pointer must point into device memory. */
#define GAS __attribute__((address_space(1)))
typedef uint32_t gu32x4 __attribute__((ext_vector_type(4)));
typedef gu32x4 __attribute__((aligned(2))) gu32x4_a2;
typedef uint32_t gu32x2 __attribute__((ext_vector_type(2)));
typedef gu32x2 __attribute__((aligned(2))) gu32x2_a2;
typedef uint32_t gu32x3 __attribute__((ext_vector_type(3)));
typedef float gf32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 gld_u4(const void *p)          /* 16-byte aligned */
{
    const gu32x4 v = *(const GAS gu32x4 *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint4 gld_u4a2(const void *p)        /* 2-byte aligned */
{
    const gu32x4 v = *(const GAS gu32x4_a2 *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint3 gld_u3(const void *p)           /* 16-byte aligned, 12 bytes read */
{
    const gu32x3 v = *(const GAS gu32x3 *)p;
    return make_uint3(v.x, v.y, v.z);
}
__device__ __forceinline__ uint2 gld_u2(const void *p)           /* 8-byte aligned */
{
    const gu32x2 v = *(const GAS gu32x2 *)p;
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint2 gld_u2a2(const void *p)
{
    const gu32x2 v = *(const GAS gu32x2_a2 *)p;
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t gld_u16(const void *p) { return *(const GAS uint16_t *)p; }
__device__ __forceinline__ uint32_t gld_u32(const void *p) { return *(const GAS uint32_t *)p; }
__device__ __forceinline__ float4 gld_f4(const void *p)
{
    const gf32x4 v = *(const GAS gf32x4 *)p;
    return make_float4(v.x, v.y, v.z, v.w);
}

/* Raw bytes of one lane's share of a super-block. */
struct QChunk {
    uint4 q;       /* Q4_K: qs bytes;  Q6_K: ql bytes */
    uint4 h;       /* Q4_K: header (d, dmin, scales); Q6_K: qh bytes */
    uint2 s;       /* Q6_K: scales[8n .. 8n+8) */
    uint32_t dd;   /* Q6_K: d (low 16 bits) */
};

/* Chunks of one gate row and one up row. */
struct QChunk2 { QChunk g, u; };

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

template <bool q6>
__device__ __forceinline__ QChunk q_load(const uint8_t *blk, int c)
{
    QChunk ch;
    if (!q6) {
        ch.h = gld_u4(blk);                             /* 144-byte blocks are 16-byte aligned */
        ch.q = gld_u4(blk + 16 + 16 * c);
        ch.s = make_uint2(0, 0);
        ch.dd = 0;
    } else {
        const int n = c >> 2, p = c & 3;
        ch.q = gld_u4a2(blk + 16 * c);
        ch.h = gld_u4a2(blk + 128 + 32 * n + 16 * (p & 1));
        ch.s = gld_u2a2(blk + 192 + 8 * n);
        ch.dd = gld_u16(blk + 208);
    }
    return ch;
}

/* Column offsets (within the block) of runs A and B for chunk c. */
template <bool q6>
__device__ __forceinline__ int q_run_a(int c)
{
    return q6 ? (128 * (c >> 2) + 32 * ((c & 3) >> 1) + 16 * (c & 1)) : (64 * (c >> 1) + 16 * (c & 1));
}
template <bool q6>
__device__ __forceinline__ int q_run_b_off() { return q6 ? 64 : 32; }

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xFFu; }

/* Scale factors for the lane: sA, mA, sB, mB. */
template <bool q6>
__device__ __forceinline__ void q_scales(const QChunk &ch, int c, float &sA, float &mA, float &sB, float &mB)
{
    if (!q6) {
        const float d = f16_bits_to_f32(ch.h.x & 0xFFFFu), dmin = f16_bits_to_f32(ch.h.x >> 16);
        /* scales bytes s[0..11] = h.y (0-3), h.z (4-7), h.w (8-11) */
        const int g = c >> 1;
        const int j0 = 2 * g, j1 = 2 * g + 1;
        uint32_t s03 = ch.h.y, s47 = ch.h.z, s811 = ch.h.w;
        int sc0, m0, sc1, m1;
        if (g < 2) {           /* j0, j1 < 4 */
            sc0 = byte_of(s03, j0) & 63; m0 = byte_of(s47, j0) & 63;
            sc1 = byte_of(s03, j1) & 63; m1 = byte_of(s47, j1) & 63;
        } else {               /* j >= 4: low nibble / high nibble of s[j+4], top bits of s[j-4] / s[j] */
            const int i0 = j0 - 4, i1 = j1 - 4;
            sc0 = (byte_of(s811, i0) & 15) | ((byte_of(s03, i0) >> 6) << 4);
            m0  = (byte_of(s811, i0) >> 4) | ((byte_of(s47, i0) >> 6) << 4);
            sc1 = (byte_of(s811, i1) & 15) | ((byte_of(s03, i1) >> 6) << 4);
            m1  = (byte_of(s811, i1) >> 4) | ((byte_of(s47, i1) >> 6) << 4);
        }
        sA = d * (float)sc0; mA = dmin * (float)m0;
        sB = d * (float)sc1; mB = dmin * (float)m1;
    } else {
        const float d = f16_bits_to_f32(ch.dd);
        const int p = c & 3;
        const int ia = (p & 1) + 2 * (p >> 1);     /* index within the 8 scales of this half */
        const int ib = ia + 4;
        const int sa = (int)(int8_t)byte_of(ia < 4 ? ch.s.x : ch.s.y, ia & 3);
        const int sb = (int)(int8_t)byte_of(ch.s.y, ib & 3);
        sA = d * (float)sa; mA = 32.0f * sA;
        sB = d * (float)sb; mB = 32.0f * sB;
    }
}

/* Quant values of word i (4 consecutive columns) of runs A and B, as 4 bytes each. */
template <bool q6>
__device__ __forceinline__ void q_word(const QChunk &ch, int i, int c, uint32_t &a, uint32_t &b)
{
    const uint32_t v = i == 0 ? ch.q.x : i == 1 ? ch.q.y : i == 2 ? ch.q.z : ch.q.w;
    a = v & 0x0F0F0F0Fu;
    b = (v >> 4) & 0x0F0F0F0Fu;
    if (q6) {
        const uint32_t hv = i == 0 ? ch.h.x : i == 1 ? ch.h.y : i == 2 ? ch.h.z : ch.h.w;
        const int sh = 2 * ((c & 3) >> 1);
        a |= ((hv >> sh) & 0x03030303u) << 4;
        b |= ((hv >> (sh + 4)) & 0x03030303u) << 4;
    }
    /* opaque to the compiler: otherwise it folds each mask into the byte
     * extraction of dot4u8 (a bit-field extract plus a convert per quant)
     * instead of converting bytes 0..3 of the word directly (one
     * v_cvt_f32_ubyteN per quant) */
    asm("" : "+v"(a), "+v"(b));
}

__device__ __forceinline__ float dot4u8(uint32_t q, const float4 x, float acc)
{
    acc = fmaf((float)(q & 0xFFu), x.x, acc);
    acc = fmaf((float)((q >> 8) & 0xFFu), x.y, acc);
    acc = fmaf((float)((q >> 16) & 0xFFu), x.z, acc);
    acc = fmaf((float)(q >> 24), x.w, acc);
    return acc;
}

/* Lane partial of sum_i w_i x_i over its 32 weights, x already in registers:
 * xa / xb are the 16 floats of runs A / B, sxa / sxb their sums. */
template <bool q6>
__device__ __forceinline__ float q_chunk_dot_r(const QChunk &ch, int c, const float4 (&xa)[4], const float4 (&xb)[4],
                                               float sxa, float sxb)
{
    float sA, mA, sB, mB;
    q_scales<q6>(ch, c, sA, mA, sB, mB);
    float accA = 0.0f, accB = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t qa, qb;
        q_word<q6>(ch, i, c, qa, qb);
        accA = dot4u8(qa, xa[i], accA);
        accB = dot4u8(qb, xb[i], accB);
    }
    float r = sA * accA;
    r = fmaf(-mA, sxa, r);
    r = fmaf(sB, accB, r);
    r = fmaf(-mB, sxb, r);
    return r;
}

/* The same with x read from memory (16-byte aligned, global or LDS). */
template <bool q6>
__device__ __forceinline__ float q_chunk_dot(const QChunk &ch, int c, const float *xa, const float *xb,
                                             float sxa, float sxb)
{
    float4 a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        a[i] = *(const float4 *)(xa + 4 * i);
        b[i] = *(const float4 *)(xb + 4 * i);
    }
    return q_chunk_dot_r<q6>(ch, c, a, b, sxa, sxb);
}

__device__ __forceinline__ float sum16(const float *x)
{
    float4 a = *(const float4 *)x, b = *(const float4 *)(x + 4), c = *(const float4 *)(x + 8), d = *(const float4 *)(x + 12);
    return ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w)) + (((c.x + c.y) + (c.z + c.w)) + ((d.x + d.y) + (d.z + d.w)));
}

/* ---- cross-lane reductions with DPP (no LDS crossbar round trips) ---------- */
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v)
{
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v)
{
    return __builtin_bit_cast(float, dpp_i<CTRL>(__builtin_bit_cast(int, v)));
}
__device__ __forceinline__ float lane_f(float v, int l)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

#define DPP_XOR1 0xB1          /* quad_perm [1,0,3,2] */
#define DPP_XOR2 0x4E          /* quad_perm [2,3,0,1] */
#define DPP_HALF_MIRROR 0x141  /* lane i <-> 7-i within 8 */
#define DPP_MIRROR 0x140       /* lane i <-> 15-i within 16 */
#define DPP_ROW_BCAST15 0x142  /* lane 15 of each row -> the next row (row_mask selects receivers) */
#define DPP_ROW_BCAST31 0x143  /* lane 31 -> rows 2 and 3 */

/* Sum over aligned groups of W lanes (W a power of two <= 64); every lane of a
 * group receives the group's sum (fixed order, so results are deterministic). */
template <int W>
__device__ __forceinline__ float group_sum(float v)
{
    if (W >= 2) v += dpp_f<DPP_XOR1>(v);
    if (W >= 4) v += dpp_f<DPP_XOR2>(v);
    if (W >= 8) v += dpp_f<DPP_HALF_MIRROR>(v);
    if (W >= 16) v += dpp_f<DPP_MIRROR>(v);
    if (W == 32) {
        const float lo = lane_f(v, 0) + lane_f(v, 16), hi = lane_f(v, 32) + lane_f(v, 48);
        v = (threadIdx.x & 32) ? hi : lo;
    }
    if (W == 64) v = (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
    return v;
}

/* Maximum of v over each 32-lane half of the wave: lo = lanes 0..31, hi =
 * lanes 32..63 (wave-uniform results). */
__device__ __forceinline__ void half_max(float v, float &lo, float &hi)
{
    v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f<DPP_MIRROR>(v));
    lo = fmaxf(lane_f(v, 0), lane_f(v, 16));
    hi = fmaxf(lane_f(v, 32), lane_f(v, 48));
}

/* Lanes serving one row of nb super-blocks: 8 per block, rounded up to the
 * power of two group_sum_w reduces over (lanes past 8 * nb stay idle). */
__host__ __device__ __forceinline__ int lanes_per_row(int nb) { return nb >= 5 ? 64 : nb >= 3 ? 32 : 8 * nb; }

/* Runtime group width (8, 16, 32 or 64). */
__device__ __forceinline__ float group_sum_w(float v, int w)
{
    if (w == 16) return group_sum<16>(v);
    if (w == 64) return group_sum<64>(v);
    if (w == 8) return group_sum<8>(v);
    return group_sum<32>(v);
}

#endif
