/*
 * synth.h -- deterministic counter-based generator for synthetic MoE inputs.
 *
 * Every byte is a pure function of (seed, stream, counter), so the host (C) and
 * the device (HIP) produce identical Q4_K / Q6_K blocks: the GPU can fill a
 * 21 GB expert table in HBM while a CPU check regenerates any expert it needs.
 * Only integer arithmetic, one fmaf and an integer f32->f16 rounding are used
 * for quantised blocks, so both sides agree bit for bit.  Floating-point
 * vectors (x, router weights) use Box-Muller with libm and are produced on the
 * host only.
 *
 * Distributions (per block):
 *   Q4_K: bytes 4..143 uniform (6-bit scales/mins and 4-bit quants are packed
 *         densely, so uniform bytes give uniform fields); d, dmin = f16(U(lo, hi)).
 *   Q6_K: ql/qh bytes uniform (uniform 6-bit quants); scales int8 U[-32, 31];
 *         d = f16(U(lo, hi)).
 */
#ifndef ROASTER_SYNTH_H
#define ROASTER_SYNTH_H

#include <stdint.h>
#include <math.h>

#if defined(__HIPCC__)
#define RS_FN static inline __host__ __device__
#else
#define RS_FN static inline
#endif

#define RS_GOLDEN 0x9E3779B97F4A7C15ull

RS_FN uint64_t rs_mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Key of one independent stream (a matrix, a vector). */
RS_FN uint64_t rs_key(uint64_t seed, uint64_t stream)
{
    return rs_mix64(seed * RS_GOLDEN + rs_mix64(stream + 0x632BE59BD9B4E019ull));
}

RS_FN uint64_t rs_at(uint64_t key, uint64_t ctr)
{
    return rs_mix64(key + (ctr + 1ull) * RS_GOLDEN);
}

/* Stream id of (layer, expert, kind): kind 0..2 = gate/up/down, 3 = router,
 * 4 = shared-gate vector; expert == n_experts is the shared expert. */
RS_FN uint64_t rs_stream(int layer, int expert, int kind)
{
    return ((uint64_t)(unsigned)kind << 40) | ((uint64_t)(unsigned)layer << 20) | (uint64_t)(unsigned)expert;
}

/* Uniform in [0, 1) with 24 random bits (exact in f32). */
RS_FN float rs_unit(uint64_t r) { return (float)(uint32_t)(r >> 40) * 0x1p-24f; }

/* Round a positive normal-range f32 to f16 bits, round-to-nearest-even. */
RS_FN uint16_t rs_f32_to_f16(float f)
{
    union { float f; uint32_t u; } v;
    v.f = f;
    uint32_t u = v.u;
    uint32_t sign = (u >> 16) & 0x8000u;
    int32_t e = (int32_t)((u >> 23) & 0xFF) - 127 + 15;
    uint32_t m = u & 0x7FFFFFu;
    if (e <= 0) {                      /* f16 subnormal */
        if (e < -10) return (uint16_t)sign;
        m |= 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t hm = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    uint32_t hm = m >> 13, rem = m & 0x1FFFu;
    uint32_t h = sign | ((uint32_t)e << 10) | hm;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) h++;
    return (uint16_t)h;
}

RS_FN uint16_t rs_f16_uniform(uint64_t r, float lo, float hi)
{
    return rs_f32_to_f16(fmaf(rs_unit(r), hi - lo, lo));
}

/* Block `b` of the stream `key`: 144 bytes of Q4_K. */
RS_FN void rs_q4k_block(uint64_t key, uint64_t b, float lo, float hi, uint8_t *out)
{
    for (int i = 0; i < 18; i++) {
        uint64_t r = rs_at(key, b * 32u + (uint64_t)i);
        for (int j = 0; j < 8; j++) out[8 * i + j] = (uint8_t)(r >> (8 * j));
    }
    uint16_t d = rs_f16_uniform(rs_at(key, b * 32u + 20u), lo, hi);
    uint16_t dm = rs_f16_uniform(rs_at(key, b * 32u + 21u), lo, hi);
    out[0] = (uint8_t)d; out[1] = (uint8_t)(d >> 8);
    out[2] = (uint8_t)dm; out[3] = (uint8_t)(dm >> 8);
}

/* Block `b` of the stream `key`: 210 bytes of Q6_K. */
RS_FN void rs_q6k_block(uint64_t key, uint64_t b, float lo, float hi, uint8_t *out)
{
    for (int i = 0; i < 24; i++) {
        uint64_t r = rs_at(key, b * 32u + (uint64_t)i);
        for (int j = 0; j < 8; j++) out[8 * i + j] = (uint8_t)(r >> (8 * j));
    }
    for (int i = 0; i < 2; i++) {
        uint64_t r = rs_at(key, b * 32u + 24u + (uint64_t)i);
        for (int j = 0; j < 8; j++) out[192 + 8 * i + j] = (uint8_t)((int)((r >> (8 * j)) & 63u) - 32);
    }
    uint16_t d = rs_f16_uniform(rs_at(key, b * 32u + 28u), lo, hi);
    out[208] = (uint8_t)d; out[209] = (uint8_t)(d >> 8);
}

#endif
