/*
 * tk_gen.c -- replays the deterministic inputs of the reference's kernel test
 * (src/test_kernels.c:9-29): xorshift64 state 88172645463325252, random bytes
 * per quantised matrix with d / dmin overwritten by its h16() encoding (which
 * maps 0.0f to 0x4000 = 2.0, a quirk kept so the bytes match), and frnd()
 * activations in [-1, 1].  Test infrastructure only.
 *
 * Calls must follow the reference test's order: every make_w / frnd_fill call
 * consumes the shared state.
 */
#include <stdint.h>
#include <string.h>

static uint64_t rs = 88172645463325252ULL;

void tk_reset(void) { rs = 88172645463325252ULL; }

static uint32_t rnd(void)
{
    rs ^= rs << 13;
    rs ^= rs >> 7;
    rs ^= rs << 17;
    return (uint32_t)(rs >> 11);
}

static uint16_t h16(float f)
{
    union { float f; uint32_t u; } v = { f };
    uint32_t e = ((v.u >> 23) & 255) - 127 + 15;
    return (uint16_t)((e << 10) | ((v.u >> 13) & 0x3FF));
}

/* test_kernels.c:18-29 (the reference build contracts 0.001f*k + 0.002f into one fma) */
void tk_make_w(int q6, size_t rows, size_t cols, uint8_t *w)
{
    size_t bpr = cols / 256, bs = q6 ? 210 : 144, n = rows * bpr * bs;
    for (size_t i = 0; i < n; i++) w[i] = (uint8_t)rnd();
    for (size_t b = 0; b < rows * bpr; b++) {
        uint8_t *blk = w + b * bs;
        if (q6) {
            uint16_t d = h16(__builtin_fmaf(0.001f, (float)(rnd() % 8), 0.002f));
            memcpy(blk + 208, &d, 2);
            for (int i = 0; i < 16; i++) ((int8_t *)blk + 192)[i] = (int8_t)((int)(rnd() % 64) - 32);
        } else {
            uint16_t d = h16(__builtin_fmaf(0.001f, (float)(rnd() % 8), 0.002f));
            uint16_t m = h16(0.001f * (float)(rnd() % 8));
            memcpy(blk, &d, 2);
            memcpy(blk + 2, &m, 2);
        }
    }
}

/* test_kernels.c:11 */
void tk_frnd(float *x, size_t n)
{
    for (size_t i = 0; i < n; i++) x[i] = ((rnd() & 0xFFFFF) / (float)0xFFFFF) * 2.f - 1.f;
}
