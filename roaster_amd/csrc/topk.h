/*
 * topk.h -- wave-level top-8 expert selection (model.c:869-897), shared by the
 * decode and prefill kernels.
 */
#ifndef ROASTER_TOPK_H
#define ROASTER_TOPK_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qdot.h"

#ifndef RTOPK
#define RTOPK 8
#endif

/* Order-preserving key of a logit: larger float -> larger unsigned key; NaN
 * and -inf map to 0 and are never selected (model.c:879 enters a value only
 * if it is > the current slot, which starts at -inf). */
__device__ __forceinline__ uint32_t logit_key(float v)
{
    if (!(v > -INFINITY)) return 0u;
    const uint32_t u = __builtin_bit_cast(uint32_t, v + 0.0f);   /* -0 and +0 compare equal */
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_logit(uint32_t k)
{
    const uint32_t u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
    return __builtin_bit_cast(float, u);
}

/* Wave-level top-8 of one token (model.c:869-897).  Each logit becomes a
 * distinct 40-bit key (logit key << 8 | 255 - expert), so the order is "larger
 * logit, then lower index" and no two keys tie; NaN / -inf get key 0.  A radix
 * select over the 40 bits (ballot counts per bit) finds the 8th largest key,
 * the (at most 8) keys >= it are ranked in 8 lanes, and the softmax over the
 * selected logits is summed in slot order like the reference.  v4[i] holds the
 * logit of expert lane + 64*i (E <= 256).  sk: 16 entries of LDS scratch. */
static __device__ void topk8_wave(const float v4in[4], int E, int *ids, float *w, int *bad, unsigned long long *sk)
{
    const int lane = threadIdx.x & 63;
    unsigned long long key[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int e = lane + 64 * i;
        const uint32_t k32 = e < E ? logit_key(v4in[i]) : 0u;
        key[i] = k32 ? (((unsigned long long)k32 << 8) | (unsigned long long)(255 - e)) : 0ull;
    }
    unsigned long long P = 0ull;
    for (int b = 39; b >= 0; b--) {
        const unsigned long long C = P | (1ull << b);
        int cnt = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) cnt += __popcll(__ballot(key[i] >= C));
        if (cnt >= RTOPK) P = C;
    }
    /* the selected keys: >= P and valid; compact them into sk[0..nsel) */
    int base = 0;
    const unsigned long long lt = (1ull << lane) - 1ull;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const bool sel = key[i] != 0ull && key[i] >= P;
        const unsigned long long m = __ballot(sel);
        if (sel) {
            const int pos = base + __popcll(m & lt);
            if (pos < RTOPK) sk[pos] = key[i];
        }
        base += __popcll(m);
    }
    const int nsel = base < RTOPK ? base : RTOPK;
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    /* rank the selected keys (descending) in lanes 0..7 */
    if (lane < nsel) {
        const unsigned long long my = sk[lane];
        int r = 0;
        for (int j = 0; j < nsel; j++) r += sk[j] > my;
        sk[8 + r] = my;
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    const unsigned long long kk = lane < nsel ? sk[8 + lane] : 0ull;
    const int e = kk ? 255 - (int)(kk & 0xFFull) : -1;
    const float v = kk ? key_logit((uint32_t)(kk >> 8)) : -INFINITY;
    const float mx = lane_f(v, 0);
    const float ex = expf(v - mx);
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < RTOPK; k++) sum += lane_f(ex, k);
    const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    if (lane < RTOPK) {
        ids[lane] = e;
        w[lane] = ex * inv;
    }
    if (lane == 0 && nsel < RTOPK) *bad = 1;
}

#endif
