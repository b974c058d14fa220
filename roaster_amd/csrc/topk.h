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

/* Wave-level top-8 of one token (model.c:869-897).  Each logit becomes an
 * order-preserving 32-bit key (NaN and -inf: key 0, never selected).  Eight
 * rounds each take the wave maximum of the keys (DPP within 16-lane rows, then
 * the four row maxima) and, among the experts holding it, the lowest index
 * (ballot, first set bit): "larger logit, then lower index", the order the
 * reference's strict-greater insertion produces.  The softmax over the selected
 * logits is then summed in slot order like the reference.  v4[i] holds the
 * logit of expert lane + 64*i (E <= 256).  Fewer than 8 selectable logits:
 * the remaining ids are -1 and *bad is set. */
static __device__ void topk8_wave(const float v4in[4], int E, int *ids, float *w, int *bad)
{
    const int lane = threadIdx.x & 63;
    uint32_t key[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int e = lane + 64 * i;
        key[i] = e < E ? logit_key(v4in[i]) : 0u;
    }
    float v = -INFINITY;
    int myid = -1, nsel = 0;
    for (int r = 0; r < RTOPK; r++) {
        uint32_t m = max(max(key[0], key[1]), max(key[2], key[3]));
        m = max(m, (uint32_t)dpp_i<DPP_XOR1>((int)m));
        m = max(m, (uint32_t)dpp_i<DPP_XOR2>((int)m));
        m = max(m, (uint32_t)dpp_i<DPP_HALF_MIRROR>((int)m));
        m = max(m, (uint32_t)dpp_i<DPP_MIRROR>((int)m));
        const uint32_t M = max(max((uint32_t)__builtin_amdgcn_readlane((int)m, 0), (uint32_t)__builtin_amdgcn_readlane((int)m, 16)),
                               max((uint32_t)__builtin_amdgcn_readlane((int)m, 32), (uint32_t)__builtin_amdgcn_readlane((int)m, 48)));
        if (M == 0u) break;                               /* no selectable logit left */
        int e = -1;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const unsigned long long b = __ballot(key[i] == M);
            if (e < 0 && b) e = 64 * i + (int)__builtin_ctzll(b);
        }
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (e == lane + 64 * i) key[i] = 0u;
        if (lane == r) {
            v = key_logit(M);
            myid = e;
        }
        nsel++;
    }
    const float mx = lane_f(v, 0);
    const float ex = expf(v - mx);
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < RTOPK; k++) sum += lane_f(ex, k);
    const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    if (lane < RTOPK) {
        ids[lane] = myid;
        w[lane] = ex * inv;
    }
    if (lane == 0 && nsel < RTOPK) *bad = 1;
}

#endif
