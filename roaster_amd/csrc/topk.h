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

/* Wave reductions (all 64 lanes): DPP within each 16-lane row, then row
 * broadcasts fold the rows into lane 63, read once into a scalar. */
__device__ __forceinline__ uint32_t topk_wave_max(uint32_t m)
{
    m = max(m, (uint32_t)dpp_i<DPP_XOR1>((int)m));
    m = max(m, (uint32_t)dpp_i<DPP_XOR2>((int)m));
    m = max(m, (uint32_t)dpp_i<DPP_HALF_MIRROR>((int)m));
    m = max(m, (uint32_t)dpp_i<DPP_MIRROR>((int)m));
    m = max(m, (uint32_t)__builtin_amdgcn_update_dpp((int)m, (int)m, DPP_ROW_BCAST15, 0xA, 0xF, false));
    m = max(m, (uint32_t)__builtin_amdgcn_update_dpp((int)m, (int)m, DPP_ROW_BCAST31, 0xC, 0xF, false));
    return (uint32_t)__builtin_amdgcn_readlane((int)m, 63);
}

__device__ __forceinline__ int topk_wave_min(int m)
{
    m = min(m, dpp_i<DPP_XOR1>(m));
    m = min(m, dpp_i<DPP_XOR2>(m));
    m = min(m, dpp_i<DPP_HALF_MIRROR>(m));
    m = min(m, dpp_i<DPP_MIRROR>(m));
    m = min(m, __builtin_amdgcn_update_dpp(m, m, DPP_ROW_BCAST15, 0xA, 0xF, false));
    m = min(m, __builtin_amdgcn_update_dpp(m, m, DPP_ROW_BCAST31, 0xC, 0xF, false));
    return __builtin_amdgcn_readlane(m, 63);
}

/* Keys of one token's logits: v4[i] holds the logit of expert lane + 64*i
 * (E <= 256); experts past E get key 0. */
__device__ __forceinline__ void topk_keys(const float v4in[4], int E, uint32_t key[4])
{
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < 4; i++) key[i] = lane + 64 * i < E ? logit_key(v4in[i]) : 0u;
}

/* Round r of the wave top-8: the wave maximum M of the keys and then, among
 * the experts holding M, the lowest index (each lane offers its lowest such
 * index, a wave minimum picks one): "larger logit, then lower index", the
 * order the reference's strict-greater insertion produces.  The expert's key
 * is cleared; lane r keeps its logit and id.  Returns the expert (the same in
 * every lane), or -1 when no selectable logit is left. */
__device__ __forceinline__ int topk_round(uint32_t key[4], int r, float &v, int &myid)
{
    const int lane = threadIdx.x & 63;
    const uint32_t M = topk_wave_max(max(max(key[0], key[1]), max(key[2], key[3])));
    if (M == 0u) return -1;
    const int cand = key[0] == M ? lane : key[1] == M ? 64 + lane : key[2] == M ? 128 + lane
                   : key[3] == M ? 192 + lane : 1 << 20;
    const int e = topk_wave_min(cand);
#pragma unroll
    for (int i = 0; i < 4; i++)
        if (e == lane + 64 * i) key[i] = 0u;
    if (lane == r) {
        v = key_logit(M);
        myid = e;
    }
    return e;
}

/* Softmax over the selected logits (lane k holds slot k's), summed in slot
 * order like the reference; lanes 0..7 write ids and weights, and *bad is set
 * when fewer than 8 logits were selectable (the remaining ids are -1). */
__device__ __forceinline__ void topk_finish(float v, int myid, int nsel, int *ids, float *w, int *bad)
{
    const int lane = threadIdx.x & 63;
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

/* Wave-level top-8 of one token (model.c:869-897).  Each logit becomes an
 * order-preserving 32-bit key (NaN and -inf: key 0, never selected); eight
 * rounds of topk_round, then the softmax over the selected logits. */
static __device__ void topk8_wave(const float v4in[4], int E, int *ids, float *w, int *bad)
{
    uint32_t key[4];
    topk_keys(v4in, E, key);
    float v = -INFINITY;
    int myid = -1, nsel = 0;
#pragma unroll
    for (int r = 0; r < RTOPK; r++) {
        if (topk_round(key, r, v, myid) < 0) break;     /* no selectable logit left */
        nsel++;
    }
    topk_finish(v, myid, nsel, ids, w, bad);
}

#endif
