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
__device__ __forceinline__ void topk_finish(float v, int myid, int nsel, int *ids, float *w, int *bad,
                                            int *ready = nullptr, int ready_val = 0)
{
    const int lane = threadIdx.x & 63;
    if (ready) {
        /* ids first, then the flag (release: the ids' LDS stores complete
         * before it), then the weights */
        if (lane < RTOPK) ids[lane] = myid;
        if (lane == 0) __hip_atomic_store(ready, ready_val, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
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

/* Wave-level top-8 of one token (model.c:869-897).  Each logit becomes an
 * order-preserving 32-bit key (NaN and -inf: key 0, never selected); eight
 * rounds of topk_round, then the softmax over the selected logits. */
static __device__ void topk8_wave(const float v4in[4], int E, int *ids, float *w, int *bad, int *ready = nullptr,
                                  int ready_val = 0)
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
    topk_finish(v, myid, nsel, ids, w, bad, ready, ready_val);
}

/* LDS scratch of topk8_fast, per wave. */
struct TopkScratch {
    unsigned long long cand[64];    /* candidates' composite keys */
    unsigned long long slot[RTOPK]; /* slot k's composite key */
};

/* Composite key: the logit key in the high word, 255 - expert in the low
 * word, so that a larger composite is "larger logit, then lower index". */
__device__ __forceinline__ unsigned long long topk_ck(uint32_t key, int e)
{
    return ((unsigned long long)key << 32) | (uint32_t)(255 - e);
}

/* Wave-level top-8 of one token (model.c:869-897) by ranking a candidate
 * set, the same selection as topk8_wave.  The 256 keys fall into 8 groups of
 * 32 (the 4 keys of each 8-lane group); T = the smallest of the 8 group
 * maxima is at most the 8th largest key, so every selected key is >= T (the
 * maxima by DPP, their minimum by a row mirror and permlane16 / permlane32
 * swaps, so T reaches every lane without readlane round trips).  The
 * candidates (key >= T, key != 0) are compacted into LDS and each candidate's
 * rank is the number of candidates with a larger composite key; rank r < 8
 * fills slot r.  The rounds of topk8_wave run instead when more than 64 keys
 * qualify (many ties at the threshold, or a group without a selectable
 * logit).  All 64 lanes must be active; S is this wave's scratch. */
template <bool OPAQUE = false>
static __device__ void topk8_fast(const float v4in[4], int E, int *ids, float *w, int *bad, TopkScratch *S,
                                  int *ready = nullptr, int ready_val = 0)
{
    /* OPAQUE: the scratch addresses are computed at each call, not hoisted
     * out of a caller's loop (where, held across its other work, they were
     * spilled to scratch memory in the batched decode stack) */
    int lane_v = (int)threadIdx.x & 63;
    if constexpr (OPAQUE) asm volatile("" : "+v"(lane_v));
    const int lane = lane_v;
    uint32_t key[4];
    topk_keys(v4in, E, key);
    uint32_t g = max(max(key[0], key[1]), max(key[2], key[3]));
    g = max(g, (uint32_t)dpp_i<DPP_XOR1>((int)g));
    g = max(g, (uint32_t)dpp_i<DPP_XOR2>((int)g));
    g = max(g, (uint32_t)dpp_i<DPP_HALF_MIRROR>((int)g));          /* group maximum in each 8-lane group */
    g = min(g, (uint32_t)dpp_i<DPP_MIRROR>((int)g));              /* smaller of the row's two groups */
    const auto p16 = __builtin_amdgcn_permlane16_swap(g, g, false, false);
    g = min((uint32_t)p16[0], (uint32_t)p16[1]);                   /* rows 0-1 and rows 2-3 */
    const auto p32 = __builtin_amdgcn_permlane32_swap(g, g, false, false);
    const uint32_t T = min((uint32_t)p32[0], (uint32_t)p32[1]);    /* all eight groups, in every lane */
    bool c[4];
    uint64_t b[4];
    int n = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        c[i] = key[i] >= T && key[i] != 0u;
        b[i] = __builtin_amdgcn_ballot_w64(c[i]);
        n += __builtin_popcountll(b[i]);
    }
    if (n > 64) {                                   /* wave-uniform */
        topk8_wave(v4in, E, ids, w, bad, ready, ready_val);
        return;
    }
    S->cand[lane] = 0ull;                           /* entries past the candidates compare below every key */
    int base = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int pos = base + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(b[i] >> 32),
                                                           __builtin_amdgcn_mbcnt_lo((uint32_t)b[i], 0u));
        if (c[i]) S->cand[pos] = topk_ck(key[i], lane + 64 * i);
        base += __builtin_popcountll(b[i]);
    }
    if (lane < RTOPK) S->slot[lane] = 0ull;
    __builtin_amdgcn_s_waitcnt(0xC07F);             /* lgkmcnt(0): the wave's LDS writes are done */
    __builtin_amdgcn_wave_barrier();
    /* candidate p's rank = the number of candidates with a larger composite
     * key; with at most 16 (32) candidates four (two) lanes share candidate p,
     * each counting over a quarter (half) of the list, and permlane swaps add
     * the parts: a dependent chain of 4 (8) compares instead of n */
    const ulonglong2 *c2 = (const ulonglong2 *)S->cand;
    unsigned long long my;
    int rank = 0;
    if (n <= 16) {
        my = S->cand[lane & 15];
        const int q = lane >> 4;
        const ulonglong2 x = c2[2 * q], y = c2[2 * q + 1];
        rank = (x.x > my) + (x.y > my) + (y.x > my) + (y.y > my);
        const auto p16 = __builtin_amdgcn_permlane16_swap(rank, rank, false, false);
        rank = (int)p16[0] + (int)p16[1];
        const auto p32 = __builtin_amdgcn_permlane32_swap(rank, rank, false, false);
        rank = (int)p32[0] + (int)p32[1];
    } else if (n <= 32) {
        my = S->cand[lane & 31];
        const int hf = lane >> 5;
        ulonglong2 x[8];
#pragma unroll
        for (int u = 0; u < 8; u++) x[u] = c2[8 * hf + u];
#pragma unroll
        for (int u = 0; u < 8; u++) rank += (x[u].x > my) + (x[u].y > my);
        const auto p32 = __builtin_amdgcn_permlane32_swap(rank, rank, false, false);
        rank = (int)p32[0] + (int)p32[1];
    } else {
        my = S->cand[lane];                         /* lanes >= n read an entry they never write */
        for (int j0 = 0; j0 < n; j0 += 16) {        /* 8 reads of two candidates in flight, then the compares */
            ulonglong2 cj[8];
#pragma unroll
            for (int u = 0; u < 8; u++) cj[u] = c2[(j0 >> 1) + u];
#pragma unroll
            for (int u = 0; u < 8; u++) rank += (cj[u].x > my) + (cj[u].y > my);
        }
    }
    if (lane < n && rank < RTOPK) S->slot[rank] = my;
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_wave_barrier();
    const unsigned long long sk = S->slot[lane & (RTOPK - 1)];
    const bool sel = lane < RTOPK && sk != 0ull;
    const float v = sel ? key_logit((uint32_t)(sk >> 32)) : -INFINITY;
    const int myid = sel ? 255 - (int)(uint32_t)sk : -1;
    topk_finish(v, myid, min(n, RTOPK), ids, w, bad, ready, ready_val);
}

#endif
