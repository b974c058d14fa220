/*
 * pf_gemm.hip -- grouped expert GEMMs of the prefill path on MFMA.
 *
 * Both launch forms take a device tile list (group, first row) built by the
 * caller and a group table (prefill.h); a tile is `chunk` consecutive rows of
 * one group.  Launch grids are sized for the worst case and surplus
 * workgroups exit at once.
 *
 * v2 (PF_F16, the default) -- weight-stationary, 512 threads (two waves per
 * SIMD, up to 256 registers each):
 *   A workgroup owns up to 96 rows of one group (MS = 1..3 row blocks of 32)
 *   and 256 weight rows; every wave owns 32 of those rows as one 32-row MFMA
 *   column block (gate/up: 16 gate rows and the 16 up rows of the same
 *   columns, so the SiLU(gate) * up epilogue pairs lanes n and n + 16).  Each lane
 *   dequantises, for one weight row, the half super-block that forms its MFMA
 *   B operand, straight into registers: weights never pass through LDS.
 *   Inside a super-block the K order is permuted so that the 8 k-items a lane
 *   feeds per v_mfma_f32_32x32x16_f16 come from one dword of Q6_K ql / qh (or
 *   Q4_K qs): items i = 0..3 / 4..7 of k-slice kk in half h are super-block
 *   positions 128h + 64(kk/8) + 4(kk%8) + i and + 32 + i - 4.  Activations are
 *   stored in that permuted order (fp16, scaled per row by a power of two), so
 *   A and B agree and the dot product is unchanged.
 *   Q6_K: 1024 + q is built as an fp16 bit pattern with v_perm_b32, then
 *   fma(1024 + q, sc, -1056 sc) = sc (q - 32) exactly and one multiply by d
 *   rounds once: the fp16 weight is the reference's f32 weight (kernels.c:
 *   1855-1874) rounded to nearest even.  Q4_K: d sc q - dmin m in f32 with one
 *   fused multiply-add (kernels.c:1844-1852), then rounded to fp16.
 *
 * v1 (PF_SPLIT, PF_BF16) -- 64 x 64 output tiles, 256 threads, operands of
 * both sides dequantised / converted into LDS (gemm.h).
 */
#include <type_traits>

#include "internal.h"
#include "gemm.h"
#include "prefill.h"
#include "tile.h"

/* Opt-in timing (build with -DROASTER_PF_TS): thread 0 of each of the first
 * 4096 workgroups of a GEMM launch records the 100 MHz real-time counter at
 * its entry, after its first barrier, after each K step and at its end, with
 * its CU / XCD ids; roaster_pf_ts() copies the table out. */
#ifdef ROASTER_PF_TS
__device__ unsigned long long g_pf_ts[4096][16];
extern "C" int roaster_pf_ts(unsigned long long *out)
{
    return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(g_pf_ts), sizeof(g_pf_ts));
}
#define PF_TS(i)                                                                              \
    do {                                                                                      \
        if (threadIdx.x == 0 && blockIdx.x < 4096) g_pf_ts[blockIdx.x][i] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#define PF_TSV(i, v)                                                                          \
    do {                                                                                      \
        if (threadIdx.x == 0 && blockIdx.x < 4096) g_pf_ts[blockIdx.x][i] = (v);              \
    } while (0)
/* the persistent gate/up grid records by unit instead of workgroup */
/* the balanced down GEMM: [workgroup][event] */
__device__ unsigned long long g_pf_ts2[256][40];
extern "C" int roaster_pf_ts2(unsigned long long *out)
{
    return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(g_pf_ts2), sizeof(g_pf_ts2));
}
#define PF_TSD(i)                                                                             \
    do {                                                                                      \
        const int pf_i_ = (i);                                                                \
        if (threadIdx.x == 0 && blockIdx.x < 256 && pf_i_ < 40)                               \
            g_pf_ts2[blockIdx.x][pf_i_] = __builtin_amdgcn_s_memrealtime();                   \
    } while (0)
#define PF_TSU(u, i)                                                                          \
    do {                                                                                      \
        if (threadIdx.x == 0 && (u) >= 0 && (u) < 4096) g_pf_ts[u][i] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#define PF_TSUV(u, i, v)                                                                      \
    do {                                                                                      \
        if (threadIdx.x == 0 && (u) >= 0 && (u) < 4096) g_pf_ts[u][i] = (v);                 \
    } while (0)
#else
#define PF_TS(i) do { } while (0)
#define PF_TSV(i, v) do { } while (0)
#define PF_TSU(u, i) do { } while (0)
#define PF_TSD(i) do { } while (0)
#define PF_TSUV(u, i, v) do { } while (0)
#endif

static __device__ __forceinline__ float pf_silu_mul(float g, float u) { return (g / (1.0f + expf(-g))) * u; }
/* The exponent s of row_scale(amax): fwd = 2^s, clamped to [-100, 100]. */
static __device__ __forceinline__ int pf_scale_exp(float amax)
{
    const int s = (int)((__builtin_bit_cast(uint32_t, amax) >> 23) & 255u) - 127 - 14;
    return s < -100 ? -100 : (s > 100 ? 100 : s);
}
/* SiLU(g) * u with the hardware exp and reciprocal (v_exp_f32, v_rcp_f32: a
 * few ulp in f32; the result is rounded to fp16 for the next GEMM anyway). */
static __device__ __forceinline__ float pf_silu_mul_fast(float g, float u)
{
    return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

/* A workgroup barrier that orders LDS accesses only: every wave's LDS reads
 * and writes complete, global loads may stay in flight (__syncthreads()
 * waits for those too). */
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

/* Virtual block id: blocks b < R = ntiles * nblk run; on a grid dispatched
 * round-robin over the 8 XCDs, XCD b % 8 takes the contiguous range of
 * virtual ids [(b % 8) * R / 8, ...), so the n-blocks of one tile and the
 * consecutive tiles of one expert share an L2. */
__device__ __forceinline__ int pf_virtual_block(int b, int R)
{
    return (R & 7) ? b : (b & 7) * (R >> 3) + (b >> 3);
}

struct PfRowMeta {
    const float *src[GM];
    int slot[GM];
    float inv[GM], fwd[GM];
};

template <int OP>
__global__ void __launch_bounds__(GT) pf_gu_kernel(PfGemmArgs A)
{
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    __shared__ PfRowMeta meta;
    const int nblk = A.I / 32;
    const int R = *A.ntiles * nblk;
    const int b = blockIdx.x;
    if (b >= R) return;
    const int v = pf_virtual_block(b, R);
    const PfTile tile = A.tiles[v / nblk];
    const int j0 = (v % nblk) * 32;
    const PfGroup &G = A.groups[tile.grp];
    const int t = threadIdx.x;
    if (t < GM) {
        const int a = tile.m0 + t;
        if (a < G.n) {
            const int tok = G.tok ? G.tok[a] : G.tok0 + a;
            meta.src[t] = A.X + (size_t)tok * A.H;
            meta.slot[t] = G.slot0 + a;
            meta.inv[t] = A.xinv ? A.xinv[tok] : 1.0f;
            meta.fwd[t] = A.xfwd ? A.xfwd[tok] : 1.0f;
        } else {
            meta.src[t] = nullptr;
            meta.slot[t] = -1;
            meta.inv[t] = 1.0f;
            meta.fwd[t] = 1.0f;
        }
    }
    uint16_t *Xh = smem, *Wh = smem + G_TILE_ELEMS;
    uint16_t *Xl = smem + 2 * G_TILE_ELEMS, *Wl = smem + 3 * G_TILE_ELEMS;
    /* weight row of this thread: tile rows 0..31 gate rows j0.., 32..63 up rows j0.. */
    const int wr = t >> 2;
    const bool is_up = wr >= 32;
    const bool q6 = is_up ? G.uq6 : G.gq6;
    const size_t bb = q6 ? RQ6K_BYTES : RQ4K_BYTES;
    const int nkb = A.H / GK;
    const uint8_t *wrow = (is_up ? G.u : G.g) + (size_t)(j0 + (wr & 31)) * nkb * bb;
    __syncthreads();
    const float *xsrc = meta.src[wr];
    const float xinv = meta.inv[wr];
    const int w = t >> 6, wm = w & 1, wn = w >> 1;
    f32x16 acc = {};
    for (int kb = 0; kb < nkb; kb++) {
        if (kb) __syncthreads();
        load_w_tile<OP>(wrow + kb * bb, q6, Wh, Wl);
        load_x_tile<OP>(xsrc ? xsrc + kb * GK : nullptr, xinv, Xh, Xl);
        __syncthreads();
        mfma_tile<OP>(acc, Xh, Xl, Wh, Wl, wm, wn);
    }
    /* epilogue: gate / up blocks meet in LDS */
    __syncthreads();
    float *Cs = (float *)smem;                 /* [64][65] */
    const int l = t & 63;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int m = 32 * wm + 8 * (i >> 2) + 4 * (l >> 5) + (i & 3);
        Cs[m * 65 + 32 * wn + (l & 31)] = acc[i];
    }
    __syncthreads();
    const int m = t >> 2, q = t & 3;
    const int slot = meta.slot[m];
    const float fwd = meta.fwd[m];
    float e8[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float g = Cs[m * 65 + 8 * q + i] * fwd, u = Cs[m * 65 + 32 + 8 * q + i] * fwd;
        e8[i] = pf_silu_mul(g, u);
    }
    if (slot >= 0) {
        float4 *dst = (float4 *)(A.act + (size_t)slot * A.I + j0 + 8 * q);
        dst[0] = make_float4(e8[0], e8[1], e8[2], e8[3]);
        dst[1] = make_float4(e8[4], e8[5], e8[6], e8[7]);
    }
}

template <int OP>
__global__ void __launch_bounds__(GT) pf_down_kernel(PfGemmArgs A)
{
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    __shared__ PfRowMeta meta;
    const int nblk = A.H / GN;
    const int R = *A.ntiles * nblk;
    const int b = blockIdx.x;
    if (b >= R) return;
    const int v = pf_virtual_block(b, R);
    const PfTile tile = A.tiles[v / nblk];
    const int n0 = (v % nblk) * GN;
    const PfGroup &G = A.groups[tile.grp];
    const int t = threadIdx.x;
    if (t < GM) {
        const int a = tile.m0 + t;
        if (a < G.n) {
            const int slot = G.slot0 + a;
            meta.src[t] = A.act + (size_t)slot * A.I;
            meta.slot[t] = slot;
            meta.inv[t] = 1.0f;
            meta.fwd[t] = 1.0f;
        } else {
            meta.src[t] = nullptr;
            meta.slot[t] = -1;
            meta.inv[t] = 1.0f;
            meta.fwd[t] = 1.0f;
        }
    }
    uint16_t *Xh = smem, *Wh = smem + G_TILE_ELEMS;
    uint16_t *Xl = smem + 2 * G_TILE_ELEMS, *Wl = smem + 3 * G_TILE_ELEMS;
    const int wr = t >> 2;
    const bool q6 = G.dq6;
    const size_t bb = q6 ? RQ6K_BYTES : RQ4K_BYTES;
    const int nkb = A.I / GK;
    const uint8_t *wrow = G.d + (size_t)(n0 + wr) * nkb * bb;
    __syncthreads();
    const float *xsrc = meta.src[wr];
    const float xinv = meta.inv[wr];
    const int w = t >> 6, wm = w & 1, wn = w >> 1;
    f32x16 acc = {};
    for (int kb = 0; kb < nkb; kb++) {
        if (kb) __syncthreads();
        load_w_tile<OP>(wrow + kb * bb, q6, Wh, Wl);
        load_x_tile<OP>(xsrc ? xsrc + kb * GK : nullptr, xinv, Xh, Xl);
        __syncthreads();
        mfma_tile<OP>(acc, Xh, Xl, Wh, Wl, wm, wn);
    }
    const int l = t & 63;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int m = 32 * wm + 8 * (i >> 2) + 4 * (l >> 5) + (i & 3);
        const int slot = meta.slot[m];
        if (slot >= 0) A.out[(size_t)slot * A.H + n0 + 32 * wn + (l & 31)] = acc[i] * meta.fwd[m];
    }
}


/* ---- v2 ------------------------------------------------------------------- */
#define V2_T 512                  /* threads */
#define V2_W 8                    /* waves */
#define V2_GU_J (16 * V2_W)       /* gate/up j columns per workgroup */
#define V2_DN_N (32 * V2_W)       /* down output rows per workgroup */
static_assert(V2_DN_N == PF_DN_ROWS, "the down GEMM's unit is the plan kernel's");
#define V2_MC 96                  /* rows per tile */
#define V2_LD (GK + 8)            /* LDS row stride (fp16 elements) */
#ifndef PF_DN_NT
#define PF_DN_NT 4                /* down output tiles per workgroup (inter <= 512) */
#endif

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

/* One lane's raw share of a super-block: half h (weights 128h .. 128h+127). */
struct RawQ6 { uint32_t L[16], Hh[8], S[2], d; };
struct RawQ4 { uint32_t hd[4], Q[16]; };
template <bool Q6> struct RawOf;
template <> struct RawOf<true> { typedef RawQ6 T; };
template <> struct RawOf<false> { typedef RawQ4 T; };

/* Per super-block constants of one lane's half. */
struct ConstQ6 { f16x2 sc[8], bias[8], d; };   /* sc[s] = (S[s], S[s]), bias = -1056 sc */
struct ConstQ4 { float s[4], m[4]; };          /* sub-blocks 4h .. 4h+3: d*sc, dmin*m */
template <bool Q6> struct ConstOf;
template <> struct ConstOf<true> { typedef ConstQ6 T; };
template <> struct ConstOf<false> { typedef ConstQ4 T; };

__device__ __forceinline__ void raw_consts(const RawQ6 &r, int h, ConstQ6 &c)
{
    (void)h;
#pragma unroll
    for (int s = 0; s < 8; s++) {
        const int v = (int)(int8_t)((r.S[s >> 2] >> (8 * (s & 3))) & 0xFFu);
        const _Float16 f = (_Float16)v;
        c.sc[s] = (f16x2){ f, f };
        c.bias[s] = c.sc[s] * (f16x2){ (_Float16)-1056.0f, (_Float16)-1056.0f };   /* exact: 33 * 32 * sc */
    }
    const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)r.d);
    c.d = (f16x2){ d, d };
}

__device__ __forceinline__ void raw_consts(const RawQ4 &r, int h, ConstQ4 &c)
{
    const float d = f16_bits_to_f32(r.hd[0] & 0xFFFFu), dmin = f16_bits_to_f32(r.hd[0] >> 16);
    const uint32_t s03 = r.hd[1], s47 = r.hd[2], s811 = r.hd[3];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        int sc, m;
        if (h == 0) {
            sc = byte_of(s03, i) & 63;
            m = byte_of(s47, i) & 63;
        } else {
            sc = (byte_of(s811, i) & 15) | ((byte_of(s03, i) >> 6) << 4);
            m = (byte_of(s811, i) >> 4) | ((byte_of(s47, i) >> 6) << 4);
        }
        c.s[i] = d * (float)sc;
        c.m[i] = dmin * (float)m;
    }
}

/* fp16 pairs (1024 + b0, 1024 + b1) and (1024 + b2, 1024 + b3) of the bytes of q. */
__device__ __forceinline__ f16x2 magic_lo(uint32_t q) { return __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(q, 0x64646464u, 0x00050004u)); }
__device__ __forceinline__ f16x2 magic_hi(uint32_t q) { return __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(q, 0x64646464u, 0x00070006u)); }

__device__ __forceinline__ uint32_t q6_pair(f16x2 v, f16x2 sc, f16x2 bias, f16x2 d)
{
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(v, sc, bias) * d);
}

/* B operands of k-slices j and j + 8 (j = 0..7). */
__device__ __forceinline__ void dequant_pair(const RawQ6 &r, const ConstQ6 &c, int j, f16x8 &b0, f16x8 &b1)
{
    const uint32_t A = r.L[j], B = r.L[8 + j], C = r.Hh[j];
    const uint32_t qa = (A & 0x0F0F0F0Fu) | ((C << 4) & 0x30303030u);
    const uint32_t qb = (B & 0x0F0F0F0Fu) | ((C << 2) & 0x30303030u);
    const uint32_t qc = ((A >> 4) & 0x0F0F0F0Fu) | (C & 0x30303030u);
    const uint32_t qd = ((B >> 4) & 0x0F0F0F0Fu) | ((C >> 2) & 0x30303030u);
    const int s = j >> 2;
    const uint4 u0 = { q6_pair(magic_lo(qa), c.sc[s], c.bias[s], c.d), q6_pair(magic_hi(qa), c.sc[s], c.bias[s], c.d),
                       q6_pair(magic_lo(qb), c.sc[s + 2], c.bias[s + 2], c.d),
                       q6_pair(magic_hi(qb), c.sc[s + 2], c.bias[s + 2], c.d) };
    const uint4 u1 = { q6_pair(magic_lo(qc), c.sc[s + 4], c.bias[s + 4], c.d),
                       q6_pair(magic_hi(qc), c.sc[s + 4], c.bias[s + 4], c.d),
                       q6_pair(magic_lo(qd), c.sc[s + 6], c.bias[s + 6], c.d),
                       q6_pair(magic_hi(qd), c.sc[s + 6], c.bias[s + 6], c.d) };
    b0 = __builtin_bit_cast(f16x8, u0);
    b1 = __builtin_bit_cast(f16x8, u1);
}

__device__ __forceinline__ f16x8 q4_slice(uint32_t a, float s0, float m0, float s1, float m1)
{
    const uint32_t lo = a & 0x0F0F0F0Fu, hi = (a >> 4) & 0x0F0F0F0Fu;
    f32x8 v;
#pragma unroll
    for (int b = 0; b < 4; b++) {
        v[b] = fmaf(s0, (float)((lo >> (8 * b)) & 0xFFu), -m0);
        v[4 + b] = fmaf(s1, (float)((hi >> (8 * b)) & 0xFFu), -m1);
    }
    return __builtin_convertvector(v, f16x8);
}

__device__ __forceinline__ void dequant_pair(const RawQ4 &r, const ConstQ4 &c, int j, f16x8 &b0, f16x8 &b1)
{
    b0 = q4_slice(r.Q[j], c.s[0], c.m[0], c.s[1], c.m[1]);
    b1 = q4_slice(r.Q[8 + j], c.s[2], c.m[2], c.s[3], c.m[3]);
}

/* Natural position p (multiple of 4) of a super-block -> its permuted slot. */
__device__ __forceinline__ int perm_slot4(int p)
{
    const int h = p >> 7, q = p & 127, hi = q >> 6, r = q & 63;
    const int l0 = r < 32 ? r : r - 32, i0 = r < 32 ? 0 : 4;
    return (8 * hi + (l0 >> 2)) * 16 + 8 * h + i0;
}


/* ---- v2 workgroup: 8 waves, two per SIMD -------------------------------------
 * Each wave owns one 32-row MFMA column block of weights: for gate/up, lanes
 * n = 0..15 hold gate row j0 + 16w + n and lanes 16..31 the up row of the same
 * column, so SiLU(gate) * up pairs lane n with lane n + 16 in the epilogue; for
 * down, output rows n0 + 32w + n.  Two waves per SIMD let one wave's dequant
 * VALU work run under the other's MFMAs.  Activations (MS x 32 rows x 256
 * fp16 per K step, permuted K order) are double-buffered in LDS. */
#define V3_XBUF (V2_MC * V2_LD)            /* fp16 elements per activation buffer */

/* MFMA work of one K step: MS row blocks x this wave's 32 weight columns, one
 * accumulator per row block.  Xs: activation buffer, row stride V2_LD. */
template <int MS, bool Q6>
__device__ __forceinline__ void v4_mfma(f32x16 (&acc)[MS], const _Float16 *Xs, const typename RawOf<Q6>::T &r,
                                        int h)
{
    typename ConstOf<Q6>::T c;
    raw_consts(r, h, c);
    const int l = threadIdx.x & 63;
    const _Float16 *xa = Xs + (l & 31) * V2_LD + 8 * (l >> 5);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        f16x8 b0, b1;
        dequant_pair(r, c, j, b0, b1);
#pragma unroll
        for (int ms = 0; ms < MS; ms++) {
            const f16x8 x0 = *(const f16x8 *)(xa + ms * 32 * V2_LD + 16 * j);
            const f16x8 x1 = *(const f16x8 *)(xa + ms * 32 * V2_LD + 16 * (j + 8));
            acc[ms] = __builtin_amdgcn_mfma_f32_32x32x16_f16(x0, b0, acc[ms], 0, 0, 0);
            acc[ms] = __builtin_amdgcn_mfma_f32_32x32x16_f16(x1, b1, acc[ms], 0, 0, 0);
        }
    }
}

#define V5_MAXPART 128                 /* inter / 16 for inter <= 2048 */
struct V4Shared {
    int tok[V2_MC];
    int slot[V2_MC];
    float inv[V2_MC], fwd[V2_MC];
    int8_t psh[V2_MC][V5_MAXPART];     /* down: part scale exponent - row scale exponent (<= 0) */
};

/* v4_mfma for a wave whose lanes n < 16 hold gate rows of type QG and lanes
 * n >= 16 up rows of type QU != QG: each lane dequantises its own record
 * (divergent VALU work, exec-masked), then every MFMA runs with the whole
 * wave active: an MFMA ignores the exec mask and reads all 64 lanes. */
template <int MS, bool QG, bool QU>
__device__ __forceinline__ void v4_mfma_mixed(f32x16 (&acc)[MS], const _Float16 *Xs, const typename RawOf<QG>::T &rg,
                                              const typename RawOf<QU>::T &ru, bool up, int h)
{
    typename ConstOf<QG>::T cg;
    typename ConstOf<QU>::T cu;
    if (up) raw_consts(ru, h, cu);
    else raw_consts(rg, h, cg);
    const int l = threadIdx.x & 63;
    const _Float16 *xa = Xs + (l & 31) * V2_LD + 8 * (l >> 5);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        f16x8 b0, b1;
        if (up) dequant_pair(ru, cu, j, b0, b1);
        else dequant_pair(rg, cg, j, b0, b1);
#pragma unroll
        for (int ms = 0; ms < MS; ms++) {
            const f16x8 x0 = *(const f16x8 *)(xa + ms * 32 * V2_LD + 16 * j);
            const f16x8 x1 = *(const f16x8 *)(xa + ms * 32 * V2_LD + 16 * (j + 8));
            acc[ms] = __builtin_amdgcn_mfma_f32_32x32x16_f16(x0, b0, acc[ms], 0, 0, 0);
            acc[ms] = __builtin_amdgcn_mfma_f32_32x32x16_f16(x1, b1, acc[ms], 0, 0, 0);
        }
    }
}

/* ---- v5: weights straight from the MFMA tile layout into registers ----------
 * Workgroup shape, MFMA work and activation staging as in v4 (8 waves, two per
 * SIMD; activations double-buffered in LDS through registers), but every lane
 * loads its raw super-block half directly from the tile copy of the matrix
 * (tile.h): seven 16-byte loads (Q6_K) or five (Q4_K), each instruction
 * covering contiguous runs of a wave's records (one
 * kilobyte for down; two 256-byte runs for gate/up, whose waves pair 16 gate
 * rows with 16 up rows).  The raw registers are double-buffered per wave: step
 * kb + 1's loads are issued before step kb's MFMA work, with no workgroup
 * barrier for them, and the LDS holds activations only. */
__device__ __forceinline__ void tile_load(RawQ6 &r, const uint8_t *tile, int lane)
{
    const uint8_t *p = tile + 16 * lane;
    uint4 s[6];
#pragma unroll
    for (int i = 0; i < 6; i++) s[i] = gld_u4(p + 1024 * i);
    const uint3 s6 = gld_u3(p + 1024 * 6);          /* the record's last dword is padding */
#pragma unroll
    for (int i = 0; i < 4; i++) {
        r.L[4 * i] = s[i].x; r.L[4 * i + 1] = s[i].y; r.L[4 * i + 2] = s[i].z; r.L[4 * i + 3] = s[i].w;
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {
        r.Hh[4 * i] = s[4 + i].x; r.Hh[4 * i + 1] = s[4 + i].y; r.Hh[4 * i + 2] = s[4 + i].z; r.Hh[4 * i + 3] = s[4 + i].w;
    }
    r.S[0] = s6.x;
    r.S[1] = s6.y;
    r.d = s6.z & 0xFFFFu;
}

__device__ __forceinline__ void tile_load(RawQ4 &r, const uint8_t *tile, int lane)
{
    const uint8_t *p = tile + 16 * lane;
    uint4 s[5];
#pragma unroll
    for (int i = 0; i < 5; i++) s[i] = gld_u4(p + 1024 * i);
    r.hd[0] = s[0].x; r.hd[1] = s[0].y; r.hd[2] = s[0].z; r.hd[3] = s[0].w;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        r.Q[4 * i] = s[1 + i].x; r.Q[4 * i + 1] = s[1 + i].y; r.Q[4 * i + 2] = s[1 + i].z; r.Q[4 * i + 3] = s[1 + i].w;
    }
}

/* Slice i of a lane's record (one 16-byte load, the last Q6_K slice 12
 * bytes): the pieces of tile_load, issued one at a time. */
__device__ __forceinline__ void tile_slice(RawQ6 &r, const uint8_t *tile, int lane, int i)
{
    const uint8_t *p = tile + 16 * lane + 1024 * i;
    if (i < 4) {
        const uint4 s = gld_u4(p);
        r.L[4 * i] = s.x; r.L[4 * i + 1] = s.y; r.L[4 * i + 2] = s.z; r.L[4 * i + 3] = s.w;
    } else if (i < 6) {
        const uint4 s = gld_u4(p);
        const int k = 4 * (i - 4);
        r.Hh[k] = s.x; r.Hh[k + 1] = s.y; r.Hh[k + 2] = s.z; r.Hh[k + 3] = s.w;
    } else {
        const uint3 s = gld_u3(p);
        r.S[0] = s.x; r.S[1] = s.y; r.d = s.z & 0xFFFFu;
    }
}

__device__ __forceinline__ void tile_slice(RawQ4 &r, const uint8_t *tile, int lane, int i)
{
    const uint4 s = gld_u4(tile + 16 * lane + 1024 * i);
    if (i == 0) {
        r.hd[0] = s.x; r.hd[1] = s.y; r.hd[2] = s.z; r.hd[3] = s.w;
    } else {
        const int k = 4 * (i - 1);
        r.Q[k] = s.x; r.Q[k + 1] = s.y; r.Q[k + 2] = s.z; r.Q[k + 3] = s.w;
    }
}

/* v4_mfma with the next K step's loads spread over its eight groups and the
 * dequantisation software-pipelined: group j runs piece(j) (a share of the
 * next step's loads), its activation reads, then the dequantisation of group
 * j + 1 interleaved with group j's MFMAs (one MFMA, then a share of the VALU
 * work, in turn), so that loads queue at the vector memory unit a few at a
 * time and the VALU work runs while the matrix core is busy.  A scheduling
 * fence after each group keeps every piece in its slot. */
template <int MS, bool Q6, class Piece>
__device__ __forceinline__ void v8_mfma(f32x16 (&acc)[MS], const _Float16 *Xs, const typename RawOf<Q6>::T &r,
                                        int h, Piece &&piece)
{
    typename ConstOf<Q6>::T c;
    raw_consts(r, h, c);
    const int l = threadIdx.x & 63;
    const _Float16 *xa = Xs + (l & 31) * V2_LD + 8 * (l >> 5);
    f16x8 b0, b1;
    dequant_pair(r, c, 0, b0, b1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        piece(j);
        f16x8 x0[MS], x1[MS];
#pragma unroll
        for (int ms = 0; ms < MS; ms++) {
            x0[ms] = *(const f16x8 *)(xa + ms * 32 * V2_LD + 16 * j);
            x1[ms] = *(const f16x8 *)(xa + ms * 32 * V2_LD + 16 * (j + 8));
        }
        f16x8 n0 = b0, n1 = b1;
        if (j < 7) dequant_pair(r, c, j + 1, n0, n1);
#pragma unroll
        for (int ms = 0; ms < MS; ms++) {
            acc[ms] = __builtin_amdgcn_mfma_f32_32x32x16_f16(x0[ms], b0, acc[ms], 0, 0, 0);
            acc[ms] = __builtin_amdgcn_mfma_f32_32x32x16_f16(x1[ms], b1, acc[ms], 0, 0, 0);
        }
        constexpr int VPM = (34 + 2 * MS - 1) / (2 * MS);
        __builtin_amdgcn_sched_group_barrier(0x0020, 8, 0);      /* the piece's loads */
        __builtin_amdgcn_sched_group_barrier(0x0100, 2 * MS, 0); /* activation reads */
        __builtin_amdgcn_sched_group_barrier(0x0002, 6, 0);
#pragma unroll
        for (int i = 0; i < 2 * MS; i++) {
            __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x0002, VPM, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        b0 = n0;
        b1 = n1;
    }
}

/* Epilogue of a gate/up tile: lane n < 16 holds gate and lane n + 16 up of
 * column j0 + 16 w + (n & 15).  For the row pair (i, i + 1) one lane swap
 * (lane ^ 16) gives lanes n < 16 the up value of row i and lanes n >= 16 the
 * gate value of row i + 1, so all 32 lanes compute act = silu(gate) * up (f32)
 * for one row each; a 16-lane max gives the row's largest |act| over this
 * wave's 16 columns (one part), and act is rounded to fp16 scaled by that
 * part's power of two (row_scale of the part max).  Both are staged in LDS
 * (the activation buffers are free once every wave's last MFMAs have read
 * them) and written out as whole rows: the tile's 128 columns of act16 (256
 * bytes) and its 8 part maxima per row. */
template <int MS, class M = V4Shared, bool LB = false>
__device__ __forceinline__ void gu_epilogue(const PfGemmArgs &A, const M &meta, const f32x16 (&acc)[MS], int mlen,
                                            int j0, uint8_t *lds)
{
    int t = threadIdx.x;
    if constexpr (LB) asm volatile("" : "+v"(t));            /* its addressing is not hoisted into the K loop */
    const int l = t & 63, h = l >> 5, w = t >> 6, n = l & 31;
    const bool up = n >= 16;
    const int npart = A.I / 16;
    constexpr int AP = V2_GU_J + 8;                          /* fp16 pitch of a staged row */
    if constexpr (LB) lds_barrier();
    else __syncthreads();
    _Float16 *act_s = (_Float16 *)lds;                       /* [MS * 32][AP] */
    float *pmx_s = (float *)(lds + (size_t)MS * 32 * AP * 2); /* [MS * 32][8] */
#pragma unroll
    for (int ms = 0; ms < MS; ms++) {
        /* the rows' scales, read together; a row >= mlen reads whatever its
         * slot holds and its value is replaced by 0 below */
        float fw[8];
#pragma unroll
        for (int q = 0; q < 8; q++) fw[q] = meta.fwd[32 * ms + 8 * (q >> 1) + 4 * h + 2 * (q & 1) + (up ? 1 : 0)];
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
            const float v0 = acc[ms][i], v1 = acc[ms][i + 1];
            const float mine = up ? v1 : v0, other = up ? v0 : v1;
            /* lane ^ 16 (rows 0 <-> 1, 2 <-> 3): a VALU lane swap */
            const auto sw = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, other),
                                                             __builtin_bit_cast(uint32_t, other), false, false);
            const float got = __builtin_bit_cast(float, (uint32_t)(up ? sw[0] : sw[1]));
            const float gsum = up ? got : mine, usum = up ? mine : got;
            const int m = 32 * ms + 8 * (i >> 2) + 4 * h + (i & 3) + (up ? 1 : 0);
            const float f = fw[i >> 1];
            float e = pf_silu_mul_fast(gsum * f, usum * f);
            e = m < mlen ? e : 0.0f;                         /* a select: no branch */
            /* the 16-lane maximum of |e| on the bit patterns (non-negative
             * floats order as unsigned integers): one DPP max per step */
            uint32_t mb = __builtin_bit_cast(uint32_t, e) & 0x7FFFFFFFu;
            mb = max(mb, (uint32_t)dpp_i<DPP_XOR1>((int)mb));
            mb = max(mb, (uint32_t)dpp_i<DPP_XOR2>((int)mb));
            mb = max(mb, (uint32_t)dpp_i<DPP_HALF_MIRROR>((int)mb));
            mb = max(mb, (uint32_t)dpp_i<DPP_MIRROR>((int)mb));
            const float mx = __builtin_bit_cast(float, mb);
            float pinv, pfwd;
            row_scale(mx, pinv, pfwd);
            act_s[m * AP + 16 * w + (n & 15)] = (_Float16)(e * pinv);
            if ((n & 15) == 0) pmx_s[m * 8 + w] = mx;
        }
    }
    if constexpr (LB) lds_barrier();
    else __syncthreads();
    /* rows m < mlen: 16 lanes per row, 16 bytes each */
    for (int r = t >> 4; r < mlen; r += V2_T / 16) {
        const int c = t & 15;
        *(uint4 *)(A.act16 + (size_t)meta.slot[r] * A.I + j0 + 8 * c) = *(const uint4 *)(act_s + r * AP + 8 * c);
    }
    for (int r = t >> 1; r < mlen; r += V2_T / 2) {
        const int c = t & 1;
        *(float4 *)(A.pmax + (size_t)meta.slot[r] * npart + (j0 >> 4) + 4 * c) = *(const float4 *)(pmx_s + r * 8 + 4 * c);
    }
    if constexpr (!LB) PF_TS(11);
}

/* Gate/up tile: lanes n < 16 of wave w take gate row j0 + 16 w + n, lanes
 * n >= 16 the up row of the same column.  QG == QU: one raw type per wave;
 * otherwise the two halves load and dequantise on divergent paths and share
 * the MFMAs (v4_mfma_mixed). */
template <int MS, bool QG, bool QU>
__device__ __forceinline__ void v5_gu_body(const PfGemmArgs &A, const PfGroup &G, V4Shared &meta, const PfTile &tile,
                                           int mlen, int j0, uint8_t *lds)
{
    const int t = threadIdx.x, l = t & 63, h = l >> 5, w = t >> 6, n = l & 31;
    const int nkb = A.H / GK;
    _Float16 *Xb = (_Float16 *)lds;
    const bool up = n >= 16;
    const int jrow = j0 + 16 * w + (n & 15);
    const int tlane = (jrow & (TL_ROWS - 1)) + 32 * h;
    constexpr int TG = TL_BYTES(QG), TU = TL_BYTES(QU);
    const uint8_t *wt = up ? G.tu + (size_t)(jrow / TL_ROWS) * nkb * TU : G.tg + (size_t)(jrow / TL_ROWS) * nkb * TG;
    const int tb = up ? TU : TG;
    typename RawOf<QG>::T rg[2];
    typename RawOf<QU>::T ru[2];
    auto w_load = [&](int buf, int kb) {
        if (QG == QU || !up) tile_load(rg[buf], wt + (size_t)kb * tb, tlane);
        else tile_load(ru[buf], wt + (size_t)kb * tb, tlane);
    };
    /* the rows' token ids, then the first step's weights (they depend on
     * nothing; a wave's loads return in order, so the ids do not wait for
     * them) */
    int tok = 0;
    if (t < mlen) tok = G.tok ? G.tok[tile.m0 + t] : G.tok0 + tile.m0 + t;
    w_load(0, 0);
    if (t < mlen) {
        meta.tok[t] = tok;
        meta.slot[t] = G.slot0 + tile.m0 + t;
    }
    __syncthreads();
    /* activation staging: rows >= mlen read row 0 (their products are never
     * stored), so every load is unconditional and the K loop has no branches
     * around its loads */
    constexpr int NP = (MS * 32 * 32 + V2_T - 1) / V2_T;
    uint4 xr[NP];
    uint32_t xoff[NP];                  /* byte offsets into X16 (< 2^28: T <= 65536, H <= 2048) */
#pragma unroll
    for (int i = 0; i < NP; i++) {
        const int idx = t + i * V2_T, row = idx >> 5;
        xoff[i] = 2u * ((uint32_t)meta.tok[row < mlen ? row : 0] * (uint32_t)A.H + 8u * (idx & 31));
    }
    const uint8_t *x16 = (const uint8_t *)A.X16;
    auto x_load = [&](int kb) {
#pragma unroll
        for (int i = 0; i < NP; i++) xr[i] = gld_u4(x16 + xoff[i] + 2 * kb * GK);
    };
    auto x_store = [&](_Float16 *dst) {
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const int idx = t + i * V2_T, row = idx >> 5;
            if ((MS * 32 * 32) % V2_T == 0 || row < MS * 32) *(uint4 *)(dst + row * V2_LD + 8 * (idx & 31)) = xr[i];
        }
    };
    f32x16 acc[MS];
#pragma unroll
    for (int ms = 0; ms < MS; ms++) acc[ms] = (f32x16){};
    /* a step's MFMA work; the scheduling fences keep the next step's loads
     * ahead of it and the activation store (which waits for those loads)
     * after it */
    auto step = [&](int buf, const _Float16 *Xs) {
        __builtin_amdgcn_sched_barrier(0);
        if (QG == QU) v4_mfma<MS, QG>(acc, Xs, rg[buf], h);
        else v4_mfma_mixed<MS, QG, QU>(acc, Xs, rg[buf], ru[buf], up, h);
        __builtin_amdgcn_sched_barrier(0);
    };
    x_load(0);
    if (t < mlen) meta.fwd[t] = A.xfwd ? A.xfwd[meta.tok[t]] : 1.0f;   /* read in the epilogue */
    x_store(Xb);
    __syncthreads();
    PF_TS(2);
    int tsk = 3;
    (void)tsk;
    int kb = 0;
    if constexpr (QG == QU) {
        /* step kb's MFMA work on raw buffer buf with step kn's loads spread
         * over it: the activations in the first group (a wave's loads complete
         * in order, so the activation store waits for them only), then one
         * weight slice per group */
        auto step_ld = [&](int buf, const _Float16 *Xs, int kn) {
            const uint8_t *wn = wt + (size_t)kn * tb;
            __builtin_amdgcn_sched_barrier(0);
            v8_mfma<MS, QG>(acc, Xs, rg[buf], h, [&](int j) {
                if (j == 0) x_load(kn);
                if (j < TL_SLICES(QG)) tile_slice(rg[buf ^ 1], wn, tlane, j);
            });
        };
        /* bare barriers: __syncthreads()'s release fence would drain the
         * next step's weight loads, which are only needed after the barrier */
        for (; kb + 2 < nkb; kb += 2) {
            step_ld(0, Xb, kb + 1);
            x_store(Xb + V3_XBUF);
            lds_barrier();
            PF_TS(tsk++);
            step_ld(1, Xb + V3_XBUF, kb + 2);
            x_store(Xb);
            lds_barrier();
            PF_TS(tsk++);
        }
        if (kb + 1 < nkb) {
            step_ld(0, Xb, kb + 1);
            x_store(Xb + V3_XBUF);
            lds_barrier();
            PF_TS(tsk++);
            step(1, Xb + V3_XBUF);
        } else {
            step(0, Xb);
        }
        PF_TS(tsk++);
    } else {
        /* steady state: steps kb (raw buffer 0, activation buffer 0) and kb +
         * 1 (buffers 1), each issuing the next step's loads first, activations
         * before weights: a wave's loads complete in order, so the activation
         * store (and with it the barrier) waits for the activation loads only,
         * not for the next step's weights from HBM */
        for (; kb + 2 < nkb; kb += 2) {
            x_load(kb + 1);
            w_load(1, kb + 1);
            step(0, Xb);
            x_store(Xb + V3_XBUF);
            __syncthreads();
            x_load(kb + 2);
            w_load(0, kb + 2);
            step(1, Xb + V3_XBUF);
            x_store(Xb);
            __syncthreads();
        }
        /* last one or two steps */
        if (kb + 1 < nkb) {
            x_load(kb + 1);
            w_load(1, kb + 1);
            step(0, Xb);
            x_store(Xb + V3_XBUF);
            __syncthreads();
            step(1, Xb + V3_XBUF);
        } else {
            step(0, Xb);
        }
    }
    gu_epilogue<MS>(A, meta, acc, mlen, j0, lds);
}

/* A wave's down products of one output tile: lane n of half h holds column
 * orow (= its tile column + n) of rows 32 ms + 8 (i >> 2) + 4 h + (i & 3).
 * f32: one store per value.  fp16 (already scaled by each row's 2^-oexp):
 * lanes n and n ^ 1 swap one value of each row pair (i, i + 1), so the even
 * lane stores row i's columns (n, n + 1) and the odd lane row i + 1's as one
 * 4-byte store: half the store instructions. */
template <int MS, bool ALL = false>
__device__ __forceinline__ void dn_store_tile(const PfGemmArgs &A, const V4Shared &meta, const f32x16 (&acc)[MS],
                                              int mlen, int orow)
{
    /* ALL: fp16 products, every row stored (rows past the tile's end carry
     * the spare slot), no branches */
    if constexpr (ALL) mlen = MS * 32;
    const int l = threadIdx.x & 63, h = l >> 5;
    if (!ALL && !A.out16) {
#pragma unroll
        for (int ms = 0; ms < MS; ms++)
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int m = 32 * ms + 8 * (i >> 2) + 4 * h + (i & 3);
                if (m < mlen) A.out[(size_t)meta.slot[m] * A.H + orow] = acc[ms][i] * meta.fwd[m];
            }
        return;
    }
    const bool odd = (l & 1) != 0;
#pragma unroll
    for (int ms = 0; ms < MS; ms++)
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
            const int m0 = 32 * ms + 8 * (i >> 2) + 4 * h + (i & 3);     /* value i + 1 is row m0 + 1 */
            const float v0 = acc[ms][i] * meta.fwd[m0], v1 = acc[ms][i + 1] * meta.fwd[m0 + 1];
            const float got = dpp_f<DPP_XOR1>(odd ? v0 : v1);
            const float lo = odd ? got : v0, hi = odd ? v1 : got;
            const int m = odd ? m0 + 1 : m0;
            if (m < mlen) {
                const f16x2 pk = { (_Float16)lo, (_Float16)hi };
                *(uint32_t *)(A.out16 + (size_t)meta.slot[m] * A.H + orow - (odd ? 1 : 0)) = __builtin_bit_cast(uint32_t, pk);
            }
        }
}

/* Down tile: wave w takes output rows n0 + 32 w .. + 31 (one tile row group,
 * its lane records in lane order). */
template <int MS, bool QD>
__device__ __forceinline__ void v5_dn_body(const PfGemmArgs &A, const PfGroup &G, const V4Shared &meta, int mlen, int n0,
                                           uint8_t *lds)
{
    const int t = threadIdx.x, l = t & 63, h = l >> 5, w = t >> 6, n = l & 31;
    const int nkb = A.I / GK;
    _Float16 *Xb = (_Float16 *)lds;
    constexpr int TD = TL_BYTES(QD);
    const int orow = n0 + 32 * w + n;
    const uint8_t *wt = G.td + (size_t)((n0 + 32 * w) / TL_ROWS) * nkb * TD;
    /* activation staging: act16 rows (natural order, each 16-column part at
     * its own power of two) -> fp16 at the row's power of two (ldexp by the
     * part's shift, exact unless the value turns subnormal), in the permuted K
     * order; 4-element pieces idx = t + i * V2_T, row idx / 64 */
    constexpr int NP = MS * 32 * 64 / V2_T;
    const uint8_t *a16 = (const uint8_t *)A.act16;
    auto x_stage = [&](int kb, _Float16 *dst) {
        uint2 xr[NP];
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const int idx = t + i * V2_T, row = idx >> 6;
            const int slot = meta.slot[row < mlen ? row : 0];
            xr[i] = gld_u2(a16 + 2 * ((size_t)slot * A.I + kb * GK + 4 * (idx & 63)));
        }
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const int idx = t + i * V2_T, row = idx >> 6, c4 = 4 * (idx & 63);
            const int sh = row < mlen ? (int)meta.psh[row][(kb * GK + c4) >> 4] : -200;
            const f16x4 hv = __builtin_bit_cast(f16x4, xr[i]);
            const f32x8 e = { __builtin_ldexpf((float)hv[0], sh), __builtin_ldexpf((float)hv[1], sh),
                              __builtin_ldexpf((float)hv[2], sh), __builtin_ldexpf((float)hv[3], sh),
                              0.f, 0.f, 0.f, 0.f };
            const uint4 cu = __builtin_bit_cast(uint4, __builtin_convertvector(e, f16x8));
            *(uint2 *)(dst + row * V2_LD + perm_slot4(c4)) = make_uint2(cu.x, cu.y);
        }
    };
    f32x16 acc[MS];
#pragma unroll
    for (int ms = 0; ms < MS; ms++) acc[ms] = (f32x16){};
    typename RawOf<QD>::T r[2];
    tile_load(r[0], wt, l);
    if (nkb > 1) tile_load(r[1], wt + TD, l);
    x_stage(0, Xb);
    if (nkb > 1) x_stage(1, Xb + V3_XBUF);
    __syncthreads();
    for (int kb = 0; kb < nkb; kb += 2) {
        v4_mfma<MS, QD>(acc, Xb, r[0], h);
        if (kb + 1 >= nkb) break;
        if (kb + 2 < nkb) tile_load(r[0], wt + (size_t)(kb + 2) * TD, l);
        v4_mfma<MS, QD>(acc, Xb + V3_XBUF, r[1], h);
        if (kb + 2 >= nkb) break;
        if (kb + 3 < nkb) tile_load(r[1], wt + (size_t)(kb + 3) * TD, l);
        __syncthreads();                    /* every wave is done with both buffers */
        x_stage(kb + 2, Xb);
        if (kb + 3 < nkb) x_stage(kb + 3, Xb + V3_XBUF);
        __syncthreads();
    }
    dn_store_tile<MS>(A, meta, acc, mlen, orow);
}

/* Down, K <= 512 (one or two K steps): a workgroup keeps the whole activation
 * tile in LDS (both K steps, staged once) and walks nt_count consecutive
 * 256-row output tiles; the next tile's weight registers are loaded while the
 * current tile computes, with no workgroup barrier after the staging. */
template <int MS, bool QD>
__device__ __forceinline__ void v6_dn_body(const PfGemmArgs &A, const PfGroup &G, const V4Shared &meta, int mlen, int n0,
                                           int nt_count, uint8_t *lds, int &ev)
{
    (void)ev;
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));                 /* addressing computed per unit, not held across units */
    const int l = t & 63, h = l >> 5, w = t >> 6, n = l & 31;
    const int nkb = A.I / GK;                  /* 1 or 2 */
    _Float16 *Xb = (_Float16 *)lds;
    constexpr int TD = TL_BYTES(QD);
    constexpr int NP = MS * 32 * 32 / V2_T;   /* 16-byte pieces (8 columns) per thread per K step */
    const uint8_t *a16 = (const uint8_t *)A.act16;
    uint4 xr[NP];
    auto x_load = [&](int kb) {
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const int idx = t + i * V2_T, row = idx >> 5;
            const int slot = meta.slot[row < mlen ? row : 0];
            xr[i] = gld_u4(a16 + 2 * ((size_t)slot * A.I + kb * GK + 8 * (idx & 31)));
        }
    };
    /* each piece onto its part's scale (8 columns lie in one 16-column part),
     * stored as two 4-column groups at their permuted K positions */
    auto x_store = [&](int kb, _Float16 *dst) {
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const int idx = t + i * V2_T, row = idx >> 5, c8 = 8 * (idx & 31);
            const int sh = row < mlen ? (int)meta.psh[row][(kb * GK + c8) >> 4] : -200;
            const f16x8 hv = __builtin_bit_cast(f16x8, xr[i]);
            f32x8 e;
#pragma unroll
            for (int k = 0; k < 8; k++) e[k] = __builtin_ldexpf((float)hv[k], sh);
            const uint4 cu = __builtin_bit_cast(uint4, __builtin_convertvector(e, f16x8));
            *(uint2 *)(dst + row * V2_LD + perm_slot4(c8)) = make_uint2(cu.x, cu.y);
            *(uint2 *)(dst + row * V2_LD + perm_slot4(c8 + 4)) = make_uint2(cu.z, cu.w);
        }
    };
    auto tile_base = [&](int nt) {
        return G.td + (size_t)((n0 + nt * V2_DN_N + 32 * w) / TL_ROWS) * nkb * TD;
    };
    /* each K step's activations are fetched before its weights (a wave's
     * loads complete in order, so the staging stores wait for the
     * activations only), and the barrier orders LDS only: the weights stay in
     * flight */
    typename RawOf<QD>::T r[2];
    const uint8_t *wt = tile_base(0);
    x_load(0);
    tile_load(r[0], wt, l);
    x_store(0, Xb);
    if (nkb > 1) {
        x_load(1);
        tile_load(r[1], wt + TD, l);
        x_store(1, Xb + V3_XBUF);
    }
    lds_barrier();
    PF_TSD(ev++);
    for (int nt = 0; nt < nt_count; nt++) {
        const bool more = nt + 1 < nt_count;
        const uint8_t *wn = tile_base(more ? nt + 1 : nt);
        f32x16 acc[MS];
#pragma unroll
        for (int ms = 0; ms < MS; ms++) acc[ms] = (f32x16){};
        __builtin_amdgcn_sched_barrier(0);
        v4_mfma<MS, QD>(acc, Xb, r[0], h);
        __builtin_amdgcn_sched_barrier(0);
        if (more) tile_load(r[0], wn, l);
        if (nkb > 1) {
            __builtin_amdgcn_sched_barrier(0);
            v4_mfma<MS, QD>(acc, Xb + V3_XBUF, r[1], h);
            __builtin_amdgcn_sched_barrier(0);
            if (more) tile_load(r[1], wn + TD, l);
        }
        const int orow = n0 + nt * V2_DN_N + 32 * w + n;
        dn_store_tile<MS>(A, meta, acc, mlen, orow);
        PF_TSD(ev++);
    }
}

__device__ __forceinline__ bool v2_tile(const PfGemmArgs &A, int nblk, int &v, PfTile &tile)
{
    const int R = *A.ntiles * nblk;
    const int b = blockIdx.x;
    if (b >= R) return false;
    v = pf_virtual_block(b, R);
    tile = A.tiles[v / nblk];
    return true;
}

extern "C" __global__ void __launch_bounds__(V2_T) pf2_gu_kernel(PfGemmArgs A)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t lds4[];
    __shared__ V4Shared meta;
    const int nblk = A.I / V2_GU_J;
    int v;
    PfTile tile;
    if (!v2_tile(A, nblk, v, tile)) return;
    PF_TS(1);
#ifdef ROASTER_PF_TS
    {
        unsigned hw, xc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xc));
        PF_TSV(0, ((unsigned long long)xc << 32) | hw);
        PF_TSV(13, (unsigned long long)v);
    }
#endif
    const PfGroup &G = A.groups[tile.grp];
    const int mlen = min(A.chunk, G.n - tile.m0);
    PF_TSV(12, (unsigned long long)mlen);
    const int j0 = (v % nblk) * V2_GU_J;
    const int ms = (mlen + 31) >> 5;
    const int ty = (G.gq6 ? 2 : 0) | (G.uq6 ? 1 : 0);
    /* three row blocks come with one weight type only (pf_gemm_chunk) */
    if (ms == 3) {
        if (ty == 3) v5_gu_body<3, true, true>(A, G, meta, tile, mlen, j0, lds4);
        else if (ty == 0) v5_gu_body<3, false, false>(A, G, meta, tile, mlen, j0, lds4);
        return;
    }
#define GU_CASE(M)                                                                   \
    if (ms == M) {                                                                   \
        if (ty == 3) v5_gu_body<M, true, true>(A, G, meta, tile, mlen, j0, lds4);    \
        else if (ty == 2) v5_gu_body<M, true, false>(A, G, meta, tile, mlen, j0, lds4);\
        else if (ty == 1) v5_gu_body<M, false, true>(A, G, meta, tile, mlen, j0, lds4);\
        else v5_gu_body<M, false, false>(A, G, meta, tile, mlen, j0, lds4);          \
        return;                                                                      \
    }
    GU_CASE(1)
    GU_CASE(2)
#undef GU_CASE
}

/* ---- gate/up on a persistent grid ------------------------------------------
 * One workgroup per CU takes (tile, 128-column block) units through work
 * counters over eight ranges of the unit list (its own XCD's range first,
 * then the others'), so the units of one XCD share their tiles' activations
 * in its L2 and no CU sits idle while another still holds several units.
 * While a unit runs, the next one is prepared in the K steps' shadow: its
 * index (taken at the unit's start), tile (step 1) and group (step 2), its
 * rows' tokens (step 3, stored with the slots at step 4) and scales (step 5)
 * into the second meta buffer; the last K step issues its first step's
 * activations and weights, so those loads are in flight during this unit's
 * epilogue.  The epilogue stages its rows above the two activation buffers,
 * so the next unit's first activations are stored into buffer 0 before the
 * unit ends.
 * Each unit's arithmetic is v5_gu_body's (bit-identical results).  Every unit
 * of a launch has one weight type, and nkb is even and >= 8. */
#define GP_STAGE (2 * V3_XBUF * 2)                               /* epilogue staging (bytes into LDS) */
#define GP_LDS (GP_STAGE + V2_MC * (V2_GU_J + 8) * 2 + V2_MC * 8 * 4)

struct GuMeta {
    int tok[V2_MC];
    int slot[V2_MC];
    float fwd[V2_MC];
};

/* A unit as the workgroup sees it (wave-uniform). */
struct GuUnit {
    int u;                          /* unit index, or -1 */
    int mlen, j0, m0, slot0, tok0;
    const int *tok;
    const uint8_t *tg, *tu;
};

/* A unit's tile and group fields come in by vector loads a K step ahead of
 * their use (scalar loads would share the LDS wait counter with the MFMA
 * operand reads, flat loads both counters), one dword per lane: lane k holds
 * dword k of the record, and the fields are read out by lane.  u < 0 reads
 * unit 0's (valid addresses, unused). */
__device__ __forceinline__ uint32_t gp_tile_load(const PfGemmArgs &A, int u, int nblk)
{
    return gld_u32((const uint8_t *)(A.tiles + (u >= 0 ? u / nblk : 0)) + 4 * (threadIdx.x & 1));
}

__device__ __forceinline__ uint32_t gp_group_load(const PfGemmArgs &A, uint32_t tw)
{
    constexpr int NW = (int)(sizeof(PfGroup) / 4);
    const uint8_t *g = (const uint8_t *)(A.groups + __builtin_amdgcn_readlane((int)tw, 0));
    return gld_u32(g + 4 * min((int)(threadIdx.x & 63), NW - 1));
}

__device__ __forceinline__ int gp_field(uint32_t gw, size_t off) { return __builtin_amdgcn_readlane((int)gw, (int)(off / 4)); }

__device__ __forceinline__ const void *gp_ptr(uint32_t gw, size_t off)
{
    const uint64_t p = ((uint64_t)(uint32_t)gp_field(gw, off + 4) << 32) | (uint32_t)gp_field(gw, off);
    return (const void *)p;
}

__device__ __forceinline__ void gp_fill(const PfGemmArgs &A, uint32_t tw, uint32_t gw, int u, int nblk, GuUnit &N)
{
    N.u = u;
    N.m0 = __builtin_amdgcn_readlane((int)tw, 1);
    N.j0 = (u >= 0 ? u % nblk : 0) * V2_GU_J;
    N.mlen = min(A.chunk, gp_field(gw, offsetof(PfGroup, n)) - N.m0);
    N.slot0 = gp_field(gw, offsetof(PfGroup, slot0));
    N.tok0 = gp_field(gw, offsetof(PfGroup, tok0));
    N.tok = (const int *)gp_ptr(gw, offsetof(PfGroup, tok));
    N.tg = (const uint8_t *)gp_ptr(gw, offsetof(PfGroup, tg));
    N.tu = (const uint8_t *)gp_ptr(gw, offsetof(PfGroup, tu));
}

/* Row t's token of unit N, clamped to its last row (loads nothing
 * conditionally: the shared expert's tile reads A.ntiles and ignores it). */
__device__ __forceinline__ int gp_tok(const PfGemmArgs &A, const GuUnit &N, int t)
{
    const int r = min(t, N.mlen - 1);
    const int *tp = N.tok ? N.tok + N.m0 + r : A.ntiles;
    const int tv = (int)gld_u32(tp);
    return N.tok ? tv : N.tok0 + N.m0 + r;
}

__device__ __forceinline__ float gp_fwd(const PfGemmArgs &A, int tok)
{
    return A.xfwd ? __builtin_bit_cast(float, gld_u32(A.xfwd + tok)) : 1.0f;
}

/* Thread 0: unit index of an issued take (old value of counter x0 + xs);
 * a range that has run out moves on to the next XCD's. */
template <bool FUSED = false>
__device__ __forceinline__ int gp_resolve(const PfGemmArgs &A, int old, int &xs, int x0, int U)
{
    if constexpr (FUSED) {
        /* this XCD's tiles only: their SiLU*up rows stay in its L2 for its
         * own down chunks */
        const int nblk = A.I / V2_GU_J, lo = A.xcd_tb[x0] * nblk, hi = A.xcd_tb[x0 + 1] * nblk;
        (void)xs; (void)U;
        return lo + old < hi ? lo + old : -1;
    }
    for (;;) {
        const int x = (x0 + xs) & 7;
        const int lo = (int)((long long)x * U / 8), hi = (int)((long long)(x + 1) * U / 8);
        if (lo + old < hi) return lo + old;
        if (++xs == 8) return -1;
        old = __hip_atomic_fetch_add(A.gu_ctr + ((x0 + xs) & 7), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int MS, bool Q6, bool FUSED = false>
__device__ __forceinline__ void gp_unit(const PfGemmArgs &A, GuMeta (&meta)[2], int cur, const GuUnit &U, GuUnit &N,
                                        int *s_unit, typename RawOf<Q6>::T (&rg)[2], uint4 (&xr)[6], uint8_t *lds,
                                        int &xs, int x0, int Uall, int nblk, int sig = -1)
{
    const int t = threadIdx.x, l = t & 63, h = l >> 5, w = t >> 6, n = l & 31;
    const int nkb = A.H / GK;
    _Float16 *Xb = (_Float16 *)lds;
    const bool up = n >= 16;
    constexpr int TB = TL_BYTES(Q6), WS = TL_SLICES(Q6), NP = 2 * MS;
    const int tlane = ((16 * w + (n & 15)) & (TL_ROWS - 1)) + 32 * h;   /* j0 is a multiple of 128 */
    const int rblk = (16 * w + (n & 15)) / TL_ROWS;
    const uint8_t *wt = (up ? U.tu : U.tg) + (size_t)(U.j0 / TL_ROWS + rblk) * nkb * TB;
    GuMeta &mc = meta[cur], &mn = meta[cur ^ 1];
    const uint8_t *x16 = (const uint8_t *)A.X16;
    uint32_t xoff[NP];
#pragma unroll
    for (int i = 0; i < NP; i++) {
        const int idx = t + i * V2_T, row = idx >> 5;
        xoff[i] = 2u * ((uint32_t)mc.tok[row < U.mlen ? row : 0] * (uint32_t)A.H + 8u * (idx & 31));
    }
    auto x_load = [&](int kb) {
#pragma unroll
        for (int i = 0; i < NP; i++) xr[i] = gld_u4(x16 + xoff[i] + 2 * kb * GK);
    };
    auto x_store = [&](_Float16 *dst) {
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const int idx = t + i * V2_T, row = idx >> 5;
            *(uint4 *)(dst + row * V2_LD + 8 * (idx & 31)) = xr[i];
        }
    };
    PF_TSU(U.u, 1);
#ifdef ROASTER_PF_TS
    {
        unsigned hw, xc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xc));
        PF_TSUV(U.u, 0, ((unsigned long long)xc << 32) | hw);
        PF_TSUV(U.u, 12, (unsigned long long)U.mlen);
        PF_TSUV(U.u, 13, (unsigned long long)blockIdx.x);
    }
#endif
    int tk = 0;
    if (t == 0) tk = __hip_atomic_fetch_add(A.gu_ctr + ((x0 + xs) & 7), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    f32x16 acc[MS];
#pragma unroll
    for (int ms = 0; ms < MS; ms++) acc[ms] = (f32x16){};
    /* step kb on raw and activation buffer buf, loading step kb + 1 into
     * buffer buf ^ 1 */
    auto step = [&](auto bc, int kb) {
        constexpr int buf = decltype(bc)::value;
        const uint8_t *wn = wt + (size_t)(kb + 1) * TB;
        __builtin_amdgcn_sched_barrier(0);
        v8_mfma<MS, Q6>(acc, Xb + buf * V3_XBUF, rg[buf], h, [&](int j) {
            if (j == 0) x_load(kb + 1);
            if (j < WS) tile_slice(rg[buf ^ 1], wn, tlane, j);
        });
        __builtin_amdgcn_sched_barrier(0);
        x_store(Xb + (buf ^ 1) * V3_XBUF);
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    step(B0(), 0);
    if (t == 0) s_unit[cur ^ 1] = gp_resolve<FUSED>(A, tk, xs, x0, Uall);
    lds_barrier();
    if constexpr (FUSED) {
        /* the previous unit's rows are stored: every thread has waited for
         * step 0's activation loads, issued after them (a wave's memory
         * operations complete in order), before the barrier */
        if (t == 0 && sig >= 0) __hip_atomic_fetch_add(A.tile_done + sig, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    PF_TSU(U.u, 2);
    const int nu = __builtin_amdgcn_readfirstlane(s_unit[cur ^ 1]);
    const uint32_t ntl = gp_tile_load(A, nu, nblk); /* step 1: the next unit's tile */
    step(B1(), 1);
    lds_barrier();
    PF_TSU(U.u, 3);
    const uint32_t ngr = gp_group_load(A, ntl);    /* step 2: its group */
    step(B0(), 2);
    lds_barrier();
    PF_TSU(U.u, 4);
    gp_fill(A, ntl, ngr, nu, nblk, N);
    const int ntok = gp_tok(A, N, t);              /* step 3: its rows' tokens */
    step(B1(), 3);
    lds_barrier();
    PF_TSU(U.u, 5);
    if (t < V2_MC) {                                /* step 4: stored, their scales loaded */
        mn.tok[t] = ntok;
        mn.slot[t] = N.slot0 + N.m0 + t;
    }
    const float nfwd = gp_fwd(A, ntok);
    step(B0(), 4);
    lds_barrier();
    PF_TSU(U.u, 6);
    if (t < V2_MC) mn.fwd[t] = nfwd;                /* step 5 */
    step(B1(), 5);
    lds_barrier();
    PF_TSU(U.u, 7);
    int kb = 6;
    for (; kb + 2 <= nkb - 2; kb += 2) {
        step(B0(), kb);
        lds_barrier();
        step(B1(), kb + 1);
        lds_barrier();
    }
    step(B0(), kb);                           /* kb = nkb - 2 */
    lds_barrier();
    PF_TSU(U.u, 8);
    /* the last step (raw and activation buffer 1), with the next unit's
     * first activations (all 96 rows; rows >= mlen read row 0) and step 0
     * weights into buffer 0 */
    {
        uint32_t nxo[6];
#pragma unroll
        for (int i = 0; i < 6; i++) {
            const int idx = t + i * V2_T, row = idx >> 5;
            nxo[i] = 2u * ((uint32_t)mn.tok[row < N.mlen ? row : 0] * (uint32_t)A.H + 8u * (idx & 31));
        }
        const uint8_t *nwt = (up ? N.tu : N.tg) + (size_t)(N.j0 / TL_ROWS + rblk) * nkb * TB;
        __builtin_amdgcn_sched_barrier(0);
        v8_mfma<MS, Q6>(acc, Xb + V3_XBUF, rg[1], h, [&](int j) {
            if (j == 0) {
#pragma unroll
                for (int i = 0; i < 6; i++) xr[i] = gld_u4(x16 + nxo[i]);
            }
            if (j < WS) tile_slice(rg[0], nwt, tlane, j);
        });
        __builtin_amdgcn_sched_barrier(0);
    }
    PF_TSU(U.u, 9);
    gu_epilogue<MS, GuMeta, true>(A, mc, acc, U.mlen, U.j0, lds + GP_STAGE);
    PF_TSU(U.u, 10);
#pragma unroll
    for (int i = 0; i < 6; i++) {                   /* the next unit's step 0 activations */
        const int idx = t + i * V2_T, row = idx >> 5;
        *(uint4 *)(Xb + row * V2_LD + 8 * (idx & 31)) = xr[i];
    }
    lds_barrier();
    PF_TSU(U.u, 11);
}

template <bool Q6, bool FUSED = false>
__device__ __forceinline__ void gp_body(const PfGemmArgs &A, uint8_t *lds, GuMeta (&meta)[2], int *s_unit)
{
    const int t = threadIdx.x, l = t & 63, h = l >> 5, w = t >> 6, n = l & 31;
    const int nkb = A.H / GK, nblk = A.I / V2_GU_J;
    const int Uall = *A.ntiles * nblk;
    const bool up = n >= 16;
    constexpr int TB = TL_BYTES(Q6);
    unsigned xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    const int x0 = (int)(xcc & 7);
    int xs = 0;
    if (t == 0) {
        const int old = __hip_atomic_fetch_add(A.gu_ctr + x0, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_unit[0] = gp_resolve<FUSED>(A, old, xs, x0, Uall);
    }
    __syncthreads();
    GuUnit U;
    {
        const int u0 = __builtin_amdgcn_readfirstlane(s_unit[0]);
        if (u0 < 0) return;                         /* workgroup-uniform */
        const uint32_t tl = gp_tile_load(A, u0, nblk);
        gp_fill(A, tl, gp_group_load(A, tl), u0, nblk, U);
    }
    /* the first unit's meta, step 0 weights and step 0 activations */
    typename RawOf<Q6>::T rg[2];
    uint4 xr[6];
    {
        const int tv = gp_tok(A, U, t);
        if (t < V2_MC) {
            meta[0].tok[t] = tv;
            meta[0].slot[t] = U.slot0 + U.m0 + t;
            meta[0].fwd[t] = gp_fwd(A, tv);
        }
        const int tlane = ((16 * w + (n & 15)) & (TL_ROWS - 1)) + 32 * h;
        const uint8_t *wt = (up ? U.tu : U.tg) + (size_t)(U.j0 / TL_ROWS + (16 * w + (n & 15)) / TL_ROWS) * nkb * TB;
        tile_load(rg[0], wt, tlane);
        __syncthreads();
        const uint8_t *x16 = (const uint8_t *)A.X16;
#pragma unroll
        for (int i = 0; i < 6; i++) {
            const int idx = t + i * V2_T, row = idx >> 5;
            xr[i] = gld_u4(x16 + 2u * ((uint32_t)meta[0].tok[row < U.mlen ? row : 0] * (uint32_t)A.H + 8u * (idx & 31)));
        }
        _Float16 *Xb = (_Float16 *)lds;
#pragma unroll
        for (int i = 0; i < 6; i++) {
            const int idx = t + i * V2_T, row = idx >> 5;
            *(uint4 *)(Xb + row * V2_LD + 8 * (idx & 31)) = xr[i];
        }
        lds_barrier();
    }
    int cur = 0, sig = -1;
    for (;;) {
        GuUnit N;
        const int ms = (U.mlen + 31) >> 5;
        if (ms == 1) gp_unit<1, Q6, FUSED>(A, meta, cur, U, N, s_unit, rg, xr, lds, xs, x0, Uall, nblk, sig);
        else if (ms == 2) gp_unit<2, Q6, FUSED>(A, meta, cur, U, N, s_unit, rg, xr, lds, xs, x0, Uall, nblk, sig);
        else gp_unit<3, Q6, FUSED>(A, meta, cur, U, N, s_unit, rg, xr, lds, xs, x0, Uall, nblk, sig);
        sig = U.u / nblk;
        if (N.u < 0) break;                         /* workgroup-uniform */
        U = N;
        cur ^= 1;
    }
    if constexpr (FUSED) {
        /* the last unit's rows: its stores complete, then counted */
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        lds_barrier();
        if (t == 0) __hip_atomic_fetch_add(A.tile_done + sig, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

extern "C" __global__ void __launch_bounds__(V2_T) pf2_gu_pers_kernel(PfGemmArgs A)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t lds4[];
    __shared__ GuMeta meta[2];
    __shared__ int s_unit[2];
    if (A.gu_pers == 2) gp_body<true>(A, lds4, meta, s_unit);
    else gp_body<false>(A, lds4, meta, s_unit);
}

/* Per-row meta of the down GEMM for tile rows [0, mlen): slot, the row's
 * power-of-two scale (from its part maxima) and each part's shift onto it.
 * With fp16 products (A.out16) the row's products are also scaled by 2^-e,
 * e the exponent row_scale gives their bound max|act| * G.dbnd (no product
 * of the row exceeds it, so the scaled products stay below 2^15), and fwd
 * folds both scales; e goes to A.oexp[slot] (first: the workgroup writing
 * the row's first output columns). */
__device__ __forceinline__ void dn_meta(const PfGemmArgs &A, const PfGroup &G, const PfTile &tile, int mlen,
                                        V4Shared &meta, bool first)
{
    const int t = threadIdx.x;
    if (t < mlen) {
        const int slot = G.slot0 + tile.m0 + t;
        const int nb = A.I / 16;
        const float *pr = A.pmax + (size_t)slot * nb;
        float mx = 0.0f;
        float4 v[8];
        if (nb <= 32) {
            /* the row's part maxima in one batch of 16-byte loads (a row is
             * 16-byte aligned: nb is a multiple of 16) */
#pragma unroll
            for (int q = 0; q < 8; q++) v[q] = 4 * q < nb ? gld_f4(pr + 4 * q) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int q = 0; q < 8; q++) mx = fmaxf(fmaxf(fmaxf(mx, v[q].x), fmaxf(v[q].y, v[q].z)), v[q].w);
        } else {
            for (int b = 0; b < nb; b++) mx = fmaxf(mx, pr[b]);
        }
        float inv, fwd;
        row_scale(mx, inv, fwd);
        meta.slot[t] = slot;
        meta.inv[t] = inv;
        meta.fwd[t] = fwd;
        if (A.out16) {
            const int sp = pf_scale_exp(mx * G.dbnd), sf = pf_scale_exp(mx) - sp;
            meta.fwd[t] = __builtin_bit_cast(float, (uint32_t)(127 + max(-126, min(126, sf))) << 23);
            if (first) A.oexp[slot] = (int8_t)sp;
        }
        /* shift of part b: exponent of its scale minus the row's (fp16 mode);
         * 2^-64 is 0 in fp16 */
        const int er = pf_scale_exp(mx);
        auto sh = [&](float pmx) { return (uint32_t)(uint8_t)(int8_t)max(pf_scale_exp(pmx) - er, -64); };
        if (nb <= 32) {
#pragma unroll
            for (int q = 0; q < 8; q++)
                if (4 * q < nb)
                    *(uint32_t *)&meta.psh[t][4 * q] = sh(v[q].x) | sh(v[q].y) << 8 | sh(v[q].z) << 16 | sh(v[q].w) << 24;
        } else {
            for (int b = 0; b < nb && b < V5_MAXPART; b++) meta.psh[t][b] = (int8_t)sh(pr[b]);
        }
    }
}

/* Tile ti's down record spread over the wave: lane k holds its dword k (k < 8). */
__device__ __forceinline__ uint32_t dn_rec_load(const PfGemmArgs &A, int ti)
{
    return gld_u32((const uint32_t *)(A.dn_tiles + ti) + (threadIdx.x & 7));
}

/* One tile range of the balanced down GEMM (inter <= 512): dn_meta's row
 * meta, the activation staging and the output tiles of v6_dn_body, with the
 * range's loads issued as one batch in the order their data is needed — the
 * rows' part maxima, both K steps' activations, then the first output tile's
 * weights — so that the maxima and the activations (L2) return without
 * waiting behind the weights (HBM): a wave's loads complete in order.  The
 * part maxima are spread over the workgroup, four parts (one 16-byte load)
 * per thread and up to two pieces each: piece p holds parts 4 (p % ppr) ..
 * + 3 of row p / ppr, ppr = inter / 64, and the row maximum is taken over the
 * row's ppr neighbouring lanes by DPP (fmaxf, so the order does not change
 * it).  An activation row's slot is the tile's first slot plus the row. */
template <int MS, bool QD, int NKB>
__device__ __forceinline__ void v7_dn_range(const PfGemmArgs &A, const uint8_t *td, int sbase, int mlen, float dbnd,
                                            V4Shared &meta, int n0, int nt_count, bool first, int nti, uint32_t &rec,
                                            uint8_t *lds, int &ev)
{
    (void)ev;
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));                 /* addressing computed per range, not held across ranges */
    const int l = t & 63, h = l >> 5, w = t >> 6, n = l & 31;
    constexpr int nkb = NKB;                   /* K steps: inter / 256, 1 or 2 */
    constexpr int nb = 16 * NKB, lp = NKB == 2 ? 3 : 2, ppr = 1 << lp;
    _Float16 *Xb = (_Float16 *)lds;
    constexpr int TD = TL_BYTES(QD);
    constexpr int NP = MS * 32 * 32 / V2_T;   /* 16-byte pieces (8 columns) per thread per K step */
    const uint8_t *a16 = (const uint8_t *)A.act16;
    float4 pm[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int p = t + V2_T * i, row = p >> lp;
        pm[i] = gld_f4(A.pmax + (size_t)(sbase + (row < mlen ? row : 0)) * nb + 4 * (p & (ppr - 1)));
    }
    uint4 xr[2][NP];
    auto x_load = [&](int kb, uint4 (&dst)[NP]) {
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const int idx = t + i * V2_T, row = idx >> 5;
            dst[i] = gld_u4(a16 + 2 * ((size_t)(sbase + (row < mlen ? row : 0)) * A.I + kb * GK + 8 * (idx & 31)));
        }
    };
    auto x_store = [&](int kb, const uint4 (&src)[NP], _Float16 *dst) {
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const int idx = t + i * V2_T, row = idx >> 5, c8 = 8 * (idx & 31);
            const int sh = row < mlen ? (int)meta.psh[row][(kb * GK + c8) >> 4] : -200;
            const f16x8 hv = __builtin_bit_cast(f16x8, src[i]);
            f32x8 e;
#pragma unroll
            for (int k = 0; k < 8; k++) e[k] = __builtin_ldexpf((float)hv[k], sh);
            const uint4 cu = __builtin_bit_cast(uint4, __builtin_convertvector(e, f16x8));
            *(uint2 *)(dst + row * V2_LD + perm_slot4(c8)) = make_uint2(cu.x, cu.y);
            *(uint2 *)(dst + row * V2_LD + perm_slot4(c8 + 4)) = make_uint2(cu.z, cu.w);
        }
    };
    auto tile_base = [&](int nt) {
        return td + (size_t)((n0 + nt * V2_DN_N + 32 * w) / TL_ROWS) * nkb * TD;
    };
    x_load(0, xr[0]);
    if constexpr (NKB > 1) x_load(1, xr[1]);
    typename RawOf<QD>::T r[2];
    const uint8_t *wt = tile_base(0);
    tile_load(r[0], wt, l);
    if constexpr (NKB > 1) tile_load(r[1], wt + TD, l);
    rec = dn_rec_load(A, nti);                  /* the next range's record, read at its start */
    /* the rows' meta (dn_meta's values) */
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int p = t + V2_T * i, row = p >> lp, q = p & (ppr - 1);
        const float4 v = pm[i];
        float mx = fmaxf(fmaxf(fmaxf(0.0f, v.x), fmaxf(v.y, v.z)), v.w);
        mx = fmaxf(mx, dpp_f<DPP_XOR1>(mx));
        mx = fmaxf(mx, dpp_f<DPP_XOR2>(mx));
        if constexpr (ppr == 8) mx = fmaxf(mx, dpp_f<DPP_HALF_MIRROR>(mx));
        if (row < mlen) {
            const int er = pf_scale_exp(mx);
            auto sh = [&](float pmx) { return (uint32_t)(uint8_t)(int8_t)max(pf_scale_exp(pmx) - er, -64); };
            *(uint32_t *)&meta.psh[row][4 * q] = sh(v.x) | sh(v.y) << 8 | sh(v.z) << 16 | sh(v.w) << 24;
            if (q == 0) {
                const int slot = sbase + row;
                float inv, fwd;
                row_scale(mx, inv, fwd);
                meta.slot[row] = slot;
                meta.inv[row] = inv;
                meta.fwd[row] = fwd;
                if (A.out16) {
                    const int sp = pf_scale_exp(mx * dbnd), sf = er - sp;
                    meta.fwd[row] = __builtin_bit_cast(float, (uint32_t)(127 + max(-126, min(126, sf))) << 23);
                    if (first) A.oexp[slot] = (int8_t)sp;
                }
            }
        } else if (row < MS * 32 && q == 0) {
            meta.slot[row] = A.dn_spare;
            meta.fwd[row] = 0.0f;
        }
    }
    lds_barrier();                              /* the meta, for the staging and the stores */
    PF_TSD(ev++);
    x_store(0, xr[0], Xb);
    if constexpr (NKB > 1) x_store(1, xr[1], Xb + V3_XBUF);
    lds_barrier();                              /* the weights stay in flight */
    PF_TSD(ev++);
    /* the next output tile's weights are loaded unconditionally (the last
     * tile reloads its own, from L2) and every row is stored (rows past the
     * tile's end to the spare slot): with a fixed set of loads and stores per
     * tile the compiler's waits count exactly, and each K step waits for its
     * own weights only, not for the next step's or the last tile's stores */
    for (int nt = 0; nt < nt_count; nt++) {
        const uint8_t *wn = tile_base(nt + 1 < nt_count ? nt + 1 : nt);
        f32x16 acc[MS];
#pragma unroll
        for (int ms = 0; ms < MS; ms++) acc[ms] = (f32x16){};
        __builtin_amdgcn_sched_barrier(0);
        v4_mfma<MS, QD>(acc, Xb, r[0], h);
        __builtin_amdgcn_sched_barrier(0);
        tile_load(r[0], wn, l);
        if constexpr (NKB > 1) {
            __builtin_amdgcn_sched_barrier(0);
            v4_mfma<MS, QD>(acc, Xb + V3_XBUF, r[1], h);
            __builtin_amdgcn_sched_barrier(0);
            tile_load(r[1], wn + TD, l);
        }
        const int orow = n0 + nt * V2_DN_N + 32 * w + n;
        dn_store_tile<MS, true>(A, meta, acc, mlen, orow);
        PF_TSD(ev++);
    }
}

extern "C" __global__ void __launch_bounds__(V2_T) pf2_down_kernel(PfGemmArgs A)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t lds4[];
    __shared__ V4Shared meta;
    const int nt_count = A.dn_nt;              /* output tiles per workgroup */
    const int nblk = A.H / V2_DN_N / nt_count;
    int v;
    PfTile tile;
    if (!v2_tile(A, nblk, v, tile)) return;
    const PfGroup &G = A.groups[tile.grp];
    const int mlen = min(A.chunk, G.n - tile.m0);
    const int n0 = (v % nblk) * nt_count * V2_DN_N;
    dn_meta(A, G, tile, mlen, meta, n0 == 0);
    __syncthreads();
    const int ms = (mlen + 31) >> 5;
    const bool whole_k = A.I <= 2 * GK;        /* activations for every K step fit in LDS */
    int ev = 0;                                /* timestamp build: event index of this workgroup */
#define DN_CASE(M)                                                                   \
    if (ms == M) {                                                                   \
        if (whole_k) {                                                               \
            if (G.dq6) v6_dn_body<M, true>(A, G, meta, mlen, n0, nt_count, lds4, ev); \
            else v6_dn_body<M, false>(A, G, meta, mlen, n0, nt_count, lds4, ev);    \
        } else {                                                                     \
            if (G.dq6) v5_dn_body<M, true>(A, G, meta, mlen, n0, lds4);             \
            else v5_dn_body<M, false>(A, G, meta, mlen, n0, lds4);                  \
        }                                                                            \
        return;                                                                      \
    }
    DN_CASE(1)
    DN_CASE(2)
    DN_CASE(3)
#undef DN_CASE
}

/* The down GEMM for inter <= 512 on a fixed grid (one workgroup per CU): the
 * (tile, 256-row output tile) units, tile-major, are split into gridDim.x
 * contiguous ranges of about equal cost (the plan kernel's bounds, from a
 * cost per unit that grows with the tile's 32-row blocks plus one per tile
 * range started), so no last wave of workgroups runs on a few CUs while the
 * rest idle.  A range crosses at most a few tiles; each piece is one
 * v7_dn_range (meta and activations staged once, the next output tile's
 * weights loaded during the current one's MFMA work), its tile record loaded
 * during the piece before.  Workgroups of one XCD (grid dealt round-robin
 * over the 8 XCDs) take neighbouring ranges, so the activation rows of a
 * tile are fetched into one L2. */
extern "C" __global__ void __launch_bounds__(V2_T) pf2_down_bal_kernel(PfGemmArgs A)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t lds4[];
    __shared__ V4Shared meta;
    const int NT = A.H / V2_DN_N, Gd = (int)gridDim.x, b = blockIdx.x;
    const int vb = (Gd & 7) ? b : (b & 7) * (Gd >> 3) + (b >> 3);
    int u, u1;
    if (A.dn_bnd) {
        u = A.dn_bnd[vb];
        u1 = A.dn_bnd[vb + 1];
    } else {
        const int U = *A.ntiles * NT;
        u = (int)((long long)vb * U / Gd);
        u1 = (int)((long long)(vb + 1) * U / Gd);
    }
    int ev = 0;
    PF_TSD(ev++);
    /* each range's record is loaded during the range before it (the first
     * here), so a range starts with its loads, not a chain of lookups */
    uint32_t rec = dn_rec_load(A, u < u1 ? u / NT : 0);
    while (u < u1) {
        const int ti = u / NT, t0 = u % NT, cnt = min(NT - t0, u1 - u);
        const int nti = u + cnt < u1 ? (u + cnt) / NT : ti;
        auto field = [&](size_t off) { return __builtin_amdgcn_readlane((int)rec, (int)(off / 4)); };
        const uint8_t *td = (const uint8_t *)(((uint64_t)(uint32_t)field(offsetof(PfDnTile, td) + 4) << 32) |
                                              (uint32_t)field(offsetof(PfDnTile, td)));
        const int sbase = field(offsetof(PfDnTile, slot)), mlen = field(offsetof(PfDnTile, mlen));
        const bool dq6 = field(offsetof(PfDnTile, dq6)) != 0;
        const float dbnd = __builtin_bit_cast(float, field(offsetof(PfDnTile, dbnd)));
        const int ms = (mlen + 31) >> 5, n0 = t0 * V2_DN_N;
        const bool first = t0 == 0;
#define DN_RANGE(M, Q)                                                                          \
    do {                                                                                        \
        if (A.I > GK) v7_dn_range<M, Q, 2>(A, td, sbase, mlen, dbnd, meta, n0, cnt, first, nti, rec, lds4, ev); \
        else v7_dn_range<M, Q, 1>(A, td, sbase, mlen, dbnd, meta, n0, cnt, first, nti, rec, lds4, ev);          \
    } while (0)
        if (ms == 1) {
            if (dq6) DN_RANGE(1, true);
            else DN_RANGE(1, false);
        } else if (ms == 2) {
            if (dq6) DN_RANGE(2, true);
            else DN_RANGE(2, false);
        } else {
            if (dq6) DN_RANGE(3, true);
            else DN_RANGE(3, false);
        }
#undef DN_RANGE
        u += cnt;
        lds_barrier();                          /* meta and the staged activations are rewritten next */
    }
}

/* The fused kernel's down phase: chunks of PF_FX_CH output tiles of this
 * XCD's tiles, taken in tile order from the XCD's counter (whole tiles as
 * the first three quarters' chunks, or chunks of 2 or 3, measured slower:
 * coarser ends, or more activation stagings).  A chunk starts
 * once its tile's gate/up units are all counted (thread 0 polls the counter,
 * at most PF_FX_SPIN times, then reports bit 8 and goes on); the next chunk
 * is claimed while the current one runs.  The SiLU*up rows it reads were
 * written by workgroups of the same XCD, so they are in its L2 (and in no
 * CU's L1: nothing reads them before this). */
#define PF_FX_CH 4
#define PF_FX_SPIN (1 << 22)
__device__ __forceinline__ void dn_fused(const PfGemmArgs &A, uint8_t *lds, V4Shared &meta, int *s_unit)
{
    const int t = threadIdx.x;
    unsigned xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    const int x0 = (int)(xcc & 7);
    const int NT = A.H / V2_DN_N, cps = (NT + PF_FX_CH - 1) / PF_FX_CH, nblk = A.I / V2_GU_J;
    const int tb0 = A.xcd_tb[x0], ntx = A.xcd_tb[x0 + 1] - tb0;
    const int nch = ntx * cps;
    int ev = 0;
    uint32_t rec = 0;
    if (t == 0) s_unit[0] = __hip_atomic_fetch_add(A.dn_ctr + x0, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    lds_barrier();
    for (;;) {
        const int c = __builtin_amdgcn_readfirstlane(s_unit[0]);
        if (c >= nch) break;                        /* workgroup-uniform */
        const int ti = tb0 + c / cps, j0 = (c % cps) * PF_FX_CH, cnt = min(PF_FX_CH, NT - j0);
        rec = dn_rec_load(A, ti);
        int nextc = 0;
        if (t == 0) {
            nextc = __hip_atomic_fetch_add(A.dn_ctr + x0, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            int it = 0;
            while (__hip_atomic_load(A.tile_done + ti, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < nblk) {
                if (++it == PF_FX_SPIN) {
                    __hip_atomic_fetch_or(A.err, 8, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
        }
        lds_barrier();                              /* LDS only: the last chunk's stores stay in flight */
        auto field = [&](size_t off) { return __builtin_amdgcn_readlane((int)rec, (int)(off / 4)); };
        const uint8_t *td = (const uint8_t *)(((uint64_t)(uint32_t)field(offsetof(PfDnTile, td) + 4) << 32) |
                                              (uint32_t)field(offsetof(PfDnTile, td)));
        const int sbase = field(offsetof(PfDnTile, slot)), mlen = field(offsetof(PfDnTile, mlen));
        const bool dq6 = field(offsetof(PfDnTile, dq6)) != 0;
        const float dbnd = __builtin_bit_cast(float, field(offsetof(PfDnTile, dbnd)));
        const int ms = (mlen + 31) >> 5, n0 = j0 * V2_DN_N;
        const bool first = j0 == 0;
#define DN_RANGE(M, Q)                                                                          \
    do {                                                                                        \
        if (A.I > GK) v7_dn_range<M, Q, 2>(A, td, sbase, mlen, dbnd, meta, n0, cnt, first, ti, rec, lds, ev); \
        else v7_dn_range<M, Q, 1>(A, td, sbase, mlen, dbnd, meta, n0, cnt, first, ti, rec, lds, ev);          \
    } while (0)
        if (ms == 1) {
            if (dq6) DN_RANGE(1, true);
            else DN_RANGE(1, false);
        } else if (ms == 2) {
            if (dq6) DN_RANGE(2, true);
            else DN_RANGE(2, false);
        } else {
            if (dq6) DN_RANGE(3, true);
            else DN_RANGE(3, false);
        }
#undef DN_RANGE
        if (t == 0) s_unit[0] = nextc;
        lds_barrier();                              /* meta, the staged activations and the claim */
    }
}

/* Both fp16 GEMMs in one persistent grid (one workgroup per CU): each XCD's
 * workgroups take its tiles' gate/up units, then its tiles' down chunks, so
 * the CUs that run out of gate/up units work on down chunks while the last
 * units finish, and the down GEMM's start overlaps the gate/up tail. */
extern "C" __global__ void __launch_bounds__(V2_T) pf2_fused_kernel(PfGemmArgs A)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t lds4[];
    __shared__ GuMeta meta[2];
    __shared__ int s_unit[2];
    __shared__ V4Shared dmeta;
    if (A.gu_pers == 2) gp_body<true, true>(A, lds4, meta, s_unit);
    else gp_body<false, true>(A, lds4, meta, s_unit);
    __syncthreads();
    dn_fused(A, lds4, dmeta, s_unit);
}

/* ---- host ----------------------------------------------------------------- */
static int g_pf_dn_bal = 1;             /* roaster_prefill_balanced_down */
static int g_pf_gu_pers = 1;            /* roaster_prefill_persistent_gate_up */
static int g_pf_fused = 0;              /* roaster_prefill_fused_gemm */

bool pf_fused_enabled() { return g_pf_fused && g_pf_gu_pers && g_pf_dn_bal; }

extern "C" int roaster_prefill_fused_gemm(int enable)
{
    std::lock_guard<std::recursive_mutex> g(rt_lock());
    if (enable == 0 || enable == 1) g_pf_fused = enable;
    return g_pf_fused;
}

extern "C" int roaster_prefill_balanced_down(int enable)
{
    std::lock_guard<std::recursive_mutex> g(rt_lock());
    if (enable == 0 || enable == 1) g_pf_dn_bal = enable;
    return g_pf_dn_bal;
}

extern "C" int roaster_prefill_persistent_gate_up(int enable)
{
    std::lock_guard<std::recursive_mutex> g(rt_lock());
    if (enable == 0 || enable == 1) g_pf_gu_pers = enable;
    return g_pf_gu_pers;
}

template <int OP>
static int launch_v1(const PfGemmArgs &A, int max_tiles)
{
    RtState &R = rt();
    const size_t lds = gemm_lds_bytes(OP);
    const int gu_blocks = max_tiles * (A.I / 32), d_blocks = max_tiles * (A.H / GN);
    hipLaunchKernelGGL(pf_gu_kernel<OP>, dim3(gu_blocks), dim3(GT), lds, R.stream, A);
    if (rt_check(hipGetLastError(), "prefill gate/up launch")) return ROASTER_EDEVICE;
    hipLaunchKernelGGL(pf_down_kernel<OP>, dim3(d_blocks), dim3(GT), lds, R.stream, A);
    return rt_check(hipGetLastError(), "prefill down launch") ? ROASTER_EDEVICE : 0;
}

int pf_matmul_launch(const PfGemmArgs &A, int max_tiles)
{
    if (max_tiles <= 0) return 0;
    const size_t lds = gemm_lds_bytes(PF_SPLIT);
    hipLaunchKernelGGL(pf_down_kernel<PF_SPLIT>, dim3(max_tiles * (A.H / GN)), dim3(GT), lds, rt().stream, A);
    return rt_check(hipGetLastError(), "matmul launch") ? ROASTER_EDEVICE : 0;
}

/* fp16 mode: up to three 32-row blocks; two when gate and up differ in type
 * (a wave then holds both raw record types, which for three blocks exceeds
 * the register budget of two waves per SIMD). */
int pf_gemm_chunk(int op, bool mixed_gate_up) { return op == PF_F16 ? (mixed_gate_up ? 64 : V2_MC) : GM; }

int pf_gemm_launch(const PfGemmArgs &A, int max_tiles, int op)
{
    if (max_tiles <= 0) return 0;
    if (op == PF_SPLIT) return launch_v1<PF_SPLIT>(A, max_tiles);
    if (op == PF_BF16) return launch_v1<PF_BF16>(A, max_tiles);
    RtState &R = rt();
    const size_t lds_gu = 2 * (size_t)V3_XBUF * 2, lds_dn = lds_gu;
    if (A.fused && A.gu_pers && A.dn_tiles && A.out16 && A.xcd_tb) {
        /* the plan kernel set up the fused kernel's split and counters */
        hipLaunchKernelGGL(pf2_fused_kernel, dim3(R.n_cu), dim3(V2_T), (size_t)GP_LDS, R.stream, A);
        return rt_check(hipGetLastError(), "prefill fused GEMM launch") ? ROASTER_EDEVICE : 0;
    }
    if (A.gu_pers && g_pf_gu_pers)
        hipLaunchKernelGGL(pf2_gu_pers_kernel, dim3(R.n_cu), dim3(V2_T), (size_t)GP_LDS, R.stream, A);
    else
        hipLaunchKernelGGL(pf2_gu_kernel, dim3(max_tiles * (A.I / V2_GU_J)), dim3(V2_T), lds_gu, R.stream, A);
    if (rt_check(hipGetLastError(), "prefill gate/up launch")) return ROASTER_EDEVICE;
    PfGemmArgs D = A;
    if (A.I <= 2 * GK && g_pf_dn_bal && A.dn_bnd && A.dn_tiles && A.out16) {
        /* every K step's activations fit in LDS: one workgroup per CU over an
         * even split of the output tiles */
        D.dn_nt = 0;
        hipLaunchKernelGGL(pf2_down_bal_kernel, dim3(R.n_cu), dim3(V2_T), lds_dn, R.stream, D);
        return rt_check(hipGetLastError(), "prefill down launch") ? ROASTER_EDEVICE : 0;
    }
    /* several output tiles per workgroup when every K step's activations fit in
     * LDS and the tile count divides evenly, else one */
    D.dn_nt = A.I <= 2 * GK && (A.H / V2_DN_N) % PF_DN_NT == 0 ? PF_DN_NT : 1;
    hipLaunchKernelGGL(pf2_down_kernel, dim3(max_tiles * (A.H / V2_DN_N / D.dn_nt)), dim3(V2_T), lds_dn, R.stream, D);
    return rt_check(hipGetLastError(), "prefill down launch") ? ROASTER_EDEVICE : 0;
}
