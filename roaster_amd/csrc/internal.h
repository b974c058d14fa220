/*
 * internal.h -- host-side internals shared by the translation units of
 * libroaster_moe.so (runtime, expert table, decode, prefill, kernels.h API).
 */
#ifndef ROASTER_INTERNAL_H
#define ROASTER_INTERNAL_H

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include <mutex>

#include "../../include/kernels.h"
#include "../../include/roaster_moe.h"

#define RQK 256
#define RQ4K_BYTES 144
#define RQ6K_BYTES 210
#define RTOPK 8
#define RMAX_B 8                 /* decode tokens per call */
/* Every device allocation that kernels read weights or activations from carries
 * this many spare bytes: the prefill GEMM loads whole 16-byte-aligned windows
 * around each 210-byte Q6_K block, which can reach up to 14 bytes past a
 * matrix's last block (80 past a Q4_K block). */
#define RT_TAIL_PAD 256

static inline size_t rq_block_bytes(int q6) { return q6 ? RQ6K_BYTES : RQ4K_BYTES; }
static inline size_t rq_row_bytes(int q6, size_t cols) { return cols / RQK * rq_block_bytes(q6); }
static inline size_t rq_mat_bytes(int q6, size_t rows, size_t cols) { return rows * rq_row_bytes(q6, cols); }

/* ---- runtime (runtime.hip) ---- */
struct RtState {
    int inited;
    int device;
    int n_cu;
    int n_xcd;
    size_t hbm_bytes;
    hipStream_t stream;
};
RtState &rt();
std::recursive_mutex &rt_lock();          /* serialises every public entry point */
int  rt_init_locked();                      /* 0 ok, else ROASTER_EDEVICE */
int  rt_fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int  rt_check(hipError_t e, const char *what);  /* 0 or ROASTER_EDEVICE with message */
/* Grow-only device scratch slots (kept until trim/shutdown). */
enum { SCR_IN = 0, SCR_OUT, SCR_A, SCR_B, SCR_C, SCR_D, SCR_E, SCR_F, SCR_CTRL, SCR_PF, SCR_MM, SCR_N };
void *rt_scratch(int slot, size_t bytes);
void  rt_scratch_trim();
/* Pinned host staging (grow-only). */
void *rt_pinned(int slot, size_t bytes);

/* Weight pointer translation: host address of `bytes` weight bytes -> device
 * address holding the same bytes (uploads on first use).  Device addresses are
 * returned unchanged.  NULL on failure (message set). */
const void *rt_weight_dev(const void *ptr, size_t bytes);
/* Same for f32 weight matrices used by kernel_matvec_f32. */
void rt_registry_clear();
void rt_register_device_range(const void *dev, size_t bytes);   /* table allocations */
void rt_unregister_device_range(const void *dev);

/* Write tracking of host memory (wtrack.hip). */
#include <utility>
#include <vector>
size_t wt_page_size();
int wt_available();                                   /* 1 if writes can be tracked here */
int wt_register(uintptr_t start, size_t n);           /* 0: pages of the range now tracked */
void wt_unregister(uintptr_t start, size_t n);        /* its pages no longer tracked */
void wt_unregister_all();
/* Written page runs of the pages overlapping [start, start+n), re-protected
 * in the same walk; 0 ok, -1 if the range cannot be scanned. */
int wt_scan(uintptr_t start, size_t n, std::vector<std::pair<uintptr_t, uintptr_t>> &runs);

unsigned *rt_ctrl();        /* persistent-kernel control words (device) */
int rt_take_err();           /* sync the stream, report and clear kernel error bits */
void rt_set_aux_err(int *dev_word);   /* a second device error word rt_take_err reports and clears */
void rt_aux_err_used();      /* a launch that may set it was queued */
int noalloc_setup(int dev);  /* api.hip: device address of the allocation-free scratch array */

void dec_release();          /* decode.hip: frees the decode exchange buffer */
int dec_probe_placement();   /* decode.hip: whether stack-kernel workgroup b runs on XCD b % 8 */
void dec_placement_failed(); /* decode.hip: a launch found otherwise: exchanges through memory */

#endif
