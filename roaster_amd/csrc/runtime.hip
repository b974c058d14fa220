/*
 * runtime.hip -- device, stream, errors, scratch memory and the weight-pointer
 * registry behind the kernels.h memory ABI.
 *
 * The reference keeps one global Vulkan backend behind a mutex
 * (kernels.c:791-792) and maps host weight addresses to GPU buffers per call
 * (find_region / find_import, kernels.c:1140-1162, 1668-1683).  Here the
 * backend is one HIP stream on the current device; weight bytes live in HBM and
 * host addresses are translated to their HBM copy, uploaded once.
 */
#include "internal.h"

#include <algorithm>

#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>

#include <map>
#include <memory>
#include <unordered_map>
#include <utility>
#include <vector>

static RtState g_rt;
static std::recursive_mutex g_lock;
static char g_err[512];

RtState &rt() { return g_rt; }
std::recursive_mutex &rt_lock() { return g_lock; }

int rt_fail(int code, const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    fprintf(stderr, "roaster_moe: %s\n", g_err);
    return code;
}

int rt_check(hipError_t e, const char *what)
{
    if (e == hipSuccess) return 0;
    return rt_fail(ROASTER_EDEVICE, "%s: %s", what, hipGetErrorString(e));
}

extern "C" const char *roaster_last_error(void) { return g_err; }

int rt_init_locked()
{
    if (g_rt.inited) return 0;
    int dev = 0;
    if (rt_check(hipGetDevice(&dev), "hipGetDevice")) return ROASTER_EDEVICE;
    hipDeviceProp_t p;
    if (rt_check(hipGetDeviceProperties(&p, dev), "hipGetDeviceProperties")) return ROASTER_EDEVICE;
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return rt_fail(ROASTER_EDEVICE, "device %d is %s; this library is built for gfx950 (MI355X) only",
                       dev, p.gcnArchName);
    /* Default-priority, non-blocking stream: the only stream the library uses. */
    if (rt_check(hipStreamCreateWithFlags(&g_rt.stream, hipStreamNonBlocking), "hipStreamCreate"))
        return ROASTER_EDEVICE;
    g_rt.device = dev;
    g_rt.n_cu = p.multiProcessorCount;
    g_rt.n_xcd = 8;            /* MI355X: 8 XCDs of 32 CUs */
    g_rt.hbm_bytes = p.totalGlobalMem;
    g_rt.inited = 1;
    /* device address of the allocation-free entry point's scratch array; a
     * failure is reported by that entry point and leaves the others working */
    (void)noalloc_setup(dev);
    /* workgroup placement of the one-launch decode stack (a failure leaves
     * its exchanges going through memory) */
    (void)dec_probe_placement();
    return 0;
}

extern "C" int roaster_init(void)
{
    std::lock_guard<std::recursive_mutex> g(g_lock);
    return rt_init_locked();
}

extern "C" void *roaster_stream(void)
{
    std::lock_guard<std::recursive_mutex> g(g_lock);
    if (rt_init_locked()) return NULL;
    return (void *)g_rt.stream;
}

/* Control words of the decode kernels: [16] sticky error bits (1 = routing
 * found fewer than 8 finite logits, 2 = an exchange wait of the one-launch
 * stack gave up, 4 = a workgroup of it read an XCC_ID out of range), cleared
 * when reported; 4 also sends later launches' exchanges through memory. */
static unsigned *g_ctrl;
static int *g_aux_err;      /* error word of the allocation-free entry point's scratch, or NULL */
static int *g_err_pin;      /* pinned host copies of the two error words */
static bool g_aux_used;     /* a launch since the last report may have set the second word */

void rt_set_aux_err(int *dev_word) { g_aux_err = dev_word; }
void rt_aux_err_used() { g_aux_used = true; }

unsigned *rt_ctrl()
{
    if (!g_ctrl) {
        if (rt_check(hipMalloc((void **)&g_ctrl, 256), "ctrl hipMalloc")) { g_ctrl = NULL; return NULL; }
        if (rt_check(hipMemset(g_ctrl, 0, 256), "ctrl memset")) return NULL;
    }
    return g_ctrl;
}

int rt_take_err()
{
    /* the error words come back with the stream's last work: copies queued
     * behind it into pinned memory, then one synchronisation (two blocking
     * copies cost about 20 us per call) */
    int *words[2] = { g_ctrl ? (int *)(g_ctrl + 16) : NULL, g_aux_used ? g_aux_err : NULL };
    g_aux_used = false;
    if (!g_err_pin && (words[0] || words[1]) &&
        rt_check(hipHostMalloc((void **)&g_err_pin, 64, hipHostMallocDefault), "error word hipHostMalloc")) {
        g_err_pin = NULL;
        return ROASTER_EDEVICE;
    }
    for (int i = 0; i < 2; i++) {
        if (!words[i]) continue;
        g_err_pin[i] = 0;
        if (rt_check(hipMemcpyAsync(g_err_pin + i, words[i], sizeof(int), hipMemcpyDeviceToHost, g_rt.stream),
                     "error word readback"))
            return ROASTER_EDEVICE;
    }
    if (rt_check(hipStreamSynchronize(g_rt.stream), "hipStreamSynchronize")) return ROASTER_EDEVICE;
    int e = 0;
    for (int i = 0; i < 2; i++) {
        if (!words[i]) continue;
        const int w = g_err_pin[i];
        if (w && rt_check(hipMemset(words[i], 0, sizeof(int)), "error word reset")) return ROASTER_EDEVICE;
        e |= w;
    }
    if (!e) return 0;
    if (e & 4) dec_placement_failed();   /* later launches exchange through memory, groups fixed by index */
    if (e & 4) return rt_fail(ROASTER_EDEVICE, "a decode stack workgroup read an XCC_ID out of range");
    if (e & 2) return rt_fail(ROASTER_EDEVICE, "a decode layer's exchange wait timed out (workgroups not all resident?)");
    if (e & 8) return rt_fail(ROASTER_EDEVICE, "a fused prefill GEMM's tile wait timed out");
    return rt_fail(ROASTER_EROUTE, "router produced fewer than 8 finite logits for some token");
}

extern "C" int roaster_sync(void)
{
    std::lock_guard<std::recursive_mutex> g(g_lock);
    if (rt_init_locked()) return ROASTER_EDEVICE;
    return rt_take_err();
}

extern "C" int roaster_device_info(int *n_cu, int *n_xcd, size_t *hbm)
{
    std::lock_guard<std::recursive_mutex> g(g_lock);
    if (rt_init_locked()) return ROASTER_EDEVICE;
    if (n_cu) *n_cu = g_rt.n_cu;
    if (n_xcd) *n_xcd = g_rt.n_xcd;
    if (hbm) *hbm = g_rt.hbm_bytes;
    return 0;
}

/* ---- device memory helpers ---------------------------------------------- */
static std::map<uintptr_t, size_t> g_dev_ranges;    /* device allocations known to the library */

void rt_register_device_range(const void *dev, size_t bytes)
{
    g_dev_ranges[(uintptr_t)dev] = bytes;
}

void rt_unregister_device_range(const void *dev) { g_dev_ranges.erase((uintptr_t)dev); }

static bool in_device_range(const void *p)
{
    uintptr_t a = (uintptr_t)p;
    auto it = g_dev_ranges.upper_bound(a);
    if (it == g_dev_ranges.begin()) return false;
    --it;
    return a >= it->first && a < it->first + it->second;
}

extern "C" void *roaster_dev_alloc(size_t bytes)
{
    std::lock_guard<std::recursive_mutex> g(g_lock);
    if (rt_init_locked()) return NULL;
    void *p = NULL;
    if (rt_check(hipMalloc(&p, bytes + RT_TAIL_PAD), "hipMalloc")) return NULL;
    rt_register_device_range(p, bytes ? bytes : 1);
    return p;
}

extern "C" void roaster_dev_free(void *p)
{
    std::lock_guard<std::recursive_mutex> g(g_lock);
    if (!p) return;
    rt_unregister_device_range(p);
    (void)hipStreamSynchronize(g_rt.stream);
    (void)hipFree(p);
}

extern "C" int roaster_h2d(void *dst, const void *src, size_t n)
{
    std::lock_guard<std::recursive_mutex> g(g_lock);
    if (rt_init_locked()) return ROASTER_EDEVICE;
    if (!n) return 0;
    if (rt_check(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, g_rt.stream), "h2d")) return ROASTER_EDEVICE;
    return rt_check(hipStreamSynchronize(g_rt.stream), "h2d sync") ? ROASTER_EDEVICE : 0;
}

extern "C" int roaster_d2h(void *dst, const void *src, size_t n)
{
    std::lock_guard<std::recursive_mutex> g(g_lock);
    if (rt_init_locked()) return ROASTER_EDEVICE;
    if (!n) return 0;
    if (rt_check(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, g_rt.stream), "d2h")) return ROASTER_EDEVICE;
    return rt_check(hipStreamSynchronize(g_rt.stream), "d2h sync") ? ROASTER_EDEVICE : 0;
}

extern "C" int roaster_memset(void *dst, int v, size_t n)
{
    std::lock_guard<std::recursive_mutex> g(g_lock);
    if (rt_init_locked()) return ROASTER_EDEVICE;
    return rt_check(hipMemsetAsync(dst, v, n, g_rt.stream), "memset") ? ROASTER_EDEVICE : 0;
}

/* ---- scratch ------------------------------------------------------------- */
struct Buf { void *p; size_t n; };
static Buf g_scr[SCR_N];
static Buf g_pin[4];

void *rt_scratch(int slot, size_t bytes)
{
    Buf &b = g_scr[slot];
    if (b.n >= bytes && b.p) return b.p;
    if (b.p) { (void)hipStreamSynchronize(g_rt.stream); (void)hipFree(b.p); b.p = NULL; b.n = 0; }
    size_t n = bytes < 4096 ? 4096 : bytes;
    n = (n + 4095) & ~(size_t)4095;
    if (rt_check(hipMalloc(&b.p, n + RT_TAIL_PAD), "scratch hipMalloc")) { b.p = NULL; return NULL; }
    b.n = n;
    return b.p;
}

void rt_scratch_trim()
{
    (void)hipStreamSynchronize(g_rt.stream);
    for (int i = 0; i < SCR_N; i++) {
        if (g_scr[i].p) (void)hipFree(g_scr[i].p);
        g_scr[i].p = NULL;
        g_scr[i].n = 0;
    }
}

void *rt_pinned(int slot, size_t bytes)
{
    Buf &b = g_pin[slot];
    if (b.n >= bytes && b.p) return b.p;
    if (b.p) { (void)hipStreamSynchronize(g_rt.stream); (void)hipHostFree(b.p); b.p = NULL; b.n = 0; }
    size_t n = (bytes < 65536 ? 65536 : bytes);
    if (rt_check(hipHostMalloc(&b.p, n, hipHostMallocDefault), "hipHostMalloc")) { b.p = NULL; return NULL; }
    b.n = n;
    return b.p;
}

/* ---- weight registry ------------------------------------------------------
 * Host weight addresses are served from HBM twins that always hold the host
 * bytes as they are when a call uses them (the reference's GPU reads the host
 * memory itself, kernels.c:1445-1475, so a write before a call is seen by that
 * call):
 * (1) allocs: kernel_vk_alloc_weights hands out host addresses in 256 MB
 *     anonymous mappings; each allocation's twin sits at the same offset of
 *     the arena's HBM block;
 * (2) regions: kernel_vk_register_region records a host range with a twin;
 * (3) imports: any other host range, with a twin per (pointer, size).
 * Each use copies what changed: the used range's pages that a write-tracking
 * scan (wtrack.hip) finds written since their last copy, or -- where tracking
 * is unavailable -- the whole used range.  A page found written gets a new
 * version number; every twin records per page the version it copied, so
 * twins that share a page (adjacent imports, a region over an import) each
 * refresh it.  Copies go through pinned staging so that the DMA engine never
 * pins (and so never marks written) the tracked pages themselves.          */
#define ARENA_BYTES (256ull << 20)
static const uint32_t VER_NEVER = 0xFFFFFFFFu;

struct Twin {
    size_t size;                    /* host bytes [start, start + size) */
    uint8_t *dev;                   /* device copy of the same bytes */
    bool tracked;                   /* pages registered for write tracking */
    bool owns_dev;                  /* dev is this twin's own allocation */
    std::vector<uint32_t> synced;   /* per page of the span: version copied (VER_NEVER: none) */
    uintptr_t last_a = 0;           /* the range last brought up to date, and g_epoch then */
    size_t last_n = 0;
    uint32_t last_epoch = 0;
};
struct Arena { uint8_t *host; uint8_t *dev; size_t used, size; bool tracked; };

static std::vector<Arena> g_arenas;
static std::map<uintptr_t, Twin> g_allocs;
static std::map<uintptr_t, Twin> g_regions;
static std::map<std::pair<uintptr_t, size_t>, Twin> g_imports;

/* Page versions, in chunks of 512 pages; a page never found written has 0. */
static uint32_t g_epoch;
static std::unordered_map<uintptr_t, std::unique_ptr<uint32_t[]>> g_pver;
static unsigned long long g_sync_bytes;

static uint32_t page_ver(uintptr_t pn)
{
    auto it = g_pver.find(pn >> 9);
    return it == g_pver.end() ? 0 : it->second[pn & 511];
}

static void set_page_ver(uintptr_t pn, uint32_t v)
{
    auto &c = g_pver[pn >> 9];
    if (!c) {
        c.reset(new uint32_t[512]);
        memset(c.get(), 0, 512 * sizeof(uint32_t));
    }
    c[pn & 511] = v;
}

template <class M>
static typename M::iterator find_containing(M &m, uintptr_t a)
{
    auto it = m.upper_bound(a);
    if (it == m.begin()) return m.end();
    --it;
    if (a >= it->first && a < it->first + it->second.size) return it;
    return m.end();
}

static bool is_device_pointer(const void *p)
{
    if (in_device_range(p)) return true;
    hipPointerAttribute_t at;
    hipError_t e = hipPointerGetAttributes(&at, p);
    if (e != hipSuccess) { (void)hipGetLastError(); return false; }
    return at.type == hipMemoryTypeDevice;
}

/* Host -> device copy through two pinned 8 MB buffers, ordered on the library
 * stream (kernels launched later on it see the bytes).  Returns when the host
 * bytes have been read. */
static uint8_t *g_stage[2];
static hipEvent_t g_stage_ev[2];
static bool g_stage_busy[2];
#define STAGE_BYTES (8u << 20)

static int stage_upload(uint8_t *dst, const uint8_t *src, size_t n)
{
    if (!g_stage[0]) {
        for (int b = 0; b < 2; b++) {
            if (rt_check(hipHostMalloc((void **)&g_stage[b], STAGE_BYTES, hipHostMallocDefault), "staging hipHostMalloc") ||
                rt_check(hipEventCreateWithFlags(&g_stage_ev[b], hipEventDisableTiming), "staging event"))
                return ROASTER_EDEVICE;
            g_stage_busy[b] = false;
        }
    }
    static int next;
    for (size_t off = 0; off < n; off += STAGE_BYTES) {
        const size_t len = n - off < STAGE_BYTES ? n - off : STAGE_BYTES;
        const int b = next;
        next ^= 1;
        if (g_stage_busy[b] && rt_check(hipEventSynchronize(g_stage_ev[b]), "staging wait")) return ROASTER_EDEVICE;
        memcpy(g_stage[b], src + off, len);
        if (rt_check(hipMemcpyAsync(dst + off, g_stage[b], len, hipMemcpyHostToDevice, g_rt.stream), "weight upload") ||
            rt_check(hipEventRecord(g_stage_ev[b], g_rt.stream), "staging record"))
            return ROASTER_EDEVICE;
        g_stage_busy[b] = true;
    }
    g_sync_bytes += n;
    return 0;
}

static void stage_release()
{
    for (int b = 0; b < 2; b++) {
        if (!g_stage[b]) continue;
        if (g_stage_busy[b]) (void)hipEventSynchronize(g_stage_ev[b]);
        (void)hipEventDestroy(g_stage_ev[b]);
        (void)hipHostFree(g_stage[b]);
        g_stage[b] = NULL;
        g_stage_busy[b] = false;
    }
}

static void twin_init(Twin &T, size_t size, uint8_t *dev, bool owns, uintptr_t host, bool tracked)
{
    const size_t P = wt_page_size();
    const uintptr_t p0 = host & ~(uintptr_t)(P - 1), p1 = (host + size + P - 1) & ~(uintptr_t)(P - 1);
    T.size = size;
    T.dev = dev;
    T.owns_dev = owns;
    T.tracked = tracked;
    T.synced.assign(tracked ? (p1 - p0) / P : 0, VER_NEVER);
}

/* Make the twin hold the current host bytes of [a, a + bytes) (a inside the
 * twin that starts at host address h). */
static int twin_sync(Twin &T, uintptr_t h, uintptr_t a, size_t bytes)
{
    if (!T.tracked || !wt_available()) return stage_upload(T.dev + (a - h), (const uint8_t *)a, bytes);
    const size_t P = wt_page_size();
    const uintptr_t s0 = h & ~(uintptr_t)(P - 1);
    const uintptr_t p_lo = a & ~(uintptr_t)(P - 1), p_hi = (a + bytes + P - 1) & ~(uintptr_t)(P - 1);
    std::vector<std::pair<uintptr_t, uintptr_t>> runs;
    if (wt_scan(p_lo, p_hi - p_lo, runs)) {
        /* The range is no longer tracked (remapped behind the library's back):
         * copy on every use from now on.  The scan may have re-protected
         * written pages before it failed, so every page of the range counts
         * as written: every other twin holding one copies it again. */
        ++g_epoch;
        for (uintptr_t pg = p_lo; pg < p_hi; pg += P) set_page_ver(pg / P, g_epoch);
        T.tracked = false;
        T.synced.clear();
        return stage_upload(T.dev + (a - h), (const uint8_t *)a, bytes);
    }
    if (!runs.empty()) {
        ++g_epoch;
        for (auto &r : runs)
            for (uintptr_t pg = r.first; pg < r.second; pg += P) set_page_ver(pg / P, g_epoch);
    } else if (T.last_n && a == T.last_a && bytes == T.last_n && T.last_epoch == g_epoch) {
        /* no page anywhere found written since this range was last brought up
         * to date (every write found bumps g_epoch): nothing to copy */
        return 0;
    }
    /* Whole pages (clipped to the twin): the scan re-protected them, so this
     * twin must now hold all of each, not only the part inside [a, a+bytes). */
    uintptr_t run0 = 0, run1 = 0;
    for (uintptr_t pg = p_lo; pg < p_hi; pg += P) {
        uint32_t &s = T.synced[(pg - s0) / P];
        const uint32_t v = page_ver(pg / P);
        const bool stale = s == VER_NEVER || v > s;
        if (stale) {
            s = v;
            const uintptr_t lo = pg > h ? pg : h, hi = pg + P < h + T.size ? pg + P : h + T.size;
            if (run1 == lo) run1 = hi;
            else {
                if (run1 > run0 && stage_upload(T.dev + (run0 - h), (const uint8_t *)run0, run1 - run0)) return ROASTER_EDEVICE;
                run0 = lo;
                run1 = hi;
            }
        }
    }
    if (run1 > run0 && stage_upload(T.dev + (run0 - h), (const uint8_t *)run0, run1 - run0)) return ROASTER_EDEVICE;
    T.last_a = a;
    T.last_n = bytes;
    T.last_epoch = g_epoch;
    return 0;
}

const void *rt_weight_dev(const void *ptr, size_t bytes)
{
    if (!ptr) { rt_fail(ROASTER_EINVAL, "NULL weight pointer"); return NULL; }
    const uintptr_t a = (uintptr_t)ptr;
    auto al = find_containing(g_allocs, a);
    if (al != g_allocs.end()) {
        Twin &T = al->second;
        if (a + bytes > al->first + T.size) { rt_fail(ROASTER_EINVAL, "weight range overruns its allocation"); return NULL; }
        if (twin_sync(T, al->first, a, bytes)) return NULL;
        return T.dev + (a - al->first);
    }
    auto rg = find_containing(g_regions, a);
    if (rg != g_regions.end()) {
        Twin &T = rg->second;
        if (a + bytes > rg->first + T.size) { rt_fail(ROASTER_EINVAL, "weight range overruns its region"); return NULL; }
        if (twin_sync(T, rg->first, a, bytes)) return NULL;
        return T.dev + (a - rg->first);
    }
    if (is_device_pointer(ptr)) return ptr;
    auto key = std::make_pair(a, bytes);
    auto im = g_imports.find(key);
    if (im == g_imports.end()) {
        void *d = NULL;
        if (rt_check(hipMalloc(&d, bytes + RT_TAIL_PAD), "import hipMalloc")) return NULL;
        Twin T;
        twin_init(T, bytes, (uint8_t *)d, true, a, wt_register(a, bytes) == 0);
        im = g_imports.emplace(key, std::move(T)).first;
    }
    if (twin_sync(im->second, a, a, bytes)) return NULL;
    return im->second.dev;
}

static void free_twin(Twin &T)
{
    if (T.owns_dev && T.dev) (void)hipFree(T.dev);
    T.dev = NULL;
}

void rt_registry_clear()
{
    (void)hipDeviceSynchronize();
    wt_unregister_all();
    for (auto &kv : g_imports) free_twin(kv.second);
    g_imports.clear();
    for (auto &kv : g_regions) free_twin(kv.second);
    g_regions.clear();
    g_allocs.clear();
    for (auto &ar : g_arenas) {
        (void)hipFree(ar.dev);
        munmap(ar.host, ar.size);
    }
    g_arenas.clear();
    g_pver.clear();
    stage_release();
}

/* kernels.h:103 -- 4 KB-aligned bump allocation from 256 MB blocks (kernels.c:1445-1537);
 * freed only at shutdown.  Returns a host address whose bytes the caller fills. */
extern "C" void *kernel_vk_alloc_weights(size_t size, size_t *granted)
{
    std::lock_guard<std::recursive_mutex> g(g_lock);
    if (granted) *granted = 0;
    if (!size || rt_init_locked()) return NULL;
    size_t need = (size + 4095) & ~(size_t)4095;
    Arena *ar = NULL;
    if (!g_arenas.empty() && g_arenas.back().size - g_arenas.back().used >= need) ar = &g_arenas.back();
    if (!ar) {
        size_t asz = need > ARENA_BYTES ? need : ARENA_BYTES;
        Arena na;
        na.host = (uint8_t *)mmap(NULL, asz, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
        if (na.host == MAP_FAILED) { rt_fail(ROASTER_ENOMEM, "mmap of %zu bytes failed", asz); return NULL; }
        if (hipMalloc((void **)&na.dev, asz + RT_TAIL_PAD) != hipSuccess) {
            (void)hipGetLastError();
            munmap(na.host, asz);
            rt_fail(ROASTER_ENOMEM, "HBM arena of %zu bytes unavailable", asz);
            return NULL;
        }
        /* Base pages keep write tracking at 4 KB granularity. */
        (void)madvise(na.host, asz, MADV_NOHUGEPAGE);
        na.tracked = wt_register((uintptr_t)na.host, asz) == 0;
        na.used = 0;
        na.size = asz;
        g_arenas.push_back(na);
        ar = &g_arenas.back();
    }
    uint8_t *h = ar->host + ar->used;
    Twin T;
    twin_init(T, need, ar->dev + ar->used, false, (uintptr_t)h, ar->tracked);
    g_allocs.emplace((uintptr_t)h, std::move(T));
    ar->used += need;
    if (granted) *granted = need;
    return h;
}

extern "C" int kernel_vk_owns_weights(const void *ptr)
{
    std::lock_guard<std::recursive_mutex> g(g_lock);
    return find_containing(g_allocs, (uintptr_t)ptr) != g_allocs.end();
}

/* 1 if ptr is arena memory (nothing more to do: released at shutdown). */
extern "C" int kernel_vk_free_weights(void *ptr)
{
    return kernel_vk_owns_weights(ptr);
}

/* kernels.c:1431-1443: one twin for a whole host range (weights.c:527-529
 * registers its expert-cache slab); ranges inside it are then served from it. */
extern "C" int kernel_vk_register_region(const void *ptr, size_t size)
{
    std::lock_guard<std::recursive_mutex> g(g_lock);
    if (!ptr || !size || rt_init_locked()) return 0;
    if (find_containing(g_regions, (uintptr_t)ptr) != g_regions.end()) return 1;
    uint8_t *dev = NULL;
    if (hipMalloc((void **)&dev, size + RT_TAIL_PAD) != hipSuccess) { (void)hipGetLastError(); return 0; }
    Twin T;
    twin_init(T, size, dev, true, (uintptr_t)ptr, wt_register((uintptr_t)ptr, size) == 0);
    g_regions.emplace((uintptr_t)ptr, std::move(T));
    return 1;
}

/* kernels.c:1402-1429: drop every import and region that starts at ptr (the
 * caller is about to free that memory; weights.c:333-339).  Imports that lie
 * inside a dropped region go with it.  Arena memory is the library's own and
 * is released at shutdown only. */
/* Pages of the dropped ranges that no remaining twin covers stop being
 * tracked, so that memory mapped there later is registered afresh. */
static void untrack_dropped(std::vector<std::pair<uintptr_t, uintptr_t>> &dropped)
{
    if (dropped.empty() || !wt_available()) return;
    const size_t P = wt_page_size();
    std::vector<std::pair<uintptr_t, uintptr_t>> live;
    auto add_live = [&](uintptr_t s, size_t n) {
        if (n) live.push_back(std::make_pair(s & ~(uintptr_t)(P - 1), (s + n + P - 1) & ~(uintptr_t)(P - 1)));
    };
    for (auto &ar : g_arenas) add_live((uintptr_t)ar.host, ar.size);
    for (auto &kv : g_regions) add_live(kv.first, kv.second.size);
    for (auto &kv : g_imports) add_live(kv.first.first, kv.second.size);
    std::sort(live.begin(), live.end());
    for (auto &d : dropped) {
        uintptr_t at = d.first & ~(uintptr_t)(P - 1);
        const uintptr_t end = (d.second + P - 1) & ~(uintptr_t)(P - 1);
        for (auto &lv : live) {
            if (lv.second <= at) continue;
            if (lv.first >= end) break;
            if (lv.first > at) wt_unregister(at, lv.first - at);
            at = lv.second > at ? lv.second : at;
        }
        if (at < end) wt_unregister(at, end - at);
    }
}

extern "C" void kernel_vk_release_host_ptr(const void *ptr)
{
    std::lock_guard<std::recursive_mutex> g(g_lock);
    if (!ptr) return;
    const uintptr_t a = (uintptr_t)ptr;
    uintptr_t lo = a, hi = a + 1;
    auto rg = g_regions.find(a);
    if (rg != g_regions.end()) hi = a + rg->second.size;
    bool synced = false;
    std::vector<std::pair<uintptr_t, uintptr_t>> dropped;
    for (auto it = g_imports.begin(); it != g_imports.end();) {
        const uintptr_t s = it->first.first;
        if (s == a || (s >= lo && s + it->first.second <= hi)) {
            if (!synced) { (void)hipStreamSynchronize(g_rt.stream); synced = true; }
            dropped.push_back(std::make_pair(s, s + it->first.second));
            free_twin(it->second);
            it = g_imports.erase(it);
        } else {
            ++it;
        }
    }
    if (rg != g_regions.end()) {
        if (!synced) (void)hipStreamSynchronize(g_rt.stream);
        dropped.push_back(std::make_pair(a, hi));
        free_twin(rg->second);
        g_regions.erase(rg);
    }
    untrack_dropped(dropped);
}

/* Bytes copied host -> HBM by the registry since load, and whether writes are
 * tracked (1) or every used range is copied on each use (0). */
extern "C" int roaster_weight_sync_stats(unsigned long long *bytes_copied, int *tracking)
{
    std::lock_guard<std::recursive_mutex> g(g_lock);
    if (bytes_copied) *bytes_copied = g_sync_bytes;
    if (tracking) *tracking = wt_available();
    return 0;
}

extern "C" void kernel_vk_trim_scratch(void)
{
    std::lock_guard<std::recursive_mutex> g(g_lock);
    if (!g_rt.inited) return;
    rt_scratch_trim();
}

/* kernels.h:105 -- the reference destroys its backend here (kernels.c, called
 * from weights.c:1171).  Everything the library holds goes: scratch, control
 * words, the decode exchange buffer, pinned and staging buffers, the weight
 * registry and its HBM twins, and the stream, so that nothing of the library
 * is left for the HIP runtime to tear down at process exit.  Expert tables
 * belong to the caller (roaster_table_destroy).  A later call initialises
 * the library again. */
extern "C" void kernel_vk_shutdown(void)
{
    std::lock_guard<std::recursive_mutex> g(g_lock);
    if (!g_rt.inited) return;
    kernel_matvec_quant_end();
    (void)hipStreamSynchronize(g_rt.stream);
    rt_scratch_trim();
    rt_registry_clear();
    for (int i = 0; i < 4; i++) {
        if (g_pin[i].p) (void)hipHostFree(g_pin[i].p);
        g_pin[i].p = NULL;
        g_pin[i].n = 0;
    }
    dec_release();
    if (g_ctrl) {
        (void)hipFree(g_ctrl);
        g_ctrl = NULL;
    }
    if (g_err_pin) {
        (void)hipHostFree(g_err_pin);
        g_err_pin = NULL;
    }
    (void)hipStreamDestroy(g_rt.stream);
    g_rt.stream = NULL;
    g_rt.inited = 0;
}
