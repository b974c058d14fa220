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

#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>

#include <map>
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

/* Control words of the persistent kernels: [0] grid-barrier arrivals (reset
 * before each launch), [16] sticky error bits (1 = routing found fewer than 8
 * finite logits, 2 = a grid barrier wait timed out), cleared when reported. */
static unsigned *g_ctrl;

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
    if (rt_check(hipStreamSynchronize(g_rt.stream), "hipStreamSynchronize")) return ROASTER_EDEVICE;
    if (!g_ctrl) return 0;
    int e = 0;
    if (rt_check(hipMemcpy(&e, g_ctrl + 16, sizeof(int), hipMemcpyDeviceToHost), "error word readback"))
        return ROASTER_EDEVICE;
    if (!e) return 0;
    if (rt_check(hipMemset(g_ctrl + 16, 0, sizeof(int)), "error word reset")) return ROASTER_EDEVICE;
    if (e & 2) return rt_fail(ROASTER_EDEVICE, "a grid barrier timed out (workgroups not co-resident?)");
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
 * (1) arenas: kernel_vk_alloc_weights hands out host addresses in 256 MB
 *     anonymous mappings; each allocation has an HBM twin, uploaded whole on
 *     its first use (weights are written once by the loader, then read).
 * (2) regions: kernel_vk_register_region records a host range with an HBM
 *     twin; sub-ranges are uploaded on their first use.
 * (3) imports: any other host range, uploaded and cached per (pointer, size).
 * kernel_vk_release_host_ptr(p) forgets uploads that start at p, so rewritten
 * bytes are uploaded again on next use.                                      */
#define ARENA_BYTES (256ull << 20)

struct Arena { uint8_t *host; uint8_t *dev; size_t used, size; };
struct Alloc { size_t size; uint8_t *dev; bool uploaded; };
struct Region { size_t size; uint8_t *dev; std::map<uintptr_t, size_t> up; };

static std::vector<Arena> g_arenas;
static std::map<uintptr_t, Alloc> g_allocs;
static std::map<uintptr_t, Region> g_regions;
static std::map<std::pair<uintptr_t, size_t>, void *> g_imports;

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

const void *rt_weight_dev(const void *ptr, size_t bytes)
{
    if (!ptr) { rt_fail(ROASTER_EINVAL, "NULL weight pointer"); return NULL; }
    uintptr_t a = (uintptr_t)ptr;
    auto al = find_containing(g_allocs, a);
    if (al != g_allocs.end()) {
        Alloc &A = al->second;
        if (a + bytes > al->first + A.size) { rt_fail(ROASTER_EINVAL, "weight range overruns its allocation"); return NULL; }
        if (!A.uploaded) {
            if (rt_check(hipMemcpy(A.dev, (const void *)al->first, A.size, hipMemcpyHostToDevice), "weight upload"))
                return NULL;
            A.uploaded = true;
        }
        return A.dev + (a - al->first);
    }
    auto rg = find_containing(g_regions, a);
    if (rg != g_regions.end()) {
        Region &R = rg->second;
        if (a + bytes > rg->first + R.size) { rt_fail(ROASTER_EINVAL, "weight range overruns its region"); return NULL; }
        auto u = R.up.find(a);
        if (u == R.up.end() || u->second < bytes) {
            if (rt_check(hipMemcpy(R.dev + (a - rg->first), ptr, bytes, hipMemcpyHostToDevice), "region upload"))
                return NULL;
            R.up[a] = bytes;
        }
        return R.dev + (a - rg->first);
    }
    if (is_device_pointer(ptr)) return ptr;
    auto key = std::make_pair(a, bytes);
    auto im = g_imports.find(key);
    if (im != g_imports.end()) return im->second;
    void *d = NULL;
    if (rt_check(hipMalloc(&d, bytes + RT_TAIL_PAD), "import hipMalloc")) return NULL;
    if (rt_check(hipMemcpy(d, ptr, bytes, hipMemcpyHostToDevice), "import upload")) { (void)hipFree(d); return NULL; }
    g_imports[key] = d;
    return d;
}

void rt_registry_clear()
{
    (void)hipDeviceSynchronize();
    for (auto &kv : g_imports) (void)hipFree(kv.second);
    g_imports.clear();
    for (auto &kv : g_regions) (void)hipFree(kv.second.dev);
    g_regions.clear();
    g_allocs.clear();
    for (auto &ar : g_arenas) {
        (void)hipFree(ar.dev);
        munmap(ar.host, ar.size);
    }
    g_arenas.clear();
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
        na.used = 0;
        na.size = asz;
        g_arenas.push_back(na);
        ar = &g_arenas.back();
    }
    uint8_t *h = ar->host + ar->used;
    Alloc A;
    A.size = need;
    A.dev = ar->dev + ar->used;
    A.uploaded = false;
    g_allocs[(uintptr_t)h] = A;
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

extern "C" int kernel_vk_register_region(const void *ptr, size_t size)
{
    std::lock_guard<std::recursive_mutex> g(g_lock);
    if (!ptr || !size || rt_init_locked()) return 0;
    if (find_containing(g_regions, (uintptr_t)ptr) != g_regions.end()) return 1;
    Region R;
    R.size = size;
    R.dev = NULL;
    if (hipMalloc((void **)&R.dev, size + RT_TAIL_PAD) != hipSuccess) { (void)hipGetLastError(); return 0; }
    g_regions[(uintptr_t)ptr] = R;
    return 1;
}

extern "C" void kernel_vk_release_host_ptr(const void *ptr)
{
    std::lock_guard<std::recursive_mutex> g(g_lock);
    uintptr_t a = (uintptr_t)ptr;
    for (auto it = g_imports.begin(); it != g_imports.end();) {
        if (it->first.first == a) {
            (void)hipStreamSynchronize(g_rt.stream);
            (void)hipFree(it->second);
            it = g_imports.erase(it);
        } else {
            ++it;
        }
    }
    auto al = g_allocs.find(a);
    if (al != g_allocs.end()) al->second.uploaded = false;
    auto rg = find_containing(g_regions, a);
    if (rg != g_regions.end()) rg->second.up.erase(a);
}

extern "C" void kernel_vk_trim_scratch(void)
{
    std::lock_guard<std::recursive_mutex> g(g_lock);
    if (!g_rt.inited) return;
    rt_scratch_trim();
}

extern "C" void kernel_vk_shutdown(void)
{
    std::lock_guard<std::recursive_mutex> g(g_lock);
    if (!g_rt.inited) return;
    kernel_matvec_quant_end();
    rt_scratch_trim();
    rt_registry_clear();
    for (int i = 0; i < 4; i++) {
        if (g_pin[i].p) (void)hipHostFree(g_pin[i].p);
        g_pin[i].p = NULL;
        g_pin[i].n = 0;
    }
}

int rt_coop_grid(const void *kernel, int threads, size_t lds, int *blocks_out)
{
    int per_cu = 0;
    if (rt_check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, lds), "occupancy"))
        return ROASTER_EDEVICE;
    if (per_cu < 1) return rt_fail(ROASTER_EDEVICE, "kernel cannot be resident (threads %d, lds %zu)", threads, lds);
    *blocks_out = per_cu * g_rt.n_cu;
    return 0;
}
