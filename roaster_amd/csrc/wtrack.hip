/*
 * wtrack.hip -- write tracking of host memory whose bytes have an HBM twin.
 *
 * The reference keeps weights in host-visible memory that its GPU reads in
 * place (kernels.c:1445-1475), so a write made before a call is seen by that
 * call; weights.c relies on it when it reads a new expert into an expert-cache
 * slot at the same address on every miss (weights.c:615-645).  Here weights
 * are read from an HBM twin, so the library must learn which host pages
 * changed since it last copied them.
 *
 * Mechanism: userfaultfd write protection in asynchronous mode
 * (UFFD_FEATURE_WP_ASYNC, Linux 6.7+).  A registered, write-protected page
 * takes one minor fault on its next write -- from user code or from the
 * kernel on the process's behalf (pread, O_DIRECT pinning) -- which the kernel
 * resolves by itself and records as "written" in the page table; no handler
 * thread runs.  The PAGEMAP_SCAN ioctl on /proc/self/pagemap then reports the
 * written pages of a range and write-protects them again in the same atomic
 * walk, so every later write is seen by the next scan.  mprotect() could not
 * serve here: a pread() into a read-only page fails with EFAULT instead of
 * faulting.
 *
 * When the running kernel lacks any of these (older kernel, userfaultfd
 * disabled), wt_available() is 0 and callers re-copy every range they use.
 * The ABI constants below are the kernel's (include/uapi/linux/userfaultfd.h
 * and fs.h); they are defined here because the build image's headers predate
 * them.
 */
#include "internal.h"

#include <errno.h>
#include <fcntl.h>
#include <stdlib.h>
#include <string.h>
#include <sys/ioctl.h>
#include <sys/mman.h>
#include <sys/syscall.h>
#include <unistd.h>
#include <linux/userfaultfd.h>

#include <iterator>
#include <map>

#ifndef UFFD_USER_MODE_ONLY
#define UFFD_USER_MODE_ONLY 1
#endif
#define WT_FEATURE_WP_UNPOPULATED (1ull << 13)
#define WT_FEATURE_WP_ASYNC (1ull << 15)

struct wt_page_region { uint64_t start, end, categories; };
struct wt_scan_arg {
    uint64_t size, flags, start, end, walk_end, vec, vec_len, max_pages;
    uint64_t category_inverted, category_mask, category_anyof_mask, return_mask;
};
#define WT_SCAN_WP_MATCHING (1ull << 0)
#define WT_SCAN_CHECK_WPASYNC (1ull << 1)
#define WT_PAGE_IS_WRITTEN (1ull << 1)
#define WT_PAGEMAP_SCAN _IOWR('f', 16, struct wt_scan_arg)

static int g_state;          /* 0 not probed, 1 available, -1 unavailable */
static int g_enabled = 1;    /* roaster_weight_tracking(0) switches tracking off */
static int g_uffd = -1;
static int g_pagemap = -1;
static size_t g_page;

size_t wt_page_size()
{
    if (!g_page) {
        long p = sysconf(_SC_PAGESIZE);
        g_page = p > 0 ? (size_t)p : 4096;
    }
    return g_page;
}

static int wt_open()
{
    /* User-mode-only descriptors are what unprivileged processes may create;
     * asynchronous write protection is resolved in the fault path itself, so
     * kernel-mode writes are recorded all the same. */
    int fd = (int)syscall(SYS_userfaultfd, O_CLOEXEC | O_NONBLOCK | UFFD_USER_MODE_ONLY);
    if (fd < 0) return -1;
    struct uffdio_api api;
    memset(&api, 0, sizeof(api));
    api.api = UFFD_API;
    api.features = WT_FEATURE_WP_ASYNC | WT_FEATURE_WP_UNPOPULATED;
    if (ioctl(fd, UFFDIO_API, &api) != 0 ||
        (api.features & (WT_FEATURE_WP_ASYNC | WT_FEATURE_WP_UNPOPULATED)) !=
            (WT_FEATURE_WP_ASYNC | WT_FEATURE_WP_UNPOPULATED)) {
        close(fd);
        return -1;
    }
    return fd;
}

static int wt_register_fd(int fd, uintptr_t p0, uintptr_t p1)
{
    struct uffdio_register r;
    memset(&r, 0, sizeof(r));
    r.range.start = p0;
    r.range.len = p1 - p0;
    r.mode = UFFDIO_REGISTER_MODE_WP;
    if (ioctl(fd, UFFDIO_REGISTER, &r) != 0) return -1;
    struct uffdio_writeprotect wp;
    memset(&wp, 0, sizeof(wp));
    wp.range.start = p0;
    wp.range.len = p1 - p0;
    wp.mode = UFFDIO_WRITEPROTECT_MODE_WP;
    return ioctl(fd, UFFDIO_WRITEPROTECT, &wp) == 0 ? 0 : -1;
}

static long wt_scan_fd(int pm, uintptr_t p0, uintptr_t p1, std::vector<std::pair<uintptr_t, uintptr_t>> &runs)
{
    struct wt_page_region vec[64];
    uintptr_t at = p0;
    while (at < p1) {
        struct wt_scan_arg a;
        memset(&a, 0, sizeof(a));
        a.size = sizeof(a);
        a.flags = WT_SCAN_WP_MATCHING | WT_SCAN_CHECK_WPASYNC;
        a.start = at;
        a.end = p1;
        a.vec = (uint64_t)(uintptr_t)vec;
        a.vec_len = 64;
        a.category_mask = WT_PAGE_IS_WRITTEN;
        a.return_mask = WT_PAGE_IS_WRITTEN;
        long k = ioctl(pm, WT_PAGEMAP_SCAN, &a);
        if (k < 0) return -1;
        for (long i = 0; i < k; i++) runs.push_back(std::make_pair((uintptr_t)vec[i].start, (uintptr_t)vec[i].end));
        if (a.walk_end <= at) return -1;          /* no progress: refuse rather than spin */
        at = (uintptr_t)a.walk_end;
    }
    return 0;
}

/* Probe once: a scratch mapping must report exactly the pages written by a
 * store, by a store to a never-touched page and by a read(2) into it. */
static int wt_probe()
{
    if (const char *m = getenv("ROASTER_WEIGHT_SYNC"))
        if (!strcmp(m, "copy")) g_enabled = 0;
    int fd = wt_open();
    if (fd < 0) return -1;
    int pm = open("/proc/self/pagemap", O_RDONLY | O_CLOEXEC);
    const size_t P = wt_page_size();
    uint8_t *m = (uint8_t *)mmap(NULL, 8 * P, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0);
    int ok = pm >= 0 && m != MAP_FAILED;
    int pfd[2] = { -1, -1 };
    if (ok) {
        memset(m, 1, 2 * P);
        madvise(m, 8 * P, MADV_NOHUGEPAGE);
        const uintptr_t p0 = (uintptr_t)m, p1 = p0 + 8 * P;
        std::vector<std::pair<uintptr_t, uintptr_t>> runs;
        ok = wt_register_fd(fd, p0, p1) == 0 && wt_scan_fd(pm, p0, p1, runs) == 0 && runs.empty();
        if (ok) {
            m[1 * P + 5] = 7;                                  /* populated page */
            m[6 * P] = 9;                                      /* never-touched page */
            ok = pipe(pfd) == 0 && write(pfd[1], "wt", 2) == 2 && read(pfd[0], m + 3 * P + 100, 2) == 2;
        }
        if (ok) {
            runs.clear();
            ok = wt_scan_fd(pm, p0, p1, runs) == 0 && runs.size() == 3 &&
                 runs[0] == std::make_pair(p0 + 1 * P, p0 + 2 * P) &&
                 runs[1] == std::make_pair(p0 + 3 * P, p0 + 4 * P) &&
                 runs[2] == std::make_pair(p0 + 6 * P, p0 + 7 * P);
        }
        if (ok) {
            runs.clear();
            ok = wt_scan_fd(pm, p0, p1, runs) == 0 && runs.empty();   /* the scan re-protected them */
        }
    }
    if (pfd[0] >= 0) close(pfd[0]);
    if (pfd[1] >= 0) close(pfd[1]);
    if (m != MAP_FAILED) munmap(m, 8 * P);
    if (!ok) {
        if (pm >= 0) close(pm);
        close(fd);
        return -1;
    }
    g_uffd = fd;
    g_pagemap = pm;
    return 1;
}

int wt_available()
{
    if (!g_state) g_state = wt_probe();
    return g_state > 0 && g_enabled;
}

/* Page spans registered so far (merged, disjoint).  A page is registered and
 * write-protected once only: protecting it again would erase a "written"
 * state that no scan has collected yet. */
static std::map<uintptr_t, uintptr_t> g_spans;

int wt_register(uintptr_t start, size_t n)
{
    if (!wt_available() || !n) return -1;
    const size_t P = wt_page_size();
    uintptr_t p0 = start & ~(uintptr_t)(P - 1), p1 = (start + n + P - 1) & ~(uintptr_t)(P - 1);
    /* the gaps of [p0, p1) not yet registered */
    auto it = g_spans.upper_bound(p0);
    if (it != g_spans.begin()) {
        auto pv = std::prev(it);
        if (pv->second > p0) it = pv;
    }
    uintptr_t at = p0;
    std::vector<std::pair<uintptr_t, uintptr_t>> gaps;
    for (; it != g_spans.end() && it->first < p1; ++it) {
        if (it->first > at) gaps.push_back(std::make_pair(at, it->first));
        if (it->second > at) at = it->second;
    }
    if (at < p1) gaps.push_back(std::make_pair(at, p1));
    for (auto &gp : gaps)
        if (wt_register_fd(g_uffd, gp.first, gp.second)) return -1;
    /* merge [p0, p1) into the span set */
    it = g_spans.upper_bound(p0);
    if (it != g_spans.begin()) {
        auto pv = std::prev(it);
        if (pv->second >= p0) it = pv;
    }
    while (it != g_spans.end() && it->first <= p1) {
        if (it->first < p0) p0 = it->first;
        if (it->second > p1) p1 = it->second;
        it = g_spans.erase(it);
    }
    g_spans[p0] = p1;
    return 0;
}

/* Stop tracking the pages of [start, start + n): they leave the span set, so
 * a later registration of the same addresses (a new mapping there) is
 * registered and protected again, and are unregistered from the descriptor
 * (which fails harmlessly for memory that is no longer mapped). */
void wt_unregister(uintptr_t start, size_t n)
{
    if (g_state <= 0 || !n) return;
    const size_t P = wt_page_size();
    const uintptr_t p0 = start & ~(uintptr_t)(P - 1), p1 = (start + n + P - 1) & ~(uintptr_t)(P - 1);
    auto it = g_spans.upper_bound(p0);
    if (it != g_spans.begin()) {
        auto pv = std::prev(it);
        if (pv->second > p0) it = pv;
    }
    std::vector<std::pair<uintptr_t, uintptr_t>> keep;
    while (it != g_spans.end() && it->first < p1) {
        if (it->first < p0) keep.push_back(std::make_pair(it->first, p0));
        if (it->second > p1) keep.push_back(std::make_pair(p1, it->second));
        it = g_spans.erase(it);
    }
    for (auto &k : keep) g_spans[k.first] = k.second;
    struct uffdio_range r;
    r.start = p0;
    r.len = p1 - p0;
    (void)ioctl(g_uffd, UFFDIO_UNREGISTER, &r);
}

/* Every span (at shutdown, before the library's own mappings go away). */
void wt_unregister_all()
{
    while (!g_spans.empty()) {
        const auto sp = *g_spans.begin();
        wt_unregister(sp.first, sp.second - sp.first);
    }
}

int wt_scan(uintptr_t start, size_t n, std::vector<std::pair<uintptr_t, uintptr_t>> &runs)
{
    if (!wt_available()) return -1;
    const size_t P = wt_page_size();
    const uintptr_t p0 = start & ~(uintptr_t)(P - 1), p1 = (start + n + P - 1) & ~(uintptr_t)(P - 1);
    return wt_scan_fd(g_pagemap, p0, p1, runs) == 0 ? 0 : -1;
}

/* enable = 1: track writes where the kernel allows it; 0: copy every used
 * range on each use (for memory that a device writes by DMA into pages it
 * pinned earlier, which no page-table mechanism sees); -1: query only.
 * Returns 1 if writes are tracked after the call.  Needs no GPU. */
extern "C" int roaster_weight_tracking(int enable)
{
    std::lock_guard<std::recursive_mutex> g(rt_lock());
    if (!g_state) g_state = wt_probe();
    if (enable == 0 || enable == 1) g_enabled = enable;
    return wt_available();
}
