"""Weight memory rewritten in place between calls.

weights.c allocates its expert-cache slab from kernel_vk_alloc_weights memory
(weights.c:522-532), or mallocs it and registers it as a region (527-529), and
on every cache miss reads a new expert into a slot at the same address
(weights.c:615-645) -- by pread(2), i.e. a write made by the kernel.  In the
reference the GPU reads that host memory in place (kernels.c:1445-1475), so
the next kernel_ffn_fused (model.c:1103) or kernel_moe_prefill (model.c:1771)
computes on the new bytes.  These tests rewrite slots in place, by stores, by
pread and by O_DIRECT pread (weights.c's default), and require every result to
match the oracle run on the bytes the host memory holds at the time of the
call; both sync modes (write tracking, and copy-on-every-use) are exercised,
and a region mapped again at a released region's address is tracked again.  Tolerances: the reference test's 2e-4
(test_kernels.c:31) for kernel_moe_prefill, 2e-5 for the f32 decode path."""
import ctypes as C
import os
import tempfile

import numpy as np
import pytest

import roaster_amd as R
from oracle import oracle as O
from gpu_util import alloc_w, log, rel_err

pytestmark = pytest.mark.gpu

GATE_B = 512 * 8 * 144        # Q4_K [512 x 2048]
DOWN_B = 2048 * 2 * 210       # Q6_K [2048 x 512]
STRIDE = 2 * GATE_B + DOWN_B  # a slab slot (all three 4 KB multiples, as weights.c:511-514 rounds them)


def _copied():
    b = C.c_ulonglong(0)
    t = C.c_int(0)
    R.lib().roaster_weight_sync_stats(C.byref(b), C.byref(t))
    return b.value


def _store(p, arr):
    C.memmove(p, np.ascontiguousarray(arr).ctypes.data, arr.nbytes)


def _pread(p, arr):
    """Write arr's bytes at host address p with pread(2) from a file, as
    weights.c's read_full does."""
    with tempfile.NamedTemporaryFile() as f:
        f.write(np.ascontiguousarray(arr).tobytes())
        f.flush()
        fd = os.open(f.name, os.O_RDONLY)
        try:
            view = memoryview((C.c_char * arr.nbytes).from_address(p)).cast("B")
            assert os.preadv(fd, [view], 0) == arr.nbytes
        finally:
            os.close(fd)


def _expert(e):
    return R.host_expert(1, 0, e, R.table_desc())


def _oracle_expert(g, u, d, x):
    ref = np.empty(2048, np.float32)
    ex = O.OrcExpert(g, u, d, 0, 0, 1)
    O.orc().orc_expert_decode(C.byref(ex), x.ctypes.data, 512, 2048, ref.ctypes.data)
    return ref


@pytest.fixture(params=["track", "copy"])
def sync_mode(request):
    L = R.lib()
    if request.param == "track" and not L.roaster_weight_tracking(-1):
        pytest.skip("write tracking unavailable on this kernel (copy mode is tested)")
    was = L.roaster_weight_tracking(-1)
    L.roaster_weight_tracking(1 if request.param == "track" else 0)
    yield request.param
    L.roaster_weight_tracking(1 if was else 0)


def _ffn_check(slots, x, outs, fx):
    assert R.lib().kernel_ffn_fused(fx, 9, x.ctypes.data, 512, 2048) == 1
    for s, o in zip(slots, outs):
        ref = _oracle_expert(s, s + GATE_B, s + 2 * GATE_B, x)
        assert rel_err(o, ref) <= 2e-5, rel_err(o, ref)


def test_ffn_fused_sees_rewritten_slab_slots(sync_mode):
    """A 9-slot slab in kernel_vk_alloc_weights memory: slots rewritten by a
    store, by pread, and by a one-byte change between kernel_ffn_fused calls."""
    log(f"ffn_fused slab rewrite ({sync_mode})")
    L = R.lib()
    granted = C.c_size_t(0)
    slab = L.kernel_vk_alloc_weights(9 * STRIDE, C.byref(granted))
    assert slab and granted.value >= 9 * STRIDE, R.last_error()
    slots = [slab + i * STRIDE for i in range(9)]
    for s, e in zip(slots, [6, 119, 104, 200, 49, 247, 216, 123, 256]):
        g, u, d = _expert(e)
        _store(s, g)
        _store(s + GATE_B, u)
        _store(s + 2 * GATE_B, d)
    x = R.synth_normal(1, R.synth_stream(0, 0, 5), 2048)
    outs = [np.full(2048, np.nan, np.float32) for _ in range(9)]
    fx = (R.KernelFfnExpert * 9)()
    for i, (s, o) in enumerate(zip(slots, outs)):
        fx[i] = R.KernelFfnExpert(s, s + GATE_B, s + 2 * GATE_B, 0, 0, 1, o.ctypes.data)
    _ffn_check(slots, x, outs, fx)

    # cache misses: slot 2 <- expert 17 by stores, slot 5 <- expert 33 by pread
    g, u, d = _expert(17)
    _store(slots[2], g)
    _store(slots[2] + GATE_B, u)
    _store(slots[2] + 2 * GATE_B, d)
    g, u, d = _expert(33)
    _pread(slots[5], np.concatenate([g, u, d]))
    c0 = _copied()
    _ffn_check(slots, x, outs, fx)
    moved = _copied() - c0
    if sync_mode == "track":
        assert 2 * STRIDE <= moved <= 2 * STRIDE + 8 * 4096, moved
    else:
        assert moved >= 9 * STRIDE

    # nothing rewritten: tracking copies nothing
    c0 = _copied()
    _ffn_check(slots, x, outs, fx)
    if sync_mode == "track":
        assert _copied() == c0

    # one byte: a Q6_K scale in the middle of slot 7's down matrix
    before = outs[7].copy()
    p = slots[7] + 2 * GATE_B + 1000 * 210 + 195
    b = C.c_int8.from_address(p)
    b.value = 31 if b.value != 31 else -32
    _ffn_check(slots, x, outs, fx)
    assert not np.array_equal(before, outs[7])


def _moe_case(X, ns, ptrs):
    arr = (R.KernelMoeExpert * len(ns))()
    grp = (O.OrcMoeGroup * len(ns))()
    for i, (n, (g, u, d)) in enumerate(zip(ns, ptrs)):
        arr[i] = R.KernelMoeExpert(g, u, d, 0, 0, 1, n)
        grp[i] = O.OrcMoeGroup(g, u, d, 0, 0, 1, n)
    D = np.full((sum(ns), 2048), np.nan, np.float32)
    assert R.lib().kernel_moe_prefill(arr, len(ns), X.ctypes.data, D.ctypes.data, 512, 2048) == 0
    ref = np.zeros_like(D)
    O.orc().orc_moe_groups(grp, len(ns), X.ctypes.data, ref.ctypes.data, 512, 2048)
    assert rel_err(D, ref) <= 2e-4, rel_err(D, ref)


def test_moe_prefill_sees_rewritten_region(sync_mode):
    """A malloc'd slab registered with kernel_vk_register_region (the path
    weights.c takes when driver memory is unavailable): experts rewritten
    between kernel_moe_prefill calls, then the region released
    (kernel_vk_release_host_ptr) and rewritten again."""
    log(f"moe_prefill region rewrite ({sync_mode})")
    L = R.lib()
    buf = np.zeros(4 * STRIDE + 4096, np.uint8)
    base = (buf.ctypes.data + 4095) & ~4095
    assert L.kernel_vk_register_region(base, 4 * STRIDE) == 1
    slots = [base + i * STRIDE for i in range(4)]
    ptrs = [(s, s + GATE_B, s + 2 * GATE_B) for s in slots]
    for s, e in zip(slots, [3, 77, 150, 256]):
        _store(s, np.concatenate(_expert(e)))
    ns = [3, 0, 5, 2]
    X = R.synth_normal(2, 7, sum(ns) * 2048).reshape(sum(ns), 2048)
    _moe_case(X, ns, ptrs)
    _store(slots[0], np.concatenate(_expert(90)))
    _pread(slots[2], np.concatenate(_expert(91)))
    _moe_case(X, ns, ptrs)
    # release the region: later uses of these addresses are plain host ranges
    L.kernel_vk_release_host_ptr(base)
    _store(slots[3] + GATE_B, _expert(92)[1])
    _moe_case(X, ns, ptrs)
    L.kernel_vk_release_host_ptr(base)          # a second release is harmless
    _pread(slots[0], np.concatenate(_expert(93)))
    _moe_case(X, ns, ptrs)
    del buf


def test_imports_sharing_a_page_see_rewrites(sync_mode):
    """Two weight matrices adjacent in one host buffer (neither arena nor
    region memory), so that their ranges share a page: a write across the
    boundary must reach both."""
    log(f"import rewrite across a shared page ({sync_mode})")
    L = R.lib()
    A = R.synth_q4k(9, 1, 37 * 8)               # 37 rows: 42,624 B, not a page multiple
    B = R.synth_q4k(9, 2, 37 * 8)
    buf = np.concatenate([A, B])
    pa, pb = buf.ctypes.data, buf.ctypes.data + A.nbytes
    x = R.synth_normal(9, 3, 2048)
    ya = np.empty(37, np.float32)
    yb = np.empty(37, np.float32)

    def run():
        L.kernel_matvec_q4_k(pa, x.ctypes.data, ya.ctypes.data, 37, 2048)
        L.kernel_matvec_q4_k(pb, x.ctypes.data, yb.ctypes.data, 37, 2048)
        ra = O.matvec(0, np.ascontiguousarray(buf[:A.nbytes]), x, 37, 2048)
        rb = O.matvec(0, np.ascontiguousarray(buf[A.nbytes:]), x, 37, 2048)
        assert rel_err(ya, ra) <= 2e-5 and rel_err(yb, rb) <= 2e-5

    run()
    # rewrite 288 bytes straddling the boundary: the last two blocks of A's
    # last row and the first block of B's first row
    new = R.synth_q4k(9, 3, 3)
    buf[A.nbytes - 288:A.nbytes + 144] = new
    run()
    run()


def test_region_at_a_reused_address_is_tracked_again():
    """A region released by kernel_vk_release_host_ptr and unmapped, then a new
    mapping at the same address registered as a region: its writes are still
    tracked (a call with no write in between copies nothing, a store copies
    its page), and every call computes on the bytes the memory holds."""
    L = R.lib()
    if not L.roaster_weight_tracking(-1):
        pytest.skip("write tracking unavailable on this kernel")
    libc = C.CDLL(None, use_errno=True)
    libc.mmap.restype = C.c_void_p
    libc.mmap.argtypes = [C.c_void_p, C.c_size_t, C.c_int, C.c_int, C.c_int, C.c_long]
    libc.munmap.argtypes = [C.c_void_p, C.c_size_t]
    PROT_RW, MAP_PRIV_ANON, MAP_FIXED_NOREPLACE = 0x3, 0x02 | 0x20, 0x100000
    rows = 64
    A = R.synth_q4k(11, 1, rows * 8)
    B = R.synth_q4k(11, 2, rows * 8)
    N = (A.nbytes + 4095) & ~4095
    x = R.synth_normal(11, 3, 2048)
    y = np.empty(rows, np.float32)

    def check(p, data):
        L.kernel_matvec_q4_k(p, x.ctypes.data, y.ctypes.data, rows, 2048)
        ref = O.matvec(0, np.ascontiguousarray(data), x, rows, 2048)
        assert rel_err(y, ref) <= 2e-5, rel_err(y, ref)

    p1 = libc.mmap(None, N, PROT_RW, MAP_PRIV_ANON, -1, 0)
    assert p1 and p1 != C.c_void_p(-1).value
    _store(p1, A)
    assert L.kernel_vk_register_region(p1, N) == 1
    check(p1, A)
    L.kernel_vk_release_host_ptr(p1)
    assert libc.munmap(p1, N) == 0
    p2 = libc.mmap(p1, N, PROT_RW, MAP_PRIV_ANON | MAP_FIXED_NOREPLACE, -1, 0)
    if p2 != p1:
        if p2 and p2 != C.c_void_p(-1).value:
            libc.munmap(p2, N)
        pytest.skip("the address could not be mapped again")
    try:
        _store(p2, B)
        assert L.kernel_vk_register_region(p2, N) == 1
        check(p2, B)
        c0 = _copied()
        check(p2, B)
        assert _copied() == c0, "an unwritten region was copied again: its pages are not tracked"
        C2 = B.copy()
        C2[144:288] = R.synth_q4k(11, 4, 1)             # one block of row 0
        _store(p2 + 144, C2[144:288])
        check(p2, C2)
        assert 0 < _copied() - c0 <= 4096
    finally:
        L.kernel_vk_release_host_ptr(p2)
        libc.munmap(p2, N)


def _pread_direct(p, arr):
    """Write arr's bytes at the page-aligned host address p with an O_DIRECT
    pread(2), as weights.c reads experts by default (weights.c:69-74, 686):
    the kernel writes through the pages it pinned.  False where no
    directory's filesystem accepts O_DIRECT (tmpfs refuses it)."""
    n = arr.nbytes
    assert p % 4096 == 0 and n % 4096 == 0
    for d in (os.path.dirname(os.path.abspath(__file__)), "/var/tmp", tempfile.gettempdir()):
        try:
            fdw, path = tempfile.mkstemp(dir=d)
        except OSError:
            continue
        try:
            os.write(fdw, np.ascontiguousarray(arr).tobytes())
            os.fsync(fdw)
            os.close(fdw)
            try:
                fd = os.open(path, os.O_RDONLY | os.O_DIRECT)
            except OSError:
                continue
            try:
                view = memoryview((C.c_char * n).from_address(p)).cast("B")
                got = os.preadv(fd, [view], 0)
            except OSError:
                continue
            finally:
                os.close(fd)
            if got == n:
                return True
        finally:
            os.unlink(path)
    return False


def test_arena_rewritten_by_o_direct_pread(sync_mode):
    """Arena memory rewritten by an O_DIRECT pread between two matvec calls:
    the second call computes on the new bytes."""
    L = R.lib()
    rows = 64                                       # 64 x 8 Q4_K blocks: 18 pages
    A = R.synth_q4k(12, 1, rows * 8)
    B = R.synth_q4k(12, 2, rows * 8)
    p = alloc_w(A)
    x = R.synth_normal(12, 3, 2048)
    y = np.empty(rows, np.float32)

    def check(data):
        L.kernel_matvec_q4_k(p, x.ctypes.data, y.ctypes.data, rows, 2048)
        ref = O.matvec(0, np.ascontiguousarray(data), x, rows, 2048)
        assert rel_err(y, ref) <= 2e-5, rel_err(y, ref)

    check(A)
    if not _pread_direct(p, B):
        pytest.skip("O_DIRECT refused by every candidate directory's filesystem")
    check(B)
