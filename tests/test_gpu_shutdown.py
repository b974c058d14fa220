"""kernel_vk_shutdown (kernels.h:105; the reference calls it from
weights.c:1171) releases everything the library holds -- scratch, control
words, the decode exchange buffer, pinned and staging buffers, the weight
registry with its HBM twins, and the stream -- and a later call initialises
the library again.  Run in a child process: the teardown unmaps the weight
arenas that other tests' buffers live in, and the child's exit status shows
that nothing of the library is left behind for the HIP runtime's own
teardown at exit."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = r"""
import ctypes as C, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
import roaster_amd as R
from oracle import oracle as O
L = R.lib()
print("child: init", flush=True)
R.check(L.roaster_init())
desc = R.table_desc(2)
t = L.roaster_table_create(C.byref(desc)); assert t, R.last_error()
R.check(L.roaster_table_synth(t, 3, None))
h0 = R.synth_normal(3, R.synth_stream(0, 0, 5), 2048)

def stack():
    dh = L.roaster_dev_alloc(2048 * 4)
    R.check(L.roaster_h2d(dh, h0.ctypes.data, 2048 * 4))
    R.check(L.roaster_moe_decode_stack(t, dh, 1, 0, 2, None, C.c_float(1e-6), None, None))
    R.check(L.roaster_sync())
    h = np.empty(2048, np.float32)
    R.check(L.roaster_d2h(h.ctypes.data, dh, 2048 * 4))
    L.roaster_dev_free(dh)
    return h

W = R.synth_q4k(0, R.synth_stream(0, 0, 0), 512 * 8)
x = R.synth_normal(0, R.synth_stream(0, 0, 5), 2048)

def matvec():
    g = C.c_size_t(0)
    p = L.kernel_vk_alloc_weights(W.nbytes, C.byref(g)); assert p and g.value >= W.nbytes
    C.memmove(p, W.ctypes.data, W.nbytes)
    y = np.full(512, np.nan, np.float32)
    L.kernel_matvec_q4_k(p, x.ctypes.data, y.ctypes.data, 512, 2048)
    return y

h1, y1 = stack(), matvec()
assert np.array_equal(y1, O.matvec(0, W, x, 512, 2048)) or np.max(np.abs(y1 - O.matvec(0, W, x, 512, 2048))) <= 2e-5 * np.max(np.abs(y1))
print("child: shutdown", flush=True)
L.kernel_vk_shutdown()
L.kernel_vk_shutdown()                       # a second call is harmless
print("child: again after shutdown", flush=True)
h2, y2 = stack(), matvec()
assert np.array_equal(h1.view(np.uint32), h2.view(np.uint32))
assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
L.roaster_table_destroy(t)
L.kernel_vk_shutdown()
print("child: done", flush=True)
"""


def test_shutdown_releases_and_reinitialises():
    r = subprocess.run([sys.executable, "-c", CHILD, ROOT], capture_output=True, text=True, timeout=240)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0, r.returncode
    assert "child: done" in r.stdout
