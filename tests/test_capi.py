"""CPU checks of the C ABI: libroaster_moe.so loads and exports every function
include/*.h declares, and the host side of the synthetic-input generator
behaves as specified (no device calls here)."""
import ctypes as C
import glob
import os
import re

import numpy as np

import roaster_amd as R
from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        for m in re.finditer(r"\b((?:kernel|roaster)_[A-Za-z0-9_]+)\s*\(", src):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    names = declared_functions()
    assert len(names) >= 45
    lib = C.CDLL(R.LIB_PATH)
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding declares a signature for each of them
    assert names <= set(R._SIG), sorted(names - set(R._SIG))


def test_synth_deterministic_and_distributed():
    a = R.synth_q4k(9, R.synth_stream(3, 7, 0), 2000)
    b = R.synth_q4k(9, R.synth_stream(3, 7, 0), 2000)
    c = R.synth_q4k(9, R.synth_stream(3, 8, 0), 2000)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    blk = a.reshape(2000, 144)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float32).ravel()
    dm = blk[:, 2:4].copy().view(np.float16).astype(np.float32).ravel()
    for v in (d, dm):
        assert v.min() >= 1e-3 * (1 - 1e-3) and v.max() <= 2e-2 * (1 + 1e-3)
        assert abs(v.mean() - 0.0105) < 0.001
    # 6-bit scales / mins and 4-bit quants are uniform
    scs = np.empty(8, np.int32)
    mns = np.empty(8, np.int32)
    allsc = []
    for i in range(500):
        O.orc().orc_q4k_scales(blk[i].ctypes.data, scs.ctypes.data, mns.ctypes.data)
        allsc += list(scs) + list(mns)
    allsc = np.array(allsc)
    assert allsc.min() == 0 and allsc.max() == 63 and abs(allsc.mean() - 31.5) < 1.0
    q = blk[:, 16:]
    nib = np.concatenate([q & 15, q >> 4]).ravel()
    assert abs(nib.mean() - 7.5) < 0.05
    w6 = R.synth_q6k(9, 1, 2000).reshape(2000, 210)
    s6 = w6[:, 192:208].view(np.int8)
    assert s6.min() == -32 and s6.max() == 31
    d6 = w6[:, 208:210].copy().view(np.float16).astype(np.float32)
    assert d6.min() >= 1e-3 * (1 - 1e-3) and d6.max() <= 1e-2 * (1 + 1e-3)


def test_synth_normal_moments():
    x = R.synth_normal(1, 5, 200000, 0.02)
    assert abs(x.mean()) < 2e-4 and abs(x.std() - 0.02) < 2e-4
    y = R.synth_normal(1, 5, 10)
    assert np.array_equal(y, R.synth_normal(1, 5, 10))
