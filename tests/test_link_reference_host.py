"""CPU proof that the reference's host program builds against this library unchanged.

The reference links `roaster` from twelve C files (CMakeLists.txt:42-55); every one
but kernels.c calls the kernel API only through src/kernels.h.  These tests compile
the other eleven from where they lie, with include/kernels.h in place of the
reference header, and link them against libroaster_moe.so with --no-undefined: if a
name, a signature the callers use, or a symbol were missing, compiling or linking
fails.  They also check that include/kernels.h declares every function with exactly
the reference's prototype (a redeclaration with another type is a C error) and that
the four structs have the reference's size, field offsets and field sizes.

The reference sources are read from /root/reference and streamed into the compiler
(no copy is written); the tests skip where that tree is absent.  Output goes to
pytest's temporary directory only.
"""
import os
import re
import shutil
import subprocess

import pytest

import roaster_amd as R

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include")
REF_SRC = "/root/reference/src"
# CMakeLists.txt:42-55 without kernels.c, which this library replaces
HOST_SOURCES = ["main", "tokenizer", "weights", "model", "state", "slots", "server", "client", "api",
                "kvspill", "kvwindow"]
STRUCTS = {
    "KernelMatvecJob": ["is_q6", "matrix", "vector", "output", "rows", "cols"],
    "KernelMatmulJob": ["is_q6", "matrix", "X", "Y", "rows", "cols", "T"],
    "KernelMoeExpert": ["gate", "up", "down", "gate_q6", "up_q6", "down_q6", "n"],
    "KernelFfnExpert": ["gate", "up", "down", "gate_q6", "up_q6", "down_q6", "out"],
}

need_gcc = pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
need_ref = pytest.mark.skipif(not os.path.isfile(os.path.join(REF_SRC, "model.c")),
                              reason="reference tree not present")
need_lib = pytest.mark.skipif(not os.path.isfile(R.LIB_PATH), reason="libroaster_moe.so not built")


def _gcc(args, stdin=None, cwd=None):
    p = subprocess.run(["gcc"] + args, input=stdin, cwd=cwd, capture_output=True, text=True)
    assert p.returncode == 0, p.stderr[-4000:]
    return p


@need_gcc
@need_ref
@need_lib
def test_reference_host_sources_link_against_library(tmp_path):
    objs = []
    for name in HOST_SOURCES:
        with open(os.path.join(REF_SRC, name + ".c")) as f:
            text = f.read()
        obj = str(tmp_path / (name + ".o"))
        # the text comes in on stdin, so a quoted "kernels.h" is searched for in
        # -I include first, never next to the source; -H lists the headers used
        p = _gcc(["-x", "c", "-std=gnu11", "-O1", "-fopenmp", "-H", "-w",
                  "-Werror=implicit-function-declaration", "-Werror=incompatible-pointer-types",
                  "-Werror=int-conversion", "-I", INC, "-I", REF_SRC, "-c", "-o", obj, "-"],
                 stdin=text, cwd=str(tmp_path))
        used = [ln.lstrip(". ").strip() for ln in p.stderr.splitlines() if ln.startswith(".")]
        kh = [u for u in used if os.path.basename(u) == "kernels.h"]
        assert all(os.path.dirname(os.path.abspath(u)) == INC for u in kh), (name, kh)
        objs.append(obj)
    exe = str(tmp_path / "roaster")
    libdir = os.path.dirname(R.LIB_PATH)
    _gcc(["-o", exe] + objs + ["-L", libdir, "-lroaster_moe", "-Wl,-rpath," + libdir, "-Wl,--no-undefined",
                               "-fopenmp", "-lm", "-lpthread"])
    assert os.path.getsize(exe) > 0
    # every kernels.h name the callers reference is resolved by the library
    nm = subprocess.run(["nm", "-u", exe], capture_output=True, text=True).stdout
    undefined = set(re.findall(r"\b(kernel_[A-Za-z0-9_]+)\b", nm))
    exported = subprocess.run(["nm", "-D", "--defined-only", R.LIB_PATH], capture_output=True, text=True).stdout
    assert undefined and undefined <= set(re.findall(r"\b(kernel_[A-Za-z0-9_]+)\b", exported))


def _prototypes(header):
    src = open(header).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    src = re.sub(r"typedef\s+struct\s*\{.*?\}\s*\w+\s*;", "", src, flags=re.S)
    src = "\n".join(ln for ln in src.splitlines() if not ln.strip().startswith("#")
                    and ln.strip() not in ('extern "C" {', "}"))
    protos = [p.strip() + ";" for p in src.split(";") if re.search(r"\bkernel_\w+\s*\(", p)]
    return [re.sub(r"\s+", " ", p) for p in protos]


@need_gcc
@need_ref
def test_prototypes_identical_to_reference_header(tmp_path):
    protos = _prototypes(os.path.join(INC, "kernels.h"))
    ref_protos = _prototypes(os.path.join(REF_SRC, "kernels.h"))
    names = lambda ps: {re.search(r"\b(kernel_\w+)\s*\(", p).group(1) for p in ps}
    assert names(protos) == names(ref_protos)
    # the reference header, then every prototype of ours: any difference in a
    # return or parameter type is a "conflicting types" error
    tu = '#include "%s"\n%s\n' % (os.path.join(REF_SRC, "kernels.h"), "\n".join(protos))
    _gcc(["-x", "c", "-std=c11", "-Wall", "-Werror", "-fsyntax-only", "-"], stdin=tu, cwd=str(tmp_path))


def _layout_program():
    lines = ["#include <stddef.h>", "#include <stdio.h>", '#include "kernels.h"', "int main(void) {"]
    for s, fields in STRUCTS.items():
        lines.append('printf("%s %%zu %%zu\\n", sizeof(%s), _Alignof(%s));' % (s, s, s))
        for f in fields:
            lines.append('printf("%s.%s %%zu %%zu\\n", offsetof(%s, %s), sizeof(((%s *)0)->%s));'
                         % (s, f, s, f, s, f))
    lines += ["return 0;", "}"]
    return "\n".join(lines) + "\n"


def _layout(tmp_path, incdir, tag):
    exe = str(tmp_path / ("layout_" + tag))
    _gcc(["-x", "c", "-std=c11", "-I", incdir, "-o", exe, "-"], stdin=_layout_program(), cwd=str(tmp_path))
    return subprocess.run([exe], capture_output=True, text=True, check=True).stdout


@need_gcc
def test_struct_layouts_static_asserts(tmp_path):
    # x86-64 LP64 layouts (reference kernels.h:34-92), fixed in C at compile time
    tu = """#include <stddef.h>
#include "kernels.h"
_Static_assert(sizeof(KernelMatvecJob) == 48, "KernelMatvecJob");
_Static_assert(offsetof(KernelMatvecJob, matrix) == 8 && offsetof(KernelMatvecJob, cols) == 40, "KernelMatvecJob");
_Static_assert(sizeof(KernelMatmulJob) == 56, "KernelMatmulJob");
_Static_assert(offsetof(KernelMatmulJob, X) == 16 && offsetof(KernelMatmulJob, T) == 48, "KernelMatmulJob");
_Static_assert(sizeof(KernelMoeExpert) == 48, "KernelMoeExpert");
_Static_assert(offsetof(KernelMoeExpert, gate_q6) == 24 && offsetof(KernelMoeExpert, n) == 40, "KernelMoeExpert");
_Static_assert(sizeof(KernelFfnExpert) == 48, "KernelFfnExpert");
_Static_assert(offsetof(KernelFfnExpert, down_q6) == 32 && offsetof(KernelFfnExpert, out) == 40, "KernelFfnExpert");
"""
    _gcc(["-x", "c", "-std=c11", "-I", INC, "-fsyntax-only", "-"], stdin=tu, cwd=str(tmp_path))
    # and the ctypes mirrors the tests use agree with the C header
    got = _layout(tmp_path, INC, "ours")
    for s, fields in STRUCTS.items():
        cls = getattr(R, s)
        vals = dict(ln.split(" ", 1) for ln in got.splitlines())
        assert int(vals[s].split()[0]) == __import__("ctypes").sizeof(cls), s
        for f in fields:
            assert int(vals[s + "." + f].split()[0]) == getattr(cls, f).offset, (s, f)


@need_gcc
@need_ref
def test_struct_layouts_equal_reference_header(tmp_path):
    assert _layout(tmp_path, INC, "ours") == _layout(tmp_path, REF_SRC, "ref")
