# SPDX-License-Identifier: Apache-2.0
"""The C-ABI library loads and exports every function include/*.h declares
(no compute, no GPU), and the shared struct layouts are the reference's."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include")
LIB = os.path.join(ROOT, "warp_amd", "libwaste_hip.so")
SYNTH_LIB = os.path.join(ROOT, "warp_amd", "libwaste_hip_synth.so")
# The synthetic record generator's header; its library is separate.
SYNTH_H = "waste_hip_synth.h"


def declared(only=None, skip=()):
    names = []
    for f in sorted(os.listdir(INC)):
        if not f.endswith(".h") or f in skip or (only and f != only):
            continue
        src = open(os.path.join(INC, f)).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        names += re.findall(r"^[A-Za-z_][\w \*]*?\b(waste_\w+)\s*\(", src, flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB), "build first: python -m warp_amd.build"
    lib = ctypes.CDLL(LIB)
    names = declared(skip=(SYNTH_H,))
    assert len(names) >= 15
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_product_library_holds_no_generator():
    """The synthetic record generator is test and benchmark data: its
    symbols are in libwaste_hip_synth.so and not in the product."""
    lib = ctypes.CDLL(LIB)
    synth = declared(only=SYNTH_H)
    assert len(synth) == 3
    assert not [n for n in synth if hasattr(lib, n)]
    slib = ctypes.CDLL(SYNTH_LIB)
    assert not [n for n in synth if not hasattr(slib, n)]
    assert not hasattr(slib, "waste_hip_moe_forward")


def test_python_mirror_lists_every_symbol():
    import warp_amd
    from warp_amd import synth
    assert sorted(warp_amd.EXPORTS) == declared(skip=(SYNTH_H,))
    assert sorted(synth.SYNTH_EXPORTS) == declared(only=SYNTH_H)


def test_headers_compile_standalone(tmp_path):
    for h in ("waste_abi.h", "waste_hip.h"):
        src = tmp_path / "t.c"
        src.write_text(f'#include "{h}"\nint main(void){{return 0;}}\n')
        subprocess.check_call(["gcc", "-std=c11", "-Wall", "-Werror", "-I" + INC, "-c", str(src),
                               "-o", str(tmp_path / "t.o")])
        subprocess.check_call(["g++", "-std=c++17", "-Wall", "-Werror", "-x", "c++", "-I" + INC, "-c",
                               str(src), "-o", str(tmp_path / "t.o")])


REF_SRC = "/root/reference/src"


@pytest.mark.skipif(not os.path.exists(os.path.join(REF_SRC, "waste_backend.h")),
                    reason="reference headers not present")
def test_layouts_match_reference_headers(tmp_path):
    """Sizes and offsets of the shared structs, from the reference's own
    headers, against this project's declarations."""
    prog = r'''
#include <stdio.h>
#include <stddef.h>
#include "waste_backend.h"
#include "simd.h"
#include "waste_metal.h"
#include "waste_format.h"
int main(void){
 printf("%zu %zu %zu %zu %zu %zu %zu %zu %zu %zu\n", sizeof(waste_kernels),
   offsetof(waste_kernels, mvq_rows_f32), offsetof(waste_kernels, on_device),
   offsetof(waste_kernels, device_min_bytes), sizeof(mvq_arg), sizeof(lutb_arg),
   sizeof(vqp_arg), sizeof(waste_vq_job), sizeof(waste_expert_hdr), sizeof(waste_codebook_hdr));
}'''
    mine = prog.replace('#include "waste_backend.h"\n#include "simd.h"\n#include "waste_metal.h"\n#include "waste_format.h"',
                        '#include "waste_abi.h"')
    out = []
    for src, inc in ((prog, REF_SRC), (mine, INC)):
        f = tmp_path / "l.c"
        f.write_text(src)
        exe = tmp_path / "l"
        subprocess.check_call(["gcc", "-I" + inc, str(f), "-o", str(exe)])
        out.append(subprocess.check_output([str(exe)]).decode())
    assert out[0] == out[1], out


def test_empty_and_invalid_calls_fail_before_any_device_work():
    """An empty batch is an error, as in the engine's accelerator entry
    (src/metal.m:353: n <= 0 returns -1; the caller at model.c:5734 then
    falls through to its serial loop, model.c:5788-5790); a missing layer or
    T <= 0 is WASTE_HIP_EINVAL.  These
    checks come before any HIP call, so they run without a GPU."""
    lib = ctypes.CDLL(LIB)
    lib.waste_hip_vq3r.restype = ctypes.c_int
    lib.waste_hip_vq3r.argtypes = [ctypes.c_void_p, ctypes.c_int]
    assert lib.waste_hip_vq3r(None, 0) == -1
    assert lib.waste_hip_vq3r(None, -3) == -1
    f = lib.waste_hip_moe_forward
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                  ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    x = (ctypes.c_float * 8)()
    assert f(None, x, 0, 1, x, None, None, None, None) == -1
    assert f(None, x, 0, 0, x, None, None, None, None) == -1
