# SPDX-License-Identifier: Apache-2.0
"""Builds warp_amd/libwaste_hip.so in-tree: the gfx950 kernels (hipcc) and
the C host code (gcc), linked against the HIP runtime.  The synthetic record
generator (synth.hip, synth.c) links into warp_amd/libwaste_hip_synth.so
beside it: tests and the benchmark load it, the product does not.

    python -m warp_amd.build            # rebuild what changed
    python -m warp_amd.build --force    # rebuild everything

hipcc cross-compiles for gfx950 without a GPU, so this runs anywhere the
ROCm toolchain is installed.
"""
import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libwaste_hip.so")
# The synthetic record generator (tests and the benchmark's data, not the
# engine's path) is a library of its own.
SYNTH_LIB = os.path.join(PKG, "libwaste_hip_synth.so")
SYNTH_SOURCES = ("synth.hip", "synth.c")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIPCC = os.path.join(ROCM, "bin", "hipcc")
# -ffp-contract=off: every fused multiply-add in the kernels is written out;
# the bit-exact paths depend on the compiler adding none.  Packed fp32 ops
# are kept off (the compiler otherwise forms them from scalar code).
HIPFLAGS = ["--offload-arch=gfx950", "-mcode-object-version=5", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
            "-fno-gpu-flush-denormals-to-zero", "-Xclang", "-target-feature", "-Xclang",
            "-packed-fp32-ops", "-munsafe-fp-atomics", "-Wall"]
CFLAGS = ["-O2", "-std=gnu11", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter",
          "-D__HIP_PLATFORM_AMD__"]
INC = ["-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(ROCM, "include")]


def sources():
    hip = sorted(os.path.join(CSRC, "hip", f) for f in os.listdir(os.path.join(CSRC, "hip"))
                 if f.endswith(".hip"))
    c = sorted(os.path.join(CSRC, "host", f) for f in os.listdir(os.path.join(CSRC, "host"))
               if f.endswith(".c"))
    return hip, c


def headers():
    out = []
    for d in (os.path.join(CSRC, "hip"), os.path.join(CSRC, "host"), os.path.join(ROOT, "include")):
        out += [os.path.join(d, f) for f in os.listdir(d) if f.endswith(".h")]
    return out


def _stale(src, obj, deps):
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    return any(os.path.getmtime(p) > t for p in [src] + deps)


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "not a recognized feature" not in l
                    and "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError("build failed:\n" + " ".join(cmd) + "\n" + err)
    return err


def _link(lib, objs, force):
    # relinked when an object is newer or the object list changed
    listing = os.path.join(OBJ, os.path.basename(lib) + ".objs")
    want = "\n".join(objs)
    have = open(listing).read() if os.path.exists(listing) else None
    if force or have != want or not os.path.exists(lib) or \
            any(os.path.getmtime(o) > os.path.getmtime(lib) for o in objs):
        _run([HIPCC, "--offload-arch=gfx950", "-mcode-object-version=5", "-shared", "-fPIC", "-o", lib + ".tmp"] + objs +
             ["-L" + os.path.join(ROCM, "lib"), "-lamdhip64", "-lpthread"])
        os.replace(lib + ".tmp", lib)
        with open(listing, "w") as f:
            f.write(want)


def build(force=False, verbose=False):
    """Builds libwaste_hip.so (the product) and libwaste_hip_synth.so (the
    synthetic record generator); returns the product's path."""
    os.makedirs(OBJ, exist_ok=True)
    hip, c = sources()
    deps = headers()
    jobs, objs, synth = [], [], []
    for s in hip + c:
        o = os.path.join(OBJ, os.path.basename(s) + ".o")
        (synth if os.path.basename(s) in SYNTH_SOURCES else objs).append(o)
        if force or _stale(s, o, deps):
            cc = [HIPCC] + HIPFLAGS if s.endswith(".hip") else ["gcc"] + CFLAGS
            jobs.append(cc + INC + ["-c", s, "-o", o])
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        for msg in ex.map(_run, jobs):
            if verbose and msg.strip():
                print(msg)
    _link(LIB, objs, force)
    _link(SYNTH_LIB, synth, force)
    return LIB


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--force", action="store_true")
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args()
    print(build(a.force, a.verbose))


if __name__ == "__main__":
    sys.exit(main())
