"""Build the gfx950 C-ABI library in-tree: burn-rocket_amd/lib/libburn_rocket_amd.so.

    python burn-rocket_amd/build.py [-j N] [--save-temps DIR]

Each HIP source is compiled with hipcc for gfx950 only, then linked into one
shared library next to the Python binding. Objects go to burn-rocket_amd/_build/.
"""
import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libburn_rocket_amd.so")
SOURCES = ["gemm_f16.hip", "gemm_i8.hip", "misc.hip", "norm.hip", "attention.hip", "moe.hip", "noalloc.hip",
           "engine.cpp", "stage.cpp"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# Packed FP32 instructions stay off: the compiler may not emit v_pk_*_f32.
CFLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def _compile(src, extra):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *CFLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    p = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns about the device-only feature flag; drop that noise.
    noise = ("packed-fp32-ops", "is not a recognized feature")
    err = "\n".join(l for l in p.stderr.splitlines() if not any(n in l for n in noise))
    return src, obj, p.returncode, err


def build(jobs=8, save_temps=None, verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    extra = []
    if save_temps:
        os.makedirs(save_temps, exist_ok=True)
        extra = ["-save-temps=obj"]
    objs = []
    failed = []
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        for src, obj, rc, err in ex.map(lambda s: _compile(s, extra), SOURCES):
            if err.strip() and (verbose or rc != 0):
                print(f"[{src}]\n{err}", file=sys.stderr)
            if rc != 0:
                failed.append(src)
            objs.append(obj)
    if failed:
        raise RuntimeError(f"hipcc failed for {failed}")
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"link failed:\n{p.stderr}")
    os.replace(tmp, LIB)
    return LIB


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("--save-temps", default=None)
    ap.add_argument("-v", action="store_true")
    a = ap.parse_args()
    print(build(a.j, a.save_temps, a.v))


if __name__ == "__main__":
    main()
