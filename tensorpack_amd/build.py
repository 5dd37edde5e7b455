"""In-tree build of the package's native libraries.

    python -m tensorpack_amd.build            # both libraries
    python -m tensorpack_amd.build --rd-only  # host allocator search only

- lib/libmtc_rd.so  : g++ -O3 -fopenmp -ffp-contract=off (exact fp32 allocator arithmetic)
- lib/libmtc_hip.so : hipcc --offload-arch=gfx950, the kernels + C-ABI of include/mtc_hip.h

Always recompiles (it is the "does it build" check); compilation is seconds.
"""

import argparse
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_DIR = os.path.join(PKG_DIR, "lib")
INCLUDE = os.path.join(ROOT, "include")

HIP_SOURCES = ["mtc_hip.hip", "mtc_gemm.hip"]
HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    # packed fp32 VALU ops stay disabled (known to misbehave on this part)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fvisibility=hidden",
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout)
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}")
    return res.stdout


def _atomic_out(path):
    return path + ".tmp%x" % os.getpid()


def build_rd(verbose=False):
    os.makedirs(LIB_DIR, exist_ok=True)
    out = os.path.join(LIB_DIR, "libmtc_rd.so")
    tmp = _atomic_out(out)
    cxx = os.environ.get("CXX", "g++")
    _run([cxx, "-O3", "-mavx2", "-ffp-contract=off", "-fno-math-errno", "-fopenmp", "-fPIC", "-shared",
          "-std=c++17", os.path.join(CSRC, "rd_search.cpp"), "-o", tmp], verbose)
    os.replace(tmp, out)
    return out


def hipcc_path():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def build_hip(verbose=False):
    """Compiles every source to an object in parallel (each holds its own gfx950 code
    object; no device code crosses sources), then links the shared library."""
    os.makedirs(LIB_DIR, exist_ok=True)
    out = os.path.join(LIB_DIR, "libmtc_hip.so")
    tmp = _atomic_out(out)
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    objs, procs = [], []
    for s in HIP_SOURCES:
        obj = os.path.join(LIB_DIR, os.path.splitext(s)[0] + ".o.tmp%x" % os.getpid())
        cmd = [hipcc_path()] + compile_flags + ["-I", INCLUDE, "-I", CSRC, "-c", os.path.join(CSRC, s), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
        objs.append(obj)
    try:
        for cmd, p in procs:
            log, _ = p.communicate()
            if p.returncode != 0:
                sys.stderr.write(log)
                raise RuntimeError(f"build step failed ({p.returncode}): {' '.join(cmd)}")
        _run([hipcc_path(), "--offload-arch=gfx950", "-fPIC", "-shared"] + objs + ["-o", tmp], verbose)
    finally:
        for o in objs:
            if os.path.exists(o):
                os.remove(o)
    os.replace(tmp, out)
    return out


def build(verbose=False, rd_only=False):
    outs = [build_rd(verbose)]
    if not rd_only:
        outs.append(build_hip(verbose))
    return outs


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--rd-only", action="store_true")
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args()
    for p in build(a.verbose, a.rd_only):
        print("built", p)
