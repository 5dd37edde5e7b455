"""Loader for the two native libraries of the package.

- ``libmtc_rd.so``  : host-only C++ (OpenMP) scale search of the offline
  allocator. Needed to build allocations; never touches a GPU.
- ``libmtc_hip.so`` : the gfx950 HIP kernels behind the C-ABI declared in
  ``include/mtc_hip.h``. Every GPU compute call of the package goes through it;
  there is no CPU fallback, so a missing library is a hard error.

Both are built in-tree into ``tensorpack_amd/lib/`` by ``tensorpack_amd.build``.
"""

import ctypes
import os
import threading

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib")
RD_LIB_PATH = os.path.join(LIB_DIR, "libmtc_rd.so")
HIP_LIB_PATH = os.path.join(LIB_DIR, "libmtc_hip.so")

_lock = threading.Lock()
_rd = None
_hip = None

c_f32p = ctypes.POINTER(ctypes.c_float)
c_f64p = ctypes.POINTER(ctypes.c_double)
vp = ctypes.c_void_p


class NativeLibraryMissing(RuntimeError):
    pass


def _load(path: str) -> ctypes.CDLL:
    if not os.path.exists(path):
        raise NativeLibraryMissing(
            f"{os.path.basename(path)} is not built ({path}); run "
            "`python -m tensorpack_amd.build` (or __graft_entry__.build()) first")
    return ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)


def rd_lib() -> ctypes.CDLL:
    global _rd
    with _lock:
        if _rd is None:
            lib = _load(RD_LIB_PATH)
            lib.mtc_rd_search.restype = ctypes.c_int
            lib.mtc_rd_search.argtypes = [
                c_f32p, c_f64p, c_f32p, ctypes.c_int64, ctypes.c_int,
                ctypes.c_double, ctypes.c_double, ctypes.c_double,
                c_f32p, ctypes.c_int, c_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                c_f64p, c_f32p]
            lib.mtc_round_sig8.restype = None
            lib.mtc_round_sig8.argtypes = [c_f32p, c_f32p, ctypes.c_int64]
            _rd = lib
        return _rd


def hip_lib() -> ctypes.CDLL:
    global _hip
    with _lock:
        if _hip is None:
            lib = _load(HIP_LIB_PATH)
            from . import _abi
            _abi.declare(lib)
            ver = lib.mtc_abi_version()
            if ver != _abi.ABI_VERSION:
                raise RuntimeError(f"libmtc_hip.so ABI {ver} != expected {_abi.ABI_VERSION}; rebuild")
            _hip = lib
        return _hip


def ptr(a, ctype):
    """ctypes pointer to the data of a contiguous numpy array."""
    return a.ctypes.data_as(ctype)
