"""CPU oracle for the MTC quantized-weight matmul path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module (or load oracle/liboracle_cpu.so); the product path never does, and
nothing here is ever used to produce a product result. It restates the
reference's algorithm in plain numpy so GPU results can be checked against it:

  function                      reference                                       pinned by
  ----------------------------  ----------------------------------------------  ---------------------------------------
  QRANGE                        mtc/core/allocation.py:44-52                    closed form (two's complement ranges)
  quantize_blocks               mtc/core/allocation.py:89-94                    brute-force scalar loop (tests)
  qt_dequant                    mtc/core/quadtree.py:157-171                    element-grid RTN formulation
                                                                                (baselines/gptq.py:119-138,
                                                                                tests/test_gptq.py:28-35); pareto KATs
  uniform_dequant               mtc/core/allocation.py:359-369 (rd_dequant)     uniform-family pareto KATs through
                                                                                the product allocator + equality (tests)
  uniform_to_array              mtc/kernels/gemm.py:510-538 (to_array of the    equals uniform_dequant as values; its
                                uniform arena: integer codes x scale)           zero signs checked by hand (tests)
  permuted_qt_dequant/unpermute mtc/core/permutation.py:70-79                   explicit index loop (tests)
  element_grid / element_rtn    mtc/baselines/gptq.py:119-138                   equality with qt_dequant
  arena_pack / arena_unpack     mtc/kernels/gemm.py:457-478, 29-117,            exhaustive P2 256-combo + round trips
                                mtc/core/packing.py:11-45                       (tests/test_packing.py:16-69)
  qt_gemm_f64                   X @ W_hat (mtc/core/permutation.py:15-18)       textbook fp64 product
  relative_frobenius_error      mtc/kernels/reference.py:31-38                  closed form
  liboracle_cpu.so (C)          loop structure of gemm.py:124-210 generalized  agreement with qt_gemm_f64
                                to quadtree leaves and a dense X

No function here is "parity unpinned".
"""

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
CPU_LIB_PATH = os.path.join(HERE, "liboracle_cpu.so")

# literal table, allocation.py:44-52
QRANGE = {2: (-2, 1), 3: (-4, 3), 4: (-8, 7), 5: (-16, 15), 6: (-32, 31), 8: (-128, 127), 16: (-32768, 32767)}


def blocks_of(W: np.ndarray, s: int) -> np.ndarray:
    K, N = W.shape
    return W.reshape(K // s, s, N // s, s).transpose(0, 2, 1, 3)


def unblock(B: np.ndarray) -> np.ndarray:
    a, b, s, _ = B.shape
    return B.transpose(0, 2, 1, 3).reshape(a * s, b * s)


def quantize_blocks(blocks: np.ndarray, mode: int, scales: np.ndarray) -> np.ndarray:
    """fp32: clip(round_half_even(blocks / s), lo, hi), dividing by 1 where s == 0."""
    lo, hi = QRANGE[mode]
    s = np.asarray(scales, dtype=np.float32)[..., None, None]
    s = np.where(s == 0, np.float32(1.0), s)
    return np.clip(np.round(np.asarray(blocks, dtype=np.float32) / s), lo, hi)


def qt_dequant(W: np.ndarray, sizes, leaf, modes, scales) -> np.ndarray:
    """W_hat: per level, q * s at the leaves, accumulated into a +0.0 buffer."""
    W = np.asarray(W, dtype=np.float32)
    out = np.zeros_like(W)
    for s in sizes:
        lvl = np.zeros_like(blocks_of(W, s))
        bl = blocks_of(W, s)
        for m in QRANGE:
            sel = np.asarray(leaf[s], bool) & (np.asarray(modes[s]) == m)
            if sel.any():
                sc = np.asarray(scales[s], np.float32)[sel]
                lvl[sel] = quantize_blocks(bl[sel], m, sc) * sc[:, None, None]
        out += unblock(lvl)
    return out


def uniform_dequant(W: np.ndarray, modes: np.ndarray, scales: np.ndarray, block_size: int) -> np.ndarray:
    """W_hat of a uniform-block allocation: q * s written per block (so -0.0 where q = 0 and
    s < 0), +0.0 at P0 blocks. Unlike qt_dequant nothing is summed into a +0.0 buffer."""
    bs = int(block_size)
    modes = np.asarray(modes)
    sc = np.asarray(scales, np.float32)
    bl = blocks_of(np.asarray(W, np.float32), bs)
    out = np.zeros_like(bl)
    for m in QRANGE:
        sel = modes == m
        if sel.any():
            out[sel] = quantize_blocks(bl[sel], m, sc[sel]) * sc[sel][:, None, None]
    return unblock(out)


def uniform_to_array(W: np.ndarray, modes: np.ndarray, scales: np.ndarray, block_size: int) -> np.ndarray:
    """The uniform-block MTCMatrix rebuilt from its arena: the integer code of each weight (the
    arena holds integers, so a weight that rounds to zero from below is the code 0) times its
    block's scale, 0 * scale at P0 blocks. Equal to uniform_dequant as values; where
    round-half-even gives -0.0 for w / s in (-0.5, 0), rd_dequant keeps -0.0 and this gives
    0 * s."""
    bs = int(block_size)
    modes = np.asarray(modes)
    sc = np.asarray(scales, np.float32)
    bl = blocks_of(np.asarray(W, np.float32), bs)
    q = np.zeros(bl.shape, np.int64)
    for m in QRANGE:
        sel = modes == m
        if sel.any():
            q[sel] = quantize_blocks(bl[sel], m, sc[sel]).astype(np.int64)
    return unblock(q.astype(np.float32) * sc[:, :, None, None])


def unpermute(Wp: np.ndarray, pr, pc) -> np.ndarray:
    out = np.empty_like(Wp)
    out[np.ix_(np.asarray(pr), np.asarray(pc))] = Wp
    return out


def permuted_qt_dequant(W: np.ndarray, pr, pc, sizes, leaf, modes, scales) -> np.ndarray:
    Wp = np.asarray(W, dtype=np.float32)[np.asarray(pr)][:, np.asarray(pc)]
    return unpermute(qt_dequant(Wp, sizes, leaf, modes, scales), pr, pc)


def element_grid(sizes, leaf, modes, scales, shape):
    """Per-element (scale, lo, hi) arrays of a quadtree allocation."""
    K, N = shape
    S = np.zeros((K, N), np.float32)
    LO = np.zeros((K, N), np.float32)
    HI = np.zeros((K, N), np.float32)
    for s in sizes:
        lf = np.asarray(leaf[s], bool)
        mm = np.asarray(modes[s])
        rep = lambda x: np.kron(x, np.ones((s, s), dtype=x.dtype))
        mask = rep(lf.astype(np.uint8)).astype(bool)
        lo = np.zeros(mm.shape, np.float32)
        hi = np.zeros(mm.shape, np.float32)
        for m, (a, b) in QRANGE.items():
            lo[mm == m], hi[mm == m] = a, b
        S[mask] = rep(np.where(lf, np.asarray(scales[s], np.float32), 0).astype(np.float32))[mask]
        LO[mask] = rep(lo)[mask]
        HI[mask] = rep(hi)[mask]
    return S, LO, HI


def element_rtn(W: np.ndarray, S: np.ndarray, LO: np.ndarray, HI: np.ndarray) -> np.ndarray:
    """Second formulation of W_hat: elementwise RTN on the per-element grid (+0.0 canonical)."""
    safe = np.where(S == 0, np.float32(1.0), S)
    return (np.clip(np.round(np.asarray(W, np.float32) / safe), LO, HI) * S) + np.float32(0.0)


# ---- reference arena codecs (uniform-block layout) -------------------------------------------
def arena_pack(codes: np.ndarray, mode: int) -> np.ndarray:
    """(n, count) row-major codes -> bytes, one block after another (gemm.py:463-476)."""
    q = np.asarray(codes, dtype=np.int64)
    n, count = q.shape
    nbytes = mode * count // 8
    out = np.zeros((n, nbytes), dtype=np.uint8)
    u = q & ((1 << mode) - 1)
    for i in range(count):
        for b in range(mode):                      # bit b of code i -> stream bit i*mode + b
            pos = i * mode + b
            out[:, pos >> 3] |= (((u[:, i] >> b) & 1) << (pos & 7)).astype(np.uint8)
    return out


def arena_unpack(data: np.ndarray, mode: int, count: int) -> np.ndarray:
    """Bytes -> codes, reading each code's bits at [i*mode, (i+1)*mode) little-endian."""
    d = np.asarray(data, dtype=np.int64)
    out = np.zeros((d.shape[0], count), dtype=np.int64)
    for i in range(count):
        v = np.zeros(d.shape[0], dtype=np.int64)
        for b in range(mode):
            pos = i * mode + b
            v |= ((d[:, pos >> 3] >> (pos & 7)) & 1) << b
        out[:, i] = np.where(v >= (1 << (mode - 1)), v - (1 << mode), v)
    return out


# ---- products and metrics -------------------------------------------------------------------------
def qt_gemm_f64(X: np.ndarray, W_hat: np.ndarray) -> np.ndarray:
    return np.asarray(X, np.float64) @ np.asarray(W_hat, np.float64)


def relative_frobenius_error(y_true, y_pred) -> float:
    t = np.asarray(y_true, np.float64)
    num = np.linalg.norm(t - np.asarray(y_pred, np.float64))
    den = np.linalg.norm(t)
    return float(num) if den < 1e-12 else float(num / den)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> nearest bf16 (ties to even), returned as fp32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16
    return u.astype(np.uint32).view(np.float32)


# ---- leaf list in the reference arena layout, for the C loop -------------------------------------
class LeafArena:
    """All non-P0 leaves of a (possibly permuted) quadtree allocation, grouped by
    32-column panel, each leaf's codes packed row-major in the reference layout."""

    def __init__(self, Wp: np.ndarray, sizes, leaf, modes, scales, row_perm=None, col_perm=None):
        Wp = np.asarray(Wp, np.float32)
        K, N = Wp.shape
        rec = []
        chunks = []
        off = 0
        for s in sizes:
            bl = blocks_of(Wp, s)
            for m in QRANGE:
                ii, jj = np.nonzero(np.asarray(leaf[s], bool) & (np.asarray(modes[s]) == m))
                if ii.size == 0:
                    continue
                sc = np.asarray(scales[s], np.float32)[ii, jj]
                q = quantize_blocks(bl[ii, jj], m, sc).astype(np.int64).reshape(ii.size, s * s)
                data = arena_pack(q, m)
                nb = data.shape[1]
                for t in range(ii.size):
                    rec.append((jj[t] * s // 32, ii[t] * s, jj[t] * s, s, m, sc[t], off + t * nb))
                chunks.append(data.reshape(-1))
                off += ii.size * nb
        rec.sort(key=lambda r: (r[0], r[1], r[2]))
        self.K, self.N = K, N
        self.arena = np.concatenate(chunks) if chunks else np.zeros(1, np.uint8)
        r = np.array([x[1:] for x in rec], dtype=np.float64).reshape(-1, 6)
        self.k0 = r[:, 0].astype(np.int32)
        self.n0 = r[:, 1].astype(np.int32)
        self.size = r[:, 2].astype(np.int32)
        self.mode = r[:, 3].astype(np.int32)
        self.scale = np.array([x[5] for x in rec], dtype=np.float32)
        self.off = np.array([x[6] for x in rec], dtype=np.int64)
        panel = np.array([x[0] for x in rec], dtype=np.int64)
        self.panel_begin = np.searchsorted(panel, np.arange(N // 32 + 1)).astype(np.int64)
        self.row_perm = None if row_perm is None else np.ascontiguousarray(row_perm, np.int32)
        self.col_perm = None if col_perm is None else np.ascontiguousarray(col_perm, np.int32)

    @property
    def n_leaves(self) -> int:
        return int(self.k0.size)


_cpu = None


def cpu_lib():
    global _cpu
    if _cpu is None:
        if not os.path.exists(CPU_LIB_PATH):
            raise FileNotFoundError(f"{CPU_LIB_PATH} not built (make -C oracle)")
        lib = ctypes.CDLL(CPU_LIB_PATH)
        vp = ctypes.c_void_p
        lib.oracle_qt_gemm.restype = ctypes.c_int
        lib.oracle_qt_gemm.argtypes = [vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp, vp, vp, vp, vp, vp, vp,
                                       vp, vp, vp, vp, ctypes.c_int]
        lib.oracle_threads.restype = ctypes.c_int
        lib.oracle_threads.argtypes = []
        _cpu = lib
    return _cpu


def cpu_qt_gemm(X: np.ndarray, la: LeafArena, n_threads: int = 0) -> np.ndarray:
    """Y = X @ W_hat by the C port of the reference block loop (OpenMP over panels)."""
    X = np.ascontiguousarray(X, np.float32)
    M, K = X.shape
    assert K == la.K
    Y = np.zeros((M, la.N), np.float32)
    p = lambda a: None if a is None else a.ctypes.data
    rc = cpu_lib().oracle_qt_gemm(p(X), M, K, la.N, p(la.arena), p(la.off), p(la.k0), p(la.n0), p(la.size),
                                  p(la.mode), p(la.scale), p(la.panel_begin), p(la.row_perm), p(la.col_perm),
                                  p(Y), None, int(n_threads))
    if rc != 0:
        raise RuntimeError(f"oracle_qt_gemm failed ({rc})")
    return Y
