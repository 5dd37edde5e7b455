"""Drop-in `MTCMatrix` and `mtc_gemm` (mtc/kernels/gemm.py) executing on MI355X.

Two weight forms share one device format (the panel stream, include/mtc_hip.h):

- quadtree (QuadtreeRD / PermutedQuadtreeRD allocations): the north-star form,
  leaves 32x32 .. 4x4, bf16 scales, optional row/column permutation folded into
  an X gather and a Y scatter;
- uniform blocks (the reference's `from_allocation` arena, gemm.py:432-488):
  one leaf level of size Bs with fp32 scales. The host arena keeps the
  reference byte layout so `arena`, `offsets`, `total_bytes_allocated` mean
  what they mean in the reference.

`mtc_gemm(X, W)` with a dense X (numpy or torch, (M, K) or (K,)) is the
north-star overload; `mtc_gemm(A, B)` with two MTCMatrix keeps the reference
semantics (gemm.py:541-574): C = A_hat @ B_hat in fp32.

All arithmetic runs in libmtc_hip.so; without a GPU these calls raise.
"""

from math import ceil
from typing import Dict, Optional, Tuple

import numpy as np

from ..core.allocation import QRANGE, quantize_blocks, rd_allocate_pair, to_blocks
from ..core.arena import MemoryArena
from ..core.permutation import PermutedQTAllocation
from ..core.precision import (_BlockErrors, block_codes, block_scale, negotiate_joint_precision,
                              select_independent_precision)
from ..core.quadtree import QTAllocation
from ..core.types import PrecisionMode
from ..packer import LAYOUT_MX, LAYOUT_V1, PanelStream, check_permutation, pack_levels, weight_codes
from ..tilestream import TileStream, pack_tiles

DECODE_MAX_M = 16             # M at or below this takes the fp32 decode kernel under compute="auto"
F32_DECODE_MAX_M = 16         # fp32 compute above this many rows runs the fp32 tile path (mtc_gemm_f32)
DECODE_X_LDS_BYTES = 64 * 1024   # on-chip budget for the gathered X rows of one vector-path decode block
DECODE_MFMA_X_LDS_BYTES = 128 * 1024   # the same for a matrix-core decode block (M tiles of 8 or 16 rows)
DECODE_LDS_BYTES = 160 * 1024    # per-block LDS of gfx950
UNIFORM_BLOCK_SIZES = (4, 8, 16, 32)   # block sizes of the uniform form the device stream holds


def _decode_mt(M: int) -> int:
    """Rows of X per decode block (larger M runs several blocks along M): 1, 2 or 4 on the
    vector path; 8 or 16 on the matrix core (the library takes 8 when a unit's 16 rows of X
    would not fit on chip)."""
    return M if M <= 2 else 4 if M <= 4 else 8 if M <= 8 else 16


def _decode_x_budget(mt: int) -> int:
    """On-chip bytes for one decode block's staged X rows."""
    return DECODE_X_LDS_BYTES if mt <= 4 else DECODE_MFMA_X_LDS_BYTES


DECODE_FILL_BLOCKS = 256      # decode blocks that fill the chip (one 16-wave block per CU)
DECODE_MIN_SPLIT_ROWS = 512   # no row chunk below this when splitting only to fill the chip
DECODE_MFMA_MAX_ROWS = 2048   # row chunks of the matrix-core layout (16 X rows of one fit on chip)


def _decode_row_cap(M: int) -> int:
    """Largest row chunk of the decode layout for M rows."""
    mt = _decode_mt(M)
    cap = min(_decode_x_budget(mt) // (4 * mt) // 32 * 32, 4096)
    return cap if mt <= 4 else min(cap, DECODE_MFMA_MAX_ROWS)


def _decode_blocks_per_unit(M: int) -> int:
    """Decode blocks per unit: one per 16-column half on the vector path, one per unit on the
    matrix core."""
    return 2 if _decode_mt(M) <= 4 else 1


def gemv_chunk_rows(K: int, N: int, M: int = 1) -> int:
    """Rows per decode work unit. The whole reduction dimension when the gathered X rows
    (M_tile x rows fp32) fit the on-chip budget, so no block needs a cross-block reduction;
    otherwise the fewest chunks that fit, of equal size (a 4864-row matrix splits 2432 +
    2432, not 4096 + 768). A matrix that needs a split anyway and has too few column panels
    to fill the chip (_decode_blocks_per_unit blocks per unit) is cut into more chunks of at
    least DECODE_MIN_SPLIT_ROWS rows."""
    cap = _decode_row_cap(M)
    rows = -(-K // 32) * 32
    n = -(-rows // cap)
    if n > 1:
        panels = max(1, N // 32)
        fill = -(-DECODE_FILL_BLOCKS // (_decode_blocks_per_unit(M) * panels))
        n = max(n, min(fill, rows // DECODE_MIN_SPLIT_ROWS))
    chunk = -(-(-(-rows // n)) // 32) * 32
    return int(max(32, min(chunk, cap)))


def _decode_lds_need(ps: PanelStream, M: int) -> int:
    """LDS bytes one decode block of this stream uses for M rows, as the library computes it
    (mtc_gemv_lds_bytes)."""
    from .._native import hip_lib
    return int(hip_lib().mtc_gemv_lds_bytes(int(ps.K), int(ps.chunk_rows), int(ps.row_perm is not None), int(M)))


# ---------------------------------------------------------------------------------------
# reference arena byte layout (gemm.py:457-478 writes it, gemm.py:29-117 reads it)
# ---------------------------------------------------------------------------------------
def arena_encode(codes: np.ndarray, mode: int) -> np.ndarray:
    """(n, Bs*Bs) row-major codes -> (n, mode*Bs*Bs/8) bytes in the reference layout."""
    q = np.asarray(codes).astype(np.int32)
    n = q.shape[0]
    if mode == 8:
        return q.astype(np.int8).view(np.uint8).reshape(n, -1)
    if mode == 16:
        return q.astype("<i2").view(np.uint8).reshape(n, -1)
    if mode in (2, 4):
        per = 8 // mode
        u = (q & ((1 << mode) - 1)).reshape(n, -1, per)
        out = np.zeros(u.shape[:2], dtype=np.int32)
        for i in range(per):
            out |= u[..., i] << (mode * i)
        return out.astype(np.uint8)
    u = (q & ((1 << mode) - 1)).astype(np.uint32)
    bits = ((u[..., None] >> np.arange(mode, dtype=np.uint32)) & 1).astype(np.uint8)
    return np.packbits(bits.reshape(n, -1), axis=1, bitorder="little")


def arena_decode(data: np.ndarray, mode: int, count: int) -> np.ndarray:
    """(n, bytes) in the reference layout -> (n, count) signed codes (row-major)."""
    b = np.asarray(data, dtype=np.uint8)
    n = b.shape[0]
    if mode == 8:
        return b.view(np.int8).astype(np.int32).reshape(n, count)
    if mode == 16:
        return np.ascontiguousarray(b).view("<i2").astype(np.int32).reshape(n, count)
    bits = np.unpackbits(b, axis=1, bitorder="little")[:, : count * mode].reshape(n, count, mode).astype(np.int32)
    v = (bits << np.arange(mode, dtype=np.int32)).sum(axis=2)
    return np.where(v >= (1 << (mode - 1)), v - (1 << mode), v).astype(np.int32)


class _Levels:
    """Leaf description handed to the packer."""

    def __init__(self, shape, sizes, leaf, modes, scales, codes_of, scale_format, row_perm=None, col_perm=None):
        self.shape = (int(shape[0]), int(shape[1]))
        self.sizes, self.leaf, self.modes, self.scales = tuple(sizes), leaf, modes, scales
        self.codes_of, self.scale_format = codes_of, scale_format
        self.row_perm, self.col_perm = row_perm, col_perm


class StoredQTAllocation:
    """What a saved quadtree matrix keeps of its allocation: the leaf grids, modes and scales
    per level (in the stored, permuted order), the permutations and the accounted bit count.
    The weights are not kept; the codes travel with the matrix."""

    def __init__(self, shape, sizes, leaf, modes, scales, total_bits, row_perm=None, col_perm=None):
        self.shape = (int(shape[0]), int(shape[1]))
        self.sizes = tuple(int(x) for x in sizes)
        self.leaf, self.modes, self.scales = leaf, modes, scales
        self.total_bits = int(total_bits)
        self.row_perm, self.col_perm = row_perm, col_perm

    @property
    def permuted(self) -> bool:
        return self.row_perm is not None


SAVE_FORMAT = 1


def _check_stored(path, K, N, sizes, leaf, modes, scales, Q, pr, pc) -> None:
    """Raise ValueError unless a saved quadtree matrix is one the packers may trust: grids of
    the right shapes, leaf grids that tile the (K, N) matrix exactly once, modes in
    {0} + the code widths, finite scales, every leaf element's code inside its mode's range,
    and permutations of range(K) / range(N)."""
    def bad(msg):
        raise ValueError(f"{path}: {msg}")

    if K <= 0 or N <= 0 or not sizes or any(S not in UNIFORM_BLOCK_SIZES or K % S or N % S for S in sizes):
        bad(f"sizes {sizes} do not tile the ({K}, {N}) matrix")
    if Q.shape != (K, N) or Q.dtype not in (np.int8, np.int16):
        bad(f"codes must be an int8/int16 ({K}, {N}) grid, got {Q.dtype} {Q.shape}")
    cover = np.zeros((K, N), np.int32)
    for S in sizes:
        g = (K // S, N // S)
        if leaf[S].shape != g or modes[S].shape != g or scales[S].shape != g:
            bad(f"level {S} grids are not {g}")
        if leaf[S].dtype != bool or modes[S].dtype != np.uint8 or scales[S].dtype != np.float32:
            bad(f"level {S} grids must be bool / uint8 / float32")
        lf = leaf[S]
        if not np.isin(modes[S][lf], (0,) + tuple(QRANGE)).all():
            bad(f"level {S} has a mode outside {{0}} + {tuple(QRANGE)}")
        if not np.isfinite(scales[S][lf]).all():
            bad(f"level {S} has a non-finite scale")
        cover += np.repeat(np.repeat(lf.astype(np.int32), S, axis=0), S, axis=1)
        el_mode = np.repeat(np.repeat(np.where(lf, modes[S], 0), S, axis=0), S, axis=1)
        for P, (lo, hi) in QRANGE.items():
            sel = el_mode == P
            if sel.any() and (Q[sel].min() < lo or Q[sel].max() > hi):
                bad(f"level {S} P{P} codes outside [{lo}, {hi}]")
    if not (cover == 1).all():
        bad("leaf grids do not cover every element exactly once")
    if (pr is None) != (pc is None):
        bad("row_perm and col_perm come together")
    if pr is not None:
        check_permutation(pr, K, "row_perm")
        check_permutation(pc, N, "col_perm")


class MTCMatrix:
    """A packed (K x N) matrix: reduction along rows, as the right operand of Y = X * W."""

    def __init__(self, shape: Tuple[int, int], block_size: int, arena: MemoryArena, offsets: np.ndarray,
                 precisions: np.ndarray, scales: np.ndarray, pointer_tensor=None):
        """Uniform-block matrix over a reference-layout arena (gemm.py:222-238)."""
        self.shape = (int(shape[0]), int(shape[1]))
        self.block_size = int(block_size)
        self.arena = arena
        self.offsets = offsets
        self.precisions = precisions
        self.scales = scales
        self.pointer_tensor = pointer_tensor
        self.allocation = None
        self._levels: Optional[_Levels] = None
        self._host: Dict[object, object] = {}
        self._dev: Dict[Tuple[str, int], object] = {}

    # ---- constructors ------------------------------------------------------------------
    @classmethod
    def from_quadtree(cls, alloc, matrix: Optional[np.ndarray] = None) -> "MTCMatrix":
        """Pack a QTAllocation / PermutedQTAllocation (matrix = the ORIGINAL W; optional)."""
        if isinstance(alloc, PermutedQTAllocation):
            inner, pr, pc = alloc.inner, np.asarray(alloc.row_perm), np.asarray(alloc.col_perm)
            if matrix is not None:
                Wp = np.asarray(matrix, dtype=np.float32)[pr][:, pc]
            else:
                Wp = inner.weights
        elif isinstance(alloc, QTAllocation):
            inner, pr, pc = alloc, None, None
            Wp = np.asarray(matrix, dtype=np.float32) if matrix is not None else alloc.weights
        else:
            raise TypeError(f"expected QTAllocation or PermutedQTAllocation, got {type(alloc).__name__}")
        if Wp is None:
            raise ValueError("the allocation carries no weights; pass the original matrix")
        if tuple(Wp.shape) != tuple(inner.shape):
            raise ValueError(f"matrix shape {Wp.shape} != allocation shape {inner.shape}")
        K, N = inner.shape
        m = cls.__new__(cls)
        m.shape = (K, N)
        m.block_size = inner.sizes[0]
        m.arena = None
        m.offsets = None
        m.precisions = None
        m.scales = None
        m.pointer_tensor = None
        m.allocation = alloc
        m._levels = _Levels((K, N), inner.sizes, inner.leaf, inner.modes, inner.scales, weight_codes(Wp), "bf16",
                            pr, pc)
        m._host, m._dev = {}, {}
        return m

    @classmethod
    def from_allocation(cls, matrix: np.ndarray, modes, scales: Optional[np.ndarray] = None,
                        block_size: Optional[int] = None) -> "MTCMatrix":
        """Reference form `from_allocation(matrix, modes, scales, block_size)` packs uniform
        blocks into the arena (gemm.py:432-488); `from_allocation(matrix, qt_alloc)` packs a
        quadtree allocation."""
        if isinstance(modes, (QTAllocation, PermutedQTAllocation)):
            return cls.from_quadtree(modes, matrix)
        if scales is None or block_size is None:
            raise TypeError("uniform form needs modes, scales and block_size")
        arr = np.asarray(matrix, dtype=np.float32)
        H, W = arr.shape
        Bs = int(block_size)
        assert H % Bs == 0 and W % Bs == 0, f"Dimensions ({H}, {W}) must be divisible by block_size {Bs}"
        blocks = to_blocks(arr, Bs)
        nbh, nbw = blocks.shape[:2]
        modes = np.asarray(modes).reshape(nbh, nbw)
        if not np.isin(modes, (0,) + tuple(QRANGE)).all():
            raise ValueError(f"modes must be in {{0}} + {tuple(QRANGE)}")
        modes = modes.astype(np.uint8)
        scales = np.asarray(scales, dtype=np.float32).reshape(nbh, nbw)
        nbytes = (modes.astype(np.int64) * Bs * Bs) // 8
        starts = np.concatenate([[0], np.cumsum(nbytes.ravel())[:-1]])
        total = int(nbytes.sum())
        arena = MemoryArena(capacity_bytes=max(total, 1))
        base = arena.allocate(total, alignment=2)
        offsets = (starts + base).astype(np.uint32).reshape(nbh, nbw)
        buf = arena.raw_buffer
        for m in QRANGE:
            sel = modes == m
            if not sel.any():
                continue
            q = quantize_blocks(blocks[sel][None], m, scales[sel][None])[0]
            packed = arena_encode(q.reshape(q.shape[0], Bs * Bs), m)
            buf[offsets[sel].astype(np.int64)[:, None] + np.arange(packed.shape[1])] = packed
        return cls((H, W), Bs, arena, offsets, modes.copy(), np.where(modes == 0, 0.0, scales).astype(np.float32))

    @classmethod
    def _from_block_modes(cls, arr: np.ndarray, Bs: int, modes: np.ndarray, scales: Optional[np.ndarray],
                          arena: Optional[MemoryArena]) -> "MTCMatrix":
        """Uniform-block matrix whose block (i, j) is quantized at modes[i, j] the way
        MicroTensor.from_array does (microtensor.py:63-160), with scales[i, j] or, where a
        scale is NaN / scales is None, the block's own symmetric max-abs scale; blocks are
        written in row-major order, P16 payloads on 2-byte boundaries."""
        H, W = arr.shape
        blocks = to_blocks(arr, Bs)
        nbh, nbw = blocks.shape[:2]
        if arena is None:
            arena = MemoryArena(capacity_bytes=max(1024 * 1024, H * W * 2))
        offsets = np.zeros((nbh, nbw), dtype=np.uint32)
        sc32 = np.zeros((nbh, nbw), dtype=np.float32)
        for bi in range(nbh):
            for bj in range(nbw):
                m = int(modes[bi, bj])
                given = None if scales is None or np.isnan(scales[bi, bj]) else float(scales[bi, bj])
                sc = block_scale(blocks[bi, bj], m, given)
                q = block_codes(blocks[bi, bj], m, sc)
                offsets[bi, bj] = arena.write_bytes(arena_encode(q.reshape(1, Bs * Bs), m),
                                                    alignment=2 if m == 16 else 1)
                sc32[bi, bj] = sc
        return cls((H, W), Bs, arena, offsets, np.asarray(modes, dtype=np.uint8).copy(), sc32)

    @classmethod
    def from_numpy(cls, matrix: np.ndarray, block_size: int = 16, precision_mode=None, epsilon: float = 0.05,
                   arena: Optional[MemoryArena] = None, use_pointer_hierarchy: bool = True) -> "MTCMatrix":
        """Uniform-block matrix with one fixed precision or per-block adaptive precision
        (gemm.py:255-328): with `precision_mode` every block uses that mode (P2, P4, P8 or
        P16) and the scale max|block| / qmax (1.0 for a block whose max is <= 1e-7); without
        it each block takes the lowest of P2/P4/P8 whose relative error is <= epsilon, else
        P16 at scale 1.0. The pointer hierarchy (`PointerTensor`) is not built here:
        `pointer_tensor` stays None whatever `use_pointer_hierarchy` says."""
        arr = np.asarray(matrix, dtype=np.float32)
        H, W = arr.shape
        Bs = int(block_size)
        assert H % Bs == 0 and W % Bs == 0, f"Dimensions ({H}, {W}) must be divisible by block_size {Bs}"
        if Bs not in UNIFORM_BLOCK_SIZES:
            raise ValueError(f"block_size {Bs} is not one of {UNIFORM_BLOCK_SIZES}")
        blocks = to_blocks(arr, Bs)
        nbh, nbw = blocks.shape[:2]
        if precision_mode is not None:
            mode = int(precision_mode)
            if mode not in (2, 4, 8, 16):
                raise ValueError(f"Unsupported precision: {PrecisionMode(mode)!r}")
            modes = np.full((nbh, nbw), mode, dtype=np.uint8)
            scales = None
        else:
            modes = np.zeros((nbh, nbw), dtype=np.uint8)
            scales = np.zeros((nbh, nbw), dtype=np.float64)
            for bi in range(nbh):
                for bj in range(nbw):
                    p, sc = select_independent_precision(blocks[bi, bj], epsilon)
                    modes[bi, bj], scales[bi, bj] = int(p), sc
        return cls._from_block_modes(arr, Bs, modes, scales, arena)

    @classmethod
    def from_numpy_joint(cls, matrix_a: np.ndarray, matrix_b: np.ndarray, block_size: int = 16,
                         target_epsilon: float = 0.05, use_pointer_hierarchy: bool = True
                         ) -> Tuple["MTCMatrix", "MTCMatrix"]:
        """A and B of C = A @ B with block modes negotiated over every interacting block pair
        (gemm.py:330-430): each of A's blocks (and B's) takes the highest mode any of its
        pairs asked for (starting from P2), then is quantized at its own max-abs scale."""
        A = np.asarray(matrix_a, dtype=np.float32)
        B = np.asarray(matrix_b, dtype=np.float32)
        M, K = A.shape
        K2, N = B.shape
        assert K == K2
        Bs = int(block_size)
        if Bs not in UNIFORM_BLOCK_SIZES:
            raise ValueError(f"block_size {Bs} is not one of {UNIFORM_BLOCK_SIZES}")
        ab, bb = to_blocks(A, Bs), to_blocks(B, Bs)
        nbm, nbk, nbn = M // Bs, K // Bs, N // Bs
        ea = [[_BlockErrors(ab[i, k]) for k in range(nbk)] for i in range(nbm)]
        eb = [[_BlockErrors(bb[k, j]) for j in range(nbn)] for k in range(nbk)]
        pa = np.full((nbm, nbk), 2, dtype=np.uint8)
        pb = np.full((nbk, nbn), 2, dtype=np.uint8)
        for k in range(nbk):
            for i in range(nbm):
                for j in range(nbn):
                    a, b = negotiate_joint_precision(ea[i][k], eb[k][j], target_epsilon, nbk)
                    pa[i, k] = max(pa[i, k], a)
                    pb[k, j] = max(pb[k, j], b)
        arena_a = MemoryArena(capacity_bytes=max(1024 * 1024, M * K * 2))
        arena_b = MemoryArena(capacity_bytes=max(1024 * 1024, K * N * 2))
        return cls._from_block_modes(A, Bs, pa, None, arena_a), cls._from_block_modes(B, Bs, pb, None, arena_b)

    @classmethod
    def from_numpy_rd_pair(cls, matrix_a: np.ndarray, matrix_b: np.ndarray, bits_per_element: float,
                           block_size: int = 16) -> Tuple["MTCMatrix", "MTCMatrix"]:
        """Joint RD allocation of C = A @ B packed into real arenas (gemm.py:490-508)."""
        a, b = rd_allocate_pair(matrix_a, matrix_b, bits_per_element, block_size)
        return (cls.from_allocation(matrix_a, a.modes, a.scales, block_size),
                cls.from_allocation(matrix_b, b.modes, b.scales, block_size))

    # ---- on-disk form ----------------------------------------------------------------------
    def save(self, path) -> None:
        """Write a quadtree matrix to one .npz of plain arrays (no pickled objects): per level
        the leaf grid, modes and scales; the permutations; the accounted bit count; and the
        code of every leaf element as one dense (K x N) int8 grid (int16 when a leaf is P16) in
        the stored order. `load` rebuilds a matrix whose streams are byte-identical to this
        one's without the allocator or the weights. (The reference keeps allocations in
        memory only; the uniform-block form is its arena and is not written here.)"""
        if self._levels is None:
            raise ValueError("save() writes quadtree matrices; a uniform-block matrix is its arena")
        lv = self._levels
        K, N = self.shape
        wide = any(bool(np.any(lv.modes[S][lv.leaf[S]] > 8)) for S in lv.sizes)
        Q = np.zeros((K, N), np.int16 if wide else np.int8)
        for S in lv.sizes:
            blocks = Q.reshape(K // S, S, N // S, S)                  # view: [bi, r, bj, c]
            for P in np.unique(lv.modes[S][lv.leaf[S]]):
                if P == 0:
                    continue
                ii, jj = np.nonzero(lv.leaf[S] & (lv.modes[S] == P))
                blocks[ii, :, jj, :] = np.asarray(lv.codes_of(S, int(P), ii, jj, lv.scales[S][ii, jj]))
        arrays = {"format": np.array([SAVE_FORMAT]), "shape": np.array([K, N]), "sizes": np.array(lv.sizes),
                  "total_bits": np.array([self.total_bits], np.int64), "codes": Q}
        for S in lv.sizes:
            arrays[f"leaf_{S}"] = np.asarray(lv.leaf[S], bool)
            arrays[f"modes_{S}"] = np.asarray(lv.modes[S], np.uint8)
            arrays[f"scales_{S}"] = np.asarray(lv.scales[S], np.float32)
        if lv.row_perm is not None:
            arrays["row_perm"] = np.asarray(lv.row_perm, np.int64)
            arrays["col_perm"] = np.asarray(lv.col_perm, np.int64)
        with open(path, "wb") as f:
            np.savez_compressed(f, **arrays)

    @classmethod
    def load(cls, path) -> "MTCMatrix":
        """Read a matrix written by `save` (plain arrays only: allow_pickle stays off)."""
        with np.load(path, allow_pickle=False) as z:
            if int(z["format"][0]) != SAVE_FORMAT:
                raise ValueError(f"{path}: format {int(z['format'][0])}, expected {SAVE_FORMAT}")
            K, N = (int(x) for x in z["shape"])
            sizes = tuple(int(x) for x in z["sizes"])
            leaf = {S: z[f"leaf_{S}"] for S in sizes}
            modes = {S: z[f"modes_{S}"] for S in sizes}
            scales = {S: z[f"scales_{S}"] for S in sizes}
            Q = z["codes"]
            pr = z["row_perm"] if "row_perm" in z.files else None
            pc = z["col_perm"] if "col_perm" in z.files else None
            total_bits = int(z["total_bits"][0])
        _check_stored(path, K, N, sizes, leaf, modes, scales, Q, pr, pc)
        views: Dict[int, np.ndarray] = {}

        def codes_of(S, P, ii, jj, sc):
            if S not in views:
                views[S] = to_blocks(Q, S)
            return views[S][ii, jj]

        m = cls.__new__(cls)
        m.shape = (K, N)
        m.block_size = sizes[0]
        m.arena = m.offsets = m.precisions = m.scales = m.pointer_tensor = None
        m.allocation = StoredQTAllocation((K, N), sizes, leaf, modes, scales, total_bits, pr, pc)
        m._levels = _Levels((K, N), sizes, leaf, modes, scales, codes_of, "bf16", pr, pc)
        m._host, m._dev = {}, {}
        return m

    # ---- reference properties ------------------------------------------------------------
    @property
    def is_quadtree(self) -> bool:
        return self.allocation is not None

    @property
    def num_blocks(self) -> Tuple[int, int]:
        if self.offsets is not None:
            return self.offsets.shape
        return (self.shape[0] // self.block_size, self.shape[1] // self.block_size)

    @property
    def total_bits(self) -> int:
        """Allocator-accounted bits: payload + per-leaf metadata (+ split flags, permutation indices)."""
        if self.is_quadtree:
            return int(self.allocation.total_bits)
        return int(self.arena.bytes_allocated * 8)

    @property
    def total_bytes_allocated(self) -> int:
        if self.arena is not None:
            return self.arena.bytes_allocated
        return int(ceil(self.total_bits / 8))

    @property
    def packed_bytes(self) -> float:
        return self.total_bits / 8.0

    @property
    def average_bits_per_element(self) -> float:
        n = self.shape[0] * self.shape[1]
        return 0.0 if n == 0 else self.total_bytes_allocated * 8.0 / n

    # ---- packing ---------------------------------------------------------------------------
    def _uniform_levels(self) -> _Levels:
        Bs = self.block_size
        buf = self.arena.raw_buffer

        def codes_of(S, P, ii, jj, sc):
            nb = P * Bs * Bs // 8
            raw = buf[self.offsets[ii, jj].astype(np.int64)[:, None] + np.arange(nb)]
            return arena_decode(raw, P, Bs * Bs).reshape(-1, Bs, Bs)

        leaf = {Bs: np.ones(self.precisions.shape, dtype=bool)}
        return _Levels(self.shape, (Bs,), leaf, {Bs: self.precisions}, {Bs: self.scales}, codes_of, "fp32")

    def panel_stream(self, chunk_rows: int, layout: int = LAYOUT_V1) -> PanelStream:
        """Host image of the decode layout cut into `chunk_rows`-row units, with the payload in
        `layout` (LAYOUT_V1: every decode kernel; LAYOUT_MX: the matrix-core decode of one X row)."""
        key = (int(chunk_rows), int(layout))
        ps = self._host.get(key)
        if ps is None:
            lv = self._levels if self._levels is not None else self._uniform_levels()
            ps = pack_levels(lv.shape, lv.sizes, lv.leaf, lv.modes, lv.scales, lv.codes_of, chunk_rows,
                             lv.scale_format, lv.row_perm, lv.col_perm, layout=layout)
            self._host[key] = ps
        return ps

    @staticmethod
    def decode_layout(M: int = 1) -> int:
        """Payload layout of the decode stream for M rows of X: the chunk-contiguous layout
        (vector decode for M <= 4, 4x4x1 matrix core above). The matrix-core layout for one row
        (LAYOUT_MX: every multiply-accumulate on the matrix core, the vector units only decode)
        is available through device_stream(layout=LAYOUT_MX); measured slower at every benchmark
        shape, whose decode blocks are bound by memory latency rather than by vector issue."""
        return LAYOUT_V1

    def decode_chunk_rows(self, M: int = 1) -> int:
        """Rows per unit of the decode layout for M rows: gemv_chunk_rows, halved
        until the largest unit's on-chip staging fits the LDS budget (host only)."""
        chunk_rows = gemv_chunk_rows(self.shape[0], self.shape[1], M)
        while chunk_rows > 32 and _decode_lds_need(self.panel_stream(chunk_rows), M) > DECODE_LDS_BYTES:
            self._host.pop((chunk_rows, LAYOUT_V1), None)
            chunk_rows = max(32, (chunk_rows // 2) // 32 * 32)
        return chunk_rows

    def device_stream(self, chunk_rows: Optional[int] = None, device=None, M: int = 1,
                      layout: Optional[int] = None):
        """Device copy of the stream cut into `chunk_rows`-row units (default: the
        decode layout for M rows, shrunk until one unit fits on chip), payload in `layout`
        (default: decode_layout(M)). Any stream serves any M; the defaults are the fast ones."""
        from ..device import DeviceStream, require_gpu
        dev = require_gpu(device)
        if chunk_rows is None:
            chunk_rows = self.decode_chunk_rows(M)
        if layout is None:
            layout = self.decode_layout(M)
        key = (str(dev), int(chunk_rows), int(layout))
        ds = self._dev.get(key)
        if ds is None:
            ds = DeviceStream(self.panel_stream(int(chunk_rows), int(layout)), dev)
            self._dev[key] = ds
        return ds

    def tile_stream(self) -> TileStream:
        """Host image of the prefill (bf16 MFMA) layout."""
        ts = self._host.get("tiles")
        if ts is None:
            lv = self._levels if self._levels is not None else self._uniform_levels()
            ts = pack_tiles(lv.shape, lv.sizes, lv.leaf, lv.modes, lv.scales, lv.codes_of, lv.scale_format,
                            lv.row_perm, lv.col_perm)
            self._host["tiles"] = ts
        return ts

    def device_tiles(self, device=None):
        """Device copy of the prefill layout."""
        from ..device import DeviceTiles, require_gpu
        dev = require_gpu(device)
        key = (str(dev), "tiles")
        dt = self._dev.get(key)
        if dt is None:
            dt = DeviceTiles(self.tile_stream(), dev)
            self._dev[key] = dt
        return dt

    def release_host_streams(self) -> None:
        """Drop host copies of packed streams (device copies stay)."""
        self._host.clear()

    def dequant_device(self, device=None):
        """W_hat as a (K, N) fp32 device tensor in the original channel order."""
        return self.device_stream(None, device).dequant()

    def to_array(self) -> np.ndarray:
        """Reconstruct the full float32 matrix (gemm.py:510-538), dequantized on the GPU."""
        return self.dequant_device().cpu().numpy()


# ---------------------------------------------------------------------------------------
# mtc_gemm
# ---------------------------------------------------------------------------------------
def _as_device_tensor(x, device):
    import torch
    if isinstance(x, torch.Tensor):
        return x.to(device) if x.device != device else x
    arr = np.asarray(x)
    if arr.dtype not in (np.float32,):
        arr = arr.astype(np.float32)
    return torch.from_numpy(np.ascontiguousarray(arr)).to(device)


def _kernel_layout(X):
    """X itself when the kernels can read it in place (row-major rows: unit column stride, a
    row stride of at least K, and for bf16 16-byte aligned rows), else a contiguous copy.
    Views the reference accepts, such as X[:, 4:] or an expanded row, then run too."""
    import torch
    K = X.shape[1]
    ok = X.stride(1) == 1 and X.stride(0) >= K
    if ok and X.dtype == torch.bfloat16:
        ok = X.stride(0) % 8 == 0 and X.data_ptr() % 16 == 0
    return X if ok else X.contiguous()


def _gemm_f32(B: "MTCMatrix", Xf, dev):
    """fp32 Y = Xf @ W_hat: the decode kernels over the panel stream up to F32_DECODE_MAX_M rows,
    the fp32 matrix-core tile path above. The tile path is faster from 16 rows on (c2: M = 16 23.0
    against 24.0 µs, M = 64 52 against 73 µs, M = 256 176 against 276 µs) but its cell
    descriptors and split-K partials move 40 MB per call at c2 M = 16 against 14 MB for the
    decode path, so the decode path keeps M <= 16."""
    M = Xf.shape[0]
    if M > F32_DECODE_MAX_M:
        if Xf.stride(0) % 4 or Xf.data_ptr() % 16:   # the tile kernel reads rows in 16-byte pieces
            Xf = Xf.contiguous()
        return B.device_tiles(dev).gemm_f32(Xf)
    return B.device_stream(None, dev, M).gemv_f32(Xf)


def mtc_gemm(A, B: MTCMatrix, *, compute: str = "auto", out_dtype=None):
    """Y = A @ W_hat.

    - A MTCMatrix (reference form): returns np.ndarray fp32 C = A_hat @ B_hat.
    - A dense (M, K) or (K,), numpy or torch: returns the same kind (device
      tensor for torch input). compute="fp32" runs the fp32 path (default for
      M <= 16: the decode kernel; above 16 rows the fp32 matrix-core tile kernel),
      compute="bf16" the bf16 MFMA kernel (default above 16 rows).
    """
    if not isinstance(B, MTCMatrix):
        raise TypeError(f"right operand must be an MTCMatrix, got {type(B).__name__}")
    import torch
    from ..device import require_gpu
    dev = require_gpu()
    if isinstance(A, MTCMatrix):
        M, K = A.shape
        K2, N = B.shape
        assert K == K2, f"Shape mismatch: {A.shape} vs {B.shape}"
        assert A.block_size == B.block_size, "Block size mismatch"
        a_hat = A.dequant_device(dev)
        return _gemm_f32(B, a_hat, dev).cpu().numpy()

    from_numpy = not isinstance(A, torch.Tensor)
    X = _as_device_tensor(A, dev)
    squeeze = X.dim() == 1
    if squeeze:
        X = X.unsqueeze(0)
    if X.dim() != 2:
        raise ValueError(f"X must be 1-D or 2-D, got shape {tuple(X.shape)}")
    M, K = X.shape
    if K != B.shape[0]:
        raise ValueError(f"Shape mismatch: X {tuple(X.shape)} vs W {B.shape}")
    if compute == "auto":
        compute = "fp32" if M <= DECODE_MAX_M else "bf16"
    if M == 0:
        Y = torch.zeros((0, B.shape[1]), dtype=out_dtype or torch.float32, device=dev)
    elif compute == "fp32":
        Xf = _kernel_layout(X.float())
        Y = _gemm_f32(B, Xf, dev)
        if out_dtype is not None and out_dtype != torch.float32:
            Y = Y.to(out_dtype)
    elif compute == "bf16":
        Xb = _kernel_layout(X if X.dtype in (torch.float32, torch.bfloat16) else X.float())
        Y = B.device_tiles(dev).gemm_bf16(Xb, out_dtype=out_dtype)
    else:
        raise ValueError(f"compute must be 'auto', 'fp32' or 'bf16', got {compute!r}")
    if squeeze:
        Y = Y.squeeze(0)
    if from_numpy:
        return Y.float().cpu().numpy()
    return Y


def mtc_gemm_group(A, Bs, *, compute: str = "auto"):
    """[A @ W_hat_i for W_i in Bs] for weights that share the input A (the q/k/v or gate/up
    projections of a decoder layer; in the reference each is its own
    LinearMTCAdaptive.forward call, mtc/nn/layers.py:150-151).

    At decode sizes (fp32 path, up to F32_DECODE_MAX_M rows) matrices whose decode streams have
    a single row chunk run MAX_GROUP at a time in one launch (mtc_gemv_f32_group); above that the
    fp32 path runs one mtc_gemm_f32 call per matrix; at prefill sizes (bf16 path)
    MAX_GROUP at a time through one launch per kernel (mtc_gemm_bf16_group). Each result
    is bit-identical to mtc_gemm(A, W_i); other members launch one matrix at a time.
    Returns a list in the order of Bs, each of the kind mtc_gemm returns.
    """
    import torch
    from .. import _abi
    from ..device import gemv_f32_group, require_gpu
    Bs = list(Bs)
    if not Bs:
        return []
    for B in Bs:
        if not isinstance(B, MTCMatrix):
            raise TypeError(f"weights must be MTCMatrix, got {type(B).__name__}")
    dev = require_gpu()
    from_numpy = not isinstance(A, torch.Tensor)
    X = _as_device_tensor(A, dev)
    squeeze = X.dim() == 1
    if squeeze:
        X = X.unsqueeze(0)
    if X.dim() != 2:
        raise ValueError(f"X must be 1-D or 2-D, got shape {tuple(X.shape)}")
    M, K = X.shape
    for B in Bs:
        if B.shape[0] != K:
            raise ValueError(f"Shape mismatch: X {tuple(X.shape)} vs W {B.shape}")
    if compute == "auto":
        compute = "fp32" if M <= DECODE_MAX_M else "bf16"
    outs = [None] * len(Bs)
    if compute == "fp32" and M > F32_DECODE_MAX_M:
        Xf = _kernel_layout(X.float())
        outs = [_gemm_f32(B, Xf, dev) for B in Bs]
        if squeeze:
            outs = [y.squeeze(0) for y in outs]
        if from_numpy:
            return [y.cpu().numpy() for y in outs]
        return outs
    if compute == "fp32" and M > 0:
        Xf = _kernel_layout(X.float())
        streams = [B.device_stream(None, dev, M) for B in Bs]
        # members that can share a launch: one row chunk, same scale format and permutation presence
        groups: Dict[Tuple[bool, bool], list] = {}
        for i, s in enumerate(streams):
            if s.host.n_chunks == 1:
                key = (s.host.leaf_scale is not None, s.host.row_perm is not None)
                groups.setdefault(key, []).append(i)
        for idx in groups.values():
            for j in range(0, len(idx), _abi.MAX_GROUP):
                part = idx[j:j + _abi.MAX_GROUP]
                for i, y in zip(part, gemv_f32_group([streams[i] for i in part], Xf)):
                    outs[i] = y
        for i, s in enumerate(streams):
            if outs[i] is None:
                outs[i] = s.gemv_f32(Xf)
        if squeeze:
            outs = [y.squeeze(0) for y in outs]
        if from_numpy:
            return [y.cpu().numpy() for y in outs]
        return outs
    if compute == "bf16" and M > 0:
        from ..device import gemm_bf16_group
        Xb = _kernel_layout(X if X.dtype in (torch.float32, torch.bfloat16) else X.float())
        tiles = [B.device_tiles(dev) for B in Bs]
        # members that can share a launch: same scale format
        groups: Dict[bool, list] = {}
        for i, t in enumerate(tiles):
            groups.setdefault(t.host.fp32_scales, []).append(i)
        for idx in groups.values():
            for j in range(0, len(idx), _abi.MAX_GROUP):
                part = idx[j:j + _abi.MAX_GROUP]
                for i, y in zip(part, gemm_bf16_group([tiles[i] for i in part], Xb)):
                    outs[i] = y
        if squeeze:
            outs = [y.squeeze(0) for y in outs]
        if from_numpy:
            return [y.float().cpu().numpy() for y in outs]
        return outs
    return [mtc_gemm(A, B, compute=compute) for B in Bs]
