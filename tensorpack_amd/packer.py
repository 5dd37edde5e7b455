"""Packer: quadtree (or uniform-block) allocation -> device "panel stream".

Replaces the reference's arena packer (mtc/kernels/gemm.py:432-488,
MTCMatrix.from_allocation) for quadtree leaves. The byte layout is defined in
include/mtc_hip.h; in short:

- work unit = (panel of 32 output columns, chunk of `chunk_rows` reduction rows);
  a panel is 8 column groups (cg) of 4 columns
- a lane chunk is 32 codes that all land in ONE column group: 4 columns x 8
  rows of a leaf of size 8/16/32, or two 4x4 leaves of one column group
- inside a unit, chunks are grouped by cg, then bucketed by (leaf size S,
  code width P), S = 32, 16, 8, 4 then P ascending, leaves by row, then row block
- each bucket is P dwords per chunk, 16-byte aligned
- one 32-bit word per leaf (row/4, pad flag, bf16 scale), stored once and shared
  by every column group the leaf covers; P0 leaves are not stored at all

Codes are computed exactly as the reference quantizer does
(clip(round_half_even(w / s)), fp32 division; allocation.py:89-94), so the
device dequantization q * s reproduces W_hat bit for bit.
"""

from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional, Sequence, Tuple

import numpy as np

from .core.allocation import quantize_blocks, to_blocks

PANEL = 32
GROUP = 4                              # columns per column group
N_GROUPS = PANEL // GROUP              # 8
LEAF_SIZES = (32, 16, 8, 4)
CODE_WIDTHS = (2, 3, 4, 5, 6, 8, 16)
LEAF_PAD = 1 << 13
ROW_BITS = 10                          # leaf word: row/4 in bits 0-9
MAX_CHUNK_ROWS = 4 << ROW_BITS         # 4096
UNIT_HDR_WORDS = 32
STREAM_FORMAT = 10                     # panel stream layout version (the C-ABI version that introduced it)
PAYLOAD_PAD = 4                        # dwords after the last bucket
STEP_GROUPS = 4                        # column groups one decode step covers
STEP_LANES = 16                        # lanes (chunks) per column group in a step
STEP_WORDS = 8                         # words per step record: (slot word, kind-and-counts word) x 4
MAX_FIXED_STEPS = 48                   # records per block stored at block-computable positions
BLOCKS_PER_UNIT = 2                    # decode blocks (of STEP_GROUPS column groups) per unit
_NULL_KEY = 3 | (2 << 8)               # kind of a record with no chunks (any valid kind)
SLOT_OFFSET_LIMIT = 1 << 16            # step payload offset / 4 and first leaf, relative to the unit
_LOG2 = {32: 5, 16: 4, 8: 3, 4: 2}
MAX_DEVICE_ARRAY_BYTES = 0x7FFFFFFF    # the kernels address every stream array with 32-bit byte offsets


def check_permutation(p, n: int, name: str) -> None:
    """Raise ValueError unless p is an integer array holding each of 0 .. n-1 exactly once
    (permutations index device memory directly: anything else reads or writes out of bounds)."""
    a = np.asarray(p)
    if a.shape != (n,) or not np.issubdtype(a.dtype, np.integer):
        raise ValueError(f"{name} must be an integer array of shape ({n},), got {a.dtype} {a.shape}")
    if n and (a.min() < 0 or a.max() >= n or np.bincount(a.astype(np.int64), minlength=n).max() != 1):
        raise ValueError(f"{name} is not a permutation of range({n})")

CodeSource = Callable[[int, int, np.ndarray, np.ndarray, np.ndarray], np.ndarray]


@dataclass
class PanelStream:
    """Host image of a panel stream (uploaded as-is by tensorpack_amd.device)."""
    K: int
    N: int
    chunk_rows: int
    payload: np.ndarray                 # uint32
    buckets: np.ndarray                 # uint32 (n_buckets, 4)
    unit_hdr: np.ndarray                # int32 (n_units, 32)
    leaf_word: np.ndarray               # uint32
    leaf_scale: Optional[np.ndarray]    # float32 or None (bf16 scales in leaf_word)
    steps: Optional[np.ndarray] = None  # uint32 (n_records, 16): decode step records
    fixed_steps: int = 0                # records per decode block at fixed positions (0, 16, 32, 48)
    row_perm: Optional[np.ndarray] = None   # int32 or None
    col_perm: Optional[np.ndarray] = None   # int32 or None
    n_real_leaves: int = 0
    max_unit_words: int = 0             # decode block of 2 column groups, max staged dwords
    max_unit_words4: int = 0            # decode block of 4 column groups
    stats: Dict[str, float] = field(default_factory=dict)
    layout: int = 0                     # LAYOUT_V1 or LAYOUT_MX (payload order; see mx_pack)

    @property
    def n_panels(self) -> int:
        return self.N // PANEL

    @property
    def n_chunks(self) -> int:
        return -(-self.K // self.chunk_rows)

    @property
    def n_units(self) -> int:
        return self.n_panels * self.n_chunks

    @property
    def n_buckets(self) -> int:
        return int(self.unit_hdr[-1, 5]) if self.n_units else 0

    @property
    def fp32_scales(self) -> bool:
        return self.leaf_scale is not None

    def nbytes(self) -> int:
        """Device bytes of the stream (payload + tables + permutations)."""
        n = self.payload.nbytes + 16 * self.n_buckets + self.unit_hdr.nbytes + self.leaf_word.nbytes
        for a in (self.leaf_scale, self.row_perm, self.col_perm, self.steps):
            if a is not None:
                n += a.nbytes
        return int(n)

    # ---- on-disk form: one .npz of plain arrays (no pickled objects) ----
    _ARRAYS = ("payload", "buckets", "unit_hdr", "leaf_word", "leaf_scale", "row_perm", "col_perm", "steps")

    def save(self, path) -> None:
        arrays = {k: getattr(self, k) for k in self._ARRAYS if getattr(self, k) is not None}
        meta = np.array([STREAM_FORMAT, self.K, self.N, self.chunk_rows, self.n_real_leaves,
                         self.max_unit_words, self.max_unit_words4, self.fixed_steps, self.layout], dtype=np.int64)
        np.savez(path, meta=meta, stats_keys=np.array(sorted(self.stats), dtype=str),
                 stats_vals=np.array([self.stats[k] for k in sorted(self.stats)], dtype=np.float64), **arrays)

    @classmethod
    def load(cls, path) -> "PanelStream":
        """Read a stream written by `save` and check it with `validate` (a file is not trusted:
        its offsets and permutations become device addresses)."""
        with np.load(path, allow_pickle=False) as z:
            meta = [int(x) for x in z["meta"]]
            if meta[0] != STREAM_FORMAT:
                raise ValueError(f"{path}: panel stream format {meta[0]}, this library reads {STREAM_FORMAT}")
            get = lambda k: np.array(z[k]) if k in z.files else None
            stats = dict(zip([str(k) for k in z["stats_keys"]], [float(v) for v in z["stats_vals"]]))
            ps = cls(K=meta[1], N=meta[2], chunk_rows=meta[3], payload=get("payload"), buckets=get("buckets"),
                     unit_hdr=get("unit_hdr"), leaf_word=get("leaf_word"), leaf_scale=get("leaf_scale"),
                     steps=get("steps"), row_perm=get("row_perm"), col_perm=get("col_perm"), n_real_leaves=meta[4],
                     max_unit_words=meta[5], max_unit_words4=meta[6], fixed_steps=meta[7], stats=stats,
                     layout=meta[8])
        ps.validate()
        return ps

    def validate(self) -> None:
        """Raise ValueError unless every index the kernels follow stays inside its array:
        unit header ranges, bucket payload and leaf ranges, leaf rows within the unit's rows,
        permutations of range(K) / range(N), array sizes the 32-bit device offsets reach."""
        K, N, kc = int(self.K), int(self.N), int(self.chunk_rows)

        def bad(msg):
            raise ValueError(f"panel stream: {msg}")

        if K <= 0 or N <= 0 or N % PANEL or K % 8:
            bad(f"shape ({K}, {N}) (N must be a multiple of {PANEL}, K of 8)")
        if kc % 32 or not 32 <= kc <= MAX_CHUNK_ROWS:
            bad(f"chunk_rows={kc}")
        if self.layout not in (LAYOUT_V1, LAYOUT_MX):
            bad(f"layout={self.layout}")
        mx = self.layout == LAYOUT_MX
        arrays = {"payload": (self.payload, np.uint32), "leaf_word": (self.leaf_word, np.uint32),
                  "unit_hdr": (self.unit_hdr, np.int32), "buckets": (self.buckets, np.uint32)}
        for name, (a, dt) in arrays.items():
            if not isinstance(a, np.ndarray) or a.dtype != dt:
                bad(f"{name} must be a {np.dtype(dt).name} array")
        n_units = self.n_units
        if self.unit_hdr.shape != (n_units, UNIT_HDR_WORDS) or self.buckets.ndim != 2 or self.buckets.shape[1] != 4:
            bad("unit_hdr / buckets shape")
        for name, a in (("payload", self.payload), ("leaf_word", self.leaf_word)):
            if a.ndim != 1 or a.size * 4 > MAX_DEVICE_ARRAY_BYTES:
                bad(f"{name} of {a.size} words (at most {MAX_DEVICE_ARRAY_BYTES // 4})")
        if self.leaf_scale is not None and (self.leaf_scale.dtype != np.float32 or self.leaf_scale.shape != self.leaf_word.shape):
            bad("leaf_scale must be float32 with one scale per leaf word")
        for name, p, n in (("row_perm", self.row_perm, K), ("col_perm", self.col_perm, N)):
            if p is not None:
                check_permutation(p, n, name)
        if (self.row_perm is None) != (self.col_perm is None):
            bad("row_perm and col_perm come together")
        h = self.unit_hdr.astype(np.int64)
        nb = self.buckets.shape[0]
        if (h[:, 0] < 0).any() or (h[:, 0] % 4).any() or (h[:, 1] < h[:, 0]).any() or \
                (h[:, 1] > self.payload.size - PAYLOAD_PAD).any():
            bad("unit payload ranges")
        if (h[:, 2] < 0).any() or (h[:, 3] < h[:, 2]).any() or (h[:, 3] > self.leaf_word.size).any():
            bad("unit leaf-word ranges")
        if (h[:, 4] < 0).any() or (h[:, 5] < h[:, 4]).any() or (h[:, 5] > nb).any() or \
                (h[:, 8] != 0).any() or (np.diff(h[:, 8:17], axis=1) < 0).any() or (h[:, 16] != h[:, 5] - h[:, 4]).any():
            bad("unit bucket ranges")
        if nb:
            unit = np.repeat(np.arange(n_units), (h[:, 5] - h[:, 4]))
            if unit.size != nb:
                bad("buckets not covered exactly once by the unit headers")
            b = self.buckets.astype(np.int64)
            ls, P = b[:, 3] & 0xFF, b[:, 3] >> 8
            if not np.isin(ls, (2, 3, 4, 5)).all() or not np.isin(P, CODE_WIDTHS).all():
                bad("bucket kind")
            n = b[:, 2] & 0xFFFF
            S = np.left_shift(1, ls)
            n_pay = ((n + 3) // 4) * 4 if mx else n                 # mx: whole quads of chunks
            if (b[:, 0] % 4).any() or (h[unit, 0] + b[:, 0] + n_pay * P > h[unit, 1]).any():
                bad("bucket payload outside its unit")
            n_leaf = np.where(S == 4, 2 * n, -(-n * 8 // np.maximum(S, 8)))
            first = h[unit, 2] + b[:, 1]
            if (b[:, 1] < 0).any() or (first + n_leaf > h[unit, 3]).any():
                bad("bucket leaf words outside its unit")
            # every leaf of a bucket: its rows lie inside the unit's rows
            idx = np.repeat(first - np.cumsum(n_leaf) + n_leaf, n_leaf) + np.arange(int(n_leaf.sum()))
            size = np.repeat(S, n_leaf)
            kb = np.repeat((unit % self.n_chunks) * kc, n_leaf)
            w = self.leaf_word[idx].astype(np.int64)
            row = (w & ((1 << ROW_BITS) - 1)) * 4
            real = (w & LEAF_PAD) == 0
            if (real & (row + size > np.minimum(kc, K - kb))).any():
                bad("leaf rows outside their unit")
        if self.steps is not None:
            blocks = n_units * BLOCKS_PER_UNIT
            if self.steps.ndim != 2 or self.steps.shape[1] != STEP_WORDS or \
                    self.steps.shape[0] < blocks * int(self.fixed_steps) + 1 or self.steps.size * 4 > MAX_DEVICE_ARRAY_BYTES:
                bad("step records shape")
            kc = self.steps[:, 1::2].astype(np.int64)
            ls, P = kc[:, 0] & 7, (kc[:, 0] >> 3) & 31
            counts = (kc[:, :1] >> (8 + 5 * np.arange(4))) & 31
            if np.any(kc != kc[:, :1]) or np.any((ls < 2) | (ls > 5)) or \
                    np.any(~np.isin(P, CODE_WIDTHS)) or np.any(counts > STEP_LANES):
                bad("step record kind or chunk counts")
            self._validate_records(h, blocks, ls, P, counts, bad)
        elif nb:
            bad("step records missing")
        if self.fixed_steps not in (0, 16, 32, 48):
            bad(f"fixed_steps={self.fixed_steps}")

    def _validate_records(self, h, blocks, ls, P, counts, bad) -> None:
        """Step records against the unit headers: each decode block's record count and overflow
        start (unit header words 27 + 2b, 28 + 2b) stay inside the record array, the null record
        has no chunks, and every record a block executes (all of its fixed places, which the
        decode reads whatever the count, and its overflow records) names payload and leaf words
        inside its own unit for every chunk it counts."""
        F = int(self.fixed_steps)
        n_rec = self.steps.shape[0]
        null = blocks * F
        if counts[null].any():
            bad("the null step record has chunks")
        cb = np.arange(BLOCKS_PER_UNIT)
        ovf = h[:, 27 + 2 * cb].reshape(-1)                # per block, block = unit * 2 + cb
        nrec = h[:, 28 + 2 * cb].reshape(-1)
        extra = np.maximum(nrec - F, 0)
        if (nrec < 0).any() or ((extra > 0) & ((ovf < null + 1) | (ovf + extra > n_rec))).any():
            bad("decode block record count or overflow start outside the step records")
        # every (record, owning unit) pair a block executes
        fixed_rec = np.arange(null, dtype=np.int64)
        fixed_unit = fixed_rec // max(F, 1) // BLOCKS_PER_UNIT
        blk = np.repeat(np.arange(blocks), extra)
        pos = np.arange(int(extra.sum())) - np.repeat(np.cumsum(extra) - extra, extra)
        rec = np.concatenate([fixed_rec, ovf[blk] + pos])
        unit = np.concatenate([fixed_unit, blk // BLOCKS_PER_UNIT])
        if rec.size == 0:
            return
        slot = self.steps[rec][:, 0::2].astype(np.int64)   # (n, 4) slot words
        n = counts[rec]                                      # (n, 4) chunks per slot
        Pr, lsr = P[rec][:, None], ls[rec][:, None]
        n_pay = ((n + 3) // 4) * 4 if self.layout == LAYOUT_MX else n
        pay_end = (slot & 0xFFFF) * 4 + n_pay * Pr
        leaves = np.where(lsr == 2, 2 * n, ((np.maximum(n, 1) - 1) >> np.maximum(lsr - 3, 0)) + 1)
        leaf_end = (slot >> 16) + leaves
        pay_len = (h[unit, 1] - h[unit, 0])[:, None]
        leaf_len = (h[unit, 3] - h[unit, 2])[:, None]
        on = n > 0
        if (on & (pay_end > pay_len)).any():
            bad("step record payload outside its unit")
        if (on & (leaf_end > leaf_len)).any():
            bad("step record leaf words outside its unit")


def _code_bits(P: int, i: int):
    """Where code i of a chunk lives: [(dword, shift, bits of the code taken, shift into the
    code)], one entry per dword it touches. P = 3 uses byte lanes: byte b of the 3 dwords,
    dword 0's byte lowest, is a 24-bit string holding codes 8b .. 8b+7 at bits 3a (a = i % 8),
    so a shift and a mask extract one code of every lane at once. Other widths run code i
    over bits [i*P, i*P+P) of the chunk's little-endian bit string."""
    if P == 3:
        b, s = i // 8, 3 * (i % 8)
        k, o = s // 8, s % 8
        first = min(3, 8 - o)
        parts = [(k, 8 * b + o, first, 0)]
        if first < 3:
            parts.append((k + 1, 8 * b, 3 - first, first))
        return parts
    bit = i * P
    j, sh = bit >> 5, bit & 31
    first = min(P, 32 - sh)
    parts = [(j, sh, first, 0)]
    if first < P:
        parts.append((j + 1, 0, P - first, first))
    return parts


# ---- the matrix-core decode layout ("mx", MTC_FLAG_MX_LAYOUT) ----
# A bucket's chunks are taken in quads (4 consecutive chunks; the last quad is padded with
# zero codes) and a quad's 4P dwords are 4 lanes of P dwords: lane j holds column j of the
# quad's 4 chunks, the 8 codes of each chunk in chunk-row order r = 0..7 (for S = 4 rows 0-3
# are the chunk's first leaf, rows 4-7 its second). The decode turns a lane's 32 codes into 16
# dwords o = 0..15 of two f16 operands each: dword o holds chunk t = o / 4, rows r = 2 (o % 4)
# (low half) and r + 1 (high half). The codes of the low halves form one bit string over the
# low 16-bit halves of the lane's dwords (dword d holds bits [16 d, 16 d + 16)), those of the
# high halves the same string over the high halves, so one shift and one masked OR build an
# operand dword. Code o sits at bits [o W, o W + W) of its string (W = P; P = 16 is two planes
# of W = 8, the low bytes in dwords 0-7 and the high bytes in dwords 8-15).
LAYOUT_V1, LAYOUT_MX = 0, 1
MX_PLANES = {2: (2, 1), 3: (3, 1), 4: (4, 1), 5: (5, 1), 6: (6, 1), 8: (8, 1), 16: (8, 2)}   # P -> (W, planes)


def mx_rows(S: int) -> np.ndarray:
    """(4 columns, 8 chunk rows) -> the chunk's code index (the panel stream's chunk code order)."""
    j, r = np.meshgrid(np.arange(4), np.arange(8), indexing="ij")
    return np.where(S == 4, 16 * (r // 4) + 4 * j + r % 4, 8 * j + r)


_MX_TABLES: Dict[Tuple[int, int], Tuple[np.ndarray, ...]] = {}


def _mx_table(S: int, P: int):
    """Every code bit of a quad in the mx layout, as flat index arrays: the code (chunk t,
    chunk code index c), its bit v (8 * plane + k), and where it is stored (lane l, dword d,
    bit b). Cached per (S == 4, P)."""
    key = (int(S == 4), int(P))
    if key not in _MX_TABLES:
        W, npl = MX_PLANES[P]
        ci = mx_rows(S)
        rows = []
        for j in range(4):
            for o in range(16):
                t, r = o // 4, 2 * (o % 4)
                for half, rr in ((0, r), (1, r + 1)):
                    for pl in range(npl):
                        for k in range(W):
                            b = o * W + k
                            rows.append((t, ci[j, rr], 8 * pl + k, j, pl * W + b // 16, 16 * half + b % 16))
        a = np.array(rows, dtype=np.int64)
        t, c, v, l, d, bb = a.T
        po = np.lexsort((bb, d, l))                         # grouped by stored dword (pack)
        uo = np.lexsort((v, c, t))                          # grouped by code (unpack)
        _MX_TABLES[key] = (t, c, v, l, d, bb, po, uo)
    return _MX_TABLES[key]


def _segment_or(x: np.ndarray, keys: np.ndarray) -> np.ndarray:
    """OR of the columns of x (n, m) over runs of equal `keys` (sorted; bits are disjoint)."""
    starts = np.flatnonzero(np.concatenate([[True], keys[1:] != keys[:-1]]))
    return np.add.reduceat(x, starts, axis=1)


def mx_pack(codes: np.ndarray, S: int, P: int) -> np.ndarray:
    """(n, 4, 32) signed codes of n quads (4 chunks each, panel-stream chunk code order) ->
    (n, 4, P) uint32: the P dwords of lanes 0..3."""
    n = codes.shape[0]
    u = (codes.astype(np.int64) + (1 << (P - 1))).astype(np.uint64)
    if np.any(u >> np.uint64(P)):
        raise ValueError(f"codes outside the signed {P}-bit range")
    t, c, v, l, d, bb, po, _ = _mx_table(S, P)
    bits = ((u[:, t[po], c[po]] >> v[po].astype(np.uint64)) & np.uint64(1)) << bb[po].astype(np.uint64)
    return _segment_or(bits, l[po] * 64 + d[po]).reshape(n, 4, P).astype(np.uint32)


def mx_unpack(words: np.ndarray, S: int, P: int) -> np.ndarray:
    """Inverse of mx_pack: (n, 4, P) uint32 -> (n, 4, 32) signed codes."""
    n = words.shape[0]
    w = words.astype(np.uint64)
    t, c, v, l, d, bb, _, uo = _mx_table(S, P)
    bits = ((w[:, l[uo], d[uo]] >> bb[uo].astype(np.uint64)) & np.uint64(1)) << v[uo].astype(np.uint64)
    u = _segment_or(bits, t[uo] * 64 + c[uo]).reshape(n, 4, 32).astype(np.int64)
    return u - (1 << (P - 1))


def pack_codes(codes: np.ndarray, P: int) -> np.ndarray:
    """(n, 32) signed codes q -> (n, P) uint32 of offset-binary codes u = q + 2^(P-1),
    placed as _code_bits says."""
    n = codes.shape[0]
    u = (codes.astype(np.int64) + (1 << (P - 1))).astype(np.uint64)
    if np.any(u >> np.uint64(P)):
        raise ValueError(f"codes outside the signed {P}-bit range")
    out = np.zeros((n, P), dtype=np.uint64)
    for i in range(32):
        for k, sh, nb, lo in _code_bits(P, i):
            part = (u[:, i] >> np.uint64(lo)) & np.uint64((1 << nb) - 1)
            out[:, k] |= part << np.uint64(sh)
    return out.astype(np.uint32)


def unpack_codes(words: np.ndarray, P: int) -> np.ndarray:
    """Inverse of pack_codes: (n, P) uint32 -> (n, 32) int32."""
    w = words.astype(np.uint64)
    n = w.shape[0]
    out = np.zeros((n, 32), dtype=np.int64)
    for i in range(32):
        v = np.zeros(n, dtype=np.uint64)
        for k, sh, nb, lo in _code_bits(P, i):
            v |= ((w[:, k] >> np.uint64(sh)) & np.uint64((1 << nb) - 1)) << np.uint64(lo)
        out[:, i] = v.astype(np.int64) - (1 << (P - 1))
    return out.astype(np.int32)


def _bf16_bits(scale: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(scale, dtype=np.float32).view(np.uint32)
    if np.any(bits & 0xFFFF):
        raise ValueError("bf16 scale format requested but some scales are not bf16-representable")
    return bits >> 16


def weight_codes(Wp: np.ndarray) -> CodeSource:
    """Codes of leaves (level S, width P, grid rows ii, cols jj, scales sc) quantized from Wp."""
    Wp = np.asarray(Wp, dtype=np.float32)
    views: Dict[int, np.ndarray] = {}

    def source(S, P, ii, jj, sc):
        if S not in views:
            views[S] = to_blocks(Wp, S)
        return quantize_blocks(views[S][ii, jj][None], P, sc[None])[0]

    return source


def _kind_rank(S: int, P: int) -> int:
    return LEAF_SIZES.index(S) * len(CODE_WIDTHS) + CODE_WIDTHS.index(P)


_KIND_S = np.array([LEAF_SIZES[r // len(CODE_WIDTHS)] for r in range(len(LEAF_SIZES) * len(CODE_WIDTHS))])
_KIND_P = np.array([CODE_WIDTHS[r % len(CODE_WIDTHS)] for r in range(len(LEAF_SIZES) * len(CODE_WIDTHS))])

# Payload bytes a merge of two kinds may add per decode step record it saves (besides the
# record's own 64 bytes, which it also saves).
MERGE_BYTES_PER_RECORD = 256
# Bits a leaf's codes may be widened by. The fp32 decode sums x * u - 2^(P-1) * sum(x), so a
# code stored d bits wider carries an offset 2^d times larger through the same sums: its
# rounding error grows by up to 2^d.
MERGE_MAX_WIDEN = 2


def _block_records(chunks: np.ndarray) -> np.ndarray:
    """Decode step records of one kind per unit: (U, 8) lane chunks per column group ->
    (U,) records over the unit's two blocks of 4 column groups (16 chunks per slot)."""
    return (-(-chunks.reshape(-1, BLOCKS_PER_UNIT, STEP_GROUPS).max(axis=2) // STEP_LANES)).sum(axis=1)


def storage_widths(shape: Tuple[int, int], sizes: Sequence[int], leaf: Dict[int, np.ndarray],
                   modes: Dict[int, np.ndarray], chunk_rows: int) -> Dict[int, np.ndarray]:
    """Per level S, the code width each leaf is stored at: its mode P, or a wider width P' of
    the same leaf size in the same unit.

    The decode runs one kind (S, P) per step record of 4 column groups x 16 chunks, so a kind
    with a few chunks in a block still costs a whole record. Signed codes q of width P fit any
    wider offset-binary width (u' = q + 2^(P'-1)) and decode to the same q * s, so W_hat is
    unchanged. Per unit and leaf size, kinds are taken narrowest first; each is merged into
    the narrowest wider kind present in the unit when that saves records, adds at most
    MERGE_BYTES_PER_RECORD payload bytes per record saved and widens no leaf it holds (its
    own or merged into it earlier) by more than MERGE_MAX_WIDEN bits."""
    K, N = (int(x) for x in shape)
    n_chunks = -(-K // chunk_rows)
    n_units = (N // PANEL) * n_chunks
    widths = np.array(CODE_WIDTHS)
    out: Dict[int, np.ndarray] = {}
    for S in (int(s) for s in sizes):
        mode = np.asarray(modes[S])
        stored = np.asarray(leaf[S], dtype=bool) & np.isin(mode, widths)
        pw = np.where(stored, mode, 0).astype(np.int64)
        out[S] = pw
        ii, jj = np.nonzero(stored)
        if ii.size == 0:
            continue
        p_idx = np.searchsorted(widths, mode[ii, jj])
        unit = ((jj * S) // PANEL) * n_chunks + (ii * S) // chunk_rows
        ncg = max(1, S // GROUP)
        g0 = (jj * S % PANEL) // GROUP
        per_cg = 1 if S <= 8 else S // 8            # chunks per covered column group (S = 4: leaves)
        cnt = np.zeros((n_units, len(widths), N_GROUPS), dtype=np.int64)
        for c in range(ncg):
            np.add.at(cnt, (unit, p_idx, g0 + c), per_cg)

        def chunks(x):
            return -(-x // 2) if S == 4 else x       # two 4x4 leaves per chunk

        target = np.tile(np.arange(len(widths)), (n_units, 1))
        narrowest = np.tile(widths, (n_units, 1))      # narrowest mode each kind holds
        for p in range(len(widths) - 1):
            undecided = cnt[:, p].sum(axis=1) > 0
            for q in range(p + 1, len(widths)):
                cand = undecided & (cnt[:, q].sum(axis=1) > 0)
                if not cand.any():
                    continue
                merged = cnt[:, p] + cnt[:, q]
                saved = (_block_records(chunks(cnt[:, p])) + _block_records(chunks(cnt[:, q])) -
                         _block_records(chunks(merged)))
                extra = chunks(cnt[:, p]).sum(axis=1) * 4 * (widths[q] - widths[p])     # 32 codes per chunk
                ok = cand & (saved > 0) & (extra <= MERGE_BYTES_PER_RECORD * saved) & \
                    (widths[q] - narrowest[:, p] <= MERGE_MAX_WIDEN)
                cnt[ok, q] = merged[ok]
                cnt[ok, p] = 0
                narrowest[ok, q] = np.minimum(narrowest[ok, q], narrowest[ok, p])
                target[ok, p] = q
                undecided &= ~ok
        for p in range(len(widths) - 2, -1, -1):     # follow merges of merged kinds
            target[:, p] = np.where(target[:, p] != p, target[np.arange(n_units), target[:, p]], p)
        pw[ii, jj] = widths[target[unit, p_idx]]
    return out


def split_leaves(shape: Tuple[int, int], sizes: Sequence[int], leaf: Dict[int, np.ndarray],
                 store_w: Dict[int, np.ndarray], chunk_rows: int) -> Dict[int, np.ndarray]:
    """Per level S in (32, 16), the stored leaves that are packed as (S/8)^2 leaves of size 8
    (the same scale and storage width, their codes' 8 x 8 sub-blocks: W_hat is unchanged).

    Leaf sizes 8, 16 and 32 share one decode path and differ only in how many chunks share a
    leaf word, and the chunks of an S x S leaf are exactly those of its 8 x 8 sub-blocks, so a
    unit's S x S leaves of a storage width can join its 8 x 8 leaves of that width in the same
    step records. Per unit and storage width, from the largest size down, a size is split when
    that saves records and its extra leaf words ((S/8)^2 - 1 per leaf, 4 bytes each) add at
    most MERGE_BYTES_PER_RECORD bytes per record saved."""
    K, N = (int(x) for x in shape)
    n_chunks = -(-K // chunk_rows)
    n_units = (N // PANEL) * n_chunks
    widths = np.array(CODE_WIDTHS)
    sizes = {int(x) for x in sizes}

    def stored_at(S):
        st = store_w[S]
        ii, jj = np.nonzero(np.asarray(leaf[S], dtype=bool) & np.isin(st, widths))
        unit = ((jj * S) // PANEL) * n_chunks + (ii * S) // chunk_rows
        return ii, jj, unit, np.searchsorted(widths, st[ii, jj]), (jj * S % PANEL) // GROUP

    cnt8 = np.zeros((n_units, len(widths), N_GROUPS), dtype=np.int64)   # chunks of (8, P) per column group
    if 8 in sizes:
        _, _, unit, p_idx, g0 = stored_at(8)
        for c in range(2):
            np.add.at(cnt8, (unit, p_idx, g0 + c), 1)
    out: Dict[int, np.ndarray] = {}
    for S in (32, 16):
        if S not in sizes:
            continue
        ii, jj, unit, p_idx, g0 = stored_at(S)
        out[S] = np.zeros(np.asarray(leaf[S]).shape, dtype=bool)
        if ii.size == 0:
            continue
        cnt = np.zeros_like(cnt8)
        n_leaf = np.zeros((n_units, len(widths)), dtype=np.int64)
        for c in range(S // GROUP):
            np.add.at(cnt, (unit, p_idx, g0 + c), S // 8)
        np.add.at(n_leaf, (unit, p_idx), 1)
        split = np.zeros((n_units, len(widths)), dtype=bool)
        for p in range(len(widths)):
            saved = _block_records(cnt8[:, p]) + _block_records(cnt[:, p]) - _block_records(cnt8[:, p] + cnt[:, p])
            extra = n_leaf[:, p] * ((S // 8) ** 2 - 1) * 4
            split[:, p] = (n_leaf[:, p] > 0) & (saved > 0) & (extra <= MERGE_BYTES_PER_RECORD * saved)
            cnt8[split[:, p], p] += cnt[split[:, p], p]
        out[S][ii, jj] = split[unit, p_idx]
    return out


def storage_plan(shape: Tuple[int, int], sizes: Sequence[int], leaf: Dict[int, np.ndarray],
                 modes: Dict[int, np.ndarray], chunk_rows: int, merge_kinds: bool = True):
    """The levels as packed: 16 x 16 and 32 x 32 leaves split into 8 x 8 leaves (split_leaves,
    decided on the allocated widths), then storage widths chosen over those levels
    (storage_widths), split leaves counted at level 8 with their parents' modes. Returns
    (sizes, leaf, modes, storage widths, split): per level the leaf mask, mode grid and
    storage-width grid as packed, and per level 16 / 32 the leaves that were split. Without
    `merge_kinds` nothing is split and every leaf is stored at its mode."""
    K, N = (int(x) for x in shape)
    sizes = tuple(sorted({int(x) for x in sizes}, reverse=True))
    split = split_leaves((K, N), sizes, leaf, {S: np.where(np.asarray(leaf[S], bool), np.asarray(modes[S]), 0)
                                                for S in sizes}, chunk_rows) if merge_kinds else {}
    leaf_p = {S: np.asarray(leaf[S], dtype=bool) for S in sizes}
    modes_p = {S: np.asarray(modes[S]) for S in sizes}
    if any(v.any() for v in split.values()):
        if 8 not in leaf_p:
            leaf_p[8] = np.zeros((K // 8, N // 8), dtype=bool)
            modes_p[8] = np.zeros((K // 8, N // 8), dtype=np.int64)
        modes_p[8] = modes_p[8].astype(np.int64).copy()
        leaf_p[8] = leaf_p[8].copy()
        for S, sp in split.items():
            r = S // 8
            up = np.kron(sp, np.ones((r, r), dtype=bool))
            leaf_p[8] |= up
            modes_p[8][up] = np.kron(np.asarray(modes[S]).astype(np.int64), np.ones((r, r), dtype=np.int64))[up]
            leaf_p[S] = leaf_p[S] & ~sp
    sizes_p = tuple(sorted(leaf_p, reverse=True))
    if merge_kinds:
        store_w = storage_widths((K, N), sizes_p, leaf_p, modes_p, chunk_rows)
    else:
        store_w = {S: np.where(leaf_p[S] & np.isin(modes_p[S], CODE_WIDTHS), modes_p[S], 0) for S in sizes_p}
    return sizes_p, leaf_p, modes_p, store_w, split


def pack_levels(shape: Tuple[int, int], sizes: Sequence[int], leaf: Dict[int, np.ndarray],
                modes: Dict[int, np.ndarray], scales: Dict[int, np.ndarray], codes_of: CodeSource,
                chunk_rows: int = 512, scale_format: str = "bf16", row_perm: Optional[np.ndarray] = None,
                col_perm: Optional[np.ndarray] = None, merge_kinds: bool = True,
                layout: int = LAYOUT_V1) -> PanelStream:
    """Pack the leaves given per level s (leaf mask, mode grid, scale grid) of a K x N weight.

    `codes_of(S, P, ii, jj, scales)` returns the (n, S, S) integer codes of the
    listed leaves (see weight_codes). With `merge_kinds`, rare kinds are stored at a wider
    width of the same leaf size (storage_widths); W_hat is the same either way. `layout`:
    LAYOUT_V1 (chunk-contiguous payload, every decode kernel) or LAYOUT_MX (quads of chunks
    stored per lane column for the matrix-core decode of one X row; see mx_pack).
    """
    if layout not in (LAYOUT_V1, LAYOUT_MX):
        raise ValueError(f"layout={layout}")
    K, N = (int(x) for x in shape)
    if N % PANEL or K % 8:
        raise ValueError(f"panel stream needs N % {PANEL} == 0 and K % 8 == 0, got {shape}")
    if chunk_rows % 32 or not 32 <= chunk_rows <= MAX_CHUNK_ROWS:
        raise ValueError(f"chunk_rows={chunk_rows} must be a multiple of 32 in [32, {MAX_CHUNK_ROWS}]")
    if scale_format not in ("bf16", "fp32"):
        raise ValueError(scale_format)
    n_chunks = -(-K // chunk_rows)
    n_units = (N // PANEL) * n_chunks

    # per kind: leaf words (+ unit/kind keys) and chunk records
    lw_words, lw_scales, lw_unit, lw_kind = [], [], [], []
    ch_unit, ch_cg, ch_kind, ch_row, ch_leaf, ch_words, ch_codes = [], [], [], [], [], [], []
    n_real = 0
    n_lw = 0
    for S in sizes:
        if int(S) not in LEAF_SIZES:
            raise ValueError(f"leaf size {S} not supported by the panel stream (sizes {LEAF_SIZES})")
    sizes = tuple(sorted({int(x) for x in sizes}, reverse=True))
    moved: Dict[int, list] = {}                        # storage width -> 8 x 8 sub-leaves of split leaves
    sizes_p, leaf_p, modes_p, store_w, split = storage_plan((K, N), sizes, leaf, modes, chunk_rows, merge_kinds)
    for S, sp in split.items():                        # codes of split leaves, as 8 x 8 sub-leaves
        ii, jj = np.nonzero(sp)
        if ii.size == 0:
            continue
        r = S // 8
        sc = np.asarray(scales[S], dtype=np.float32)[ii, jj]
        qm = np.asarray(modes[S])[ii, jj]
        q = np.empty((ii.size, S, S), dtype=np.int32)
        for Pq in np.unique(qm):
            sel = np.flatnonzero(qm == Pq)
            q[sel] = np.asarray(codes_of(S, int(Pq), ii[sel], jj[sel], sc[sel])).astype(np.int32)
        k0, n0 = ii * S, jj * S
        unit = (n0 // PANEL) * n_chunks + k0 // chunk_rows
        pw = store_w[8][ii * r, jj * r]                 # every sub-leaf of a leaf: one unit and mode
        a_, b_ = np.divmod(np.arange(r * r), r)         # sub-block (row a, column b)
        sub = q.reshape(-1, r, 8, r, 8).transpose(0, 1, 3, 2, 4).reshape(-1, r * r, 8, 8)
        for P in np.unique(pw):
            m_ = pw == P
            moved.setdefault(int(P), []).append((
                (k0[m_][:, None] + 8 * a_).reshape(-1), (n0[m_] % PANEL)[:, None].repeat(r * r, 1).reshape(-1) +
                np.tile(8 * b_, int(m_.sum())), np.repeat(unit[m_], r * r), np.repeat(sc[m_], r * r),
                sub[m_].reshape(-1, 8, 8)))
    for S in sizes_p:
        native = S in sizes
        for P in CODE_WIDTHS:                          # storage width: the kind's P
            k0 = c0 = unit = sc = q = None
            if native:
                own = np.asarray(leaf[S], dtype=bool) if S == 8 else leaf_p[S]     # not the split sub-leaves
                ii, jj = np.nonzero(own & np.isin(modes_p[S], CODE_WIDTHS) & (store_w[S] == P))
                if ii.size:
                    sc = np.asarray(scales[S], dtype=np.float32)[ii, jj]
                    q = np.empty((ii.size, S, S), dtype=np.int32)                 # (n, S, S) row-major
                    qm = modes_p[S][ii, jj]
                    for Pq in np.unique(qm):           # codes quantized at each leaf's own width
                        sel = np.flatnonzero(qm == Pq)
                        q[sel] = np.asarray(codes_of(S, int(Pq), ii[sel], jj[sel], sc[sel])).astype(np.int32)
                    k0, n0 = ii * S, jj * S
                    unit = (n0 // PANEL) * n_chunks + k0 // chunk_rows
                    c0 = n0 % PANEL
            if S == 8 and P in moved:
                parts = ([(k0, c0, unit, sc, q)] if q is not None else []) + moved.pop(P)
                k0, c0, unit, sc, q = (np.concatenate(x) for x in zip(*parts))
            if q is None or q.shape[0] == 0:
                continue
            kr = _kind_rank(S, P)
            order = np.lexsort((k0, c0, unit))
            k0, c0, unit, sc, q = k0[order], c0[order], unit[order], sc[order], q[order]
            n_real += q.shape[0]
            words = ((k0 % chunk_rows) // 4).astype(np.uint32)
            if scale_format == "bf16":
                words = words | (_bf16_bits(sc) << 16).astype(np.uint32)
            if S == 4:
                # two leaves of one (unit, column group) per chunk; an odd group gets a pad leaf
                grp = unit * N_GROUPS + c0 // GROUP
                edges = np.flatnonzero(np.concatenate([[True], grp[1:] != grp[:-1], [True]]))
                odd = np.flatnonzero(np.diff(edges) & 1)
                if odd.size:
                    ends = edges[odd + 1]
                    q = np.insert(q, ends, 0, axis=0)
                    words = np.insert(words, ends, np.uint32(LEAF_PAD))
                    sc = np.insert(sc, ends, np.float32(0))
                    unit = np.insert(unit, ends, unit[ends - 1])
                    c0 = np.insert(c0, ends, c0[ends - 1])
                    k0 = np.insert(k0, ends, k0[ends - 1])
                n = q.shape[0]
                gidx = n_lw + np.arange(n)
                ch_unit.append(unit[0::2])
                ch_cg.append(c0[0::2] // GROUP)
                ch_kind.append(np.full(n // 2, kr))
                ch_row.append(k0[0::2])
                ch_leaf.append(gidx[0::2])
                cq = q.transpose(0, 2, 1).reshape(n // 2, 32)
                ch_words.append(pack_codes(cq, P))
                if layout == LAYOUT_MX:
                    ch_codes.append(cq.astype(np.int16))
            else:
                n = q.shape[0]
                nrb, ncg = S // 8, S // GROUP
                gidx = n_lw + np.arange(n)
                # (n, rb, r, cgi, c) -> (n, cgi, rb, c, r): chunk = 4 columns x 8 rows, column-major
                codes = q.reshape(n, nrb, 8, ncg, GROUP).transpose(0, 3, 1, 4, 2).reshape(n * ncg * nrb, 32)
                shp = (n, ncg, nrb)
                ch_unit.append(np.broadcast_to(unit[:, None, None], shp).reshape(-1))
                ch_cg.append(((c0 // GROUP)[:, None, None] + np.arange(ncg)[None, :, None] + 0 * np.arange(nrb)).reshape(-1))
                ch_kind.append(np.full(n * ncg * nrb, kr))
                ch_row.append((k0[:, None, None] + 8 * np.arange(nrb)[None, None, :] + 0 * np.arange(ncg)[None, :, None]).reshape(-1))
                ch_leaf.append(np.broadcast_to(gidx[:, None, None], shp).reshape(-1))
                ch_words.append(pack_codes(codes, P))
                if layout == LAYOUT_MX:
                    ch_codes.append(codes.astype(np.int16))
            lw_words.append(words)
            lw_scales.append(sc)
            lw_unit.append(unit)
            lw_kind.append(np.full(n, kr))
            n_lw += n

    # ---- leaf words in (unit, kind, c0, k0) order: each bucket's leaves form one run ----
    if n_lw:
        wu = np.concatenate(lw_unit).astype(np.int64)
        wk = np.concatenate(lw_kind).astype(np.int64)
        lw_order = np.lexsort((np.arange(n_lw), wk, wu))       # keeps each kind's (c0, k0) order
        lw_pos = np.empty(n_lw, dtype=np.int64)
        lw_pos[lw_order] = np.arange(n_lw)
        leaf_word = np.concatenate(lw_words)[lw_order]
        leaf_scale = np.concatenate(lw_scales)[lw_order] if scale_format == "fp32" else None
        leaf_begin = np.searchsorted(wu[lw_order], np.arange(n_units + 1)).astype(np.int64)
    else:
        leaf_word = np.zeros(1, np.uint32)
        leaf_scale = np.zeros(1, np.float32) if scale_format == "fp32" else None
        lw_pos = np.zeros(0, np.int64)
        leaf_begin = np.zeros(n_units + 1, np.int64)

    # ---- chunks in (unit, cg, kind, row) order -> buckets and payload ----
    if ch_unit:
        cu = np.concatenate(ch_unit).astype(np.int64)
        cc = np.concatenate(ch_cg).astype(np.int64)
        ck = np.concatenate(ch_kind).astype(np.int64)
        cr = np.concatenate(ch_row).astype(np.int64)
        cl = lw_pos[np.concatenate(ch_leaf).astype(np.int64)]
        cP = np.concatenate([np.full(w.shape[0], w.shape[1]) for w in ch_words]).astype(np.int64)
        src_off = np.concatenate([[0], np.cumsum(cP)[:-1]])
        src = np.concatenate([w.reshape(-1) for w in ch_words])
        corder = np.lexsort((cr, ck, cc, cu))
        cu, cc, ck, cl, cP, src_off = cu[corder], cc[corder], ck[corder], cl[corder], cP[corder], src_off[corder]
        n_ch = cu.size
        bkey = (cu * N_GROUPS + cc) * 64 + ck
        b_start = np.flatnonzero(np.concatenate([[True], bkey[1:] != bkey[:-1]]))
        n_buckets = b_start.size
        b_cnt = np.diff(np.concatenate([b_start, [n_ch]]))
        b_unit, b_cg, b_kind = cu[b_start], cc[b_start], ck[b_start]
        b_S, b_P = _KIND_S[b_kind], _KIND_P[b_kind]
        if layout == LAYOUT_MX:
            b_dw = ((b_cnt + 3) // 4) * 4 * b_P                             # whole quads of chunks
        else:
            b_dw = (b_cnt * b_P + 3) & ~3
        b_pay = np.concatenate([[0], np.cumsum(b_dw)[:-1]])
        total_dw = int(b_dw.sum())
        payload = np.zeros(total_dw + PAYLOAD_PAD, dtype=np.uint32)   # tail padding: 16-byte loads may run past a chunk
        b_of = np.repeat(np.arange(n_buckets), b_cnt)
        if layout == LAYOUT_MX:
            codes = np.concatenate(ch_codes)[corder]
            pos = np.arange(n_ch) - b_start[b_of]                        # chunk index within its bucket
            for P in np.unique(cP):
                for four in (True, False):                               # S = 4 chunks order codes by leaf
                    sel = np.flatnonzero((cP == P) & ((_KIND_S[ck] == 4) == four))
                    if sel.size == 0:
                        continue
                    qkey = b_of[sel] * (1 << 20) + pos[sel] // 4         # one entry per quad
                    uq, qi = np.unique(qkey, return_inverse=True)
                    quads = np.zeros((uq.size, 4, 32), dtype=np.int64)
                    quads[qi, pos[sel] % 4] = codes[sel]
                    words = mx_pack(quads, 4 if four else 8, int(P))     # (n_quads, 4 lanes, P)
                    qb = uq >> 20
                    qdst = b_pay[qb] + (uq & ((1 << 20) - 1)) * 4 * int(P)
                    payload[(qdst[:, None] + np.arange(4 * int(P))).reshape(-1)] = words.reshape(-1)
        else:
            dst = b_pay[b_of] + (np.arange(n_ch) - b_start[b_of]) * cP
            for P in np.unique(cP):
                sel = np.flatnonzero(cP == P)
                payload[(dst[sel][:, None] + np.arange(P)).reshape(-1)] = src[(src_off[sel][:, None] + np.arange(P)).reshape(-1)]
        # first chunk of each bucket within its column group
        gkey = cu * N_GROUPS + cc
        g_start = np.flatnonzero(np.concatenate([[True], gkey[1:] != gkey[:-1]]))
        g_of = np.repeat(np.arange(g_start.size), np.diff(np.concatenate([g_start, [n_ch]])))
        b_cstart = b_start - g_start[g_of[b_start]]
        b_leaf = cl[b_start]
        pay_after = np.concatenate([b_pay, [total_dw]])
    else:
        n_buckets, total_dw = 0, 0
        payload = np.zeros(PAYLOAD_PAD, np.uint32)
        b_unit = b_cg = b_cnt = b_cstart = b_leaf = b_pay = np.zeros(0, np.int64)
        b_S = b_P = np.zeros(0, np.int64)
        pay_after = np.zeros(1, np.int64)

    if payload.size >= 2 ** 31 or leaf_word.size >= 2 ** 31:
        raise ValueError("stream too large for 31-bit offsets")
    if n_buckets and (b_cnt.max() >= 1 << 16 or b_cstart.max() >= 1 << 16):
        raise ValueError("a column group holds 65536 or more lane chunks; use a smaller chunk_rows")

    # ---- unit headers ----
    hdr = np.zeros((n_units, UNIT_HDR_WORDS), dtype=np.int64)
    ub = np.searchsorted(b_unit, np.arange(n_units + 1))
    hdr[:, 0], hdr[:, 1] = pay_after[ub[:-1]], pay_after[ub[1:]]
    hdr[:, 2], hdr[:, 3] = leaf_begin[:-1], leaf_begin[1:]
    hdr[:, 4], hdr[:, 5] = ub[:-1], ub[1:]
    hdr[:, 6] = ub[1:] - ub[:-1]
    gb = np.searchsorted(b_unit * N_GROUPS + b_cg, np.arange(n_units * N_GROUPS + 1))
    gb = np.concatenate([gb[:-1].reshape(n_units, N_GROUPS), ub[1:, None]], axis=1)      # (n_units, 9)
    hdr[:, 8:17] = gb - hdr[:, 4:5]
    hdr[:, 17:26] = pay_after[gb] - hdr[:, 0:1]
    # dwords one decode block (a pair of column groups) stages on chip: the pair's payload and
    # bucket entries plus all of the unit's leaf words; hdr[7] is the max over the unit's pairs
    pair_pay = hdr[:, 17 + 2:26:2] - hdr[:, 17:25:2]
    pair_bk = hdr[:, 8 + 2:17:2] - hdr[:, 8:16:2]
    hdr[:, 7] = (pair_pay + 4 * pair_bk).max(axis=1) + (hdr[:, 3] - hdr[:, 2])
    # the same for blocks of four column groups
    quad_pay = hdr[:, 17 + 4:26:4] - hdr[:, 17:22:4]
    quad_bk = hdr[:, 8 + 4:17:4] - hdr[:, 8:13:4]
    hdr[:, 26] = (quad_pay + 4 * quad_bk).max(axis=1) + (hdr[:, 3] - hdr[:, 2])
    max_unit_words = int(hdr[:, 7].max()) if n_units else 0
    max_unit_words4 = int(hdr[:, 26].max()) if n_units else 0

    # ---- decode step records: one per (unit, block of 4 column groups, kind, 16-chunk step) ----
    # A block's records, in (kind, step) order, are split into its first F ("fixed") records,
    # stored at records [b*F, b*F + F) of the table (b = unit * 2 + block; unused places hold
    # null records), and the rest ("overflow"), stored after the fixed area and one null
    # record at index n_blocks * F. Word 2g (column group 4 * block + g) holds where the step
    # starts in that column group's bucket of the kind, relative to the unit: payload dwords / 4
    # (bits 0-15) and leaf-word index (bits 16-31), 0 for a slot without chunks; words 2g + 1
    # all hold the kind (log2 S | P << 3) and each slot's chunk count in this step (5 bits at
    # 8 + 5g), so that a lane of slot g reads its two words with one aligned 8-byte load.
    n_blocks = n_units * BLOCKS_PER_UNIT
    null_rec = np.zeros(STEP_WORDS, dtype=np.int64)
    null_rec[1::2] = record_kind(_NULL_KEY)
    recs = np.zeros((0, STEP_WORDS), dtype=np.int64)
    blk_begin = np.zeros(n_blocks + 1, dtype=np.int64)
    if n_buckets:
        blk = b_cg // STEP_GROUPS
        slot = b_cg % STEP_GROUPS
        order = np.lexsort((slot, b_kind, blk, b_unit))
        gk = (b_unit[order] * 2 + blk[order]) * 64 + b_kind[order]
        gstart = np.flatnonzero(np.concatenate([[True], gk[1:] != gk[:-1]]))
        n_grp = gstart.size
        gid = np.repeat(np.arange(n_grp), np.diff(np.concatenate([gstart, [n_buckets]])))
        g_steps = np.maximum.reduceat(-(-b_cnt[order] // STEP_LANES), gstart)
        gb = np.full((n_grp, STEP_GROUPS), -1, dtype=np.int64)
        gb[gid, slot[order]] = order
        first = order[gstart]
        miss = gb < 0
        gb[miss] = np.broadcast_to(first[:, None], gb.shape)[miss]          # safe offsets, no valid chunks
        g_n = np.where(miss, 0, b_cnt[gb])
        rec_g = np.repeat(np.arange(n_grp), g_steps)
        j = np.arange(rec_g.size) - np.repeat(np.concatenate([[0], np.cumsum(g_steps)[:-1]]), g_steps)
        bb = gb[rec_g]
        b_ls = np.array([_LOG2[int(v)] for v in b_S], dtype=np.int64)
        nv = np.clip(g_n[rec_g] - STEP_LANES * j[:, None], 0, STEP_LANES)
        # the step's first chunk, 16 j, and its first leaf (two 4x4 leaves per chunk, else
        # one leaf per S / 8 chunks)
        pay_rel = b_pay[bb] - hdr[b_unit[bb], 0] + STEP_LANES * j[:, None] * b_P[bb].astype(np.int64)
        leaf_rel = b_leaf[bb] - hdr[b_unit[bb], 2] + np.where(
            b_ls[bb] == 2, 2 * STEP_LANES * j[:, None], (STEP_LANES * j[:, None]) >> np.maximum(b_ls[bb] - 3, 0))
        on = nv > 0
        if np.any(pay_rel[on] % 4) or pay_rel[on].max(initial=0) >= 4 * SLOT_OFFSET_LIMIT or \
                leaf_rel[on].max(initial=0) >= SLOT_OFFSET_LIMIT:
            raise ValueError("a unit's payload or leaf words exceed the step records' 16-bit offsets")
        recs = np.zeros((rec_g.size, STEP_WORDS), dtype=np.int64)
        recs[:, 0::2] = np.where(on, (pay_rel >> 2) | (leaf_rel << 16), 0)
        kind = b_ls[bb[:, 0]] | (b_P[bb[:, 0]].astype(np.int64) << 3)
        recs[:, 1::2] = (kind | (nv << (8 + 5 * np.arange(STEP_GROUPS))).sum(axis=1))[:, None]
        rec_blk = b_unit[first][rec_g] * 2 + blk[first][rec_g]
        blk_begin = np.searchsorted(rec_blk, np.arange(n_blocks + 1)).astype(np.int64)
    blk_n = np.diff(blk_begin)
    F = int(min(MAX_FIXED_STEPS, STEP_LANES * -(-int(blk_n.max(initial=0)) // STEP_LANES)))
    fixed = np.broadcast_to(null_rec, (n_blocks, F, STEP_WORDS)).copy()
    pos = np.arange(recs.shape[0]) - np.repeat(blk_begin[:-1], blk_n)      # index within the block
    rb = np.repeat(np.arange(n_blocks), blk_n)
    inf = pos < F
    fixed[rb[inf], pos[inf]] = recs[inf]
    ovf_n = np.maximum(blk_n - F, 0)
    ovf_begin = n_blocks * F + 1 + np.concatenate([[0], np.cumsum(ovf_n)[:-1]])
    steps = np.concatenate([fixed.reshape(-1, STEP_WORDS), null_rec[None], recs[~inf]]).astype(np.uint32)
    hdr[:, 27] = ovf_begin[0::2]
    hdr[:, 28] = blk_n[0::2]
    hdr[:, 29] = ovf_begin[1::2]
    hdr[:, 30] = blk_n[1::2]

    buckets = np.zeros((max(n_buckets, 1), 4), dtype=np.uint32)
    if n_buckets:
        buckets[:n_buckets, 0] = b_pay - hdr[b_unit, 0]
        buckets[:n_buckets, 1] = b_leaf - hdr[b_unit, 2]
        buckets[:n_buckets, 2] = b_cnt | (b_cstart << 16)
        buckets[:n_buckets, 3] = np.array([_LOG2[int(s)] for s in b_S], dtype=np.uint32) | (b_P.astype(np.uint32) << 8)

    stats = {"payload_bytes": float(total_dw * 4), "n_buckets": float(n_buckets), "n_leaves": float(n_real),
             "max_unit_bytes": float(4 * max_unit_words)}
    for name, a in (("payload", payload), ("leaf words", leaf_word), ("step records", steps)):
        if a is not None and a.nbytes > MAX_DEVICE_ARRAY_BYTES:
            raise ValueError(f"panel stream {name} of {a.nbytes} bytes exceed the kernels' 32-bit offsets "
                             f"({MAX_DEVICE_ARRAY_BYTES}); split the matrix by column panels")
    return PanelStream(K=K, N=N, chunk_rows=chunk_rows, payload=payload, buckets=buckets,
                       unit_hdr=hdr.astype(np.int32), leaf_word=leaf_word, leaf_scale=leaf_scale, steps=steps,
                       fixed_steps=F,
                       row_perm=None if row_perm is None else np.ascontiguousarray(row_perm, dtype=np.int32),
                       col_perm=None if col_perm is None else np.ascontiguousarray(col_perm, dtype=np.int32),
                       n_real_leaves=n_real, max_unit_words=max_unit_words,
                       max_unit_words4=max_unit_words4, stats=stats, layout=layout)


def _place_chunks(ps: PanelStream, Wp: np.ndarray, u: int, g: int, S: int, P: int, off: int, l0: int,
                  ts: np.ndarray) -> None:
    """Dequantize chunks `ts` of the bucket whose payload starts at dword `off` and whose
    first leaf word is `l0` (both absolute) into Wp (permuted channel order)."""
    panel, chunk = divmod(u, ps.n_chunks)
    ts = np.asarray(ts, dtype=np.int64)
    if ps.layout == LAYOUT_MX and ts.size:
        nq = int(ts.max()) // 4 + 1                         # every quad up to the last chunk named
        quads = mx_unpack(ps.payload[off: off + nq * 4 * P].reshape(nq, 4, P), S, P)
    for t in (int(x) for x in ts):
        if ps.layout == LAYOUT_MX:
            cd_all = quads[t // 4, t % 4]
        else:
            cd_all = unpack_codes(ps.payload[off + t * P: off + (t + 1) * P].reshape(1, P), P)[0]
        if S == 4:
            parts = [(l0 + 2 * t, cd_all[:16], 0, 4), (l0 + 2 * t + 1, cd_all[16:], 0, 4)]
        else:
            parts = [(l0 + t // (S // 8), cd_all, 8 * (t % (S // 8)), 8)]
        for li, cd, rrel, rows in parts:
            wd = int(ps.leaf_word[li])
            if wd & LEAF_PAD:
                continue
            r0 = chunk * ps.chunk_rows + (wd & ((1 << ROW_BITS) - 1)) * 4 + rrel
            c0 = panel * PANEL + GROUP * g
            s = ps.leaf_scale[li] if ps.leaf_scale is not None else \
                np.array([wd >> 16 << 16], dtype=np.uint32).view(np.float32)[0]
            Wp[r0: r0 + rows, c0: c0 + GROUP] = cd.reshape(GROUP, rows).T.astype(np.float32) * np.float32(s)


def _to_original_order(ps: PanelStream, Wp: np.ndarray) -> np.ndarray:
    if ps.leaf_scale is None:
        Wp = Wp + np.float32(0.0)      # quadtree W_hat never holds -0.0
    if ps.row_perm is None and ps.col_perm is None:
        return Wp
    pr = np.arange(ps.K) if ps.row_perm is None else ps.row_perm
    pc = np.arange(ps.N) if ps.col_perm is None else ps.col_perm
    out = np.empty_like(Wp)
    out[np.ix_(pr, pc)] = Wp
    return out


def decode_stream(ps: PanelStream) -> np.ndarray:
    """Host decoder of a panel stream back to W_hat (original channel order), walking
    the bucket table. A debugging aid; the GPU path never calls it."""
    Wp = np.zeros((ps.K, ps.N), dtype=np.float32)
    for u in range(ps.n_units):
        h = [int(x) for x in ps.unit_hdr[u]]
        for g in range(N_GROUPS):
            for b in range(h[4] + h[8 + g], h[4] + h[9 + g]):
                prel, lrel, w2, key = (int(x) for x in ps.buckets[b])
                _place_chunks(ps, Wp, u, g, 1 << (key & 0xFF), key >> 8, h[0] + prel, h[2] + lrel,
                              np.arange(w2 & 0xFFFF))
    return _to_original_order(ps, Wp)


def record_kind(key: int) -> int:
    """Kind field of a step record, log2 S | P << 3, from a bucket key, log2 S | P << 8."""
    return (key & 0xFF) | ((key >> 8) << 3)


def record_slots(rec) -> Tuple[int, int, List[Tuple[int, int, int]]]:
    """(S, P, slots) of one step record; slot g is (payload dword, first leaf word, chunks) of
    the step in column group g of its block, offsets relative to the unit."""
    rec = [int(x) for x in rec]
    kc = rec[1]
    slots = [(4 * (w & 0xFFFF), w >> 16, (kc >> (8 + 5 * g)) & 31) for g, w in enumerate(rec[0::2])]
    return 1 << (kc & 7), (kc >> 3) & 31, slots


def step_record_index(ps: PanelStream, u: int, blk: int, r: int) -> int:
    """Table index of record r of decode block (unit u, column-group block blk): the first
    `fixed_steps` records of a block sit at block-computable positions, the rest follow
    the fixed area at the block's overflow start (unit header word 27 + 2 * blk)."""
    F = ps.fixed_steps
    if r < F:
        return (u * BLOCKS_PER_UNIT + blk) * F + r
    return int(ps.unit_hdr[u, 27 + 2 * blk]) + r - F


def decode_steps(ps: PanelStream) -> np.ndarray:
    """Host decoder that walks the step records the way the decode kernel does: block
    (unit u, column-group block b) has unit_hdr[u, 28 + 2b] records, located by
    step_record_index; slot g of a record (record_slots) names where the step starts in
    column group 4b + g (unit payload start + dwords, unit leaf start + leaves) and how many
    chunks it has, and lane li of the slot takes the step's chunk li when li is below that
    count. A debugging aid; the GPU path never calls it."""
    Wp = np.zeros((ps.K, ps.N), dtype=np.float32)
    for u in range(ps.n_units):
        pay0, leaf0 = int(ps.unit_hdr[u, 0]), int(ps.unit_hdr[u, 2])
        for blk in range(BLOCKS_PER_UNIT):
            for r in range(int(ps.unit_hdr[u, 28 + 2 * blk])):
                S, P, slots = record_slots(ps.steps[step_record_index(ps, u, blk, r)])
                for g, (pay, leaf, nv) in enumerate(slots):
                    _place_chunks(ps, Wp, u, blk * STEP_GROUPS + g, S, P, pay0 + pay, leaf0 + leaf, np.arange(nv))
    return _to_original_order(ps, Wp)
