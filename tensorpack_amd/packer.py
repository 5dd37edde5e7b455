"""Packer: quadtree (or uniform-block) allocation -> device "panel stream".

Replaces the reference's arena packer (mtc/kernels/gemm.py:432-488,
MTCMatrix.from_allocation) for quadtree leaves. The stream layout is defined
in include/mtc_hip.h; in short:

- work unit = (panel of 32 output columns, chunk of `chunk_rows` reduction rows)
- inside a unit, non-P0 leaves are bucketed by (leaf size S, code width P),
  buckets ordered S = 32, 16, 8, 4 then P ascending, leaves row-major inside
- each bucket is a run of 32-code lane chunks, P dwords each, 16-byte aligned
- one 32-bit word per leaf: row/4, col/4, pad flag, bf16 scale
- P0 leaves are not stored at all

Codes are computed exactly as the reference quantizer does
(clip(round_half_even(w / s)), fp32 division; allocation.py:89-94), so the
device dequantization q * s reproduces W_hat bit for bit.
"""

from dataclasses import dataclass, field
from typing import Callable, Dict, Optional, Sequence, Tuple

import numpy as np

from .core.allocation import quantize_blocks, to_blocks

PANEL = 32
LEAF_SIZES = (32, 16, 8, 4)
CODE_WIDTHS = (2, 3, 4, 5, 6, 8, 16)
LEAF_PAD = 1 << 11
_LOG2 = {32: 5, 16: 4, 8: 3, 4: 2}


@dataclass
class PanelStream:
    """Host image of a panel stream (uploaded as-is by tensorpack_amd.device)."""
    K: int
    N: int
    chunk_rows: int
    payload: np.ndarray                 # uint32
    buckets: np.ndarray                 # uint32 (n_buckets, 4)
    unit_buckets: np.ndarray            # int32 (n_units + 1,)
    leaf_word: np.ndarray               # uint32
    leaf_scale: Optional[np.ndarray]    # float32 or None (bf16 scales in leaf_word)
    row_perm: Optional[np.ndarray] = None   # int32 or None
    col_perm: Optional[np.ndarray] = None   # int32 or None
    n_real_leaves: int = 0
    stats: Dict[str, float] = field(default_factory=dict)

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
    def fp32_scales(self) -> bool:
        return self.leaf_scale is not None

    def nbytes(self) -> int:
        """Device bytes of the stream (payload + tables + permutations)."""
        n = self.payload.nbytes + self.buckets.nbytes + self.unit_buckets.nbytes + self.leaf_word.nbytes
        for a in (self.leaf_scale, self.row_perm, self.col_perm):
            if a is not None:
                n += a.nbytes
        return int(n)


def pack_codes(codes: np.ndarray, P: int) -> np.ndarray:
    """(n, 32) signed codes -> (n, P) uint32; code i at bits [i*P, i*P+P) of the chunk."""
    n = codes.shape[0]
    u = (codes.astype(np.int64) & ((1 << P) - 1)).astype(np.uint64)
    out = np.zeros((n, P), dtype=np.uint64)
    for i in range(32):
        bit = i * P
        j, sh = bit >> 5, bit & 31
        out[:, j] |= (u[:, i] << np.uint64(sh)) & np.uint64(0xFFFFFFFF)
        if sh + P > 32:
            out[:, j + 1] |= u[:, i] >> np.uint64(32 - sh)
    return out.astype(np.uint32)


def unpack_codes(words: np.ndarray, P: int) -> np.ndarray:
    """Inverse of pack_codes: (n, P) uint32 -> (n, 32) int32."""
    w = words.astype(np.uint64)
    n = w.shape[0]
    out = np.empty((n, 32), dtype=np.int64)
    mask = np.uint64((1 << P) - 1)
    for i in range(32):
        bit = i * P
        j, sh = bit >> 5, bit & 31
        v = w[:, j] >> np.uint64(sh)
        if sh + P > 32:
            v |= w[:, j + 1] << np.uint64(32 - sh)
        v &= mask
        out[:, i] = v.astype(np.int64)
    out[out >= (1 << (P - 1))] -= 1 << P
    return out.astype(np.int32)


def _bf16_bits(scale: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(scale, dtype=np.float32).view(np.uint32)
    if np.any(bits & 0xFFFF):
        raise ValueError("bf16 scale format requested but some scales are not bf16-representable")
    return bits >> 16


CodeSource = Callable[[int, int, np.ndarray, np.ndarray, np.ndarray], np.ndarray]


def weight_codes(Wp: np.ndarray) -> CodeSource:
    """Codes of leaves (level S, width P, grid rows ii, cols jj, scales sc) quantized from Wp."""
    Wp = np.asarray(Wp, dtype=np.float32)
    views: Dict[int, np.ndarray] = {}

    def source(S, P, ii, jj, sc):
        if S not in views:
            views[S] = to_blocks(Wp, S)
        return quantize_blocks(views[S][ii, jj][None], P, sc[None])[0]

    return source


def pack_levels(shape: Tuple[int, int], sizes: Sequence[int], leaf: Dict[int, np.ndarray],
                modes: Dict[int, np.ndarray], scales: Dict[int, np.ndarray], codes_of: CodeSource,
                chunk_rows: int = 512, scale_format: str = "bf16", row_perm: Optional[np.ndarray] = None,
                col_perm: Optional[np.ndarray] = None) -> PanelStream:
    """Pack the leaves given per level s (leaf mask, mode grid, scale grid) of a K x N weight.

    `codes_of(S, P, ii, jj, scales)` returns the (n, S, S) integer codes of the
    listed leaves (see weight_codes).
    """
    K, N = (int(x) for x in shape)
    if N % PANEL or K % 4:
        raise ValueError(f"panel stream needs N % {PANEL} == 0 and K % 4 == 0, got {Wp.shape}")
    if chunk_rows % 32 or not 32 <= chunk_rows <= 1024:
        raise ValueError(f"chunk_rows={chunk_rows} must be a multiple of 32 in [32, 1024]")
    if scale_format not in ("bf16", "fp32"):
        raise ValueError(scale_format)
    n_chunks = -(-K // chunk_rows)
    n_units = (N // PANEL) * n_chunks

    # ---- per (S, P) kind: sorted leaves, lane chunks, leaf words -------------------
    kinds = []   # (S, P, unit_of_leaf(padded), chunk words (nc, P), leaf words, leaf scales, per-unit leaf counts)
    n_real = 0
    for S in sorted((int(s) for s in sizes), reverse=True):
        if S not in LEAF_SIZES:
            raise ValueError(f"leaf size {S} not supported by the panel stream (sizes {LEAF_SIZES})")
        lv_leaf = np.asarray(leaf[S], dtype=bool)
        lv_mode = np.asarray(modes[S])
        lv_scale = np.asarray(scales[S], dtype=np.float32)
        for P in CODE_WIDTHS:
            ii, jj = np.nonzero(lv_leaf & (lv_mode == P))
            if ii.size == 0:
                continue
            k0, n0 = ii * S, jj * S
            unit = (n0 // PANEL) * n_chunks + k0 // chunk_rows
            order = np.lexsort((n0, k0, unit))
            ii, jj, k0, n0, unit = ii[order], jj[order], k0[order], n0[order], unit[order]
            sc = lv_scale[ii, jj]
            q = codes_of(S, P, ii, jj, sc)                                     # (n, S, S) codes
            codes = np.asarray(q).astype(np.int32).transpose(0, 2, 1).reshape(len(ii), S * S)   # column-major per leaf
            rowoff = (k0 % chunk_rows) // 4
            coloff = (n0 % PANEL) // 4
            if scale_format == "bf16":
                words = (rowoff | (coloff << 8) | (_bf16_bits(sc) << 16)).astype(np.uint32)
            else:
                words = (rowoff | (coloff << 8)).astype(np.uint32)
            n_real += len(ii)
            counts = np.bincount(unit, minlength=n_units)
            if S == 4:
                # pair leaves per chunk; an odd bucket gets a pad leaf (zero codes, pad flag)
                odd = np.nonzero(counts & 1)[0]
                if odd.size:
                    ends = np.cumsum(counts)[odd]                  # insert after each odd bucket's last leaf
                    codes = np.insert(codes, ends, 0, axis=0)
                    words = np.insert(words, ends, np.uint32(LEAF_PAD))
                    sc = np.insert(sc, ends, np.float32(0))
                    unit = np.insert(unit, ends, odd)
                    counts = counts + (counts & 1)
            chunk_words = pack_codes(codes.reshape(-1, 32), P)
            kinds.append((S, P, counts, chunk_words, words, sc))

    # ---- bucket table: units ascending, kinds in the order built above ----------------
    counts_mat = np.stack([k[2] for k in kinds], axis=1) if kinds else np.zeros((n_units, 0), np.int64)
    present = counts_mat > 0                                        # (n_units, n_kinds)
    unit_idx, kind_idx = np.nonzero(present)                        # row-major: unit, then kind
    n_buckets = unit_idx.size
    unit_buckets = np.zeros(n_units + 1, dtype=np.int32)
    np.cumsum(present.sum(axis=1), out=unit_buckets[1:])
    leaves_per = counts_mat[unit_idx, kind_idx].astype(np.int64)
    S_of = np.array([k[0] for k in kinds], dtype=np.int64)
    P_of = np.array([k[1] for k in kinds], dtype=np.int64)
    Sb, Pb = S_of[kind_idx], P_of[kind_idx]
    chunks_per = leaves_per * Sb * Sb // 32
    dwords = chunks_per * Pb
    aligned = (dwords + 3) & ~3
    pay_off = np.zeros(n_buckets, dtype=np.int64)
    if n_buckets:
        pay_off[1:] = np.cumsum(aligned)[:-1]
    leaf_off = np.zeros(n_buckets, dtype=np.int64)
    if n_buckets:
        leaf_off[1:] = np.cumsum(leaves_per)[:-1]
    total_dw = int(aligned.sum())
    total_leaves = int(leaves_per.sum())
    if total_dw >= 2 ** 32 or total_leaves >= 2 ** 32:
        raise ValueError("stream too large for 32-bit offsets")

    payload = np.zeros(max(total_dw, 4), dtype=np.uint32)
    leaf_word = np.zeros(max(total_leaves, 1), dtype=np.uint32)
    leaf_scale = np.zeros(max(total_leaves, 1), dtype=np.float32) if scale_format == "fp32" else None
    for ki, (S, P, counts, chunk_words, words, sc) in enumerate(kinds):
        sel = np.nonzero(kind_idx == ki)[0]                         # this kind's buckets, unit order
        if sel.size == 0:
            continue
        nl = leaves_per[sel]
        nc = chunks_per[sel]
        # payload: the kind's chunk rows are already in bucket order
        src_start = np.concatenate([[0], np.cumsum(nc)[:-1]])
        dst = np.repeat(pay_off[sel] - src_start * P, nc * P) + np.arange(int(nc.sum()) * P)
        payload[dst] = chunk_words.reshape(-1)
        lsrc = np.concatenate([[0], np.cumsum(nl)[:-1]])
        ldst = np.repeat(leaf_off[sel] - lsrc, nl) + np.arange(int(nl.sum()))
        leaf_word[ldst] = words
        if leaf_scale is not None:
            leaf_scale[ldst] = sc

    buckets = np.zeros((max(n_buckets, 1), 4), dtype=np.uint32)
    if n_buckets:
        buckets[:n_buckets, 0] = pay_off
        buckets[:n_buckets, 1] = leaf_off
        buckets[:n_buckets, 2] = chunks_per
        buckets[:n_buckets, 3] = np.array([_LOG2[int(s)] for s in Sb], dtype=np.uint32) | (Pb.astype(np.uint32) << 8)

    stats = {"payload_bytes": float(total_dw * 4), "n_buckets": float(n_buckets), "n_leaves": float(n_real)}
    return PanelStream(K=K, N=N, chunk_rows=chunk_rows, payload=payload, buckets=buckets, unit_buckets=unit_buckets,
                       leaf_word=leaf_word, leaf_scale=leaf_scale,
                       row_perm=None if row_perm is None else np.ascontiguousarray(row_perm, dtype=np.int32),
                       col_perm=None if col_perm is None else np.ascontiguousarray(col_perm, dtype=np.int32),
                       n_real_leaves=n_real, stats=stats)


def decode_stream(ps: PanelStream) -> np.ndarray:
    """Host decoder of a panel stream back to W_hat (original channel order).

    A debugging aid mirroring the device dequant kernel; the GPU path never calls it.
    """
    K, N = ps.K, ps.N
    Wp = np.zeros((K, N), dtype=np.float32)
    nb = int(ps.unit_buckets[-1])
    for b in range(nb):
        off, l0, nc, key = (int(x) for x in ps.buckets[b])
        S, P = 1 << (key & 0xFF), key >> 8
        u = int(np.searchsorted(ps.unit_buckets, b, side="right") - 1)
        panel, chunk = divmod(u, ps.n_chunks)
        codes = unpack_codes(ps.payload[off: off + nc * P].reshape(nc, P), P).reshape(-1, S * S)
        nleaf = codes.shape[0]
        words = ps.leaf_word[l0: l0 + nleaf]
        for i in range(nleaf):
            wd = int(words[i])
            if wd & LEAF_PAD:
                continue
            r0 = chunk * ps.chunk_rows + (wd & 0xFF) * 4
            c0 = panel * PANEL + ((wd >> 8) & 7) * 4
            s = ps.leaf_scale[l0 + i] if ps.leaf_scale is not None else np.uint32(wd >> 16 << 16).view(np.float32)
            blk = codes[i].reshape(S, S).T.astype(np.float32) * np.float32(s)
            Wp[r0: r0 + S, c0: c0 + S] = blk
    if ps.leaf_scale is None:
        Wp = Wp + np.float32(0.0)      # quadtree W_hat never holds -0.0
    if ps.row_perm is None and ps.col_perm is None:
        return Wp
    pr = np.arange(K) if ps.row_perm is None else ps.row_perm
    pc = np.arange(N) if ps.col_perm is None else ps.col_perm
    out = np.empty_like(Wp)
    out[np.ix_(pr, pc)] = Wp
    return out
