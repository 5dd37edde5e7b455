"""Packer for the prefill kernel: the "tile stream".

The prefill kernel (bf16 MFMA) computes a 256 x 256 output tile per block and
walks the reduction dimension in steps of 64 rows. Its weight operand for one
step is a 64 x 256 slab of Wp, cut into 512 *cells* of 8 rows x 4 columns (one
column group of a panel, one 8-row block). A cell is covered either by a single
leaf of size >= 8 (one code width P, one scale) or by two 4x4 leaves stacked
vertically (top rows 0-3, bottom rows 4-7, each with its own P and scale), so
every cell carries two (P, scale) halves.

Cells are stored in the width class of their wider half, as offset-binary codes
(u = q + 2^(w-1)):

    class W4  (P <= 4):  4 dwords, column j in dword j, byte k = u[row k] | u[row k+4] << 4
    class W8  (P <= 8):  8 dwords, column j in dwords 2j (rows 0-3), 2j+1 (rows 4-7), a byte per row
    class W16 (P = 16): 16 dwords, column j in dwords 4j+h, rows 2h (low half) and 2h+1 (high half)
    class Z   (P0):      no payload

so the device value is (u - 2^(w-1)) * s computed as one fma, exact in fp32,
then rounded once to bf16 (bf16(q * s), as the MFMA operand). Within a step,
cells are sorted by class then position, so a wavefront's 64 cells mostly share
one decode path. Cell descriptor (bf16 scales): word 0 = payload offset within
the step (dwords, bits 0-13) | class << 14 | position << 16, position =
column group in the tile (0-63) * 8 + row block (0-7); word 1 = bf16 scale of
the top half | bf16 scale of the bottom half << 16. With fp32 scales a cell is
4 words: word 0, fp32 top scale, fp32 bottom scale, 0.

Matrices with an output column permutation (QT-P) are packed with their columns
back in the original order ("gathered columns"): column n of the operand is
column inv[n] of Wp (inv the inverse of col_perm), so a tile's outputs are
adjacent columns of Y and its stores need no permutation. The four columns of
a cell then come from four unrelated leaves, so every column carries its own
(P, scale) halves: an 8-word cell, word 0 as above (the class is the widest of
its eight halves), word 1 + j = bf16 top scale | bf16 bottom scale << 16 of
column j, words 5-7 zero. Only bf16 scales take this form.

Steps are ordered column tile major: step = col_tile * n_ksteps + kstep, so a
block reads its column tile's cells and payload front to back.
"""

from dataclasses import dataclass, field
from typing import Dict, Optional, Sequence, Tuple

import numpy as np

TILE_ROWS = 64
TILE_COLS = 256
CELLS = 512
CLS_W4, CLS_W8, CLS_W16, CLS_Z = 0, 1, 2, 3
CLS_DWORDS = np.array([4, 8, 16, 0], dtype=np.int64)
CLS_OFFSET = (8, 128, 32768)
TILE_FORMAT = 2                     # 2: gathered-column cells (8 words) for permuted columns
PAYLOAD_PAD = 8                     # dwords after the last step (see pack_tiles)
_WIDTHS = (2, 3, 4, 5, 6, 8, 16)


@dataclass
class TileStream:
    K: int
    N: int
    n_ksteps: int
    n_col_tiles: int
    cells: np.ndarray                   # uint32 (n_steps * 512, 2) or (n_steps * 512, 4)
    step_off: np.ndarray                # uint32 (n_steps + 1,)
    payload: np.ndarray                 # uint32
    row_perm: Optional[np.ndarray] = None
    col_perm: Optional[np.ndarray] = None
    stats: Dict[str, float] = field(default_factory=dict)

    @property
    def n_steps(self) -> int:
        return self.n_ksteps * self.n_col_tiles

    @property
    def fp32_scales(self) -> bool:
        return self.cells.shape[1] == 4

    @property
    def cols_gathered(self) -> bool:
        """Columns in the original order with a scale per column (8-word cells)."""
        return self.cells.shape[1] == 8

    def nbytes(self) -> int:
        n = self.cells.nbytes + self.step_off.nbytes + self.payload.nbytes
        for a in (self.row_perm, self.col_perm):
            if a is not None:
                n += a.nbytes
        return int(n)


def _scale_words(s: np.ndarray, fp32: bool) -> np.ndarray:
    bits = np.ascontiguousarray(s, dtype=np.float32).view(np.uint32)
    if fp32:
        return bits
    if np.any(bits & 0xFFFF):
        raise ValueError("bf16 scale format requested but some scales are not bf16-representable")
    return bits >> 16


def pack_tiles(shape: Tuple[int, int], sizes: Sequence[int], leaf: Dict[int, np.ndarray],
               modes: Dict[int, np.ndarray], scales: Dict[int, np.ndarray], codes_of,
               scale_format: str = "bf16", row_perm: Optional[np.ndarray] = None,
               col_perm: Optional[np.ndarray] = None, gather_cols: Optional[bool] = None) -> TileStream:
    """Tile stream of the leaves given per level s (see packer.pack_levels for the arguments).
    gather_cols (default: whenever there is a column permutation and the scales are bf16): pack
    the columns in the original order with a scale per column, so the stream has no col_perm."""
    K, N = (int(x) for x in shape)
    if N % 32 or K % 8:
        raise ValueError(f"tile stream needs N % 32 == 0 and K % 8 == 0, got {shape}")
    if scale_format not in ("bf16", "fp32"):
        raise ValueError(scale_format)
    fp32 = scale_format == "fp32"
    if gather_cols is None:
        gather_cols = col_perm is not None and not fp32
    if gather_cols and (fp32 or col_perm is None):
        raise ValueError("gathered columns need a column permutation and bf16 scales")
    nks = -(-K // TILE_ROWS)
    nct = -(-N // TILE_COLS)
    R, G = nks * (TILE_ROWS // 8), nct * (TILE_COLS // 4)          # padded cell grid
    Q = np.zeros((K, N), dtype=np.int32)                            # codes, P0 -> 0
    Pt = np.zeros((R, G), dtype=np.int32)
    Pb = np.zeros((R, G), dtype=np.int32)
    St = np.zeros((R, G), dtype=np.float32)
    Sb = np.zeros((R, G), dtype=np.float32)
    n_leaves = 0
    for S in sorted((int(s) for s in sizes), reverse=True):
        if S not in (32, 16, 8, 4):
            raise ValueError(f"leaf size {S} not supported by the tile stream")
        L = np.asarray(leaf[S], dtype=bool)
        Md = np.asarray(modes[S])
        Sc = np.asarray(scales[S], dtype=np.float32)
        for P in _WIDTHS:
            ii, jj = np.nonzero(L & (Md == P))
            if ii.size == 0:
                continue
            n_leaves += ii.size
            sc = Sc[ii, jj]
            q = np.asarray(codes_of(S, P, ii, jj, sc)).astype(np.int32)      # (n, S, S)
            if K % S or N % S:
                raise ValueError(f"level {S} leaves need K and N divisible by {S}, got {shape}")
            Qv = Q.reshape(K // S, S, N // S, S)
            Qv[ii, :, jj, :] = q
            if S >= 8:
                rb = ii[:, None] * (S // 8) + np.arange(S // 8)
                cg = jj[:, None] * (S // 4) + np.arange(S // 4)
                r_, g_ = rb[:, :, None], cg[:, None, :]
                Pt[r_, g_] = P
                Pb[r_, g_] = P
                St[r_, g_] = sc[:, None, None]
                Sb[r_, g_] = sc[:, None, None]
            else:
                top = ii % 2 == 0
                Pt[ii[top] // 2, jj[top]] = P
                St[ii[top] // 2, jj[top]] = sc[top]
                Pb[ii[~top] // 2, jj[~top]] = P
                Sb[ii[~top] // 2, jj[~top]] = sc[~top]
    if gather_cols:
        # per-column halves, then the original column order: operand column n = Wp column inv[n]
        inv = np.argsort(np.asarray(col_perm, dtype=np.int64), kind="stable")
        cols = np.zeros(G * 4, dtype=np.int64)
        cols[:N] = inv

        def gathered(a):
            out = np.repeat(a, 4, axis=1)[:, cols]
            out[:, N:] = 0
            return out
        Ptc, Pbc, Stc, Sbc = gathered(Pt), gathered(Pb), gathered(St), gathered(Sb)
        Q = Q[:, inv]
        Pm = np.maximum(Ptc, Pbc).reshape(R, G, 4).max(axis=2)
    else:
        Pm = np.maximum(Pt, Pb)
    cls = np.full((R, G), CLS_Z, dtype=np.int64)
    cls[(Pm >= 1) & (Pm <= 4)] = CLS_W4
    cls[(Pm >= 5) & (Pm <= 8)] = CLS_W8
    cls[Pm == 16] = CLS_W16

    # cell order: step (column tile major), then class, then position
    r_all, g_all = np.meshgrid(np.arange(R), np.arange(G), indexing="ij")
    step = (g_all // 64) * nks + r_all // 8
    pos = (g_all % 64) * 8 + r_all % 8
    key = (step.astype(np.int64) * 4 + cls) * 512 + pos
    order = np.argsort(key.reshape(-1), kind="stable")
    r_s, g_s = r_all.reshape(-1)[order], g_all.reshape(-1)[order]
    c_s, step_s, pos_s = cls.reshape(-1)[order], step.reshape(-1)[order], pos.reshape(-1)[order]
    n_steps = nks * nct
    dw = CLS_DWORDS[c_s]
    per_step = dw.reshape(n_steps, CELLS)
    step_tot = per_step.sum(axis=1)
    off_in = (np.cumsum(per_step, axis=1) - per_step).reshape(-1)
    step_off = np.concatenate([[0], np.cumsum(step_tot)]).astype(np.int64)
    if (step_off[-1] + PAYLOAD_PAD) * 4 > 0x7FFFFFFF or n_steps * CELLS * 4 * (8 if gather_cols else 4) > 0x7FFFFFFF:
        raise ValueError("tile stream payload or cells exceed the kernels' 32-bit byte offsets (2 GiB); "
                         "split the matrix by column tiles")
    # 8 dwords of tail padding: the device reads 32 bytes per cell whatever its class
    payload = np.zeros(int(step_off[-1]) + PAYLOAD_PAD, dtype=np.uint32)

    # codes of each cell: (n, 4 columns, 8 rows)
    if Q.shape != (R * 8, G * 4):
        Q = np.pad(Q, ((0, R * 8 - K), (0, G * 4 - N)))
    C = Q.reshape(R, 8, G, 4)
    for c, (width, ndw) in enumerate(zip((4, 8, 16), (4, 8, 16))):
        sel = np.flatnonzero(c_s == c)
        if sel.size == 0:
            continue
        u = (C[r_s[sel], :, g_s[sel], :].transpose(0, 2, 1) + CLS_OFFSET[c]).astype(np.uint32)   # (n, 4, 8)
        if c == CLS_W4:
            b = u[:, :, 0:4] | (u[:, :, 4:8] << 4)                                   # (n, 4, 4) bytes
            words = b[:, :, 0] | (b[:, :, 1] << 8) | (b[:, :, 2] << 16) | (b[:, :, 3] << 24)
        elif c == CLS_W8:
            h = u.reshape(-1, 4, 2, 4)
            words = (h[..., 0] | (h[..., 1] << 8) | (h[..., 2] << 16) | (h[..., 3] << 24)).reshape(-1, 8)
        else:
            h = u.reshape(-1, 4, 4, 2)
            words = (h[..., 0] | (h[..., 1] << 16)).reshape(-1, 16)
        dst = step_off[step_s[sel]] + off_in[sel]
        payload[(dst[:, None] + np.arange(ndw)).reshape(-1)] = words.astype(np.uint32).reshape(-1)

    w0 = (off_in.astype(np.uint32) | (c_s.astype(np.uint32) << 14) | (pos_s.astype(np.uint32) << 16))
    if gather_cols:
        j4 = 4 * g_s[:, None] + np.arange(4)                                    # (n, 4) operand columns
        sw = _scale_words(Stc[r_s[:, None], j4], False) | (_scale_words(Sbc[r_s[:, None], j4], False) << 16)
        z = np.zeros_like(w0)
        cells = np.stack([w0, sw[:, 0], sw[:, 1], sw[:, 2], sw[:, 3], z, z, z], axis=1)
    elif fp32:
        st, sb = St[r_s, g_s], Sb[r_s, g_s]
        cells = np.stack([w0, _scale_words(st, True), _scale_words(sb, True), np.zeros_like(w0)], axis=1)
    else:
        st, sb = St[r_s, g_s], Sb[r_s, g_s]
        cells = np.stack([w0, _scale_words(st, False) | (_scale_words(sb, False) << 16)], axis=1)
    counts = np.bincount(c_s, minlength=4)
    stats = {"payload_bytes": float(4 * step_off[-1]), "cell_bytes": float(cells.nbytes), "n_leaves": float(n_leaves),
             "frac_w4": float(counts[0] / c_s.size), "frac_w8": float(counts[1] / c_s.size),
             "frac_w16": float(counts[2] / c_s.size), "frac_zero": float(counts[3] / c_s.size)}
    return TileStream(K=K, N=N, n_ksteps=nks, n_col_tiles=nct, cells=np.ascontiguousarray(cells.astype(np.uint32)),
                      step_off=step_off.astype(np.uint32), payload=payload,
                      row_perm=None if row_perm is None else np.ascontiguousarray(row_perm, dtype=np.int32),
                      col_perm=None if col_perm is None or gather_cols else np.ascontiguousarray(col_perm, dtype=np.int32),
                      stats=stats)


def decode_tiles(ts: TileStream) -> np.ndarray:
    """Host decoder of a tile stream to W_hat in the original channel order, with
    each element rounded to bf16 exactly as the device kernel stages it. A
    debugging and test aid; the GPU path never calls it."""
    K, N = ts.K, ts.N
    R, G = ts.n_ksteps * 8, ts.n_col_tiles * 64
    Wp = np.zeros((R * 8, G * 4), dtype=np.float32)
    for step in range(ts.n_steps):
        ct, ks = divmod(step, ts.n_ksteps)
        cells = ts.cells[step * CELLS:(step + 1) * CELLS]
        base = int(ts.step_off[step])
        for cell in cells:
            w0 = int(cell[0])
            off, c, pos = w0 & 0x3FFF, (w0 >> 14) & 3, w0 >> 16
            if ts.fp32_scales:
                st, sb = (np.full(4, v, np.float32) for v in cell[1:3].view(np.float32))
            else:
                sw = cell[1:5] if ts.cols_gathered else np.full(4, cell[1], np.uint32)
                st = ((sw.astype(np.uint32) & 0xFFFF) << 16).view(np.float32)
                sb = ((sw.astype(np.uint32) >> 16) << 16).view(np.float32)
            r0, c0 = ks * TILE_ROWS + (pos & 7) * 8, ct * TILE_COLS + (pos >> 3) * 4
            if c == CLS_Z:
                continue
            wds = ts.payload[base + off: base + off + int(CLS_DWORDS[c])].astype(np.int64)
            u = np.zeros((4, 8), np.int64)
            for j in range(4):
                for r in range(8):
                    if c == CLS_W4:
                        u[j, r] = (wds[j] >> (8 * (r % 4) + 4 * (r // 4))) & 0xF
                    elif c == CLS_W8:
                        u[j, r] = (wds[2 * j + r // 4] >> (8 * (r % 4))) & 0xFF
                    else:
                        u[j, r] = (wds[4 * j + r // 2] >> (16 * (r % 2))) & 0xFFFF
            q = (u - CLS_OFFSET[c]).astype(np.float32)
            s = np.concatenate([np.repeat(st[:, None], 4, axis=1), np.repeat(sb[:, None], 4, axis=1)], axis=1)
            Wp[r0:r0 + 8, c0:c0 + 4] = (q * s).T
    Wp = Wp[:K, :N]
    Wp = _bf16_rne(Wp)
    if ts.row_perm is None and ts.col_perm is None:
        return Wp
    pr = np.arange(K) if ts.row_perm is None else ts.row_perm
    pc = np.arange(N) if ts.col_perm is None else ts.col_perm
    out = np.empty_like(Wp)
    out[np.ix_(pr, pc)] = Wp
    return out


def _bf16_rne(x: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    b = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    return (b.astype(np.uint32).view(np.float32) + np.float32(0.0)).reshape(x.shape)
