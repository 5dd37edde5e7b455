"""Packer: the panel stream must carry exactly the oracle's W_hat (host decode,
bit-exact), keep its layout invariants, and the uniform-block arena must keep
the reference byte layout."""

import numpy as np
import pytest
from hypothesis import given, settings, strategies as st

from oracle import mtc_oracle as O
from tensorpack_amd.core.allocation import rd_allocate_pair
from tensorpack_amd.core.permutation import PermutedQuadtreeRD
from tensorpack_amd.core.quadtree import QuadtreeRD
from tensorpack_amd.kernels.gemm import MTCMatrix, arena_decode, arena_encode
from tensorpack_amd.packer import (BLOCKS_PER_UNIT, LEAF_PAD, MAX_FIXED_STEPS, N_GROUPS, STEP_GROUPS, STEP_LANES,
                                   STEP_WORDS, decode_stream, decode_steps, pack_codes, pack_levels, record_slots,
                                   split_leaves, step_record_index, storage_plan, storage_widths, unpack_codes)

from conftest import kind_mix_stream, largest_unit_stream, outlier_matrix


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _oracle(alloc, W):
    if hasattr(alloc, "inner"):
        i = alloc.inner
        return O.permuted_qt_dequant(W, alloc.row_perm, alloc.col_perm, i.sizes, i.leaf, i.modes, i.scales)
    return O.qt_dequant(W, alloc.sizes, alloc.leaf, alloc.modes, alloc.scales)


@pytest.mark.parametrize("P", [2, 3, 4, 5, 6, 8, 16])
def test_pack_codes_round_trip_and_bit_order(P):
    lo, hi = -(1 << (P - 1)), (1 << (P - 1)) - 1
    q = np.random.RandomState(P).randint(lo, hi + 1, size=(9, 32))
    w = pack_codes(q, P)
    assert w.shape == (9, P)
    assert np.array_equal(unpack_codes(w, P), q)
    # offset-binary: q = -2^(P-1) packs to all-zero bits; u = 1 for code 1 starts at bit P
    # (P = 3 too: code 1 is byte lane 0's second code, at bit 3 of dword 0)
    one = np.full((1, 32), lo, np.int64)
    one[0, 1] = lo + 1
    w1 = pack_codes(one, P)
    assert w1[0, P // 32] == 1 << (P % 32) and int(w1.astype(np.int64).sum()) == 1 << (P % 32)
    assert np.all(pack_codes(np.zeros((1, 32), np.int64), P)[0] != 0)
    with pytest.raises(ValueError):
        pack_codes(np.full((1, 32), hi + 1), P)
    # every code read back from where the layout puts it, by explicit bit strings
    u = q + (1 << (P - 1))
    for n in range(q.shape[0]):
        if P == 3:          # byte lane b of the 3 dwords: codes 8b .. 8b+7 at bits 3a
            for b in range(4):
                lane = sum(((int(w[n, k]) >> (8 * b)) & 0xFF) << (8 * k) for k in range(3))
                assert [(lane >> (3 * a)) & 7 for a in range(8)] == list(u[n, 8 * b: 8 * b + 8])
        else:               # LSB-first over the chunk
            bits = sum(int(w[n, k]) << (32 * k) for k in range(P))
            assert [(bits >> (i * P)) & ((1 << P) - 1) for i in range(32)] == list(u[n])


CASES = [(QuadtreeRD, 2.2), (QuadtreeRD, 4.25), (QuadtreeRD, 9.0), (QuadtreeRD, 15.0),
         (PermutedQuadtreeRD, 2.5), (PermutedQuadtreeRD, 4.25)]


@pytest.mark.parametrize("cls,budget", CASES)
@pytest.mark.parametrize("chunk_rows", [32, 96, 256])
def test_stream_decodes_to_oracle_w_hat(cls, budget, chunk_rows):
    W = outlier_matrix(int(budget * 10), 256, 160)
    h = np.exp(np.random.RandomState(9).randn(256))
    a = cls(W, h, (32, 16, 8, 4)).select(budget)
    ps = MTCMatrix.from_quadtree(a, W).panel_stream(chunk_rows)
    assert np.array_equal(_bits(decode_stream(ps)), _bits(_oracle(a, W)))


def test_stream_layout_invariants():
    W = outlier_matrix(11, 256, 128)
    a = QuadtreeRD(W, None, (32, 16, 8, 4)).select(3.0)
    ps = MTCMatrix.from_quadtree(a, W).panel_stream(128)
    h = ps.unit_hdr
    assert np.all(h[:, 0] % 4 == 0) and np.all(h[:-1, 1] == h[1:, 0])
    assert np.all(h[:-1, 5] == h[1:, 4]) and np.all(h[:-1, 3] == h[1:, 2])
    assert np.all(np.diff(h[:, 8:17], axis=1) >= 0) and np.all(h[:, 16] == h[:, 5] - h[:, 4])
    assert np.all(np.diff(h[:, 17:26], axis=1) >= 0) and np.all(h[:, 25] == h[:, 1] - h[:, 0])
    nb = ps.n_buckets
    b = ps.buckets[:nb]
    assert np.all(b[:, 0] % 4 == 0)
    S, P = 1 << (b[:, 3] & 0xFF), b[:, 3] >> 8
    assert set(S.tolist()) <= {4, 8, 16, 32} and set(P.tolist()) <= {2, 3, 4, 5, 6, 8, 16}
    # chunk counts: every non-P0 weight once (S=4 pad leaves are zero codes)
    area = sum(int((a.leaf[s] & (a.modes[s] != 0)).sum()) * s * s for s in a.sizes)
    n_chunks = int((b[:, 2] & 0xFFFF).sum())
    pads = int(np.sum(ps.leaf_word & LEAF_PAD != 0))
    assert n_chunks * 32 == area + 16 * pads
    # per column group the chunk index restarts at 0 and runs contiguously
    for u in range(ps.n_units):
        for g in range(N_GROUPS):
            lo_, hi_ = h[u, 4] + h[u, 8 + g], h[u, 4] + h[u, 9 + g]
            start = 0
            for k in range(lo_, hi_):
                assert ps.buckets[k, 2] >> 16 == start
                start += ps.buckets[k, 2] & 0xFFFF


@pytest.mark.parametrize("merge", [False, True])
def test_payload_accounting_matches_allocator_bits(merge):
    """Unmerged, the chunk words hold exactly the allocator's payload bits (plus S = 4 pad
    leaves); merged, every leaf is stored at its storage width, which is at least its mode,
    and a split 16 x 16 or 32 x 32 leaf as its 8 x 8 sub-leaves (storage_plan)."""
    W = outlier_matrix(12, 256, 256)
    a = QuadtreeRD(W, None, (32, 16, 8, 4)).select(4.0)
    lv = MTCMatrix.from_quadtree(a, W)._levels
    ps = pack_levels(lv.shape, lv.sizes, lv.leaf, lv.modes, lv.scales, lv.codes_of, 256, lv.scale_format,
                     lv.row_perm, lv.col_perm, merge_kinds=merge)
    sizes, leaf, modes, widths, split = storage_plan((256, 256), a.sizes, a.leaf, a.modes, 256, merge)
    assert merge or not split
    for s in sizes:
        stored = leaf[s] & (modes[s] > 0)
        assert (widths[s][stored] >= modes[s][stored]).all()
    # the split levels hold the allocator's leaves: every weight of a stored leaf once, at its mode
    assert sum(int((leaf[s] & (modes[s] == m)).sum()) * s * s * m for s in sizes for m in (2, 3, 4, 5, 6, 8, 16)) == \
        sum(int((a.leaf[s] & (a.modes[s] == m)).sum()) * s * s * m for s in a.sizes for m in (2, 3, 4, 5, 6, 8, 16))
    payload_bits = sum(int((leaf[s] & (modes[s] > 0) & (widths[s] == m)).sum()) * s * s * m
                       for s in sizes for m in (2, 3, 4, 5, 6, 8, 16))
    if not merge:
        assert payload_bits == sum(int((a.leaf[s] & (a.modes[s] == m)).sum()) * s * s * m
                                   for s in a.sizes for m in (2, 3, 4, 5, 6, 8, 16))
    b = ps.buckets[:ps.n_buckets]
    n, P = (b[:, 2] & 0xFFFF).astype(np.int64), (b[:, 3] >> 8).astype(np.int64)
    # chunk words = stored payload + the zero codes of S=4 pad leaves (16 codes each)
    pad_bits = 0
    for k in np.flatnonzero((b[:, 3] & 0xFF) == 2):
        u = int(np.searchsorted(ps.unit_hdr[:, 5], k, side="right"))
        l0 = ps.unit_hdr[u, 2] + b[k, 1]
        pad_bits += 16 * int(P[k]) * int(np.sum(ps.leaf_word[l0: l0 + 2 * n[k]] & LEAF_PAD != 0))
    assert int((n * P * 32).sum()) == payload_bits + pad_bits
    # each bucket is then padded to 16 bytes
    assert ps.stats["payload_bytes"] * 8 == int((((n * P + 3) // 4) * 4 * 32).sum())


@settings(max_examples=15, deadline=None)
@given(seed=st.integers(0, 10 ** 6), budget=st.floats(1.8, 12.0), rows=st.sampled_from([64, 128]),
       perm=st.booleans(), sizes=st.sampled_from([(32, 16, 8, 4), (16, 8, 4), (8, 4), (4,), (32,)]))
def test_fuzz_leaf_mixes(seed, budget, rows, perm, sizes):
    rng = np.random.RandomState(seed)
    W = (rng.randn(rows, 64) * 10.0 ** rng.uniform(-2, 1, size=(rows, 1))).astype(np.float32)
    W[rng.rand(rows, 64) < 0.03] = 20.0
    cls = PermutedQuadtreeRD if perm else QuadtreeRD
    try:
        a = cls(W, np.exp(rng.randn(rows)), sizes).select(budget)
    except ValueError:
        return                                             # budget below this size set's floor
    ps = MTCMatrix.from_quadtree(a, W).panel_stream(32 * int(rng.randint(1, 4)))
    assert np.array_equal(_bits(decode_stream(ps)), _bits(_oracle(a, W)))


# ---------------- uniform-block arena (reference layout) ----------------
@pytest.mark.parametrize("mode", [2, 3, 4, 5, 6, 8, 16])
def test_arena_codec_matches_oracle(mode):
    lo, hi = O.QRANGE[mode]
    q = np.random.RandomState(mode + 50).randint(lo, hi + 1, size=(5, 256))
    enc = arena_encode(q, mode)
    assert np.array_equal(enc, O.arena_pack(q, mode))
    assert np.array_equal(arena_decode(enc, mode, 256), q)


def test_uniform_from_allocation_layout_and_accounting():
    rng = np.random.RandomState(5)
    A = rng.randn(128, 96).astype(np.float32)
    B = rng.randn(96, 64).astype(np.float32)
    A[:, :32] *= 1e-4
    B[32:64] *= 20.0
    a, b = rd_allocate_pair(A, B, 3.3)
    Am = MTCMatrix.from_allocation(A, a.modes, a.scales, 16)
    assert Am.total_bytes_allocated * 8 == a.payload_bits
    # the arena holds the reference byte layout: decode it block by block
    blocks = O.blocks_of(A, 16)
    for i in range(Am.offsets.shape[0]):
        for j in range(Am.offsets.shape[1]):
            m = int(Am.precisions[i, j])
            if m == 0:
                continue
            nb = m * 256 // 8
            raw = Am.arena.raw_buffer[int(Am.offsets[i, j]): int(Am.offsets[i, j]) + nb][None]
            q = O.arena_unpack(raw, m, 256).reshape(16, 16)
            want = O.quantize_blocks(blocks[i, j][None], m, np.array([a.scales[i, j]], np.float32))[0]
            assert np.array_equal(q, want)
    # and its panel stream decodes to the allocator's dequant (fp32 scales)
    ps = Am.panel_stream(64)
    assert ps.fp32_scales
    np.testing.assert_array_equal(decode_stream(ps), a.dequant)


# ---------------- decode step records ----------------

@pytest.mark.parametrize("cls,budget", [(QuadtreeRD, 2.2), (QuadtreeRD, 9.0), (PermutedQuadtreeRD, 4.25)])
@pytest.mark.parametrize("chunk_rows", [32, 256])
def test_step_records_decode_to_oracle_w_hat(cls, budget, chunk_rows):
    W = outlier_matrix(int(budget * 10) + 1, 256, 160)
    a = cls(W, np.exp(np.random.RandomState(4).randn(256)), (32, 16, 8, 4)).select(budget)
    ps = MTCMatrix.from_quadtree(a, W).panel_stream(chunk_rows)
    assert np.array_equal(_bits(decode_steps(ps)), _bits(_oracle(a, W)))


def test_step_records_cover_every_chunk_once():
    W = outlier_matrix(21, 512, 256)
    a = QuadtreeRD(W, None, (32, 16, 8, 4)).select(3.5)
    ps = MTCMatrix.from_quadtree(a, W).panel_stream(256)
    h, st = ps.unit_hdr.astype(np.int64), ps.steps.astype(np.int64)
    F, nb = ps.fixed_steps, ps.n_units * BLOCKS_PER_UNIT
    n = np.concatenate([h[:, 28:29], h[:, 30:31]], axis=1).reshape(-1)          # records per block
    assert F % STEP_LANES == 0 and F <= MAX_FIXED_STEPS and F >= min(n.max(), MAX_FIXED_STEPS)
    # table = fixed area, one null record, then the blocks' overflow records in block order
    assert st.shape == (nb * F + 1 + int(np.maximum(n - F, 0).sum()), STEP_WORDS)
    assert record_slots(st[nb * F])[2] == [(0, 0, 0)] * STEP_GROUPS
    used = np.zeros(st.shape[0], bool)
    seen = {}
    for u in range(ps.n_units):
        for blk in range(BLOCKS_PER_UNIT):
            steps_of = {}                                 # kind -> steps seen so far in this block
            for r in range(int(h[u, 28 + 2 * blk])):
                i = step_record_index(ps, u, blk, r)
                assert not used[i]
                used[i] = True
                S, P, slots = record_slots(st[i])
                assert max(nv for _, _, nv in slots) > 0 and max(nv for _, _, nv in slots) <= STEP_LANES
                key = (S.bit_length() - 1) | (P << 8)
                j = steps_of.get(key, 0)                  # a block's records of a kind are its steps in order
                steps_of[key] = j + 1
                for g, (pay, leaf, nv) in enumerate(slots):
                    cg = blk * STEP_GROUPS + g
                    if nv == 0:
                        assert (pay, leaf) == (0, 0)
                        continue
                    # the slot names chunk 16 j of this column group's bucket of the kind
                    b = [k for k in range(h[u, 4] + h[u, 8 + cg], h[u, 4] + h[u, 9 + cg]) if int(ps.buckets[k, 3]) == key]
                    assert len(b) == 1
                    pb, lb = int(ps.buckets[b[0], 0]), int(ps.buckets[b[0], 1])
                    assert pay == pb + STEP_LANES * j * P
                    assert leaf == lb + (2 * STEP_LANES * j if S == 4 else STEP_LANES * j // (S // 8))
                    assert nv == min(max(int(ps.buckets[b[0], 2] & 0xFFFF) - STEP_LANES * j, 0), STEP_LANES)
                    for t in range(STEP_LANES * j, STEP_LANES * j + nv):
                        assert (b[0], t) not in seen
                        seen[(b[0], t)] = 1
    # every record the blocks do not own is a null record
    assert np.all(st[~used][:, 0::2] == 0) and np.all(st[~used][:, 1::2] >> 8 == 0)
    assert np.all(st[:, 1::2] == st[:, 1:2])             # every slot carries the same kind-and-counts word
    expect = {(k, t) for k in range(ps.n_buckets) for t in range(int(ps.buckets[k, 2] & 0xFFFF))}
    assert set(seen) == expect


def test_step_records_address_the_largest_unit():
    """A 4096-row unit of P16 4x4 leaves only: the step records' 16-bit unit-relative offsets
    reach their largest values (payload dword 65536 - 256 of the last step, leaf 8192 - 32)
    and still decode to W_hat bit for bit."""
    ps, W_hat = largest_unit_stream()
    assert ps.n_units == 1 and ps.payload.size >= 65536 and ps.n_real_leaves == 8192
    seen = [record_slots(r)[2] for r in ps.steps]
    assert max(pay for sl in seen for pay, _, nv in sl if nv) == 65536 - STEP_LANES * 16
    assert max(leaf for sl in seen for _, leaf, nv in sl if nv) == 8192 - 2 * STEP_LANES
    assert np.array_equal(_bits(decode_steps(ps)), _bits(W_hat))
    assert np.array_equal(_bits(decode_stream(ps)), _bits(W_hat))


def test_step_records_overflow_past_the_fixed_area():
    ps = kind_mix_stream()
    n = np.concatenate([ps.unit_hdr[:, 28], ps.unit_hdr[:, 30]])
    assert n.max() > MAX_FIXED_STEPS and ps.fixed_steps == MAX_FIXED_STEPS
    assert ps.steps.shape[0] > ps.n_units * BLOCKS_PER_UNIT * MAX_FIXED_STEPS + 1
    assert np.array_equal(_bits(decode_steps(ps)), _bits(decode_stream(ps)))
    ps.validate()                         # the overflow records pass the record bounds checks


def _records(ps):
    return int((ps.steps[:, 1] >> 8 > 0).sum())


def test_storage_widths_merge_rare_kinds_within_the_byte_limit():
    """One unit of 256 rows x 32 columns of 8x8 leaves (leaf (i, j): rows 8i.., column groups
    2j, 2j + 1; blocks of 4 column groups). Worked by hand: a lone P2 leaf among 31 P3 leaves
    of its column pair costs a record of its own; stored at P3 it fits the P3 records (32
    chunks per group either way: 2 records), so it is merged. Fifteen P2 leaves (one full
    record) and one P16 leaf: merged they fit one record, but the 30 P2 chunks would grow by
    14 bits per code, 1680 bytes for one record saved, so they stay."""
    shape, S = (256, 32), 8
    leaf = {S: np.ones((32, 4), bool)}
    modes = {S: np.zeros((32, 4), np.int64)}
    modes[S][:, 0] = 3
    modes[S][0, 0] = 2
    w = storage_widths(shape, (S,), leaf, modes, 256)[S]
    assert w[0, 0] == 3 and (w[1:, 0] == 3).all() and (w[:, 1:] == 0).all()
    modes[S][:, 0] = 0
    modes[S][:15, 1] = 2
    modes[S][15, 1] = 16
    w = storage_widths(shape, (S,), leaf, modes, 256)[S]
    assert (w[:15, 1] == 2).all() and w[15, 1] == 16
    # the decision covers the unit: a P2 leaf in the other block (column groups 4-7) keeps
    # its record either way (2 + 1 records before, 2 merged: one saved for 32 chunks x 56
    # bytes), so nothing is merged
    modes[S][0, 2] = 2
    w = storage_widths(shape, (S,), leaf, modes, 256)[S]
    assert (w[:15, 1] == 2).all() and w[15, 1] == 16 and w[0, 2] == 2


def test_split_leaves_join_the_8x8_records_within_the_byte_limit():
    """One unit of 256 rows x 32 columns. Worked by hand: column groups 0-1 hold 30 P3 8x8
    leaves (rows 0-239, 30 chunks per group: 2 records) and the rows 240-255 hold one P3
    16 x 16 leaf over column groups 0-3 (2 chunks per group: a record of its own). Split into
    four 8 x 8 leaves it adds 2 chunks to groups 0-1 (32: still 2 records) and 2 to groups 2-3,
    so one record is saved for 3 extra leaf words (12 bytes): it is split. A 32 x 32 P16 leaf
    alone in the other block has no 8 x 8 leaves to join and stays."""
    shape = (256, 32)
    leaf = {32: np.zeros((8, 1), bool), 16: np.zeros((16, 2), bool), 8: np.zeros((32, 4), bool)}
    modes = {S: np.zeros(g.shape, np.int64) for S, g in leaf.items()}
    leaf[8][:30, 0], modes[8][:30, 0] = True, 3
    leaf[16][15, 0], modes[16][15, 0] = True, 3
    sizes = (32, 16, 8)
    w = storage_widths(shape, sizes, leaf, modes, 256)
    sp = split_leaves(shape, sizes, leaf, w, 256)
    assert sp[16][15, 0] and sp[16].sum() == 1 and not sp[32].any()
    # a lone 32 x 32 leaf: splitting it would add 15 leaf words and save no record
    leaf[32][0, 0], modes[32][0, 0] = True, 16
    leaf[8][:4, :] = False
    sp = split_leaves(shape, sizes, leaf, storage_widths(shape, sizes, leaf, modes, 256), 256)
    assert not sp[32].any()
    # the split stream decodes to the same W_hat as the unsplit one
    rng = np.random.RandomState(3)
    scales = {S: (2.0 ** rng.randint(-8, -2, size=g.shape)).astype(np.float32) for S, g in leaf.items()}
    base = {S: rng.randint(0, 1 << 16, size=g.shape + (S, S)) for S, g in leaf.items()}
    codes = lambda S, P, ii, jj, sc: base[S][ii, jj] % (1 << P) - (1 << (P - 1))
    p0 = pack_levels(shape, sizes, leaf, modes, scales, codes, 256, merge_kinds=False)
    p1 = pack_levels(shape, sizes, leaf, modes, scales, codes, 256, merge_kinds=True)
    assert p1.n_real_leaves == p0.n_real_leaves + 3                # the 16 x 16 leaf as four 8 x 8
    assert _records(p1) == _records(p0) - 1
    ref = _bits(decode_stream(p0))
    assert np.array_equal(_bits(decode_stream(p1)), ref) and np.array_equal(_bits(decode_steps(p1)), ref)


@pytest.mark.parametrize("budget,chunk_rows,perm", [(2.5, 128, False), (3.25, 256, True), (4.0, 64, True)])
def test_merged_kinds_decode_to_the_same_w_hat(budget, chunk_rows, perm):
    """Merged and unmerged streams of one allocation decode to the same W_hat bit for bit, by
    the bucket walk and by the step-record walk; merging never adds records."""
    W = outlier_matrix(31, 512, 256)
    h = np.exp(np.random.RandomState(5).randn(512))
    a = (PermutedQuadtreeRD(W, h, (32, 16, 8, 4)) if perm else QuadtreeRD(W, None, (32, 16, 8, 4))).select(budget)
    lv = MTCMatrix.from_quadtree(a, W)._levels
    args = (lv.shape, lv.sizes, lv.leaf, lv.modes, lv.scales, lv.codes_of, chunk_rows, lv.scale_format,
            lv.row_perm, lv.col_perm)
    p0, p1 = pack_levels(*args, merge_kinds=False), pack_levels(*args, merge_kinds=True)
    ref = _bits(decode_stream(p0))
    assert np.array_equal(_bits(decode_stream(p1)), ref)
    assert np.array_equal(_bits(decode_steps(p1)), ref)
    assert _records(p1) <= _records(p0)
    widths = storage_widths(lv.shape, lv.sizes, lv.leaf, lv.modes, chunk_rows)
    assert any((widths[s] != np.where(lv.leaf[s] & (lv.modes[s] > 0), lv.modes[s], 0)).any() for s in lv.sizes)


@settings(max_examples=20, deadline=None)
@given(seed=st.integers(0, 10 ** 6), rows=st.sampled_from([64, 128, 256]), chunk=st.sampled_from([32, 64, 128]),
       sizes=st.sampled_from([(32, 16, 8, 4), (16, 8, 4), (8, 4), (4,), (32,), (32, 16, 4), (32, 4)]))
def test_fuzz_storage_widths(seed, rows, chunk, sizes):
    """Random leaf mixes: a stored width is never narrower than the mode and at most
    MERGE_MAX_WIDEN bits wider, P0 leaves are never stored, and the merged stream (rare kinds
    widened, large leaves split into 8 x 8 ones, also where the allocation has no 8 x 8 level)
    decodes to the unmerged stream's W_hat bit for bit (bucket walk and step-record walk) with
    no more step records."""
    from tensorpack_amd.packer import CODE_WIDTHS, MERGE_MAX_WIDEN
    rng = np.random.RandomState(seed)
    K, N = rows, 64
    chunk = min(chunk, K)
    # a random quadtree-like cover: each 32 x 32 root tile is split to one leaf size of `sizes`
    leaf = {s: np.zeros((K // s, N // s), bool) for s in sizes}
    modes = {s: np.zeros((K // s, N // s), np.int64) for s in sizes}
    scales = {s: (2.0 ** rng.randint(-8, 0, size=(K // s, N // s))).astype(np.float32) for s in sizes}
    widths_all = np.array((0,) + tuple(CODE_WIDTHS))
    for i in range(K // 32):
        for j in range(N // 32):
            s = int(rng.choice(sizes))
            r = 32 // s
            leaf[s][i * r:(i + 1) * r, j * r:(j + 1) * r] = True
            modes[s][i * r:(i + 1) * r, j * r:(j + 1) * r] = widths_all[rng.randint(0, len(widths_all), size=(r, r))]
    # codes a fixed function of the leaf (packing calls it per kind, in any grouping)
    base = {s: rng.randint(0, 1 << 16, size=(K // s, N // s, s, s)) for s in sizes}
    codes = lambda S, P, ii, jj, sc: base[S][ii, jj] % (1 << P) - (1 << (P - 1))
    args = ((K, N), sizes, leaf, modes, scales, codes, chunk)
    w = storage_widths((K, N), sizes, leaf, modes, chunk)
    for s in sizes:
        stored = leaf[s] & (modes[s] > 0)
        assert (w[s][~stored] == 0).all()
        d = w[s][stored] - modes[s][stored]
        assert (d >= 0).all() and (d <= MERGE_MAX_WIDEN).all()
        assert np.isin(w[s][stored], CODE_WIDTHS).all()
    p0, p1 = pack_levels(*args, merge_kinds=False), pack_levels(*args, merge_kinds=True)
    ref = _bits(decode_stream(p0))
    assert np.array_equal(_bits(decode_stream(p1)), ref)
    assert np.array_equal(_bits(decode_steps(p1)), ref)
    assert _records(p1) <= _records(p0)


@pytest.mark.parametrize("chunk", [64, 256])
def test_negative_scales_decode_exactly(chunk):
    """Scales may be negative: both host walks of the panel stream, and the tile stream's
    host decode, give W_hat = q * s (+0.0 for a zero code) from the grids directly."""
    from tensorpack_amd.tilestream import decode_tiles, pack_tiles
    from conftest import signed_scale_levels
    args, W_hat = signed_scale_levels()
    assert any((args[4][s] < 0).any() for s in args[1])
    ps = pack_levels(*args, chunk_rows=chunk)
    assert np.array_equal(_bits(decode_stream(ps)), _bits(W_hat))
    assert np.array_equal(_bits(decode_steps(ps)), _bits(W_hat))
    ts = pack_tiles(*args)
    assert np.array_equal(_bits(decode_tiles(ts) + np.float32(0.0)), _bits(O.bf16_round(W_hat) + np.float32(0.0)))


def test_step_records_survive_save_load(tmp_path):
    W = outlier_matrix(22, 128, 64)
    a = QuadtreeRD(W, None, (32, 16, 8, 4)).select(4.0)
    ps = MTCMatrix.from_quadtree(a, W).panel_stream(64)
    f = tmp_path / "s.npz"
    ps.save(str(f))
    back = type(ps).load(str(f))
    assert np.array_equal(back.steps, ps.steps) and np.array_equal(back.unit_hdr, ps.unit_hdr)
    assert np.array_equal(_bits(decode_steps(back)), _bits(decode_stream(ps)))


@pytest.mark.parametrize("K,N,M", [(4096, 4096, 1), (4096, 4096, 16), (8192, 8192, 1), (4864, 896, 1),
                                   (4864, 896, 16), (896, 896, 1), (896, 4864, 1), (896, 128, 1), (10000, 64, 1),
                                   (100, 64, 1)])
def test_decode_row_chunks_are_even_and_fill_the_chip(K, N, M):
    from tensorpack_amd.kernels.gemm import DECODE_FILL_BLOCKS, DECODE_MIN_SPLIT_ROWS, _decode_blocks_per_unit, \
        _decode_mt, _decode_row_cap, _decode_x_budget, gemv_chunk_rows
    c = gemv_chunk_rows(K, N, M)
    rows = -(-K // 32) * 32
    cap = _decode_row_cap(M)
    assert cap * 4 * _decode_mt(M) <= _decode_x_budget(_decode_mt(M))   # the staged X rows fit on chip
    n = -(-rows // c)
    assert c % 32 == 0 and 32 <= c <= cap
    if rows <= cap:
        assert n == 1                                   # no split when the X rows fit on chip
    else:
        need = -(-rows // cap)
        assert n >= need
        assert rows - (n - 1) * c > 0 and (n - 1) * c < rows      # every chunk holds rows
        assert c - (rows - (n - 1) * c) < 32 * n        # chunks are equal up to 32-row rounding
        if n > need:                                    # a split beyond the minimum only to fill the chip
            assert _decode_blocks_per_unit(M) * (N // 32) * (n - 1) < DECODE_FILL_BLOCKS \
                and c >= DECODE_MIN_SPLIT_ROWS - 32


# ---------------- matrix-core (mx) payload layout ----------------

@pytest.mark.parametrize("S", [4, 8])
@pytest.mark.parametrize("P", [2, 3, 4, 5, 6, 8, 16])
def test_mx_pack_round_trip_and_bit_order(P, S):
    """mx_pack stores quad lane j's codes as half-strings: over the W-bit plane pl of every
    code, dwords pl W .. pl W + W - 1 of lane j read as two 16 W-bit strings (their low
    16-bit halves, their high halves); code o of a string sits at bits [o W, o W + W) and is
    chunk o // 4's code at column j, chunk row 2 (o % 4) (low halves) or 2 (o % 4) + 1
    (high halves), chunk rows indexed into the chunk's code order by mx_rows."""
    from tensorpack_amd.packer import MX_PLANES, mx_pack, mx_rows, mx_unpack
    lo, hi = -(1 << (P - 1)), (1 << (P - 1)) - 1
    q = np.random.RandomState(P + S).randint(lo, hi + 1, size=(3, 4, 32))
    w = mx_pack(q, S, P)
    assert w.shape == (3, 4, P) and w.dtype == np.uint32
    assert np.array_equal(mx_unpack(w, S, P), q)
    with pytest.raises(ValueError):
        mx_pack(np.full((1, 4, 32), hi + 1), S, P)
    # chunk row order: 8x8 leaves keep column-major rows of 8, a 4x4 leaf pair splits at row 4
    ci = mx_rows(S)
    assert sorted(ci.reshape(-1)) == list(range(32))
    assert ci[1, 0] == (4 if S == 4 else 8) and ci[0, 4] == (16 if S == 4 else 4)
    W, npl = MX_PLANES[P]
    assert W * npl == P
    u = q + (1 << (P - 1))
    for n in range(q.shape[0]):
        for j in range(4):
            for pl in range(npl):
                dw = [int(w[n, j, pl * W + k]) for k in range(W)]
                for half in (0, 1):
                    s = sum(((d >> (16 * half)) & 0xFFFF) << (16 * k) for k, d in enumerate(dw))
                    for o in range(16):
                        code = int(u[n, o // 4, ci[j, 2 * (o % 4) + half]])
                        assert (s >> (o * W)) & ((1 << W) - 1) == (code >> (8 * pl)) & ((1 << W) - 1)


@pytest.mark.parametrize("cls,budget", [(QuadtreeRD, 2.2), (QuadtreeRD, 9.0), (QuadtreeRD, 15.0),
                                        (PermutedQuadtreeRD, 4.25)])
@pytest.mark.parametrize("chunk_rows", [32, 256])
def test_mx_stream_decodes_to_oracle_w_hat(cls, budget, chunk_rows, tmp_path):
    """The mx layout carries the same W_hat as the chunk-contiguous one: both host walks
    (bucket table, step records) decode it bit for bit, its buckets are padded to whole
    quads, it validates, and the layout survives save/load."""
    from tensorpack_amd.packer import LAYOUT_MX
    W = outlier_matrix(int(budget * 10) + 3, 256, 160)
    a = cls(W, np.exp(np.random.RandomState(5).randn(256)), (32, 16, 8, 4)).select(budget)
    m = MTCMatrix.from_quadtree(a, W)
    ps = m.panel_stream(chunk_rows, LAYOUT_MX)
    v1 = m.panel_stream(chunk_rows)
    assert ps.layout == LAYOUT_MX and v1.layout == 0
    ref = _bits(_oracle(a, W))
    assert np.array_equal(_bits(decode_stream(ps)), ref)
    assert np.array_equal(_bits(decode_steps(ps)), ref)
    ps.validate()
    # same buckets and records; each bucket's payload padded to a multiple of 4 chunks
    assert np.array_equal(ps.buckets[:, 1:], v1.buckets[:, 1:]) and np.array_equal(ps.leaf_word, v1.leaf_word)
    P = ps.buckets[:, 3].astype(np.int64) >> 8
    n = ps.buckets[:, 2].astype(np.int64) & 0xFFFF
    assert ps.payload.size >= int((((n + 3) // 4) * 4 * P).sum()) >= v1.payload.size
    f = tmp_path / "mx.npz"
    ps.save(str(f))
    back = type(ps).load(str(f))
    assert back.layout == LAYOUT_MX
    assert np.array_equal(_bits(decode_stream(back)), ref)


def test_mx_stream_rejects_a_short_payload():
    from tensorpack_amd.packer import LAYOUT_MX
    W = outlier_matrix(31, 128, 64)
    m = MTCMatrix.from_quadtree(QuadtreeRD(W, None, (32, 16, 8, 4)).select(3.0), W)
    ps = m.panel_stream(64, LAYOUT_MX)
    ps.validate()
    ps.payload = ps.payload[:-1]
    with pytest.raises(ValueError):
        ps.validate()
