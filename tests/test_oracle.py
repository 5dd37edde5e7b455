"""Pins the CPU oracle itself (oracle/mtc_oracle.py, oracle/cpu_gemm.c) against
independent formulations, so a slip in it (a dropped term, a transposed
operand, a wrong rounding) cannot hide behind agreement with the GPU path:

- quantize_blocks vs a scalar loop with explicit half-even ties
- qt_dequant vs the per-element (scale, lo, hi) RTN grid (the reference's second
  formulation, baselines/gptq.py:119-138 / tests/test_gptq.py:28-35), and vs the
  allocator's own dequant
- permuted dequant vs an explicit index loop
- arena codecs: exhaustive P2 256-combo round trip (tests/test_packing.py:16-27),
  hand-computed bytes, random round trips at every width
- the C block-loop GEMM vs an fp64 product of W_hat
"""

import os
import subprocess

import numpy as np
import pytest

from oracle import mtc_oracle as O
from tensorpack_amd.core.permutation import PermutedQuadtreeRD
from tensorpack_amd.core.quadtree import QuadtreeRD

from conftest import outlier_matrix


@pytest.fixture(scope="module")
def cpu_lib():
    if not os.path.exists(O.CPU_LIB_PATH):
        subprocess.run(["make", "-C", os.path.dirname(O.CPU_LIB_PATH), "-s"], check=True)
    return O.cpu_lib()


def test_qrange_is_twos_complement():
    for m, (lo, hi) in O.QRANGE.items():
        assert lo == -(2 ** (m - 1)) and hi == 2 ** (m - 1) - 1


def test_quantize_blocks_scalar_loop():
    rng = np.random.RandomState(0)
    blocks = (rng.randn(6, 4, 4) * 3).astype(np.float32)
    scales = np.array([0.5, -0.25, 1.0, 0.0, 2.0, -1.0], np.float32)
    blocks[0, 0, :] = [0.25, 0.75, -0.25, -0.75]          # x/s = +-0.5, +-1.5: ties to even
    for m in (2, 3, 4, 8):
        got = O.quantize_blocks(blocks, m, scales)
        lo, hi = O.QRANGE[m]
        for b in range(6):
            s = scales[b] if scales[b] != 0 else np.float32(1.0)
            for i in range(4):
                for j in range(4):
                    v = float(np.float32(blocks[b, i, j] / s))
                    r = round(v)                             # Python round: half to even
                    assert got[b, i, j] == min(max(r, lo), hi)
    assert list(O.quantize_blocks(blocks[:1], 4, scales[:1])[0, 0]) == [0.0, 2.0, -0.0, -2.0]


@pytest.mark.parametrize("budget", [2.2, 3.5, 6.0, 12.0])
def test_qt_dequant_equals_element_grid_rtn(budget):
    W = outlier_matrix(budget.__hash__() % 100, 128, 96)
    a = QuadtreeRD(W, np.exp(np.random.RandomState(1).randn(128)), (32, 16, 8, 4)).select(budget)
    ref = O.qt_dequant(W, a.sizes, a.leaf, a.modes, a.scales)
    S, LO, HI = O.element_grid(a.sizes, a.leaf, a.modes, a.scales, W.shape)
    rtn = O.element_rtn(W, S, LO, HI)
    assert np.array_equal(ref.view(np.uint32), rtn.view(np.uint32))
    assert np.array_equal(ref, a.dequant)
    assert not np.signbit(ref[ref == 0]).any()


def test_permuted_dequant_index_loop():
    rng = np.random.RandomState(2)
    W = (rng.randn(64, 64) * np.exp(rng.randn(64, 1))).astype(np.float32)
    a = PermutedQuadtreeRD(W, np.exp(rng.randn(64)), (32, 16, 8)).select(3.0)
    i = a.inner
    got = O.permuted_qt_dequant(W, a.row_perm, a.col_perm, i.sizes, i.leaf, i.modes, i.scales)
    Wp = W[a.row_perm][:, a.col_perm]
    inner = O.qt_dequant(Wp, i.sizes, i.leaf, i.modes, i.scales)
    want = np.empty_like(W)
    for r in range(64):
        for c in range(64):
            want[a.row_perm[r], a.col_perm[c]] = inner[r, c]
    assert np.array_equal(got, want)
    assert np.array_equal(got, a.dequant)


def test_arena_p2_exhaustive_and_layout():
    combos = np.array([[a, b, c, d] for a in range(-2, 2) for b in range(-2, 2) for c in range(-2, 2)
                       for d in range(-2, 2)], dtype=np.int64)
    packed = O.arena_pack(combos, 2)
    assert packed.shape == (256, 1) and len(set(packed[:, 0].tolist())) == 256
    assert np.array_equal(O.arena_unpack(packed, 2, 4), combos)
    # element 4j at bits 0-1 (packing.py:11-19)
    assert O.arena_pack(np.array([[1, -2, 0, -1]]), 2)[0, 0] == (1 | (2 << 2) | (0 << 4) | (3 << 6))
    # P4: low nibble first (gemm.py:466-468)
    assert O.arena_pack(np.array([[1, -2]]), 4)[0, 0] == 0xE1
    # P3 LSB-first bitstream (gemm.py:99-117): codes 3, -1, 2 -> bits 011 111 010
    assert list(O.arena_pack(np.array([[3, -1, 2, 0, 0, 0, 0, 0]]), 3)[0]) == [0b10111011, 0b00000000, 0]


@pytest.mark.parametrize("mode", [2, 3, 4, 5, 6, 8, 16])
def test_arena_round_trip(mode):
    lo, hi = O.QRANGE[mode]
    q = np.random.RandomState(mode).randint(lo, hi + 1, size=(7, 64))
    data = O.arena_pack(q, mode)
    assert data.shape[1] == mode * 64 // 8
    assert np.array_equal(O.arena_unpack(data, mode, 64), q)


def test_relative_frobenius_error_closed_form():
    y = np.array([[3.0, 4.0]])
    assert O.relative_frobenius_error(y, y * 0.0) == pytest.approx(1.0)
    assert O.relative_frobenius_error(y, y + np.array([[0.0, 5e-1]])) == pytest.approx(0.1)
    assert O.relative_frobenius_error(np.zeros((1, 2)), np.array([[3.0, 4.0]])) == pytest.approx(5.0)


@pytest.mark.parametrize("perm", [False, True])
def test_cpu_block_loop_gemm_matches_fp64(cpu_lib, perm):
    W = outlier_matrix(7, 192, 96)
    h = np.exp(np.random.RandomState(3).randn(192))
    if perm:
        a = PermutedQuadtreeRD(W, h, (32, 16, 8, 4)).select(4.0)
        i = a.inner
        la = O.LeafArena(W[a.row_perm][:, a.col_perm], i.sizes, i.leaf, i.modes, i.scales, a.row_perm, a.col_perm)
    else:
        a = QuadtreeRD(W, h, (32, 16, 8, 4)).select(4.0)
        la = O.LeafArena(W, a.sizes, a.leaf, a.modes, a.scales)
    X = np.random.RandomState(4).randn(5, 192).astype(np.float32)
    Y = O.cpu_qt_gemm(X, la, n_threads=2)
    assert O.relative_frobenius_error(O.qt_gemm_f64(X, a.dequant), Y) < 1e-6
    # a wrong transpose or a dropped scale is far outside that bar
    assert O.relative_frobenius_error(O.qt_gemm_f64(X, a.dequant), Y * 1.001) > 1e-4


def test_bf16_round_ties_to_even():
    x = np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -1.5, 0.0], np.float32)
    assert list(O.bf16_round(x)) == [1.0, 1.0 + 2 ** -6, -1.5, 0.0]


def test_uniform_to_array_zero_signs_and_values():
    """The uniform arena's rebuild (integer codes x scale, gemm.py:510-538) against rd_dequant
    (allocation.py:359-369): equal as values; worked by hand on one 4x4 block at P2, scale 0.5:
    w = -0.1 rounds to the code 0, so rd_dequant keeps np.round's -0.0 and the arena gives
    0 * 0.5 = +0.0; w = 0.2 and -0.3 (codes 0 and -1) and a P0 block (scale 0) give +0.0 / -0.5."""
    W = np.zeros((4, 8), np.float32)
    W[0, 0], W[0, 1], W[0, 2] = -0.1, 0.2, -0.3
    modes = np.array([[2, 0]])
    scales = np.array([[0.5, 0.0]], np.float32)
    dq = O.uniform_dequant(W, modes, scales, 4)
    ta = O.uniform_to_array(W, modes, scales, 4)
    assert np.signbit(dq[0, 0]) and not np.signbit(ta[0, 0])
    assert ta[0, 1] == 0.0 and not np.signbit(ta[0, 1]) and ta[0, 2] == -0.5
    assert not np.signbit(ta[:, 4:]).any() and (ta[:, 4:] == 0).all()
    assert np.array_equal(dq, ta)


@pytest.mark.parametrize("layout", [0, 1])
def test_uniform_to_array_is_the_stream_decode(layout):
    """Both panel-stream layouts of a uniform-form matrix decode on the host to the oracle's
    arena rebuild bit for bit (the GPU dequantizer follows the same streams)."""
    from tensorpack_amd.core.allocation import rd_allocate
    from tensorpack_amd.kernels.gemm import MTCMatrix
    from tensorpack_amd.packer import decode_stream
    rng = np.random.RandomState(7)
    W = rng.randn(64, 96).astype(np.float32)
    al = rd_allocate(W, 3.3, None, 16)
    m = MTCMatrix.from_allocation(W, al.modes, al.scales, 16)
    got = decode_stream(m.panel_stream(64, layout))
    assert np.array_equal(got.view(np.uint32), O.uniform_to_array(W, al.modes, al.scales, 16).view(np.uint32))
