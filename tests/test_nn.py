"""Host side of the linear layers (tensorpack_amd.nn): construction, accounting and the
checks that need no GPU."""

import numpy as np
import pytest

from tensorpack_amd.nn import LinearMTC, LinearMTCGroup, seeded_fp32_weight


def test_seeded_weight_is_the_reference_fp32_layer_init():
    # LinearFP32 (mtc/nn/layers.py:70-74): U(-1/sqrt(in), 1/sqrt(in)), float32, (in x out),
    # a pure function of the seed
    W = seeded_fp32_weight(64, 96, seed=42)
    assert W.shape == (64, 96) and W.dtype == np.float32
    assert np.abs(W).max() <= 1.0 / 8.0
    assert np.array_equal(W, seeded_fp32_weight(64, 96, seed=42))
    assert not np.array_equal(W, seeded_fp32_weight(64, 96, seed=43))
    # the first draws of the stream are the first row of W (row-major fill)
    u = np.random.RandomState(42).random_sample(96)
    assert np.allclose(W[0], (u * 0.25 - 0.125).astype(np.float32), atol=1e-7)


@pytest.mark.parametrize("permuted", [False, True])
def test_linear_layer_accounting(permuted):
    lin = LinearMTC(128, 64, budget_bits=4.0, seed=3, permuted=permuted)
    assert lin.W_mtc.shape == (128, 64)
    assert lin.weight_bytes == -(-lin.W_mtc.total_bits // 8) + 64 * 4
    assert lin.W_mtc.total_bits <= 4.0 * 128 * 64
    assert lin.alloc.total_bits == lin.W_mtc.total_bits


def test_linear_layer_rejects_bad_shapes():
    with pytest.raises(ValueError):
        LinearMTC(64, 64, weight=np.zeros((32, 64), np.float32))
    with pytest.raises(ValueError):
        LinearMTC(64, 64, bias=np.zeros(63, np.float32))


def test_group_requires_a_shared_input_width():
    a = LinearMTC(64, 32, budget_bits=3.0, seed=1, permuted=False)
    b = LinearMTC(96, 32, budget_bits=3.0, seed=2, permuted=False)
    with pytest.raises(ValueError):
        LinearMTCGroup([a, b])
    with pytest.raises(ValueError):
        LinearMTCGroup([])
    g = LinearMTCGroup([a, LinearMTC(64, 64, budget_bits=3.0, seed=4, permuted=False)])
    assert g.weight_bytes == a.weight_bytes + g.layers[1].weight_bytes
