"""Seeded synthetic workloads for benchmarks and tests.

Five single-matrix / stack configurations (weights stored K x N = in x out):

  c1  1024 x 1024 N(0,1), QuadtreeRD (32,16,8,4) @ 3.125 b, X 64 x 1024
  c2  4096 x 4096 Student-t(4) * 0.02, 1% outlier input channels x20,
      PermutedQuadtreeRD @ 4.25 b, X at M = 1 and 16
  c3  Qwen2.5-0.5B-shaped stack: 24 x {q,o 896x896; k,v 896x128;
      gate,up 896x4864; down 4864x896} N(0, 0.02), 0.5% outlier channels x15,
      PermutedQuadtreeRD @ 3.125 b each, M = 1 and 512
  c4  8192 x 8192 Student-t(4) * 0.02, QuadtreeRD @ 4.5 b, X 4096 x 8192 bf16
  c5  4096 x 4096 blocks N(0,1) * 10^U(-3,2) per 32x32 block, 2% entries
      +-25, h ~ LogNormal(0,1), QuadtreeRD @ 2.5 b, M = 1 and 256

Seeds: np.random.RandomState with W = 1000c, X_cal = 1000c+1, X = 1000c+2,
masks / outlier channels = 1000c+3. The Student-t weight recipe follows the
reference's llm_like generator (mtc/benchmarks/benchmark_pareto.py:141-153);
the adversarial block-scale / outlier recipes follow generate_matrix
(mtc/benchmarks/benchmark_runner.py:21-51).
"""

from dataclasses import dataclass
from typing import Callable, List, Optional, Tuple

import numpy as np

from .core.permutation import PermutedQuadtreeRD
from .core.quadtree import QuadtreeRD

SIZES = (32, 16, 8, 4)


@dataclass
class MatrixWorkload:
    name: str
    W: np.ndarray
    h: Optional[np.ndarray]
    permuted: bool
    budget: float
    chan_scale: Optional[np.ndarray]     # per-input-channel activation scale (None = 1)
    seed: int

    def allocate(self, n_threads: int = 0):
        cls = PermutedQuadtreeRD if self.permuted else QuadtreeRD
        return cls(self.W, self.h, SIZES, n_threads=n_threads).select(self.budget)

    def activations(self, M: int, dtype=np.float32) -> np.ndarray:
        rng = np.random.RandomState(self.seed + 2)
        X = rng.randn(M, self.W.shape[0])
        if self.chan_scale is not None:
            X = X * self.chan_scale
        return X.astype(dtype)


def _outlier_channels(K: int, frac_count: int, factor: float, seed: int) -> np.ndarray:
    scale = np.ones(K)
    idx = np.random.RandomState(seed).choice(K, size=max(1, frac_count), replace=False)
    scale[idx] = factor
    return scale


def c1() -> MatrixWorkload:
    base = 1000
    W = np.random.RandomState(base).randn(1024, 1024).astype(np.float32)
    X_cal = np.random.RandomState(base + 1).randn(256, 1024).astype(np.float32)
    h = (X_cal.astype(np.float64) ** 2).mean(axis=0)
    return MatrixWorkload("c1-1024x1024-qt-3.125", W, h, False, 3.125, None, base)


def c2() -> MatrixWorkload:
    base, K, N = 2000, 4096, 4096
    W = (np.random.RandomState(base).standard_t(4, size=(K, N)) * 0.02).astype(np.float32)
    chan = _outlier_channels(K, K // 100, 20.0, base + 3)
    X_cal = (np.random.RandomState(base + 1).randn(512, K) * chan).astype(np.float32)
    h = (X_cal.astype(np.float64) ** 2).mean(axis=0)
    return MatrixWorkload("c2-4096x4096-qtp-4.25", W, h, True, 4.25, chan, base)


def c4() -> MatrixWorkload:
    base, K, N = 4000, 8192, 8192
    W = (np.random.RandomState(base).standard_t(4, size=(K, N)) * 0.02).astype(np.float32)
    X_cal = np.random.RandomState(base + 1).randn(512, K).astype(np.float32)
    h = (X_cal.astype(np.float64) ** 2).mean(axis=0)
    return MatrixWorkload("c4-8192x8192-qt-4.5", W, h, False, 4.5, None, base)


def c5() -> MatrixWorkload:
    base, K, N = 5000, 4096, 4096
    rng = np.random.RandomState(base)
    W = rng.randn(K, N).astype(np.float32)
    u = rng.uniform(-3.0, 2.0, size=(K // 32, N // 32))
    W *= np.repeat(np.repeat(10.0 ** u, 32, axis=0), 32, axis=1).astype(np.float32)
    mrng = np.random.RandomState(base + 3)
    mask = mrng.rand(K, N) < 0.02
    W[mask] = np.where(mrng.rand(int(mask.sum())) < 0.5, -25.0, 25.0).astype(np.float32)
    h = np.random.RandomState(base + 1).lognormal(0.0, 1.0, K)
    return MatrixWorkload("c5-4096x4096-adversarial-qt-2.5", W, h, False, 2.5, None, base)


QWEN_LAYER = (("q", 896, 896), ("k", 896, 128), ("v", 896, 128), ("o", 896, 896),
              ("gate", 896, 4864), ("up", 896, 4864), ("down", 4864, 896))


def c3_matrices(n_layers: int = 24) -> List[MatrixWorkload]:
    base = 3000
    out = []
    for layer in range(n_layers):
        for j, (name, K, N) in enumerate(QWEN_LAYER):
            s = base + 10 * (layer * len(QWEN_LAYER) + j)
            W = (np.random.RandomState(s).randn(K, N) * 0.02).astype(np.float32)
            chan = _outlier_channels(K, int(round(K * 0.005)), 15.0, s + 3)
            X_cal = (np.random.RandomState(s + 1).randn(256, K) * chan).astype(np.float32)
            h = (X_cal.astype(np.float64) ** 2).mean(axis=0)
            out.append(MatrixWorkload(f"c3-L{layer}-{name}-{K}x{N}", W, h, True, 3.125, chan, s))
    return out


CONFIGS = {"c1": c1, "c2": c2, "c4": c4, "c5": c5}


def _allocate_one(w: MatrixWorkload):
    return w.allocate(n_threads=1)


def allocate_many(mats: List[MatrixWorkload], processes: int = 0) -> list:
    """Allocations of many matrices at once: one forked worker process per CPU (at most 16, the
    size of a GPU host's share), each running one matrix's allocator single-threaded. Results are
    those of `w.allocate()` (the allocator is deterministic; its thread count does not change
    its decisions). Fork only from a process that has not initialised the GPU yet."""
    import multiprocessing as mp
    import os
    n = processes or min(16, len(os.sched_getaffinity(0)))
    if n <= 1 or len(mats) <= 1:
        return [w.allocate() for w in mats]
    with mp.get_context("fork").Pool(min(n, len(mats))) as pool:
        return pool.map(_allocate_one, mats, chunksize=1)
