"""Row-invariant linear layer on the CPU (numpy) -- oracle restatement.

linear             restates respect/kernels/gemm.py:11-41: C = X . W^T with
                   bf16 inputs, fp32 accumulation over the K axis in fixed
                   BK-wide blocks (the block's dot product modelled as an exact
                   sum rounded once to fp32, bf16 x bf16 products being exact in
                   fp32), cast to the output dtype (bf16, or fp32 for the
                   vocabulary projection, patch.py:23).
linear_exact       float64 X . W^T (the mathematical definition).
linear_error_bound per-element bound on |fp32-accumulated result - exact|
                   before the output rounding: K u sum|x w|, u = 2^-24.

Pinned by (tests/test_oracle_gemm.py): linear vs linear_exact rounded to bf16
(at most 1 bf16 ulp, and equal on nearly every element); vs PyTorch's CPU
fp32 matmul; the known answer of one-hot rows (a row of the identity picks
a column of W exactly); row-count invariance of the restatement itself.
"""
from __future__ import annotations

import numpy as np

from .bf16 import round_bf16


def linear_exact(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    return np.asarray(x, np.float64) @ np.asarray(w, np.float64).T


def linear(x: np.ndarray, w: np.ndarray, out_fp32: bool = False, BK: int = 128) -> np.ndarray:
    """gemm.py:30 linear(x, w, BK=...) -- returns float32 arrays (bf16 values unless out_fp32)."""
    x = np.asarray(x, np.float32)
    w = np.asarray(w, np.float32)
    M, K = x.shape
    acc = np.zeros((M, w.shape[0]), np.float32)
    for k0 in range(0, K, BK):  # fixed order, gemm.py:19
        blk = (x[:, k0:k0 + BK].astype(np.float64) @ w[:, k0:k0 + BK].astype(np.float64).T).astype(np.float32)
        acc = (acc + blk).astype(np.float32)
    return acc if out_fp32 else round_bf16(acc)


def linear_error_bound(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    K = x.shape[1]
    return K * 2.0 ** -24 * (np.abs(np.asarray(x, np.float64)) @ np.abs(np.asarray(w, np.float64)).T)
