"""The tiled weight layout on the host: TiledWeight.dense() inverts the layout
include/respect_amd.h documents for rspx_linear_tile_weight (the GPU tests check
the packing kernel against the same element-by-element placement)."""
import numpy as np
import pytest
import torch


def _tiled(w, pad=64):
    N, K = w.shape
    out = np.zeros((N // 16) * (16 * K + pad), dtype=w.dtype)
    n, k = np.meshgrid(np.arange(N), np.arange(K), indexing="ij")
    off = (n // 16) * (16 * K + pad) + (k // 32) * 512 + ((n % 16) + 16 * ((k % 32) // 8)) * 8 + k % 8
    out[off.ravel()] = w.ravel()
    return out


@pytest.mark.parametrize("N,K", [(16, 32), (32, 256), (48, 768)])
def test_dense_inverts_the_layout(N, K):
    from respect_amd.kernels.gemm import TiledWeight
    w = np.random.default_rng(N * K).integers(-30000, 30000, (N, K)).astype(np.int16)
    t = TiledWeight(torch.from_numpy(_tiled(w)), N, K)
    assert t.shape == (N, K)
    assert np.array_equal(t.dense().numpy(), w)


def test_layout_places_tiles_in_order_of_k():
    """A wave's 16 rows of one k-block are one contiguous 1 KB tile, and the next
    k-block's tile follows it: lane n + 16 g reads k 8 g .. 8 g + 7."""
    N, K = 16, 64
    w = np.arange(N * K, dtype=np.int32).reshape(N, K)
    t = _tiled(w, pad=0)
    lanes = t[:512].reshape(64, 8)            # first tile, 16-byte chunks by lane
    for lane in range(64):
        n, g = lane % 16, lane // 16
        assert np.array_equal(lanes[lane], w[n, 8 * g:8 * g + 8])
    assert np.array_equal(t[512:1024].reshape(64, 8)[0], w[0, 32:40])
