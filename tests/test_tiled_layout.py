"""The tiled activation layout (RSPX_TILED): the test helpers follow the header's
formula, and the entry points reject what the layout cannot hold before any GPU
work (CPU-only test)."""
import numpy as np
import pytest
import torch

from _tiled import from_tiled, tiled_index, tiled_rows, to_tiled


@pytest.mark.parametrize("M,K", [(1, 32), (7, 64), (64, 96), (130, 256)])
def test_to_tiled_follows_the_formula(M, K):
    a = torch.arange(M * K, dtype=torch.float64).view(M, K)
    t = to_tiled(a, fill=-1.0)
    assert t.numel() == tiled_rows(M) * K
    idx = np.array([[tiled_index(m, k, K) for k in range(K)] for m in range(M)])
    assert np.array_equal(t.numpy()[idx], a.numpy())
    # every position is hit once: valid rows by their element, rows past M by the fill
    assert int((t == -1.0).sum()) == (tiled_rows(M) - M) * K
    assert torch.equal(from_tiled(t, M, K), a)


def test_tile_is_one_mfma_operand():
    """Lane n16 + 16 g of tile (block 0, k-block 0, row tile 1) holds row 16 + n16, k 8 g .. 8 g + 7."""
    K = 64
    a = torch.arange(64 * K, dtype=torch.float64).view(64, K)
    tile = to_tiled(a)[512:1024].view(64, 8)
    for lane in range(64):
        n16, g = lane % 16, lane // 16
        assert torch.equal(tile[lane], a[16 + n16, 8 * g:8 * g + 8])


@pytest.fixture(scope="module")
def lib():
    from respect_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.skip("librespect_amd.so not built")
    return _lib.lib()


def test_entry_points_check_tiled_sizes(lib):
    from respect_amd import _lib
    T = _lib.RSPX_TILED
    p = 1 << 20           # 16-byte aligned stand-in pointer: every call below returns before using it
    # RMSNorm: tiled output needs n % 32 == 0; other negative strides are invalid
    assert lib.rspx_rmsnorm(p, 40, p, p, T, 4, 40, 1e-6, None) == -2
    assert lib.rspx_rmsnorm(p, 64, p, p, -8, 4, 64, 1e-6, None) == -1
    assert lib.rspx_add_rmsnorm_partials(p, 40, p, 1, p, p, 40, p, T, 4, 40, 1e-6, None) == -2
    # SwiGLU epilogue: a tiled output of N / 2 columns needs N / 2 % 32 == 0
    assert lib.rspx_linear_silu(p, T, p, 256, p, T, 4, 32, 256, None) == -1
    # rspx_linear writes row-major only
    assert lib.rspx_linear(p, T, p, 256, p, T, 4, 64, 256, 0, p, 0, None) == -1
