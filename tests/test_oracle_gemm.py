"""CPU pinning of the linear-layer oracle."""
import numpy as np
import torch

from oracle import bf16, gen
from oracle import gemm as G


def _xw(seed, M, N, K):
    rng = np.random.default_rng(seed)
    return gen.bf16_normal(rng, (M, K)), bf16.round_bf16(0.02 * rng.standard_normal((N, K)).astype(np.float32))


def test_linear_close_to_exact():
    x, w = _xw(0, 9, 96, 512)
    out = G.linear(x, w)
    ex = G.linear_exact(x, w)
    d = bf16.ulp_diff(out, bf16.round_bf16(ex.astype(np.float32)))
    assert d.max() <= 1.0
    assert (out == bf16.round_bf16(ex.astype(np.float32))).mean() > 0.98
    assert np.all(np.abs(G.linear(x, w, out_fp32=True) - ex) <= G.linear_error_bound(x, w))


def test_linear_vs_torch_fp32():
    x, w = _xw(1, 5, 64, 256)
    ref = (torch.from_numpy(x) @ torch.from_numpy(w).T).numpy()
    out = G.linear(x, w, out_fp32=True)
    assert np.all(np.abs(out - ref) <= 2 * G.linear_error_bound(x, w) + 1e-30)


def test_one_hot_rows_pick_columns_exactly():
    _, w = _xw(2, 1, 48, 256)
    x = np.zeros((3, 256), np.float32)
    for i, k in enumerate((0, 77, 255)):
        x[i, k] = 1.0
    out = G.linear(x, w)
    assert np.array_equal(out, w[:, [0, 77, 255]].T)


def test_restatement_is_row_invariant():
    x, w = _xw(3, 16, 32, 256)
    full = G.linear(x, w)
    for m in (1, 7):
        assert np.array_equal(G.linear(x[:m], w), full[:m])
