"""GPU parity of the Prefill / Flow element-wise kernels (respect/system/fused.py).

Bars: square, add_sq and rope_vision bitwise against the oracle (the
reference's arithmetic = PyTorch's fp32 / bf16 operations); the Prefill
RMSNorm bitwise against the oracle's norm_apply fed with the same mean of the
squares (the mean is PyTorch's in both, as in the reference); row-count
invariance bitwise.
"""
import numpy as np
import pytest
import torch

from oracle import bf16, gen
from oracle import norm as N

pytestmark = pytest.mark.gpu


def _dev(x, dt=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dt).cuda()


def _np(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("rows,n", [(64, 4096), (3, 1024), (1, 128), (17, 12288)])
def test_add_sq_and_square_bitwise(rows, n):
    from respect_amd.system.fused import _square, add_sq
    print(f"[add_sq] rows={rows} n={n}", flush=True)
    rng = np.random.default_rng(n + rows)
    r = gen.bf16_normal(rng, (rows, n))
    h = gen.bf16_normal(rng, (rows, n))
    x, q = add_sq(_dev(r), _dev(h))
    ex, eq = N.add_sq(r, h)
    assert np.array_equal(_np(x), ex)
    assert np.array_equal(q.cpu().numpy(), eq)
    sq = _square(_dev(r))
    assert np.array_equal(sq.cpu().numpy(), N.square(r))


@pytest.mark.parametrize("rows,n", [(64, 4096), (5, 2048), (2, 128)])
def test_prefill_rmsnorm_bitwise(rows, n):
    from respect_amd.system.fused import rmsnorm
    print(f"[prefill rmsnorm] rows={rows} n={n}", flush=True)
    rng = np.random.default_rng(3 * n + rows)
    x = gen.bf16_normal(rng, (rows, n))
    w = bf16.round_bf16(1 + 0.02 * rng.standard_normal(n).astype(np.float32))
    xd = _dev(x)
    y = _np(rmsnorm(xd, _dev(w), 1e-6))
    var = (xd.float() ** 2).mean(-1).cpu().numpy()     # PyTorch's mean, as the wrapper takes it
    assert np.array_equal(y, N.norm_apply(x, var, w, 1e-6))
    # against the decode-path formula (float64 mean): within 1 bf16 ulp
    assert bf16.ulp_diff(y, N.rmsnorm(x, w, 1e-6)).max() <= 1.0


def test_prefill_kernels_row_count_invariant():
    from respect_amd.system.fused import add_sq, norm_from
    rng = np.random.default_rng(11)
    r = gen.bf16_normal(rng, (40, 1024))
    h = gen.bf16_normal(rng, (40, 1024))
    w = _dev(bf16.round_bf16(1 + 0.02 * rng.standard_normal(1024).astype(np.float32)))
    x, q = add_sq(_dev(r), _dev(h))
    y = norm_from(x, q, w, 1e-6)
    for lo, hi in ((0, 1), (7, 9), (13, 40)):
        x2, q2 = add_sq(_dev(r[lo:hi]), _dev(h[lo:hi]))
        assert torch.equal(x2, x[lo:hi]) and torch.equal(q2, q[lo:hi])
        assert torch.equal(norm_from(x2, q2, w, 1e-6), y[lo:hi])


@pytest.mark.parametrize("L,NH,D", [(64, 16, 80), (7, 3, 128), (1, 1, 16)])
def test_rope_vision_bitwise(L, NH, D):
    from respect_amd.system.fused import rope_vision
    print(f"[rope_vision] L={L} NH={NH} D={D}", flush=True)
    rng = np.random.default_rng(L * NH + D)
    x = gen.bf16_normal(rng, (L, NH, D))
    ang = (rng.standard_normal((L, D)) * 3).astype(np.float32)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    y = _np(rope_vision(_dev(x), _dev(cos, torch.float32), _dev(sin, torch.float32)))
    assert np.array_equal(y, N.rope_vision(x, cos, sin))
    # a strided view (q of a packed qkv) gives the same bits
    packed = torch.zeros((L, 3, NH, D), dtype=torch.bfloat16, device="cuda")
    packed[:, 1] = _dev(x)
    y2 = _np(rope_vision(packed[:, 1], _dev(cos, torch.float32), _dev(sin, torch.float32)))
    assert np.array_equal(y2, y)


def test_prefill_errors():
    from respect_amd import _lib
    from respect_amd.system.fused import add_sq, norm_from, rope_vision
    L = _lib.lib()
    x = torch.zeros((4, 12), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(_lib.RspxError):
        add_sq(x, x)                                       # n % 8 != 0
    with pytest.raises(TypeError):
        add_sq(x.float(), x.float())
    with pytest.raises(ValueError):
        norm_from(torch.zeros((4, 16), dtype=torch.bfloat16, device="cuda"),
                  torch.zeros((4, 16)), torch.zeros(16, dtype=torch.bfloat16, device="cuda"), 1e-6)
    with pytest.raises(RuntimeError):
        rope_vision(torch.zeros((2, 2, 16), dtype=torch.bfloat16, device="cuda"), torch.zeros(2, 16), torch.zeros(2, 16))
    assert L.rspx_rope_vision(0, 16, 16, 0, 0, 16, 0, 2, 2, 24, 0) == -2   # D % 16 != 0
    assert L.rspx_square(0, 8, 0, 8, 0, 8, 0) == 0                          # no rows: nothing to do
