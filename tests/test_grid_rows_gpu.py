"""Calls with more rows than one grid's y dimension holds (65,535).

The element-wise kernels, the split-K reduction of the linear layer, the vision
RoPE and the decoder's q/k/v epilogue take a row (token) from `blockIdx.y` and
run one launch per 65,535 rows.
Every row of a 66,000-row call must match the oracle (bitwise where the kernel
is bitwise), and the rows on either side of the launch boundary must equal the
same rows computed in a small call.
"""
import numpy as np
import pytest
import torch

from oracle import bf16, gen
from oracle import gemm as G
from oracle import norm as N

pytestmark = pytest.mark.gpu

ROWS = 66000          # two launches: 65,535 rows, then 465
EDGE = slice(65530, 65540)


def _dev(x, dt=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dt).cuda()


def _np(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("cols", [8, 7])
def test_silu_mul_past_grid_rows(cols):
    """Two bf16 per thread (even width) and one (odd width)."""
    from respect_amd.system.fused import silu_mul
    print(f"[silu_mul] rows={ROWS} cols={cols}", flush=True)
    rng = np.random.default_rng(cols)
    g = gen.bf16_normal(rng, (ROWS, cols))
    u = gen.bf16_normal(rng, (ROWS, cols))
    out = silu_mul(_dev(g), _dev(u))
    d = bf16.ulp_diff(_np(out), N.silu_mul(g, u), 1e-30)
    assert d.max() <= 1.0
    assert torch.equal(silu_mul(_dev(g[EDGE]), _dev(u[EDGE])), out[EDGE])


def test_prefill_kernels_past_grid_rows():
    from respect_amd.system.fused import _square, add_sq, rope_vision
    print(f"[prefill] rows={ROWS}", flush=True)
    rng = np.random.default_rng(11)
    r = gen.bf16_normal(rng, (ROWS, 16))
    h = gen.bf16_normal(rng, (ROWS, 16))
    x, q = add_sq(_dev(r), _dev(h))
    ex, eq = N.add_sq(r, h)
    assert np.array_equal(_np(x), ex)
    assert np.array_equal(q.cpu().numpy(), eq)
    assert np.array_equal(_square(_dev(r)).cpu().numpy(), N.square(r))
    # vision RoPE: one row per token, L past the grid's y dimension
    xv = gen.bf16_normal(rng, (ROWS, 1, 16))
    ang = (rng.standard_normal((ROWS, 16)) * 3).astype(np.float32)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    y = _np(rope_vision(_dev(xv), _dev(cos, torch.float32), _dev(sin, torch.float32)))
    assert np.array_equal(y, N.rope_vision(xv, cos, sin))


def test_linear_split_k_reduction_past_grid_rows():
    """[66000, 512] . [16, 512]^T: two K chunks, so the chunk partials are summed
    by the reduction kernel, one launch per 65,535 rows."""
    from respect_amd import _lib
    from respect_amd.kernels.gemm import linear
    assert _lib.lib().rspx_linear_splits(16, 512) > 1
    print(f"[linear] M={ROWS} N=16 K=512", flush=True)
    rng = np.random.default_rng(3)
    x = bf16.round_bf16(rng.standard_normal((ROWS, 512)).astype(np.float32))
    w = bf16.round_bf16(0.02 * rng.standard_normal((16, 512)).astype(np.float32))
    xd, wd = _dev(x), _dev(w)
    out = linear(xd, wd)
    assert torch.equal(linear(xd[EDGE], wd), out[EDGE])
    assert torch.equal(linear(xd[-3:], wd), out[-3:])
    rows = np.r_[0:4, 65530:65540, ROWS - 4:ROWS]
    ex = G.linear_exact(x[rows], w)
    bound = G.linear_error_bound(x[rows], w)
    o = _np(out[torch.from_numpy(rows).cuda()])
    assert np.all(np.abs(o - ex) <= bound + bf16.ulp(np.abs(ex) + bound))


def test_qkv_rope_cache_past_grid_tokens():
    """The decoder's q/k/v epilogue (grid: head rows x tokens) over 66,000 tokens: q, K and
    V rows bitwise those of rspx_qk_norm_rope (a flat grid) and of the packed projection."""
    from respect_amd import _lib
    from respect_amd.system.fused import qk_norm_rope
    T, HQ, HK, D = ROWS, 1, 1, 128
    print(f"[qkv_rope_cache] T={T}", flush=True)
    rng = np.random.default_rng(17)
    q = gen.bf16_normal(rng, (T, HQ, D))
    k = gen.bf16_normal(rng, (T, HK, D))
    v = gen.bf16_normal(rng, (T, HK, D))
    wq = bf16.round_bf16(1 + 0.02 * rng.standard_normal(D).astype(np.float32))
    wk = bf16.round_bf16(1 + 0.02 * rng.standard_normal(D).astype(np.float32))
    cos, sin = N.rope_tables(rng.integers(0, 8192, T), head_dim=D)
    wqd, wkd, cosd, sind = _dev(wq), _dev(wk), _dev(cos), _dev(sin)
    qo, ko = qk_norm_rope(_dev(q), _dev(k), wqd, wkd, 1e-6, cosd, sind)
    L = _lib.lib()
    s = _lib.stream_ptr(torch.device("cuda"))
    qkv = _dev(np.concatenate([q.reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1)], axis=1))
    n = (HQ + 2 * HK) * D
    P = T + 5
    slots = torch.arange(2, 2 + T, dtype=torch.int32, device="cuda")
    ck = torch.zeros(HK, P, D, device="cuda", dtype=torch.bfloat16)
    cv = torch.zeros_like(ck)
    q2 = torch.empty(T, HQ, D, device="cuda", dtype=torch.bfloat16)
    _lib.check("rspx_qkv_rope_cache", L.rspx_qkv_rope_cache(
        qkv.data_ptr(), n, wqd.data_ptr(), wkd.data_ptr(), cosd.data_ptr(), sind.data_ptr(), D,
        slots.data_ptr(), P, ck.data_ptr(), P * D, D, cv.data_ptr(), P * D, D, q2.data_ptr(), T, HQ, HK, D, 1e-6, s))
    torch.cuda.synchronize()
    assert torch.equal(q2, qo)
    assert torch.equal(ck[:, 2:2 + T].transpose(0, 1), ko)
    assert torch.equal(cv[:, 2:2 + T].transpose(0, 1), _dev(v))
