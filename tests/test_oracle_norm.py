"""CPU pinning of the norm / RoPE / SwiGLU oracle against PyTorch's CPU arithmetic."""
import numpy as np
import torch

from oracle import bf16, gen
from oracle import norm as N


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(torch.bfloat16)


def test_rope_bitwise_vs_torch_bf16_ops():
    rng = np.random.default_rng(0)
    x = gen.bf16_normal(rng, (2, 4, 9, 128))
    cos, sin = N.rope_tables(np.arange(9) + 3000)
    cos, sin = np.broadcast_to(cos, (2, 9, 128)), np.broadcast_to(sin, (2, 9, 128))
    ours = N.rope(x, cos[:, None], sin[:, None])
    xt, ct, st = _t(x), _t(cos)[:, None], _t(sin)[:, None]
    h = 64
    rot = torch.cat((-xt[..., h:], xt[..., :h]), dim=-1)
    ref = (xt * ct) + (rot * st)
    assert np.array_equal(ours, ref.float().numpy())


def test_rmsnorm_vs_hf_formula():
    rng = np.random.default_rng(1)
    x = gen.bf16_normal(rng, (64, 4096))
    w = bf16.round_bf16(1 + 0.02 * rng.standard_normal(4096).astype(np.float32))
    ours = N.rmsnorm(x, w, 1e-6)
    xt = _t(x).float()
    var = xt.pow(2).mean(-1, keepdim=True)
    ref = (_t(w) * (xt * torch.rsqrt(var + 1e-6)).to(torch.bfloat16)).float().numpy()
    d = bf16.ulp_diff(ours, ref)
    assert d.max() <= 1.0 and (ours == ref).mean() > 0.999


def test_rmsnorm_constant_row_closed_form():
    x = np.full((3, 256), 0.75, np.float32)
    w = bf16.round_bf16(np.linspace(0.5, 1.5, 256).astype(np.float32))
    y = N.rmsnorm(x, w, 1e-6)
    # x / rms(x) = 1 up to eps: xh = bf16(~1) = 1 (or 1 - 2^-8), y = bf16(w * xh)
    xh = bf16.round_bf16(np.float32(0.75) * np.float32(1.0 / np.sqrt(0.5625 + 1e-6)))
    assert np.array_equal(y, bf16.round_bf16(w * xh)[None].repeat(3, 0))


def test_silu_mul_vs_torch_and_limits():
    rng = np.random.default_rng(2)
    g = gen.bf16_normal(rng, (64, 1024), 3.0)
    u = gen.bf16_normal(rng, (64, 1024))
    ours = N.silu_mul(g, u)
    ref = (torch.nn.functional.silu(_t(g)) * _t(u)).float().numpy()
    assert bf16.ulp_diff(ours, ref, 1e-30).max() <= 1.0
    z = N.silu_mul(np.array([0.0, 200.0, -200.0], np.float32), np.ones(3, np.float32))
    assert z[0] == 0 and z[1] == 200.0 and z[2] == 0


def test_prefill_square_and_add_sq_bitwise_vs_torch():
    rng = np.random.default_rng(5)
    r = gen.bf16_normal(rng, (7, 256))
    h = gen.bf16_normal(rng, (7, 256))
    assert np.array_equal(N.square(r), (_t(r).float() ** 2).numpy())
    x, q = N.add_sq(r, h)
    xt = _t(r) + _t(h)                       # bf16 add on the CPU: fp32 add, one rounding
    assert np.array_equal(x, xt.float().numpy())
    assert np.array_equal(q, (xt.float() ** 2).numpy())


def test_prefill_norm_apply_vs_torch_and_exact_rsqrt():
    rng = np.random.default_rng(6)
    x = gen.bf16_normal(rng, (16, 512))
    w = bf16.round_bf16(1 + 0.02 * rng.standard_normal(512).astype(np.float32))
    var = (x.astype(np.float32) ** 2).mean(-1).astype(np.float32)
    ours = N.norm_apply(x, var, w, 1e-6)
    xt = _t(x).float()
    ref = (_t(w) * (xt * torch.rsqrt(torch.from_numpy(var)[:, None] + 1e-6)).to(torch.bfloat16)).float().numpy()
    assert bf16.ulp_diff(ours, ref).max() <= 1.0
    # var + eps = 4^k: rsqrt is exact, so y = bf16(w * bf16(x * 2^-k)) exactly
    v = np.array([4.0, 0.25, 16.0, 1.0], np.float32)
    xs = gen.bf16_normal(rng, (4, 64))
    wn = bf16.round_bf16(np.linspace(0.5, 1.5, 64).astype(np.float32))
    y = N.norm_apply(xs, v, wn, 0.0)
    exact = bf16.round_bf16(wn * bf16.round_bf16(xs * (1.0 / np.sqrt(v))[:, None].astype(np.float32)))
    assert np.array_equal(y, exact)


def test_prefill_rope_vision_bitwise_vs_hf_formula():
    rng = np.random.default_rng(7)
    L, NH, D = 9, 3, 80
    x = gen.bf16_normal(rng, (L, NH, D))
    ang = rng.standard_normal((L, D)).astype(np.float32)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    ours = N.rope_vision(x, cos, sin)
    q = _t(x).float()
    c, s = torch.from_numpy(cos)[:, None], torch.from_numpy(sin)[:, None]
    rot = torch.cat((-q[..., D // 2:], q[..., :D // 2]), dim=-1)
    ref = ((q * c) + (rot * s)).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ours, ref)
