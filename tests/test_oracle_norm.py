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
