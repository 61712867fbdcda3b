"""GPU parity and row-invariance tests of RMSNorm, RoPE, q/k-norm+RoPE and SwiGLU.

Parity bars: RoPE bitwise against the oracle (= PyTorch's bf16 elementwise
ops); RMSNorm and SwiGLU within 1 bf16 ulp of the oracle (the reduction order,
the rsqrt and the exp differ from PyTorch's CPU implementation); q/k norm +
RoPE bitwise equal to RMSNorm followed by RoPE.  Row invariance is bitwise.
"""
import numpy as np
import pytest
import torch

from oracle import bf16, gen
from oracle import norm as N

pytestmark = pytest.mark.gpu


def _dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(torch.bfloat16).cuda()


def _np(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("rows,n", [(64, 4096), (64, 128), (5, 512), (3, 1024), (2, 12288), (2, 16384), (9, 2048)])
def test_rmsnorm_parity(rows, n):
    from respect_amd.kernels.rmsnorm import rmsnorm
    print(f"[rmsnorm] rows={rows} n={n}", flush=True)
    rng = np.random.default_rng(n)
    x = gen.bf16_normal(rng, (rows, n))
    w = bf16.round_bf16(1 + 0.02 * rng.standard_normal(n).astype(np.float32))
    out = _np(rmsnorm(_dev(x), _dev(w), 1e-6))
    ref = N.rmsnorm(x, w, 1e-6)
    d = bf16.ulp_diff(out, ref)
    print(f"  max ulp {d.max():.2f}, equal {(out == ref).mean():.5f}", flush=True)
    assert d.max() <= 1.0


def test_rmsnorm_row_count_invariant():
    """tests/test_kernel_invariance.py:20-27 of the reference, plus more row counts."""
    from respect_amd.kernels.rmsnorm import rmsnorm
    torch.manual_seed(0)
    x = torch.randn(64, 4096, device="cuda", dtype=torch.bfloat16)
    w = torch.randn(4096, device="cuda", dtype=torch.bfloat16)
    full = rmsnorm(x, w, 1e-6)
    for m in (1, 7, 33):
        assert torch.equal(rmsnorm(x[:m], w, 1e-6), full[:m])
    # rows taken from the middle, and a 3-D input
    assert torch.equal(rmsnorm(x[20:21], w, 1e-6), full[20:21])
    assert torch.equal(rmsnorm(x.view(4, 16, 4096), w, 1e-6).view(64, 4096), full)


def test_rope_bitwise():
    from respect_amd.system.fused import rope
    rng = np.random.default_rng(3)
    B, H, L, D = 1, 32, 64, 128
    x = gen.bf16_normal(rng, (B, H, L, D))
    pos = 3072 + rng.integers(0, 24, L)          # KV offset + trie depth
    cos, sin = N.rope_tables(pos)
    out = _np(rope(_dev(x), _dev(cos[None]), _dev(sin[None])))
    assert np.array_equal(out, N.rope(x, cos[None, None], sin[None, None]))
    # strided x (heads and tokens swapped in memory) gives the same bits
    xs = _dev(x).transpose(1, 2).contiguous().transpose(1, 2)
    assert np.array_equal(_np(rope(xs, _dev(cos[None]), _dev(sin[None]))), out)


def test_qk_norm_rope_equals_norm_then_rope():
    from respect_amd.kernels.rmsnorm import rmsnorm
    from respect_amd.system.fused import qk_norm_rope, rope
    rng = np.random.default_rng(4)
    T, HQ, HK, D = 64, 32, 8, 128
    q = gen.bf16_normal(rng, (T, HQ, D))
    k = gen.bf16_normal(rng, (T, HK, D))
    wq = bf16.round_bf16(1 + 0.02 * rng.standard_normal(D).astype(np.float32))
    wk = bf16.round_bf16(1 + 0.02 * rng.standard_normal(D).astype(np.float32))
    cos, sin = N.rope_tables(3072 + rng.integers(0, 24, T))
    qo, ko = qk_norm_rope(_dev(q), _dev(k), _dev(wq), _dev(wk), 1e-6, _dev(cos), _dev(sin))
    # composition of the two kernels, in the [B, H, L, D] layout rope expects
    qn = rmsnorm(_dev(q), _dev(wq), 1e-6).transpose(0, 1)[None]
    kn = rmsnorm(_dev(k), _dev(wk), 1e-6).transpose(0, 1)[None]
    q2 = rope(qn, _dev(cos)[None], _dev(sin)[None])[0].transpose(0, 1)
    k2 = rope(kn, _dev(cos)[None], _dev(sin)[None])[0].transpose(0, 1)
    assert torch.equal(qo, q2) and torch.equal(ko, k2)
    # oracle composition (RMSNorm within 1 ulp, so compare through the oracle's own norm)
    ref_q = N.rope(N.rmsnorm(q, wq, 1e-6), cos[:, None], sin[:, None])
    assert bf16.ulp_diff(_np(qo), ref_q).max() <= 2.0
    # token-count invariance
    q1, k1 = qk_norm_rope(_dev(q[5:6]), _dev(k[5:6]), _dev(wq), _dev(wk), 1e-6, _dev(cos[5:6]), _dev(sin[5:6]))
    assert torch.equal(q1[0], qo[5]) and torch.equal(k1[0], ko[5])


def test_silu_mul_parity_packed_gate_up():
    """Config shape: gate/up packed as [64, 2 x 12288] -> [64, 12288]."""
    from respect_amd.system.fused import silu_mul
    rng = np.random.default_rng(5)
    F = 12288
    gu = gen.bf16_normal(rng, (64, 2 * F))
    gud = _dev(gu)
    out = silu_mul(gud[:, :F], gud[:, F:])
    ref = N.silu_mul(gu[:, :F], gu[:, F:])
    o = _np(out)
    d = bf16.ulp_diff(o, ref, 1e-30)
    print(f"  silu_mul max ulp {d.max():.2f}, equal {(o == ref).mean():.5f}", flush=True)
    assert d.max() <= 1.0
    assert torch.equal(silu_mul(gud[7:8, :F], gud[7:8, F:]), out[7:8])
    # contiguous separate tensors give the same bits
    assert torch.equal(silu_mul(gud[:, :F].contiguous(), gud[:, F:].contiguous()), out)


def test_kernel_errors():
    from respect_amd._lib import RspxError
    from respect_amd.kernels.rmsnorm import rmsnorm
    from respect_amd.system.fused import rope, silu_mul
    x = torch.randn(4, 100, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError):   # w shorter than the row
        rmsnorm(x, torch.ones(96, device="cuda", dtype=torch.bfloat16), 1e-6)
    with pytest.raises(TypeError):
        silu_mul(x.float(), x.float())
    with pytest.raises(RspxError):   # head_dim not a multiple of 16
        c = torch.ones(1, 2, 72, device="cuda", dtype=torch.bfloat16)
        rope(torch.ones(1, 1, 2, 72, device="cuda", dtype=torch.bfloat16), c, c)


@pytest.mark.parametrize("rows,n", [(1, 4096), (7, 4096), (64, 4096), (130, 4096), (9, 256), (64, 12288)])
def test_rmsnorm_tiled_output(rows, n):
    """y written in the tiled layout (RSPX_TILED) holds the row-major result's bits, for
    rspx_rmsnorm and rspx_add_rmsnorm_partials, and nothing outside rows [0, rows)."""
    from _tiled import from_tiled, tiled_rows
    from respect_amd import _lib
    print(f"[rmsnorm tiled] rows={rows} n={n}", flush=True)
    L = _lib.lib()
    s = _lib.stream_ptr(torch.device("cuda"))
    g = torch.Generator(device="cuda").manual_seed(rows * 13 + n)
    x = torch.randn((rows, n), generator=g, device="cuda").to(torch.bfloat16)
    w = (1 + 0.02 * torch.randn(n, generator=g, device="cuda")).to(torch.bfloat16)
    hp = torch.randn((2, rows, n), generator=g, device="cuda")
    ref = torch.empty_like(x)
    out = torch.full((tiled_rows(rows) * n,), float("nan"), dtype=torch.bfloat16, device="cuda")
    _lib.check("rspx_rmsnorm", L.rspx_rmsnorm(x.data_ptr(), n, w.data_ptr(), ref.data_ptr(), n, rows, n, 1e-6, s))
    _lib.check("rspx_rmsnorm", L.rspx_rmsnorm(x.data_ptr(), n, w.data_ptr(), out.data_ptr(), _lib.RSPX_TILED, rows,
                                              n, 1e-6, s))
    torch.cuda.synchronize()
    assert torch.equal(from_tiled(out, rows, n), ref)
    assert torch.isnan(out.float()).sum().item() == (tiled_rows(rows) - rows) * n
    xo1, xo2 = torch.empty_like(x), torch.empty_like(x)
    _lib.check("rspx_add_rmsnorm_partials", L.rspx_add_rmsnorm_partials(
        x.data_ptr(), n, hp.data_ptr(), 2, w.data_ptr(), xo1.data_ptr(), n, ref.data_ptr(), n, rows, n, 1e-6, s))
    _lib.check("rspx_add_rmsnorm_partials", L.rspx_add_rmsnorm_partials(
        x.data_ptr(), n, hp.data_ptr(), 2, w.data_ptr(), xo2.data_ptr(), n, out.data_ptr(), _lib.RSPX_TILED, rows, n,
        1e-6, s))
    torch.cuda.synchronize()
    assert torch.equal(from_tiled(out, rows, n), ref)
    assert torch.equal(xo1, xo2)


@pytest.mark.parametrize("D", [16, 32, 64, 80, 96, 256, 512])
def test_rope_any_head_dim_bitwise(D):
    """rope for head dims other than 128 (the reference's rope takes any D, fused.py:45-75):
    bitwise equal to the oracle (= PyTorch's bf16 element-wise ops), with strided x and a
    row count that leaves a partial wave."""
    from respect_amd.system.fused import rope
    rng = np.random.default_rng(D)
    B, H, L = 2, 3, 37
    x = gen.bf16_normal(rng, (B, H, L, D))
    pos = rng.integers(0, 4096, (B, L))
    tabs = [N.rope_tables(pos[b], head_dim=D) for b in range(B)]
    cos = np.stack([t[0] for t in tabs])
    sin = np.stack([t[1] for t in tabs])
    print(f"[rope] D={D}", flush=True)
    out = _np(rope(_dev(x), _dev(cos), _dev(sin)))
    assert np.array_equal(out, N.rope(x, cos[:, None], sin[:, None]))
    xs = _dev(x).transpose(1, 2).contiguous().transpose(1, 2)
    assert np.array_equal(_np(rope(xs, _dev(cos), _dev(sin))), out)


def test_rope_unsupported_head_dims():
    from respect_amd import _lib
    from respect_amd.system.fused import rope
    for D in (8, 24, 528):
        x = torch.zeros(1, 1, 2, D, dtype=torch.bfloat16, device="cuda")
        c = torch.zeros(1, 2, D, dtype=torch.bfloat16, device="cuda")
        with pytest.raises(_lib.RspxError):
            rope(x, c, c)


@pytest.mark.parametrize("rows,n", [(5, 1000), (64, 1000), (3, 20000), (2, 16392), (4, 7), (9, 100), (2, 4100)])
def test_rmsnorm_any_length(rows, n):
    """Row lengths outside n % 8 == 0, n <= 16384 (the reference's rmsnorm takes any N,
    respect/kernels/rmsnorm.py:25-32): within 1 bf16 ulp of the oracle, rows bitwise
    independent of the row count, and unaligned strided operands give the same bits; the
    residual add + RMSNorm gives bf16(r + h) and rmsnorm of it, also in place (xo = r)."""
    from respect_amd import _lib
    from respect_amd.kernels.rmsnorm import rmsnorm
    print(f"[rmsnorm any] rows={rows} n={n}", flush=True)
    rng = np.random.default_rng(n + rows)
    x = gen.bf16_normal(rng, (rows, n))
    w = bf16.round_bf16(1 + 0.02 * rng.standard_normal(n).astype(np.float32))
    xd, wd = _dev(x), _dev(w)
    out = rmsnorm(xd, wd, 1e-6)
    d = bf16.ulp_diff(_np(out), N.rmsnorm(x, w, 1e-6))
    print(f"  max ulp {d.max():.2f}", flush=True)
    assert d.max() <= 1.0
    for m in sorted({0, rows // 2, rows - 1}):
        assert torch.equal(rmsnorm(xd[m:m + 1], wd, 1e-6), out[m:m + 1])
    L = _lib.lib()
    s = _lib.stream_ptr(xd.device)
    # strided operands: one element past 16 bytes where the length takes the
    # element-wise kernel, whole 16-byte units where it takes the vector ones
    o = 8 if n % 8 == 0 and n <= 16384 else 1
    xb = torch.zeros(rows, n + o, device="cuda", dtype=torch.bfloat16)
    xb[:, o:] = xd
    wb = torch.zeros(n + o, device="cuda", dtype=torch.bfloat16)
    wb[o:] = wd
    yb = torch.full((rows, n + 2 * o), float("nan"), device="cuda", dtype=torch.bfloat16)
    _lib.check("rspx_rmsnorm", L.rspx_rmsnorm(xb.data_ptr() + 2 * o, n + o, wb.data_ptr() + 2 * o,
                                              yb.data_ptr() + 2 * o, n + 2 * o, rows, n, 1e-6, s))
    torch.cuda.synchronize()
    assert torch.equal(yb[:, o:n + o], out)
    assert torch.isnan(yb[:, :o].float()).all() and torch.isnan(yb[:, n + o:].float()).all()
    # residual add + RMSNorm, out of place and in place
    h = _dev(gen.bf16_normal(rng, (rows, n)))
    xo, y = torch.empty_like(xd), torch.empty_like(xd)
    _lib.check("rspx_add_rmsnorm", L.rspx_add_rmsnorm(xd.data_ptr(), n, h.data_ptr(), n, wd.data_ptr(), xo.data_ptr(),
                                                      n, y.data_ptr(), n, rows, n, 1e-6, s))
    r2, y2 = xd.clone(), torch.empty_like(xd)
    _lib.check("rspx_add_rmsnorm", L.rspx_add_rmsnorm(r2.data_ptr(), n, h.data_ptr(), n, wd.data_ptr(), r2.data_ptr(),
                                                      n, y2.data_ptr(), n, rows, n, 1e-6, s))
    torch.cuda.synchronize()
    assert torch.equal(xo, (xd.float() + h.float()).to(torch.bfloat16))
    assert torch.equal(y, rmsnorm(xo, wd, 1e-6))
    assert torch.equal(r2, xo) and torch.equal(y2, y)


def test_rmsnorm_any_length_errors():
    from respect_amd import _lib
    L = _lib.lib()
    s = _lib.stream_ptr(torch.device("cuda"))
    x = torch.zeros(2, 1000, device="cuda", dtype=torch.bfloat16)
    w = torch.ones(1000, device="cuda", dtype=torch.bfloat16)
    y = torch.zeros(64 * 1000, device="cuda", dtype=torch.bfloat16)
    # the tiled output layout needs n % 32 == 0; partials keep n % 8 == 0, n <= 16384
    assert L.rspx_rmsnorm(x.data_ptr(), 1000, w.data_ptr(), y.data_ptr(), _lib.RSPX_TILED, 2, 1000, 1e-6, s) == -2
    assert L.rspx_rmsnorm(x.data_ptr() + 1, 1000, w.data_ptr(), y.data_ptr(), 1000, 2, 1000, 1e-6, s) == -4
    hp = torch.zeros(2 * 1004, device="cuda", dtype=torch.float32)
    assert L.rspx_add_rmsnorm_partials(x.data_ptr(), 1004, hp.data_ptr(), 1, w.data_ptr(), x.data_ptr(), 1004,
                                       y.data_ptr(), 1004, 2, 1002, 1e-6, s) == -2
    torch.cuda.synchronize()


@pytest.mark.parametrize("D", [16, 32, 64, 96, 256, 512])
def test_qk_norm_rope_any_head_dim(D):
    """q/k RMSNorm + RoPE at head dims other than 128: bitwise equal to rmsnorm followed by
    rope at the same D, within 2 ulp of the oracle composition, token-count invariant; and
    the decoder-layer epilogue rspx_qkv_rope_cache gives the same q, K and V rows."""
    from respect_amd import _lib
    from respect_amd.kernels.rmsnorm import rmsnorm
    from respect_amd.system.fused import qk_norm_rope, rope
    print(f"[qk_norm_rope] D={D}", flush=True)
    rng = np.random.default_rng(D + 1)
    T, HQ, HK = 13, 4, 2
    q = gen.bf16_normal(rng, (T, HQ, D))
    k = gen.bf16_normal(rng, (T, HK, D))
    wq = bf16.round_bf16(1 + 0.02 * rng.standard_normal(D).astype(np.float32))
    wk = bf16.round_bf16(1 + 0.02 * rng.standard_normal(D).astype(np.float32))
    cos, sin = N.rope_tables(3072 + rng.integers(0, 24, T), head_dim=D)
    qo, ko = qk_norm_rope(_dev(q), _dev(k), _dev(wq), _dev(wk), 1e-6, _dev(cos), _dev(sin))
    qn = rmsnorm(_dev(q), _dev(wq), 1e-6).transpose(0, 1)[None]
    kn = rmsnorm(_dev(k), _dev(wk), 1e-6).transpose(0, 1)[None]
    assert torch.equal(qo, rope(qn, _dev(cos)[None], _dev(sin)[None])[0].transpose(0, 1))
    assert torch.equal(ko, rope(kn, _dev(cos)[None], _dev(sin)[None])[0].transpose(0, 1))
    ref_q = N.rope(N.rmsnorm(q, wq, 1e-6), cos[:, None], sin[:, None])
    assert bf16.ulp_diff(_np(qo), ref_q).max() <= 2.0
    q1, k1 = qk_norm_rope(_dev(q[5:6]), _dev(k[5:6]), _dev(wq), _dev(wk), 1e-6, _dev(cos[5:6]), _dev(sin[5:6]))
    assert torch.equal(q1[0], qo[5]) and torch.equal(k1[0], ko[5])
    # packed projection rows [q | k | v] through the q/k/v epilogue into a KV cache
    L = _lib.lib()
    s = _lib.stream_ptr(torch.device("cuda"))
    v = gen.bf16_normal(rng, (T, HK, D))
    qkv = _dev(np.concatenate([q.reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1)], axis=1))
    n = (HQ + 2 * HK) * D
    P = T + 5
    slots = torch.arange(2, 2 + T, dtype=torch.int32, device="cuda")
    ck = torch.zeros(HK, P, D, device="cuda", dtype=torch.bfloat16)
    cv = torch.zeros_like(ck)
    q2 = torch.empty(T, HQ, D, device="cuda", dtype=torch.bfloat16)
    wqd, wkd, cosd, sind = _dev(wq), _dev(wk), _dev(cos), _dev(sin)   # held while the kernel runs
    _lib.check("rspx_qkv_rope_cache", L.rspx_qkv_rope_cache(
        qkv.data_ptr(), n, wqd.data_ptr(), wkd.data_ptr(), cosd.data_ptr(), sind.data_ptr(), D,
        slots.data_ptr(), P, ck.data_ptr(), P * D, D, cv.data_ptr(), P * D, D, q2.data_ptr(), T, HQ, HK, D, 1e-6, s))
    torch.cuda.synchronize()
    assert torch.equal(q2, qo)
    assert torch.equal(ck[:, 2:2 + T].transpose(0, 1), ko)
    assert torch.equal(cv[:, 2:2 + T].transpose(0, 1), _dev(v))
    assert not ck[:, :2].any() and not ck[:, 2 + T:].any()


@pytest.mark.parametrize("rows,n,T,D", [(64, 4096, 64, 128), (5, 128, 3, 64), (3, 512, 7, 256), (7, 1024, 2, 128),
                                        (2, 12288, 5, 32), (9, 256, 1, 128), (4, 4000, 9, 96), (1, 16384, 64, 512)])
def test_rmsnorm_qk_norm_rope_one_launch(rows, n, T, D):
    """rspx_rmsnorm_qk_norm_rope gives bitwise the outputs of rspx_rmsnorm and
    rspx_qk_norm_rope called one after the other, for every RMSNorm split and head dim."""
    from respect_amd.kernels.rmsnorm import rmsnorm
    from respect_amd.system.fused import qk_norm_rope, rmsnorm_qk_norm_rope
    print(f"[rmsnorm+qk_norm_rope] rows={rows} n={n} T={T} D={D}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(rows * 31 + n + D)
    HQ, HK = 4, 2
    x = torch.randn(rows, n, generator=g, device="cuda").to(torch.bfloat16)
    w = (1 + 0.02 * torch.randn(n, generator=g, device="cuda")).to(torch.bfloat16)
    q = torch.randn(T, HQ, D, generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn(T, HK, D, generator=g, device="cuda").to(torch.bfloat16)
    wq = (1 + 0.02 * torch.randn(D, generator=g, device="cuda")).to(torch.bfloat16)
    wk = (1 + 0.02 * torch.randn(D, generator=g, device="cuda")).to(torch.bfloat16)
    cos, sin = N.rope_tables(3072 + np.arange(T) % 24, head_dim=D)
    cosd, sind = _dev(cos), _dev(sin)
    y, qo, ko = rmsnorm_qk_norm_rope(x, w, 1e-6, q, k, wq, wk, 1e-5, cosd, sind)
    q2, k2 = qk_norm_rope(q, k, wq, wk, 1e-5, cosd, sind)
    assert torch.equal(y, rmsnorm(x, w, 1e-6))
    assert torch.equal(qo, q2) and torch.equal(ko, k2)


@pytest.mark.parametrize("rows,F,off", [(3, 1001, 0), (5, 1000, 1), (64, 12288, 0), (1, 7, 3)])
def test_silu_mul_any_width(rows, F, off):
    """SwiGLU at widths and offsets the two-element path does not take (odd F, operands
    one element off a 4-byte boundary): within 1 ulp of the oracle, and the same bits as
    the aligned call where one exists."""
    from respect_amd import _lib
    from respect_amd.system.fused import silu_mul
    print(f"[silu_mul] rows={rows} F={F} off={off}", flush=True)
    rng = np.random.default_rng(F + off)
    gu = gen.bf16_normal(rng, (rows, 2 * F))
    ref = N.silu_mul(gu[:, :F], gu[:, F:])
    buf = torch.zeros(rows, 2 * F + off + 1, device="cuda", dtype=torch.bfloat16)
    buf[:, off:off + 2 * F] = _dev(gu)
    y = torch.full((rows, F + 1), float("nan"), device="cuda", dtype=torch.bfloat16)
    L = _lib.lib()
    s = _lib.stream_ptr(y.device)
    sb = buf.stride(0)
    _lib.check("rspx_silu_mul", L.rspx_silu_mul(buf.data_ptr() + 2 * off, sb, buf.data_ptr() + 2 * (off + F), sb,
                                                y.data_ptr(), F + 1, rows, F, s))
    torch.cuda.synchronize()
    d = bf16.ulp_diff(_np(y[:, :F]), ref, 1e-30)
    assert d.max() <= 1.0
    assert torch.isnan(y[:, F].float()).all()
    aligned = silu_mul(_dev(gu[:, :F]), _dev(gu[:, F:]))
    assert torch.equal(y[:, :F], aligned)
