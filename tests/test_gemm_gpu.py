"""GPU parity and row-count invariance of the linear layer (csrc/gemm.hip).

Parity bar: every bf16 output within the fp32-accumulation error bound
(K 2^-24 sum|x w|) plus one bf16 rounding of the float64 result, and equal
to the float64 result rounded to bf16 on at least 99% of elements (the
accumulation error is far below half a bf16 ulp except near rounding ties
and for results that cancel to much less than sum|x w|); fp32 outputs within
the accumulation bound.  Row invariance is bitwise.
"""
import numpy as np
import pytest
import torch

from oracle import bf16
from oracle import gemm as G

pytestmark = pytest.mark.gpu


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).cuda()


def _xw(seed, M, N, K):
    rng = np.random.default_rng(seed)
    x = bf16.round_bf16(rng.standard_normal((M, K)).astype(np.float32))
    w = bf16.round_bf16(0.02 * rng.standard_normal((N, K)).astype(np.float32))
    return x, w


@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (64, 6144, 4096), (7, 1024, 4096), (64, 4096, 12288),
                                   (33, 256, 256), (130, 512, 768), (64, 24576, 4096)])
def test_linear_parity_bf16(M, N, K):
    from respect_amd.kernels.gemm import linear
    print(f"[linear] M={M} N={N} K={K}", flush=True)
    x, w = _xw(M * 7 + N, M, N, K)
    out = linear(_dev(x), _dev(w)).float().cpu().numpy()
    ex = G.linear_exact(x, w)
    ref = bf16.round_bf16(ex.astype(np.float32))
    bound = G.linear_error_bound(x, w)
    allowed = bound + bf16.ulp(np.abs(ex) + bound)
    d = bf16.ulp_diff(out, ref)
    print(f"  max ulp {d.max():.2f} equal {(out == ref).mean():.5f} "
          f"max err/allowed {(np.abs(out - ex) / allowed).max():.3f}", flush=True)
    assert np.all(np.abs(out - ex) <= allowed)
    assert (out == ref).mean() >= 0.99


def test_linear_parity_fp32_out():
    from respect_amd.kernels.gemm import linear
    x, w = _xw(5, 64, 16384, 4096)
    out = linear(_dev(x), _dev(w), out_dtype=torch.float32).cpu().numpy().astype(np.float64)
    ex = G.linear_exact(x, w)
    assert np.all(np.abs(out - ex) <= G.linear_error_bound(x, w) + 1e-30)


def test_linear_is_row_count_invariant():
    """tests/test_kernel_invariance.py:8-17 of the reference, plus more row sets."""
    from respect_amd.kernels.gemm import linear
    torch.manual_seed(0)
    x = torch.randn(64, 4096, device="cuda", dtype=torch.bfloat16)
    w = torch.randn(1024, 4096, device="cuda", dtype=torch.bfloat16)
    kw = dict(BM=32, BN=128, BK=128, num_warps=4, num_stages=3)
    full = linear(x, w, **kw)
    for m in (1, 7, 33):
        assert torch.equal(linear(x[:m], w, **kw), full[:m])
    assert torch.equal(linear(x[20:23], w), full[20:23])
    big = torch.cat([x, x.flip(0), x[:5]])  # 133 rows: three 64-row tiles
    fb = linear(big, w)
    assert torch.equal(fb[:64], full) and torch.equal(fb[64:128], full.flip(0)) and torch.equal(fb[128:], full[:5])
    # fp32 output (the vocabulary projection) too
    f32 = linear(x, w, out_dtype=torch.float32)
    assert torch.equal(linear(x[7:8], w, out_dtype=torch.float32), f32[7:8])


def test_linear_strided_and_errors():
    from respect_amd._lib import RspxError, lib
    from respect_amd.kernels.gemm import linear
    x, w = _xw(9, 16, 512, 1024)
    xd, wd = _dev(x), _dev(w)
    big = torch.zeros(16, 2048, device="cuda", dtype=torch.bfloat16)
    big[:, 512:1536] = xd
    assert torch.equal(linear(big[:, 512:1536], wd), linear(xd, wd))
    # the chunk count depends on (N, K) only
    assert lib().rspx_linear_splits(4096, 4096) == lib().rspx_linear_splits(4096, 4096) > 0
    with pytest.raises(RspxError):
        linear(torch.zeros(4, 100, device="cuda", dtype=torch.bfloat16),
               torch.zeros(16, 100, device="cuda", dtype=torch.bfloat16))
    with pytest.raises(TypeError):
        linear(xd.float(), wd)


def test_partials_consumers_equal_linear_then_op():
    """rspx_linear_partials + a consumer that sums the chunks gives the bits of
    rspx_linear followed by the plain op (residual add + RMSNorm, q/k/v epilogue)."""
    from respect_amd import _lib
    from respect_amd.kernels.gemm import linear
    L = _lib.lib()
    s = _lib.stream_ptr(torch.device("cuda"))
    torch.manual_seed(3)
    T, H = 7, 4096
    for K in (4096, 12288):
        x = torch.randn(T, K, device="cuda").to(torch.bfloat16)
        w = (0.02 * torch.randn(H, K, device="cuda")).to(torch.bfloat16)
        r = torch.randn(T, H, device="cuda").to(torch.bfloat16)
        nw = (1 + 0.02 * torch.randn(H, device="cuda")).to(torch.bfloat16)
        S = L.rspx_linear_splits(H, K)
        part = torch.empty(S * T * H, device="cuda", dtype=torch.float32)
        assert L.rspx_linear_partials(x.data_ptr(), K, w.data_ptr(), K, part.data_ptr(), T, H, K, s) == 0
        h = linear(x, w)
        xo1, y1 = torch.empty_like(r), torch.empty_like(r)
        xo2, y2 = torch.empty_like(r), torch.empty_like(r)
        assert L.rspx_add_rmsnorm(r.data_ptr(), H, h.data_ptr(), H, nw.data_ptr(), xo1.data_ptr(), H, y1.data_ptr(), H,
                                  T, H, 1e-6, s) == 0
        assert L.rspx_add_rmsnorm_partials(r.data_ptr(), H, part.data_ptr(), S, nw.data_ptr(), xo2.data_ptr(), H,
                                           y2.data_ptr(), H, T, H, 1e-6, s) == 0
        assert torch.equal(xo1, xo2) and torch.equal(y1, y2)
        assert torch.equal(xo1, (r.float() + h.float()).to(torch.bfloat16))
    # q/k/v epilogue
    HQ, HK, D, P = 4, 2, 128, 16
    n = (HQ + 2 * HK) * D
    x = torch.randn(T, 512, device="cuda").to(torch.bfloat16)
    w = (0.05 * torch.randn(n, 512, device="cuda")).to(torch.bfloat16)
    S = L.rspx_linear_splits(n, 512)
    part = torch.empty(S * T * n, device="cuda", dtype=torch.float32)
    assert L.rspx_linear_partials(x.data_ptr(), 512, w.data_ptr(), 512, part.data_ptr(), T, n, 512, s) == 0
    qkv = linear(x, w)
    wq = (1 + 0.02 * torch.randn(D, device="cuda")).to(torch.bfloat16)
    wk = (1 + 0.02 * torch.randn(D, device="cuda")).to(torch.bfloat16)
    from respect_amd.system.fused import rope_tables
    cos, sin = rope_tables(torch.arange(T, device="cuda") + 100, D, 1e6, device="cuda")
    slots = torch.arange(3, 3 + T, dtype=torch.int32, device="cuda")
    outs = []
    for use_part in (False, True):
        ck = torch.zeros(HK, P, D, device="cuda", dtype=torch.bfloat16)
        cv = torch.zeros_like(ck)
        qo = torch.empty(T, HQ, D, device="cuda", dtype=torch.bfloat16)
        common = (wq.data_ptr(), wk.data_ptr(), cos.data_ptr(), sin.data_ptr(), D, slots.data_ptr(), P,
                  ck.data_ptr(), P * D, D, cv.data_ptr(), P * D, D, qo.data_ptr(), T, HQ, HK, D, 1e-6, s)
        if use_part:
            assert L.rspx_qkv_rope_cache_partials(part.data_ptr(), S, *common) == 0
        else:
            assert L.rspx_qkv_rope_cache(qkv.data_ptr(), n, *common) == 0
        outs.append((qo, ck, cv))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    assert torch.equal(outs[0][2][:, 3:3 + T].transpose(0, 1), qkv[:, (HQ + HK) * D:].view(T, HK, D))
    # Slots outside [0, cap): no K/V write anywhere, the token's q row is NaN, the other
    # tokens are unchanged.
    bad = slots.clone()
    bad[1], bad[T - 1] = P, -1
    ck = torch.zeros(HK, P + 8, D, device="cuda", dtype=torch.bfloat16)   # 8 guard slots past cap
    cv = torch.zeros_like(ck)
    qo = torch.empty(T, HQ, D, device="cuda", dtype=torch.bfloat16)
    assert L.rspx_qkv_rope_cache(qkv.data_ptr(), n, wq.data_ptr(), wk.data_ptr(), cos.data_ptr(), sin.data_ptr(), D,
                                 bad.data_ptr(), P, ck.data_ptr(), (P + 8) * D, D, cv.data_ptr(), (P + 8) * D, D,
                                 qo.data_ptr(), T, HQ, HK, D, 1e-6, s) == 0
    torch.cuda.synchronize()
    assert torch.isnan(qo[1]).all() and torch.isnan(qo[T - 1]).all()
    good = [t for t in range(T) if t not in (1, T - 1)]
    assert torch.equal(qo[good], outs[0][0][good])
    assert torch.equal(ck[:, :P][:, slots[good].long()], outs[0][1][:, slots[good].long()])
    assert not ck[:, P:].any() and not cv[:, P:].any()
    written = torch.zeros(P + 8, dtype=torch.bool)
    written[slots[good].long().cpu()] = True
    assert not ck[:, ~written.cuda()].any()


@pytest.mark.parametrize("M", [1, 7, 64, 130])
def test_linear_silu_equals_linear_then_silu_mul(M):
    """rspx_linear_silu on interleaved gate/up rows is bit for bit rspx_linear followed by
    rspx_silu_mul on the [gate | up] layout, and leaves each row independent of M."""
    from respect_amd import _lib
    from respect_amd.kernels.gemm import linear
    from respect_amd.system.fused import silu_mul
    F, K = 8192, 256
    print(f"[linear_silu] M={M} F={F} K={K}", flush=True)
    L = _lib.lib()
    assert L.rspx_linear_splits(2 * F, K) == 1
    x, w = _xw(M + 11, M, 2 * F, K)
    xd, wd = _dev(x), _dev(w)
    wil = wd.view(2, F, K).transpose(0, 1).reshape(2 * F, K).contiguous()
    gu = linear(xd, wd)
    ref = silu_mul(gu[:, :F], gu[:, F:])
    out = torch.empty((M, F), dtype=torch.bfloat16, device="cuda")
    rc = L.rspx_linear_silu(xd.data_ptr(), K, wil.data_ptr(), K, out.data_ptr(), F, M, 2 * F, K,
                            _lib.stream_ptr(xd.device))
    _lib.check("rspx_linear_silu", rc)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    one = torch.empty((1, F), dtype=torch.bfloat16, device="cuda")
    _lib.check("rspx_linear_silu", L.rspx_linear_silu(xd[M - 1:].data_ptr(), K, wil.data_ptr(), K, one.data_ptr(), F,
                                                       1, 2 * F, K, _lib.stream_ptr(xd.device)))
    torch.cuda.synchronize()
    assert torch.equal(one[0], out[M - 1])


def test_linear_silu_rejects_split_k():
    from respect_amd import _lib
    L = _lib.lib()
    N, K = 1024, 4096                      # several K chunks
    assert L.rspx_linear_splits(N, K) > 1
    x = torch.zeros((4, K), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((N, K), dtype=torch.bfloat16, device="cuda")
    out = torch.empty((4, N // 2), dtype=torch.bfloat16, device="cuda")
    rc = L.rspx_linear_silu(x.data_ptr(), K, w.data_ptr(), K, out.data_ptr(), N // 2, 4, N, K,
                            _lib.stream_ptr(x.device))
    assert rc == -2   # RSPX_EUNSUPPORTED


@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (7, 1024, 4096), (64, 6144, 4096), (130, 512, 768),
                                   (64, 24576, 4096), (200, 256, 12288)])
def test_linear_tiled_x_is_bitwise_row_major(M, N, K):
    """x in the tiled layout (RSPX_TILED) gives the row-major result bit for bit, through
    rspx_linear (bf16 and fp32 out) and rspx_linear_partials; rows past M in the last
    64-row block hold NaN and must not reach any stored output."""
    from _tiled import to_tiled
    from respect_amd import _lib
    from respect_amd.kernels.gemm import linear
    print(f"[linear tiled] M={M} N={N} K={K}", flush=True)
    L = _lib.lib()
    x, w = _xw(M * 7 + N, M, N, K)
    xd, wd = _dev(x), _dev(w)
    xt = to_tiled(xd, fill=float("nan"))
    s = _lib.stream_ptr(xd.device)
    ws = _lib.workspace(xd.device, max(L.rspx_linear_workspace_bytes(M, N, K), 16), tag="linear")
    for fp32 in (0, 1):
        ref = linear(xd, wd, out_dtype=torch.float32 if fp32 else torch.bfloat16)
        out = torch.empty_like(ref)
        _lib.check("rspx_linear", L.rspx_linear(xt.data_ptr(), _lib.RSPX_TILED, wd.data_ptr(), K, out.data_ptr(), N,
                                                M, N, K, fp32, ws.data_ptr(), ws.numel(), s))
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
    S = L.rspx_linear_splits(N, K)
    parts = []
    for xp, sx in ((xd, K), (xt, _lib.RSPX_TILED)):
        part = torch.empty((S, M, N), dtype=torch.float32, device="cuda")
        _lib.check("rspx_linear_partials", L.rspx_linear_partials(xp.data_ptr(), sx, wd.data_ptr(), K,
                                                                  part.data_ptr(), M, N, K, s))
        parts.append(part)
    torch.cuda.synchronize()
    assert torch.equal(parts[0], parts[1])


@pytest.mark.parametrize("M", [1, 7, 64, 130])
def test_linear_silu_tiled_in_and_out(M):
    """rspx_linear_silu with a tiled x and a tiled output equals the row-major call, re-tiled."""
    from _tiled import from_tiled, to_tiled
    from respect_amd import _lib
    F, K = 8192, 256
    print(f"[linear_silu tiled] M={M}", flush=True)
    L = _lib.lib()
    x, w = _xw(M + 101, M, 2 * F, K)
    xd, wd = _dev(x), _dev(w)
    s = _lib.stream_ptr(xd.device)
    ref = torch.empty((M, F), dtype=torch.bfloat16, device="cuda")
    _lib.check("rspx_linear_silu", L.rspx_linear_silu(xd.data_ptr(), K, wd.data_ptr(), K, ref.data_ptr(), F,
                                                       M, 2 * F, K, s))
    out = torch.full((-(-M // 64) * 64 * F,), float("nan"), dtype=torch.bfloat16, device="cuda")
    xt = to_tiled(xd, fill=float("nan"))
    _lib.check("rspx_linear_silu", L.rspx_linear_silu(xt.data_ptr(), _lib.RSPX_TILED, wd.data_ptr(), K,
                                                       out.data_ptr(), _lib.RSPX_TILED, M, 2 * F, K, s))
    torch.cuda.synchronize()
    assert torch.equal(from_tiled(out, M, F), ref)
    # rows past M were not written
    assert torch.isnan(out.float()).sum().item() == (-(-M // 64) * 64 - M) * F
