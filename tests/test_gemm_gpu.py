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
    from respect_amd.kernels.gemm import tile_weight
    with pytest.raises(RspxError):   # the tiled weight layout needs N % 16 == 0 and K % 32 == 0
        tile_weight(torch.zeros(20, 100, device="cuda", dtype=torch.bfloat16))
    with pytest.raises(TypeError):
        linear(xd.float(), wd)


@pytest.mark.parametrize("M,N,K", [(7, 1000, 1000), (1, 1000, 1000), (64, 1000, 4096), (5, 4096, 1000),
                                   (3, 17, 33), (130, 250, 777), (2, 24, 4104), (70, 4100, 520)])
def test_linear_any_shape(M, N, K):
    """Shapes outside N % 16 == 0 and K % 256 == 0 (the reference's linear masks any M, N, K,
    respect/kernels/gemm.py:19-27): the parity bar above in bf16, the accumulation bound in
    fp32, rows bitwise independent of M, and the same bits from unaligned, strided operands
    (two-byte loads) as from aligned ones."""
    from respect_amd import _lib
    from respect_amd.kernels.gemm import linear
    print(f"[linear any] M={M} N={N} K={K}", flush=True)
    L = _lib.lib()
    assert L.rspx_linear_splits(N, K) == 1 and L.rspx_linear_workspace_bytes(M, N, K) == 0
    x, w = _xw(M * 11 + N + K, M, N, K)
    xd, wd = _dev(x), _dev(w)
    out = linear(xd, wd)
    o = out.float().cpu().numpy()
    ex = G.linear_exact(x, w)
    ref = bf16.round_bf16(ex.astype(np.float32))
    bound = G.linear_error_bound(x, w)
    allowed = bound + bf16.ulp(np.abs(ex) + bound)
    print(f"  max ulp {bf16.ulp_diff(o, ref).max():.2f} equal {(o == ref).mean():.5f}", flush=True)
    assert np.all(np.abs(o - ex) <= allowed)
    assert (o == ref).mean() >= 0.99
    f32 = linear(xd, wd, out_dtype=torch.float32)
    assert np.all(np.abs(f32.cpu().numpy().astype(np.float64) - ex) <= bound + 1e-30)
    # rows alone and in a longer call
    for m in sorted({0, M // 2, M - 1}):
        assert torch.equal(linear(xd[m:m + 1], wd), out[m:m + 1])
    big = torch.cat([xd, xd.flip(0), xd[:1]])
    assert torch.equal(linear(big, wd)[:M], out)
    # operands one element past a 16-byte boundary, rows K + 3 apart, output rows N + 1 apart
    s = _lib.stream_ptr(xd.device)
    xb = torch.zeros(M, K + 3, device="cuda", dtype=torch.bfloat16)
    wb = torch.zeros(N, K + 3, device="cuda", dtype=torch.bfloat16)
    xb[:, 1:K + 1] = xd
    wb[:, 1:K + 1] = wd
    ob = torch.full((M, N + 1), float("nan"), device="cuda", dtype=torch.bfloat16)
    _lib.check("rspx_linear", L.rspx_linear(xb.data_ptr() + 2, K + 3, wb.data_ptr() + 2, K + 3, ob.data_ptr(), N + 1,
                                            M, N, K, 0, None, 0, s))
    torch.cuda.synchronize()
    assert torch.equal(ob[:, :N], out)
    assert torch.isnan(ob[:, N].float()).all()     # nothing written past column N


def test_linear_any_shape_errors():
    from respect_amd import _lib
    L = _lib.lib()
    s = _lib.stream_ptr(torch.device("cuda"))
    x = torch.zeros(4, 100, device="cuda", dtype=torch.bfloat16)
    w = torch.zeros(24, 100, device="cuda", dtype=torch.bfloat16)
    o = torch.zeros(4, 24, device="cuda", dtype=torch.bfloat16)
    assert L.rspx_linear(x.data_ptr(), 100, w.data_ptr(), 100, o.data_ptr(), 24, 4, 24, 100, 0, None, 0, s) == 0
    assert L.rspx_linear(x.data_ptr(), 99, w.data_ptr(), 100, o.data_ptr(), 24, 4, 24, 100, 0, None, 0, s) == -1
    assert L.rspx_linear(x.data_ptr() + 1, 100, w.data_ptr(), 100, o.data_ptr(), 24, 4, 24, 100, 0, None, 0, s) == -4
    assert L.rspx_linear(x.data_ptr(), _lib.RSPX_TILED, w.data_ptr(), 100, o.data_ptr(), 24, 4, 24, 100, 0, None, 0,
                         s) == -2
    # rspx_linear_silu and rspx_linear_partials keep the N % 16, K % 256 shapes
    assert L.rspx_linear_partials(x.data_ptr(), 100, w.data_ptr(), 100, o.data_ptr(), 4, 24, 100, s) == -2
    torch.cuda.synchronize()


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


def _tiled_weight_numpy(w, pad=64):
    """The tiled weight layout of include/respect_amd.h (rspx_linear_tile_weight),
    element by element: slab n // 16 of 16 K + pad elements, tile k // 32 of it,
    (n % 16 + 16 ((k % 32) // 8)) 8 + k % 8 inside the tile."""
    N, K = w.shape
    out = np.zeros((N // 16) * (16 * K + pad), dtype=w.dtype)
    n, k = np.meshgrid(np.arange(N), np.arange(K), indexing="ij")
    off = (n // 16) * (16 * K + pad) + (k // 32) * 512 + ((n % 16) + 16 * ((k % 32) // 8)) * 8 + k % 8
    out[off.ravel()] = w.ravel()
    return out


@pytest.mark.parametrize("N,K", [(16, 256), (48, 768), (6144, 4096)])
def test_tile_weight_layout(N, K):
    """rspx_linear_tile_weight places every element where the layout says, the slab
    pads are zero, and TiledWeight.dense() gives the matrix back; row-padded input too."""
    from respect_amd import _lib
    from respect_amd.kernels.gemm import tile_weight
    rng = np.random.default_rng(N + K)
    w = rng.integers(-30000, 30000, (N, K)).astype(np.int16)
    wd = torch.from_numpy(w).cuda().view(torch.bfloat16)
    assert _lib.lib().rspx_linear_tiled_weight_elems(N, K) == (N // 16) * (16 * K + 64)
    for src in (wd, torch.nn.functional.pad(wd.view(torch.int16), (0, 64)).view(torch.bfloat16)[:, :K]):
        t = tile_weight(src)
        got = t.buf.view(torch.int16).cpu().numpy()
        assert np.array_equal(got, _tiled_weight_numpy(w))
        assert torch.equal(t.dense().view(torch.int16), wd.view(torch.int16))


def test_tile_weight_errors():
    from respect_amd import _lib
    L = _lib.lib()
    w = torch.zeros((64, 512), dtype=torch.bfloat16, device="cuda")
    out = torch.empty(L.rspx_linear_tiled_weight_elems(64, 512), dtype=torch.bfloat16, device="cuda")
    s = _lib.stream_ptr(w.device)
    assert L.rspx_linear_tiled_weight_elems(40, 512) == -1
    assert L.rspx_linear_tiled_weight_elems(64, 500) == -1
    assert L.rspx_linear_tile_weight(w.data_ptr(), 512, 40, 512, out.data_ptr(), s) == -2   # N % 16
    assert L.rspx_linear_tile_weight(w.data_ptr(), 500, 64, 512, out.data_ptr(), s) == -1   # sw < K
    assert L.rspx_linear_tile_weight(w.data_ptr() + 2, 512, 64, 480, out.data_ptr(), s) == -4   # alignment
    assert L.rspx_linear_tile_weight(w.data_ptr(), 512, 64, 512, out.data_ptr(), s) == 0


@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (7, 1024, 4096), (64, 6144, 4096), (130, 512, 768),
                                   (64, 24576, 4096), (200, 256, 12288), (64, 16384, 4096)])
def test_linear_tiled_w_is_bitwise_row_major(M, N, K):
    """w in the tiled weight layout (TiledWeight, row stride RSPX_TILED) gives the
    row-major result bit for bit: rspx_linear (bf16 and fp32 out, row-major and
    tiled x) and rspx_linear_partials."""
    from _tiled import to_tiled
    from respect_amd import _lib
    from respect_amd.kernels.gemm import linear, tile_weight
    print(f"[linear tiled w] M={M} N={N} K={K}", flush=True)
    L = _lib.lib()
    x, w = _xw(M * 5 + N, M, N, K)
    xd, wd = _dev(x), _dev(w)
    wt = tile_weight(wd)
    for dt in (torch.bfloat16, torch.float32):
        assert torch.equal(linear(xd, wt, out_dtype=dt), linear(xd, wd, out_dtype=dt))
    s = _lib.stream_ptr(xd.device)
    S = L.rspx_linear_splits(N, K)
    xt = to_tiled(xd, fill=float("nan"))
    parts = []
    for xp, sx, wp, sw in ((xd, K, wd, K), (xd, K, wt, _lib.RSPX_TILED), (xt, _lib.RSPX_TILED, wt, _lib.RSPX_TILED)):
        part = torch.empty((S, M, N), dtype=torch.float32, device="cuda")
        _lib.check("rspx_linear_partials", L.rspx_linear_partials(xp.data_ptr(), sx, wp.data_ptr(), sw,
                                                                  part.data_ptr(), M, N, K, s))
        parts.append(part)
    torch.cuda.synchronize()
    assert torch.equal(parts[0], parts[1]) and torch.equal(parts[0], parts[2])


@pytest.mark.parametrize("M", [1, 64, 130])
def test_linear_silu_tiled_w(M):
    """rspx_linear_silu with the interleaved gate/up rows tiled equals the row-major call."""
    from respect_amd import _lib
    from respect_amd.kernels.gemm import tile_weight
    F, K = 8192, 512
    L = _lib.lib()
    x, w = _xw(M + 303, M, 2 * F, K)
    xd, wd = _dev(x), _dev(w)
    wt = tile_weight(wd)
    s = _lib.stream_ptr(xd.device)
    outs = []
    for wp, sw in ((wd, K), (wt, _lib.RSPX_TILED)):
        o = torch.empty((M, F), dtype=torch.bfloat16, device="cuda")
        _lib.check("rspx_linear_silu", L.rspx_linear_silu(xd.data_ptr(), K, wp.data_ptr(), sw, o.data_ptr(), F,
                                                           M, 2 * F, K, s))
        outs.append(o)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
