"""RoPE and SwiGLU at PyTorch's bf16 rounding points, plus the fused q/k norm + RoPE.

Signatures follow respect/system/fused.py: ``rope(x, cos, sin)`` (:67) and
``silu_mul(g, u)`` (:116).  Every multiply/add is an fp32 operation rounded once
to bf16 (no FMA contraction), so ``rope`` matches PyTorch's bf16 elementwise ops
bit for bit; ``silu_mul`` rounds silu(g) to bf16 before the product with u.
Only bf16 is built: other dtypes raise TypeError (the reference computes them
with PyTorch ops instead).
"""
from __future__ import annotations

import torch

from .. import _lib
from ..kernels._tensor import as_kernel_input


def rope(x, cos, sin):
    """q*cos + rotate_half(q)*sin.  x [B,H,L,D], cos/sin [B,L,D] -> [B,H,L,D] bf16."""
    if x.dtype != torch.bfloat16 or cos.dtype != torch.bfloat16 or sin.dtype != torch.bfloat16:
        raise TypeError("rope: respect_amd builds the bf16 path only")
    B, H, L, D = x.shape
    if tuple(cos.shape) != (B, L, D) or tuple(sin.shape) != (B, L, D):
        raise ValueError(f"rope: cos/sin must be [{B}, {L}, {D}]")
    x = as_kernel_input(x, "x")
    cos = as_kernel_input(cos.contiguous(), "cos")
    sin = as_kernel_input(sin.contiguous(), "sin")
    y = torch.empty((B, H, L, D), dtype=torch.bfloat16, device=x.device)
    rc = _lib.lib().rspx_rope(x.data_ptr(), x.stride(0), x.stride(1), x.stride(2), cos.data_ptr(),
                              sin.data_ptr(), cos.stride(0), cos.stride(1), y.data_ptr(), B, H, L, D,
                              _lib.stream_ptr(x.device))
    _lib.check("rspx_rope", rc)
    return y


def silu_mul(g, u):
    """silu(g) * u for bf16 tensors of the same shape (views into a packed gate/up are fine)."""
    if g.dtype != torch.bfloat16 or u.dtype != torch.bfloat16:
        raise TypeError("silu_mul: respect_amd builds the bf16 path only")
    if g.shape != u.shape:
        raise ValueError("silu_mul: g and u must have the same shape")
    F = g.shape[-1]
    g2 = as_kernel_input(g.reshape(-1, F) if g.is_contiguous() else _rows(g), "g")
    u2 = as_kernel_input(u.reshape(-1, F) if u.is_contiguous() else _rows(u), "u")
    M = g2.shape[0]
    y = torch.empty((M, F), dtype=torch.bfloat16, device=g.device)
    rc = _lib.lib().rspx_silu_mul(g2.data_ptr(), g2.stride(0), u2.data_ptr(), u2.stride(0), y.data_ptr(),
                                  y.stride(0), M, F, _lib.stream_ptr(g.device))
    _lib.check("rspx_silu_mul", rc)
    return y.reshape(g.shape)


def _rows(t):
    """A 2-D row view of t without copying when only the leading dims are strided."""
    F = t.shape[-1]
    if t.dim() == 2 and t.stride(-1) == 1:
        return t
    try:
        return t.view(-1, F)
    except RuntimeError:
        return t.reshape(-1, F)


def qk_norm_rope(q, k, wq, wk, eps, cos, sin):
    """q_norm / k_norm (RMSNorm over head_dim) followed by RoPE, one launch.

    q [T, HQ, D], k [T, HK, D], wq/wk [D], cos/sin [T, D] (the rotary rows of
    each token's position) -> (q_out [T, HQ, D], k_out [T, HK, D]).  Bitwise
    equal to ``rope(rmsnorm(q, wq, eps), ...)`` and the same for k.
    """
    T, HQ, D = q.shape
    HK = k.shape[1]
    q = as_kernel_input(q, "q")
    k = as_kernel_input(k, "k")
    wq = as_kernel_input(wq.contiguous(), "wq")
    wk = as_kernel_input(wk.contiguous(), "wk")
    cos = as_kernel_input(cos.reshape(T, D), "cos")
    sin = as_kernel_input(sin.reshape(T, D), "sin")
    if cos.stride(0) != sin.stride(0):
        cos, sin = cos.contiguous(), sin.contiguous()
    qo = torch.empty((T, HQ, D), dtype=torch.bfloat16, device=q.device)
    ko = torch.empty((T, HK, D), dtype=torch.bfloat16, device=q.device)
    rc = _lib.lib().rspx_qk_norm_rope(q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0),
                                      k.stride(1), wq.data_ptr(), wk.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                                      cos.stride(0), qo.data_ptr(), ko.data_ptr(), T, HQ, HK, D, float(eps),
                                      _lib.stream_ptr(q.device))
    _lib.check("rspx_qk_norm_rope", rc)
    return qo, ko


def rmsnorm_qk_norm_rope(x, w, eps, q, k, wq, wk, qk_eps, cos, sin):
    """``rmsnorm(x, w, eps)`` and ``qk_norm_rope(q, k, wq, wk, qk_eps, cos, sin)`` in one
    launch -> (y, q_out, k_out), bitwise the two calls' results.  x [..., N] with N % 8 == 0
    and N <= 16384; the rest as qk_norm_rope.  No counterpart in the reference (two
    launches there): for a caller with both inputs ready."""
    N = x.shape[-1]
    if w.numel() != N:
        raise ValueError(f"rmsnorm_qk_norm_rope: w has {w.numel()} elements for rows of {N}")
    xs = as_kernel_input(x.reshape(-1, N), "x")
    w = as_kernel_input(w.reshape(N), "w")
    T, HQ, D = q.shape
    HK = k.shape[1]
    q = as_kernel_input(q, "q")
    k = as_kernel_input(k, "k")
    wq = as_kernel_input(wq.contiguous(), "wq")
    wk = as_kernel_input(wk.contiguous(), "wk")
    cos = as_kernel_input(cos.reshape(T, D), "cos")
    sin = as_kernel_input(sin.reshape(T, D), "sin")
    if cos.stride(0) != sin.stride(0):
        cos, sin = cos.contiguous(), sin.contiguous()
    y = torch.empty((xs.shape[0], N), dtype=torch.bfloat16, device=x.device)
    qo = torch.empty((T, HQ, D), dtype=torch.bfloat16, device=q.device)
    ko = torch.empty((T, HK, D), dtype=torch.bfloat16, device=q.device)
    rc = _lib.lib().rspx_rmsnorm_qk_norm_rope(
        xs.data_ptr(), xs.stride(0), w.data_ptr(), y.data_ptr(), y.stride(0), xs.shape[0], N, float(eps),
        q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1), wq.data_ptr(), wk.data_ptr(),
        cos.data_ptr(), sin.data_ptr(), cos.stride(0), qo.data_ptr(), ko.data_ptr(), T, HQ, HK, D, float(qk_eps),
        _lib.stream_ptr(x.device))
    _lib.check("rspx_rmsnorm_qk_norm_rope", rc)
    return y.reshape(x.shape), qo, ko


def rope_tables(positions, head_dim: int = 128, theta: float = 1.0e6, device=None):
    """cos/sin rows [T, head_dim] (bf16) for integer positions, computed like HF's
    Qwen3VLTextRotaryEmbedding: fp32 inv_freq, fp32 angles, bf16 cos/sin."""
    pos = torch.as_tensor(positions, device=device).to(torch.float32)
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64, device=pos.device).float()
                                / head_dim))
    freqs = pos[:, None] * inv_freq[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)


# ------------------------------------------------------------------ Prefill / Flow
# respect/system/fused.py:126-194 and :78-103: the kernels compute the squares,
# the residual add and the normalisation at PyTorch's rounding points; the mean
# of the squares is taken with PyTorch, as the reference does, so RMSNorm's
# reduction order is PyTorch's.

def _bf16_rows(t, name):
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name}: respect_amd builds the bf16 path only")
    return as_kernel_input(t.reshape(-1, t.shape[-1]).contiguous(), name)


def _square(xs):
    M, N = xs.shape
    sq = torch.empty((M, N), device=xs.device, dtype=torch.float32)
    rc = _lib.lib().rspx_square(xs.data_ptr(), xs.stride(0), sq.data_ptr(), sq.stride(0), M, N,
                                _lib.stream_ptr(xs.device))
    _lib.check("rspx_square", rc)
    return sq


def add_sq(r, h):
    """x = r + h (bf16, rounded once) and x.float() ** 2; both [rows, n]."""
    if r.shape != h.shape:
        raise ValueError("add_sq: r and h must have the same shape")
    rs, hs = _bf16_rows(r, "r"), _bf16_rows(h, "h")
    M, N = rs.shape
    x = torch.empty((M, N), device=r.device, dtype=torch.bfloat16)
    sq = torch.empty((M, N), device=r.device, dtype=torch.float32)
    rc = _lib.lib().rspx_add_sq(rs.data_ptr(), rs.stride(0), hs.data_ptr(), hs.stride(0), x.data_ptr(), x.stride(0),
                                sq.data_ptr(), sq.stride(0), M, N, _lib.stream_ptr(r.device))
    _lib.check("rspx_add_sq", rc)
    return x, sq


def norm_from(xs, sq, w, eps):
    """xs [M, N] bf16, sq = xs.float() ** 2.  The mean is taken by PyTorch, the rest by the kernel."""
    M, N = xs.shape
    if xs.dtype != torch.bfloat16 or w.dtype != torch.bfloat16 or sq.dtype != torch.float32:
        raise TypeError("norm_from: respect_amd builds bf16 xs / w with fp32 squares only")
    if not (sq.is_cuda and sq.device == xs.device) or tuple(sq.shape) != (M, N) or tuple(w.shape) != (N,):
        raise ValueError("norm_from: sq must be [M, N] and w [N], on the device of xs")
    var = sq.mean(-1).contiguous()
    xs = as_kernel_input(xs.contiguous(), "xs")
    w = as_kernel_input(w.contiguous(), "w")
    y = torch.empty((M, N), device=xs.device, dtype=torch.bfloat16)
    rc = _lib.lib().rspx_norm_apply(xs.data_ptr(), xs.stride(0), var.data_ptr(), w.data_ptr(), y.data_ptr(),
                                    y.stride(0), M, N, float(eps), _lib.stream_ptr(xs.device))
    _lib.check("rspx_norm_apply", rc)
    return y


def rmsnorm(x, w, eps):
    """Prefill RMSNorm: squares in a kernel, mean by PyTorch, normalisation in a kernel."""
    xs = _bf16_rows(x, "x")
    return norm_from(xs, _square(xs), w, eps).reshape(x.shape)


def rope_vision(x, cos, sin):
    """One tensor of apply_rotary_pos_emb_vision: x [L, NH, D] bf16, cos/sin [L, D];
    computed in float32, returned in bf16."""
    if x.dtype != torch.bfloat16:
        raise TypeError("rope_vision: respect_amd builds the bf16 path only")
    L, NH, D = x.shape
    x = as_kernel_input(x, "x")
    if not (cos.is_cuda and sin.is_cuda and cos.device == x.device and sin.device == x.device):
        raise RuntimeError("rope_vision: cos/sin must be GPU tensors on the device of x")
    cos, sin = cos.float().reshape(L, D).contiguous(), sin.float().reshape(L, D).contiguous()
    y = torch.empty((L, NH, D), device=x.device, dtype=torch.bfloat16)
    rc = _lib.lib().rspx_rope_vision(x.data_ptr(), x.stride(0), x.stride(1), cos.data_ptr(), sin.data_ptr(),
                                     cos.stride(0), y.data_ptr(), L, NH, D, _lib.stream_ptr(x.device))
    _lib.check("rspx_rope_vision", rc)
    return y
