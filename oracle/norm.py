"""RMSNorm, RoPE and SwiGLU on the CPU (numpy) -- oracle restatements.

rmsnorm   respect/kernels/rmsnorm.py:12-22: x32 = float(x); var = sum(x32^2)/N;
          xh = bf16(x32 * rsqrt(var + eps)); y = bf16(float(w) * float(xh)).
          The sum is taken in float64 (any fixed order is a valid restatement;
          the reference's order is Triton's tl.sum tree).
rope      respect/system/fused.py:45-64 / HF apply_rotary_pos_emb: each multiply
          and the add are fp32 operations rounded to bf16.
silu_mul  respect/system/fused.py:106-113: a = bf16(g / (1 + exp(-g)));
          y = bf16(a * u).  silu in float64, rounded to fp32 then bf16.
square, add_sq, norm_apply
          respect/system/fused.py:126-159 (the Prefill RMSNorm pieces): q =
          float(x)^2; x = bf16(float(r) + float(h)); y = bf16(float(w) *
          bf16(float(x) * rsqrt(var + eps))), rsqrt = fp32(1 / fp32(sqrt)).
rope_vision
          respect/system/fused.py:78-95 / HF apply_rotary_pos_emb_vision: fp32
          x*cos + rotate_half(x)*sin, one rounding to bf16.

Pinned by (tests/test_oracle_norm.py): rope bitwise against torch's CPU bf16
ops (the reference's own arithmetic); rmsnorm against the HF formula in torch
fp32 on the CPU (<= 1 bf16 ulp) and its constant-row closed form; silu_mul
against torch F.silu(g) * u on the CPU (<= 1 bf16 ulp) and silu(0) = 0,
silu(g) -> g for large g, -> 0 for very negative g.  square, add_sq and
rope_vision bitwise against torch's CPU ops (fp32 multiply/add are correctly
rounded there too); norm_apply against torch.rsqrt on the CPU (<= 1 bf16 ulp)
and exactly where rsqrt is exact (var + eps a power of 4).
"""
from __future__ import annotations

import numpy as np

from .bf16 import round_bf16


def rmsnorm(x, w, eps) -> np.ndarray:
    x = np.asarray(x, np.float32)
    var = (x.astype(np.float64) ** 2).mean(axis=-1, keepdims=True).astype(np.float32)
    r = (1.0 / np.sqrt(var.astype(np.float64) + np.float32(eps))).astype(np.float32)
    xh = round_bf16(x * r)
    return round_bf16(np.asarray(w, np.float32) * xh)


def rotate_half(x: np.ndarray) -> np.ndarray:
    h = x.shape[-1] // 2
    return np.concatenate([-x[..., h:], x[..., :h]], axis=-1)


def rope(x, cos, sin) -> np.ndarray:
    """x [..., D] with cos/sin broadcastable to x (float32 arrays of bf16 values)."""
    x = np.asarray(x, np.float32)
    a = round_bf16(x * np.asarray(cos, np.float32))
    b = round_bf16(rotate_half(x) * np.asarray(sin, np.float32))
    return round_bf16(a + b)


def silu_mul(g, u) -> np.ndarray:
    g64 = np.asarray(g, np.float64)
    with np.errstate(over="ignore"):
        silu = g64 / (1.0 + np.exp(-g64))
    a = round_bf16(silu.astype(np.float32))
    return round_bf16(a * np.asarray(u, np.float32))


def rope_tables(positions, head_dim: int = 128, theta: float = 1.0e6):
    """cos/sin [T, head_dim] as bf16-valued float32, computed in float64 (closed form)."""
    pos = np.asarray(positions, np.float64)
    inv = 1.0 / theta ** (np.arange(0, head_dim, 2, dtype=np.float64) / head_dim)
    ang = pos[:, None] * inv[None, :]
    emb = np.concatenate([ang, ang], axis=-1)
    return round_bf16(np.cos(emb).astype(np.float32)), round_bf16(np.sin(emb).astype(np.float32))


def square(x) -> np.ndarray:
    x = np.asarray(x, np.float32)
    return x * x


def add_sq(r, h):
    x = round_bf16(np.asarray(r, np.float32) + np.asarray(h, np.float32))
    return x, x * x


def rsqrt_rn(v) -> np.ndarray:
    """fp32(1 / fp32(sqrt(v))): a correctly rounded square root, then a correctly rounded divide."""
    v = np.asarray(v, np.float32)
    return (np.float32(1.0) / np.sqrt(v)).astype(np.float32)


def norm_apply(x, var, w, eps) -> np.ndarray:
    """x [M, N] (bf16 values), var [M] fp32, w [N]."""
    x = np.asarray(x, np.float32)
    r = rsqrt_rn(np.asarray(var, np.float32) + np.float32(eps))[:, None]
    xh = round_bf16(x * r)
    return round_bf16(np.asarray(w, np.float32) * xh)


def rope_vision(x, cos, sin) -> np.ndarray:
    """x [L, NH, D] (bf16 values), cos/sin [L, D] fp32."""
    x = np.asarray(x, np.float32)
    c = np.asarray(cos, np.float32)[:, None, :]
    s = np.asarray(sin, np.float32)[:, None, :]
    return round_bf16(x * c + rotate_half(x) * s)
