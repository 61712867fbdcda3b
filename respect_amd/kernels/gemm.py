"""Linear layer whose result does not depend on the number of rows.

Same call signature and meaning as respect/kernels/gemm.py:30-41 (``linear``):
x (..., K) @ w (N, K)^T -> (..., N), bf16 inputs, fp32 accumulation, output in
``out_dtype`` (default x.dtype; torch.float32 for the vocabulary projection as
respect/kernels/patch.py:23 asks).  The Triton tuning keywords (BM, BN, BK,
num_warps, num_stages) are accepted and ignored: the HIP kernel
(respect_amd/csrc/gemm.hip) fixes its own K order from (N, K) alone.

``w`` may also be a :class:`TiledWeight` (``tile_weight``): the same matrix in
the tiled weight layout the kernel streams fastest, with the same results, bit
for bit.  That layout has no counterpart in the reference.
"""
from __future__ import annotations

import torch

from .. import _lib
from ._tensor import as_kernel_input


class TiledWeight:
    """A bf16 weight matrix [N, K] held in the tiled weight layout of
    rspx_linear_tile_weight (16-row slabs of 16 K elements plus a pad, 1 KB
    tiles of 16 x 32 in order of k inside a slab).  ``shape``, ``dtype``, ``data_ptr()``
    and ``stride(0)`` (RSPX_TILED) are what the kernel wrappers read;
    ``dense()`` gives the row-major matrix back."""

    def __init__(self, buf: torch.Tensor, N: int, K: int):
        self.buf = buf
        self.shape = (N, K)
        self.dtype = buf.dtype
        self.device = buf.device

    def data_ptr(self) -> int:
        return self.buf.data_ptr()

    def stride(self, dim: int = 0) -> int:
        if dim != 0:
            raise ValueError("TiledWeight has a row stride only")
        return _lib.RSPX_TILED

    def dense(self) -> torch.Tensor:
        """The [N, K] matrix, row-major (a copy)."""
        N, K = self.shape
        slabs = self.buf.view(N // 16, -1)[:, :16 * K]
        return slabs.reshape(N // 16, K // 32, 4, 16, 8).permute(0, 3, 1, 2, 4).reshape(N, K)


def tile_weight(w: torch.Tensor) -> TiledWeight:
    """``w`` [N, K] bf16 (N % 16 == 0, K % 32 == 0) copied into the tiled weight layout."""
    if w.dim() != 2:
        raise ValueError(f"tile_weight: w must be [N, K], got {tuple(w.shape)}")
    w2 = as_kernel_input(w, "w")
    N, K = w2.shape
    L = _lib.lib()
    n = L.rspx_linear_tiled_weight_elems(N, K)
    if n < 0:
        _lib.check("rspx_linear_tile_weight", -2)
    buf = torch.empty(n, dtype=torch.bfloat16, device=w2.device)
    _lib.check("rspx_linear_tile_weight", L.rspx_linear_tile_weight(
        w2.data_ptr(), w2.stride(0), N, K, buf.data_ptr(), _lib.stream_ptr(w2.device)))
    return TiledWeight(buf, N, K)


def linear(x, w, BM=32, BN=128, BK=64, num_warps=4, num_stages=2, out_dtype=None, out=None, workspace=None):
    """x (M, K) @ w (N, K)^T -> (M, N). Bias is handled by the caller.  ``workspace``:
    optional uint8 GPU tensor of at least rspx_linear_workspace_bytes bytes."""
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise TypeError("linear: bf16 x and w are required")
    out_dtype = out_dtype or x.dtype
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("linear: out_dtype must be bf16 or fp32")
    K = x.shape[-1]
    N = w.shape[0]
    if len(w.shape) != 2 or w.shape[1] != K:
        raise ValueError(f"linear: w must be [N, {K}], got {tuple(w.shape)}")
    xs = as_kernel_input(x.reshape(-1, K), "x")
    w2 = w if isinstance(w, TiledWeight) else as_kernel_input(w, "w")
    M = xs.shape[0]
    if out is None:
        out = torch.empty((M, N), device=x.device, dtype=out_dtype)
    L = _lib.lib()
    need = L.rspx_linear_workspace_bytes(M, N, K)
    if need < 0:
        _lib.check("rspx_linear_workspace_bytes", -2)
    ws = workspace if workspace is not None else _lib.workspace(x.device, max(need, 16), tag="linear")
    if ws.numel() < need:
        raise ValueError("linear: workspace too small")
    rc = L.rspx_linear(xs.data_ptr(), xs.stride(0), w2.data_ptr(), w2.stride(0), out.data_ptr(), out.stride(0),
                       M, N, K, 1 if out_dtype == torch.float32 else 0, ws.data_ptr(), ws.numel(),
                       _lib.stream_ptr(x.device))
    _lib.check("rspx_linear", rc)
    return out.reshape(*x.shape[:-1], N)
