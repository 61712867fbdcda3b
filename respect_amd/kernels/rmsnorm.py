"""RMS normalization whose result does not depend on the number of rows.

Same call as respect/kernels/rmsnorm.py:25 (``rmsnorm(x, w, eps)``): the last
dimension is normalised, rounding where PyTorch rounds (fp32 statistics, bf16
after the scaling, bf16 after the weight).  The HIP kernel reduces a row in an
order fixed by the row length alone (respect_amd/csrc/norm_rope.hip), for any
row length.
"""
from __future__ import annotations

import torch

from .. import _lib
from ._tensor import as_kernel_input


def rmsnorm(x, w, eps):
    """x [..., N] bf16, w [N] bf16 -> bf16 tensor shaped like x."""
    shape = x.shape
    N = shape[-1]
    if w.numel() != N:
        raise ValueError(f"rmsnorm: w has {w.numel()} elements for rows of {N}")
    xs = as_kernel_input(x.reshape(-1, N), "x")
    w = as_kernel_input(w.reshape(N), "w")
    M = xs.shape[0]
    out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    rc = _lib.lib().rspx_rmsnorm(xs.data_ptr(), xs.stride(0), w.data_ptr(), out.data_ptr(), out.stride(0),
                                 M, N, float(eps), _lib.stream_ptr(x.device))
    _lib.check("rspx_rmsnorm", rc)
    return out.reshape(shape)
