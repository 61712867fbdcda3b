"""Argument checks shared by the kernel wrappers."""
from __future__ import annotations

import torch


def _aligned(t: torch.Tensor, inner_contig: bool = True) -> bool:
    if t.data_ptr() % 16 != 0:
        return False
    if inner_contig and t.dim() > 0 and t.stride(-1) != 1 and t.shape[-1] != 1:
        return False
    return all(s % 8 == 0 for s in t.stride()[:-1])


def as_kernel_input(t: torch.Tensor, name: str, dtype=torch.bfloat16) -> torch.Tensor:
    """Check device/dtype; return ``t`` itself when its layout suits the kernels
    (contiguous last dim, 16-byte aligned rows), else a contiguous copy that
    starts 16-byte aligned (its rows are aligned too when the last dim is a
    multiple of 8; the kernels take other lengths unaligned)."""
    if not t.is_cuda:
        raise RuntimeError(f"{name}: respect_amd kernels need a GPU tensor (got {t.device})")
    if t.dtype != dtype:
        raise TypeError(f"{name}: expected {dtype}, got {t.dtype}")
    if _aligned(t):
        return t
    t = t.contiguous()
    if t.data_ptr() % 16 != 0:
        t = t.clone()
    return t
