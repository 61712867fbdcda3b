"""The tile-wise ("blocked") trie attention: the negative control of the slot-layout
experiment, with the interface of respect/kernels/reference_blocked.py:83-106.

``fused_attn(q, kp, vp, kn, vn, msk, sm_scale=None, BM=64, BN=64, num_warps=4,
num_stages=2)``: q [H, M, D], kp/vp [HK, NP, D], kn/vn [HK, NN, D], msk [M, NN] bool;
returns a new [H, M, D] bf16 tensor.  Node slots are reduced BN at a time like the prompt
(rspx_blocked_attn), so moving the same ancestors to other slots can change the output --
which is what the experiment shows and what ``fused_attn_hyb`` (respect_amd.kernels.attention)
avoids.  BM, num_warps and num_stages are accepted and ignored; BN must be 32, 64 or 128.
As the reference asserts, H must be a multiple of HK and D one of 32, 64, 128, 256; the
kernel builds D = 64 and 128 and raises for the others.
"""
from __future__ import annotations

import torch

from .. import _lib
from ._tensor import as_kernel_input


def fused_attn(q, kp, vp, kn, vn, msk, sm_scale=None, BM=64, BN=64, num_warps=4, num_stages=2):
    H, M, D = q.shape
    HK, NP, _ = kp.shape
    NN = kn.shape[1]
    assert H % HK == 0 and D in (32, 64, 128, 256)
    if sm_scale is None:
        sm_scale = D ** -0.5
    if tuple(msk.shape) != (M, NN):
        raise ValueError(f"fused_attn: msk must be [{M}, {NN}], got {tuple(msk.shape)}")
    dev = q.device
    q, kp, vp, kn, vn = (as_kernel_input(t, n) for t, n in zip((q, kp, vp, kn, vn), ("q", "kp", "vp", "kn", "vn")))
    if msk.dtype not in (torch.bool, torch.uint8):
        msk = msk != 0
    out = torch.empty((H, M, D), dtype=torch.bfloat16, device=dev)
    rc = _lib.lib().rspx_blocked_attn(
        q.data_ptr(), q.stride(0), q.stride(1), kp.data_ptr(), kp.stride(0), kp.stride(1),
        vp.data_ptr(), vp.stride(0), vp.stride(1), kn.data_ptr(), kn.stride(0), kn.stride(1),
        vn.data_ptr(), vn.stride(0), vn.stride(1), msk.data_ptr(), msk.stride(0), msk.stride(1),
        out.data_ptr(), out.stride(0), out.stride(1), H, HK, M, NP, NN, D, int(BN), float(sm_scale),
        _lib.stream_ptr(dev))
    _lib.check("rspx_blocked_attn", rc)
    return out
