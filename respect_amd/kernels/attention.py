"""Trie-verification attention with a slot-order-independent sum over nodes.

Same call signature and meaning as respect/kernels/attention.py:74-96
(``fused_attn_hyb``): q [H, M, D], kp/vp [HK, NP, D] (the prompt keys, never
masked; NP = kp.shape[1] is the prompt length), kn/vn [HK, NN, D] (node slots),
msk [M, NN] bool (True = the row may attend to that slot); returns a new
[H, M, D] bf16 tensor.  The Triton tuning keywords (BM, BN, BNB, num_warps,
num_stages) are accepted for compatibility; only ``NN % BNB == 0`` is still
checked, as the reference does.

The HIP kernel (respect_amd/csrc/trie_attn.hip) sums every row's allowed node
slots in slot order, in MFMA tiles of 32 ranks, and reduces the prompt in a
fixed tree set by NP alone, so a row's bits do not depend on M, on where its
ancestors sit in the node segment, or on the other rows.
"""
from __future__ import annotations

import torch

from .. import _lib
from ._tensor import as_kernel_input


def trie_attn(q, kp, vp, kn, vn, msk, sm_scale=None, out=None, rows_per_wave: int = 0, workspace=None,
              launches: int = 0, out_tiled: bool = False):
    """Launch the kernel on the current stream.  ``rows_per_wave`` (0/1/2) and
    ``launches`` (0 = automatic, 1 = one kernel when it fits, 2 = two kernels)
    only change the work split, never the result.  ``workspace``: a zero-filled
    uint8 GPU tensor of at least rspx_trie_attn_workspace_bytes bytes (default:
    a per-stream scratch buffer).  ``out_tiled``: ``out`` is a flat bf16 buffer
    of at least ceil(M / 64) 64 H D elements that receives the [M, H D] result
    in the tiled activation layout (RSPX_TILED) instead of [H, M, D]."""
    H, M, D = q.shape
    HK, P, D2 = kp.shape
    NN = kn.shape[1]
    if D2 != D or vp.shape != kp.shape or kn.shape != (HK, NN, D) or vn.shape != kn.shape:
        raise ValueError("fused_attn_hyb: inconsistent q/k/v shapes")
    if tuple(msk.shape) != (M, NN):
        raise ValueError(f"fused_attn_hyb: msk must be [{M}, {NN}], got {tuple(msk.shape)}")
    if sm_scale is None:
        sm_scale = D ** -0.5
    dev = q.device
    q = as_kernel_input(q, "q")
    kp = as_kernel_input(kp, "kp")
    vp = as_kernel_input(vp, "vp")
    kn = as_kernel_input(kn, "kn")
    vn = as_kernel_input(vn, "vn")
    if not msk.is_cuda:
        raise RuntimeError("fused_attn_hyb: msk must be a GPU tensor")
    if msk.dtype not in (torch.bool, torch.uint8):
        msk = msk != 0
    if out_tiled:
        if out is None or out.dtype != torch.bfloat16 or out.numel() < -(-M // 64) * 64 * H * D:
            raise ValueError("fused_attn_hyb: out_tiled needs a bf16 buffer of ceil(M/64)*64*H*D elements")
        soh, som = D, _lib.RSPX_TILED
    else:
        if out is None:
            out = torch.empty((H, M, D), dtype=torch.bfloat16, device=dev)
        soh, som = out.stride(0), out.stride(1)
    L = _lib.lib()
    need = L.rspx_trie_attn_workspace_bytes(H, HK, M, P, D)
    if need < 0:
        _lib.check("rspx_trie_attn_workspace_bytes", -2)
    ws = workspace if workspace is not None else _lib.workspace(dev, need)
    if ws.numel() < need:
        raise ValueError("fused_attn_hyb: workspace too small")
    fn = L.rspx_trie_attn if launches == 0 else L.rspx_trie_attn_launches
    extra = () if launches == 0 else (int(launches),)
    rc = fn(
        q.data_ptr(), q.stride(0), q.stride(1),
        kp.data_ptr(), kp.stride(0), kp.stride(1),
        vp.data_ptr(), vp.stride(0), vp.stride(1),
        kn.data_ptr(), kn.stride(0), kn.stride(1),
        vn.data_ptr(), vn.stride(0), vn.stride(1),
        msk.data_ptr(), msk.stride(0), msk.stride(1),
        out.data_ptr(), soh, som,
        H, HK, M, P, NN, D, float(sm_scale),
        ws.data_ptr(), ws.numel(), int(rows_per_wave), *extra,
        _lib.stream_ptr(dev))
    _lib.check("rspx_trie_attn", rc)
    return out


class AttentionWaitError(RuntimeError):
    """A one-launch attention call ran out of its bounded wait (its workgroups
    were not all resident at once): its output rows hold NaN.  Raised by the
    verification steps before anything is committed, so the caller can fall
    back (the reference falls back to stock SDPA on any kernel error,
    respect/kernels/dispatch.py:116-122)."""


def status_word(workspace: torch.Tensor) -> torch.Tensor:
    """The timeout flag of an attention workspace: an int32 [1] view of its
    first word (RSPX_ATTN_STATUS_WORD), nonzero once a call on it gave up."""
    return workspace[:4].view(torch.int32)


def raise_if_gave_up(flag: int, workspace: torch.Tensor) -> None:
    """``flag``: the host copy of ``status_word(workspace)`` taken after the
    calls to check.  Nonzero: clear the word (on the current stream) and raise
    AttentionWaitError."""
    if flag:
        status_word(workspace).zero_()
        raise AttentionWaitError("trie attention: a one-launch wait gave up (workgroups not co-resident); "
                                 "the call's output rows are NaN and nothing was committed")


def fused_attn_hyb(q, kp, vp, kn, vn, msk, sm_scale=None,
                   BM=64, BN=128, BNB=16, num_warps=4, num_stages=1):
    """q (H, M, D), kp/vp (HK, NP, D), kn/vn (HK, NN, D), msk (M, NN) bool -> (H, M, D)."""
    NN = kn.shape[1]
    assert NN % BNB == 0
    return trie_attn(q, kp, vp, kn, vn, msk, sm_scale)


def make_launcher(q, kp, vp, kn, vn, msk, sm_scale=None, out=None, workspace=None,
                  rows_per_wave: int = 0, stream=None):
    """Pre-bind every argument of one attention call and return ``(launch, out)``;
    ``launch()`` enqueues the kernel with a single C call (no per-call checks).
    The tensors must already suit the kernel (bf16, contiguous head_dim, aligned)."""
    H, M, D = q.shape
    HK, P, _ = kp.shape
    NN = kn.shape[1]
    for name, t in (("q", q), ("kp", kp), ("vp", vp), ("kn", kn), ("vn", vn)):
        if as_kernel_input(t, name) is not t:
            raise ValueError(f"make_launcher: {name} layout does not suit the kernel")
    if sm_scale is None:
        sm_scale = D ** -0.5
    if out is None:
        out = torch.empty((H, M, D), dtype=torch.bfloat16, device=q.device)
    L = _lib.lib()
    need = L.rspx_trie_attn_workspace_bytes(H, HK, M, P, D)
    if workspace is None:
        workspace = _lib.workspace(q.device, need)   # zero-filled on allocation
    if workspace.numel() < need:
        raise ValueError("make_launcher: workspace too small")
    s = stream if stream is not None else _lib.stream_ptr(q.device)
    args = (q.data_ptr(), q.stride(0), q.stride(1),
            kp.data_ptr(), kp.stride(0), kp.stride(1),
            vp.data_ptr(), vp.stride(0), vp.stride(1),
            kn.data_ptr(), kn.stride(0), kn.stride(1),
            vn.data_ptr(), vn.stride(0), vn.stride(1),
            msk.data_ptr(), msk.stride(0), msk.stride(1),
            out.data_ptr(), out.stride(0), out.stride(1),
            H, HK, M, P, NN, D, float(sm_scale),
            workspace.data_ptr(), workspace.numel(), int(rows_per_wave), s)
    fn = L.rspx_trie_attn

    def launch():
        rc = fn(*args)
        if rc != 0:
            _lib.check("rspx_trie_attn", rc)

    return launch, out
