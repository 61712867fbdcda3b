"""Install the row-invariant kernels into a Hugging Face decoder.

Same interface as respect/kernels/patch.py:22-107: ``FixedLinear``,
``FixedNorm``, ``LINEARS``, ``NORMS``, ``install(model, prompt_len) -> int``,
``uninstall(model)``, ``dedicated_kernels(model, prompt_len)`` and
``is_installed()``.  The seven linear layers of every decoder layer and the
vocabulary projection (fp32 scores) go to ``linear`` (rspx_linear), the four
RMS norms of every layer and the final one to ``rmsnorm`` (rspx_rmsnorm), and
SDPA to ``dispatch.unified_forward``: every reduction then runs in an order
that does not depend on how many rows a call carries.

``install`` finds the language model the way the reference does
(``model.vlm.model.language_model``, else ``model.vlm.model``) and also
accepts a Hugging Face model directly (``model.model.language_model``,
``model.model`` or ``model`` itself, with ``lm_head`` next to it).  Unlike the
reference, it checks before wrapping that every layer it wraps has shapes the
kernels build (bf16 weights, in_features % 256 == 0, out_features % 16 == 0)
and raises ``ValueError`` naming the first one that does not, instead of
failing at the first forward.
"""
from __future__ import annotations

import contextlib
from typing import Any, Iterator

import torch
import torch.nn as nn

from . import dispatch
from .gemm import linear
from .rmsnorm import rmsnorm

GEMM_CFG = dict(BM=32, BN=128, BK=128, num_warps=4, num_stages=3)
LM_OUT_DTYPE = torch.float32  # vocabulary scores are kept in fp32


class FixedLinear(nn.Module):
    def __init__(self, base: nn.Module, out_dtype: str | None = None) -> None:
        super().__init__()
        self.base = base
        self.out_dtype = out_dtype

    def forward(self, x):
        od = LM_OUT_DTYPE if self.out_dtype == "lm" else None
        out = linear(x, self.base.weight, out_dtype=od, **GEMM_CFG)
        if getattr(self.base, "bias", None) is not None:
            out = out + self.base.bias
        return out


class FixedNorm(nn.Module):
    def __init__(self, base: nn.Module) -> None:
        super().__init__()
        self.base = base

    def forward(self, x):
        return rmsnorm(x, self.base.weight, self.base.variance_epsilon)


LINEARS = [("self_attn", "q_proj"), ("self_attn", "k_proj"), ("self_attn", "v_proj"),
           ("self_attn", "o_proj"),
           ("mlp", "gate_proj"), ("mlp", "up_proj"), ("mlp", "down_proj")]
NORMS = [("self_attn", "q_norm"), ("self_attn", "k_norm"),
         (None, "input_layernorm"), (None, "post_attention_layernorm")]
_saved: list = []


def _language_model(model: Any):
    """(decoder with .layers, owner of lm_head)."""
    vlm = getattr(model, "vlm", None)
    if vlm is not None:
        inner = vlm.model
        return (inner.language_model if hasattr(inner, "language_model") else inner), vlm
    inner = getattr(model, "model", None)
    if inner is not None:
        return (inner.language_model if hasattr(inner, "language_model") else inner), model
    return model, model


def _check_linear(name: str, mod: nn.Module) -> None:
    w = getattr(mod, "weight", None)
    if w is None or w.dim() != 2 or w.dtype != torch.bfloat16 or w.shape[1] % 256 or w.shape[0] % 16:
        shape = None if w is None else (tuple(w.shape), w.dtype)
        raise ValueError(f"install: {name} {shape} is not a shape the row-invariant linear builds "
                         "(bf16, in_features % 256 == 0, out_features % 16 == 0)")


def _check_norm(name: str, mod: nn.Module) -> None:
    w = getattr(mod, "weight", None)
    if w is None or w.dtype != torch.bfloat16 or not hasattr(mod, "variance_epsilon"):
        raise ValueError(f"install: {name} is not a bf16 RMSNorm with variance_epsilon")


def _targets(model: Any):
    lm, head_owner = _language_model(model)
    lins, norms = [], []
    for i, layer in enumerate(lm.layers):
        for pn, cn in LINEARS:
            p = getattr(layer, pn, None)
            if p is not None and getattr(p, cn, None) is not None:
                lins.append((f"layers.{i}.{pn}.{cn}", p, cn, False))
        for pn, cn in NORMS:
            p = layer if pn is None else getattr(layer, pn, None)
            if p is not None and getattr(p, cn, None) is not None:
                norms.append((f"layers.{i}.{cn}", p, cn))
    for nm in ("norm", "final_layernorm"):
        if hasattr(lm, nm) and hasattr(getattr(lm, nm), "variance_epsilon"):
            norms.append((nm, lm, nm))
    if getattr(head_owner, "lm_head", None) is not None:
        lins.append(("lm_head", head_owner, "lm_head", True))
    return lins, norms


def _wrap(parent, name, cls, lm=False):
    base = getattr(parent, name, None)
    if base is None or isinstance(base, cls):
        return False
    _saved.append((parent, name, base))
    setattr(parent, name, cls(base, "lm") if (lm and cls is FixedLinear) else cls(base))
    return True


def is_installed() -> bool:
    return bool(_saved)


def install(model: Any, prompt_len: int) -> int:
    """Wrap every linear layer and RMS norm of the language model and route SDPA to
    the trie kernel; returns the number of modules wrapped (patch.py:70-88)."""
    lins, norms = _targets(model)
    for name, p, cn, _ in lins:
        if not isinstance(getattr(p, cn), FixedLinear):
            _check_linear(name, getattr(p, cn))
    for name, p, cn in norms:
        if not isinstance(getattr(p, cn), FixedNorm):
            _check_norm(name, getattr(p, cn))
    for _, p, cn, lm in lins:
        _wrap(p, cn, FixedLinear, lm=lm)
    for _, p, cn in norms:
        _wrap(p, cn, FixedNorm)
    dispatch.install(prompt_len)
    return len(_saved)


def uninstall(model: Any) -> None:
    dispatch.uninstall()
    while _saved:
        parent, name, base = _saved.pop()
        setattr(parent, name, base)


@contextlib.contextmanager
def dedicated_kernels(model: Any, prompt_len: int) -> Iterator[None]:
    """Run the enclosed block with the row-invariant kernels installed.

    Install after Prefill: Prefill itself runs on the default kernels.
    """
    install(model, prompt_len)
    try:
        yield
    finally:
        uninstall(model)
