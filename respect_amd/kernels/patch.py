"""Install the row-invariant kernels into a Hugging Face decoder.

Interface kept from respect/kernels/patch.py:22-107 (the names callers use):
``FixedLinear``, ``FixedNorm``, ``GEMM_CFG``, ``LM_OUT_DTYPE``, ``LINEARS``,
``NORMS``, ``install(model, prompt_len) -> int``, ``uninstall(model)``,
``dedicated_kernels(model, prompt_len)`` and ``is_installed()``.

What gets replaced: the seven linear layers of every decoder layer and the
vocabulary projection (fp32 scores) go to ``gemm.linear`` (rspx_linear), the
four RMS norms of every layer and the final norm to ``rmsnorm.rmsnorm``
(rspx_rmsnorm), and SDPA to ``dispatch.unified_forward`` -- every reduction
then runs in an order that does not depend on how many rows a call carries.

The language model is found as ``model.vlm.model[.language_model]`` (the
reference's Alpamayo wrapper) or, for a plain Hugging Face causal LM, as
``model.model[.language_model]`` with ``lm_head`` beside it.  Before anything
is swapped, every target is checked against what the kernels build (2-D bf16
weights of any shape; bf16 RMSNorms with ``variance_epsilon``); the first
misfit raises ``ValueError`` naming it and the model is left untouched.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

import torch
import torch.nn as nn

from . import dispatch
from .gemm import linear
from .rmsnorm import rmsnorm

GEMM_CFG = dict(BM=32, BN=128, BK=128, num_warps=4, num_stages=3)
LM_OUT_DTYPE = torch.float32  # vocabulary scores are kept in fp32

LINEARS = [("self_attn", "q_proj"), ("self_attn", "k_proj"), ("self_attn", "v_proj"),
           ("self_attn", "o_proj"),
           ("mlp", "gate_proj"), ("mlp", "up_proj"), ("mlp", "down_proj")]
NORMS = [("self_attn", "q_norm"), ("self_attn", "k_norm"),
         (None, "input_layernorm"), (None, "post_attention_layernorm")]


class FixedLinear(nn.Module):
    """``y = x W^T (+ b)`` through the row-invariant kernel; ``out_dtype="lm"`` keeps the
    vocabulary head's scores in ``LM_OUT_DTYPE``.  The wrapped module stays reachable as
    ``.base`` and keeps owning its parameters."""

    def __init__(self, base: nn.Module, out_dtype: str | None = None) -> None:
        super().__init__()
        self.base = base
        self.out_dtype = out_dtype

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        scores = LM_OUT_DTYPE if self.out_dtype == "lm" else None
        y = linear(x, self.base.weight, out_dtype=scores, **GEMM_CFG)
        bias = getattr(self.base, "bias", None)
        return y if bias is None else torch.add(y, bias)


class FixedNorm(nn.Module):
    """The wrapped RMSNorm's weight and epsilon through the row-invariant kernel."""

    def __init__(self, base: nn.Module) -> None:
        super().__init__()
        self.base = base

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        b = self.base
        return rmsnorm(x, b.weight, b.variance_epsilon)


@dataclass
class _Swap:
    parent: nn.Module
    attr: str
    original: nn.Module


@dataclass
class _Installation:
    """Swaps in the order they were made; undone newest first."""
    swaps: list[_Swap] = field(default_factory=list)

    def swap(self, parent: nn.Module, attr: str, make) -> None:
        cur = getattr(parent, attr)
        if isinstance(cur, (FixedLinear, FixedNorm)):
            return                  # already ours: installing twice wraps nothing new
        self.swaps.append(_Swap(parent, attr, cur))
        setattr(parent, attr, make(cur))

    def undo(self) -> None:
        for s in reversed(self.swaps):
            setattr(s.parent, s.attr, s.original)
        self.swaps.clear()


_STATE = _Installation()


def _language_model(model: Any) -> tuple[Any, Any]:
    """(module holding ``.layers``, module holding ``lm_head``)."""
    outer = getattr(model, "vlm", None)
    if outer is None:
        outer = model
    inner = getattr(outer, "model", None)
    if inner is None:
        return model, model
    return getattr(inner, "language_model", inner), outer


def _fits_linear(mod: nn.Module) -> bool:
    w = getattr(mod, "weight", None)
    return w is not None and w.dim() == 2 and w.dtype == torch.bfloat16


def _fits_norm(mod: nn.Module) -> bool:
    w = getattr(mod, "weight", None)
    return w is not None and w.dtype == torch.bfloat16 and hasattr(mod, "variance_epsilon")


def _plan(model: Any) -> list[tuple[str, nn.Module, str, Any]]:
    """Every (name, parent, attribute, wrapper factory) to swap, checked first."""
    lm, head_owner = _language_model(model)
    todo: list[tuple[str, nn.Module, str, Any]] = []

    def add(name, parent, attr, kind):
        mod = getattr(parent, attr, None) if parent is not None else None
        if mod is None:
            return
        if isinstance(mod, (FixedLinear, FixedNorm)):
            todo.append((name, parent, attr, None))
            return
        if kind == "norm":
            if not _fits_norm(mod):
                raise ValueError(f"install: {name} is not a bf16 RMSNorm with variance_epsilon")
            todo.append((name, parent, attr, FixedNorm))
            return
        if not _fits_linear(mod):
            w = getattr(mod, "weight", None)
            shape = None if w is None else (tuple(w.shape), w.dtype)
            raise ValueError(f"install: {name} {shape} is not a 2-D bf16 weight the row-invariant linear builds")
        todo.append((name, parent, attr, (lambda m: FixedLinear(m, "lm")) if kind == "lm" else FixedLinear))

    for i, layer in enumerate(lm.layers):
        for group, attr in LINEARS:
            add(f"layers.{i}.{group}.{attr}", getattr(layer, group, None), attr, "linear")
        for group, attr in NORMS:
            add(f"layers.{i}.{attr}", layer if group is None else getattr(layer, group, None), attr, "norm")
    for attr in ("norm", "final_layernorm"):
        if hasattr(getattr(lm, attr, None), "variance_epsilon"):
            add(attr, lm, attr, "norm")
    add("lm_head", head_owner, "lm_head", "lm")
    return todo


def is_installed() -> bool:
    return bool(_STATE.swaps)


def install(model: Any, prompt_len: int) -> int:
    """Swap in the row-invariant modules and route SDPA to the trie kernel
    (patch.py:70-88); returns how many modules are currently wrapped."""
    for _, parent, attr, make in _plan(model):
        if make is not None:
            _STATE.swap(parent, attr, make)
    dispatch.install(prompt_len)
    return len(_STATE.swaps)


def uninstall(model: Any) -> None:
    """Put every original module back and restore stock SDPA."""
    dispatch.uninstall()
    _STATE.undo()


class dedicated_kernels:
    """``with dedicated_kernels(model, prompt_len):`` -- the row-invariant kernels are
    installed for the block and removed afterwards, also on an exception.  Install
    after Prefill: Prefill itself runs on the stock kernels."""

    def __init__(self, model: Any, prompt_len: int) -> None:
        self.model, self.prompt_len = model, prompt_len

    def __enter__(self) -> None:
        install(self.model, self.prompt_len)

    def __exit__(self, *exc) -> bool:
        uninstall(self.model)
        return False
