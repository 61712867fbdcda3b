"""Greedy token choice and the acceptance walk (respect/decoding/acceptance.py:11-46).

``greedy_token`` runs on the GPU (rspx_argmax_rows): the index of the largest
fp32 logit with the excluded vocabulary range counted as -inf, ties to the
lowest index -- the same choice as ``mask_action_vocab(...).argmax(-1)``.
``walk`` is host code: it follows the trie while the target's choice matches.
"""
from __future__ import annotations

from typing import Callable

import torch

from .. import _lib
from ..candidates.trie import Trie


def greedy_token(logits: torch.Tensor, offset: int = 0, size: int = 0, out: torch.Tensor | None = None,
                 workspace: torch.Tensor | None = None) -> torch.Tensor:
    """logits [M, V] fp32 on the GPU -> int64 [M]."""
    if logits.dtype != torch.float32 or not logits.is_cuda or logits.dim() != 2 or logits.stride(1) != 1:
        raise TypeError("greedy_token: fp32 [M, V] GPU logits with contiguous rows are required")
    M, V = logits.shape
    if logits.stride(0) % 4 or logits.data_ptr() % 16:
        logits = logits.contiguous().clone()
    if out is None:
        out = torch.empty(M, dtype=torch.int64, device=logits.device)
    L = _lib.lib()
    need = L.rspx_argmax_workspace_bytes(M, V)
    ws = workspace if workspace is not None else _lib.workspace(logits.device, need, tag="argmax")
    rc = L.rspx_argmax_rows(logits.data_ptr(), logits.stride(0), M, V, int(offset), int(size),
                            out.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_ptr(logits.device))
    _lib.check("rspx_argmax_rows", rc)
    return out


def walk(tree: Trie, first: int, cap: int, eos: int,
         pick: Callable[[list[int], int], int]) -> tuple[list[int], list[int], int]:
    """Accept trie tokens while they match the target's choice (acceptance.py:26-46).

    Starts at the root whose token is ``first`` and takes at most ``cap`` nodes.
    After each accepted node (unless its token is ``eos``) ``pick(tokens, node)``
    gives the target's next token; the walk descends to the child carrying it, or
    stops when there is none.  Returns (node path, accepted tokens, correction
    token): the correction is the last token ``pick`` returned, ``first`` if it
    was never called.
    """
    path: list[int] = []
    tokens: list[int] = []
    correction = first
    node = tree.roots.get(first)
    for _ in range(max(cap, 0)):
        if node is None:
            break
        entry = tree.nodes[node]
        path.append(node)
        tokens.append(entry.token)
        if entry.token == eos:
            break
        correction = pick(tokens, node)
        node = entry.children.get(correction)
    return path, tokens, correction
