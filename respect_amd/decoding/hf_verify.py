"""Trie verification and 1-token decoding through a Hugging Face decoder.

``verify_trie_hf`` is respect/decoding/verify.py:12-46 on a transformers 5.x
causal LM whose kernels ``patch.install`` replaced: node ``i`` is written to
slot ``prompt_len + base + i`` (its physical slot) while its rotary position
follows its depth (``prompt_len + base + depth + rope_delta``, the same in every
M-RoPE axis); the 4-D mask opens the prompt and the committed tokens to every
node and each node only to its ancestors.  ``forward_tokens_hf`` is the 1-token
path of respect/decoding/sequential.py:17-27 on the same cache layout, the
reference every verified row must equal bit for bit.

Both raise AttentionWaitError when an attention call of theirs gave up its
bounded wait (rows of NaN), before the caller commits anything.

``model(input_ids=, position_ids=, attention_mask=, past_key_values=,
use_cache=True)`` must return an object with ``.logits`` (any Hugging Face
causal LM does); ``cache`` is a ``hf_kv.WindowCache``.
"""
from __future__ import annotations

from typing import Any

import torch

from .. import _lib
from ..candidates.trie import Trie, trie_ancestry
from ..kernels.attention import raise_if_gave_up, status_word


@torch.no_grad()
def verify_trie_hf(model: Any, cache: Any, tree: Trie, prompt_len: int, base: int, capacity: int,
                   rope_delta: int = 0) -> torch.Tensor:
    """Logits [N, V] of every trie node from one forward pass."""
    dev = cache.layers[0].keys.device
    q = len(tree.nodes)
    start = prompt_len + base
    ids = torch.tensor([[n.token for n in tree.nodes]], device=dev, dtype=torch.long)
    depth = torch.tensor([n.depth for n in tree.nodes], device=dev, dtype=torch.long)
    pos = (depth + start + rope_delta).view(1, q)
    allow = torch.zeros((1, 1, q, prompt_len + capacity), dtype=torch.bool, device=dev)
    allow[..., :start] = True
    allow[0, 0, :, start:start + q] = torch.from_numpy(trie_ancestry(tree)).to(dev)
    cache.set_positions(torch.arange(start, start + q, device=dev))
    out = model(input_ids=ids, position_ids=pos, attention_mask=allow, past_key_values=cache, use_cache=True)
    _check_attention(dev)
    return out.logits[0]


def _check_attention(dev) -> None:
    """Raise AttentionWaitError (and clear the flag) if a trie-attention call of
    the forward just run on this stream gave up its bounded wait: its rows are
    NaN, so the step must not be committed (the caller falls back, as the
    reference's dispatcher does on a kernel error, dispatch.py:116-122).  One
    word copied to the host."""
    if dev.type != "cuda":
        return
    ws = _lib.current_workspace(dev)
    if ws is not None:
        raise_if_gave_up(int(status_word(ws).item()), ws)


@torch.no_grad()
def forward_tokens_hf(model: Any, cache: Any, token_ids: list[int], slot: int, position: int,
                      prompt_len: int, capacity: int) -> torch.Tensor:
    """Feed ``token_ids`` one at a time at slots ``slot, slot + 1, ...`` and rotary
    positions ``position, position + 1, ...``; every earlier slot is visible.
    Returns the logits [len(token_ids), V] of the 1-token forwards."""
    dev = cache.layers[0].keys.device
    rows = []
    for j, t in enumerate(token_ids):
        s = slot + j
        allow = torch.zeros((1, 1, 1, prompt_len + capacity), dtype=torch.bool, device=dev)
        allow[..., :s + 1] = True
        cache.set_positions(torch.tensor([s], device=dev))
        out = model(input_ids=torch.tensor([[t]], device=dev), position_ids=torch.tensor([[position + j]], device=dev),
                    attention_mask=allow, past_key_values=cache, use_cache=True)
        rows.append(out.logits[0, -1])
    _check_attention(dev)
    return torch.stack(rows)
