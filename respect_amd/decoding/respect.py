"""Trie verification with greedy acceptance (one step of respect/decoding/respect.py):
verify every node in one forward, walk the trie with the target's greedy
choices, move the accepted path's KV to consecutive slots."""
from __future__ import annotations

import torch

from ..candidates.trie import Trie
from .acceptance import greedy_token, walk
from .verify import verify_trie, verify_trie_greedy


@torch.no_grad()
def respect_step(model, cache, tree: Trie, first: int, P: int, base: int, eos: int, offset: int = 0,
                 size: int = 0, cap: int = 1 << 30, graph: bool = False) -> tuple[list[int], int, list[int]]:
    """Returns (accepted tokens, correction token, node path).  The accepted
    tokens' KV ends up in slots P + base .. P + base + len - 1."""
    if graph and offset == 0 and size == 0:
        picks = verify_trie_greedy(model, cache, tree, P, base)
    else:
        logits = verify_trie(model, cache, tree, P, base, graph=graph)
        picks = greedy_token(logits, offset, size).tolist()
    path, acc, rec = walk(tree, first, cap, eos, lambda a, ch: picks[ch])
    cache.compact(P + base, path)
    return acc, rec, path
