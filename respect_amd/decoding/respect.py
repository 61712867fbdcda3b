"""Trie verification with greedy acceptance (one step of respect/decoding/respect.py):
verify every node in one forward, walk the trie with the target's greedy
choices, move the accepted path's KV to consecutive slots."""
from __future__ import annotations

import torch

from ..candidates.trie import Trie
from ..kernels.attention import raise_if_gave_up, status_word
from .acceptance import greedy_token, walk
from .verify import verify_trie, verify_trie_greedy


@torch.no_grad()
def respect_step(model, cache, tree: Trie, first: int, P: int, base: int, eos: int, offset: int = 0,
                 size: int = 0, cap: int = 1 << 30, graph: bool = False) -> tuple[list[int], int, list[int]]:
    """Returns (accepted tokens, correction token, node path).  The accepted
    tokens' KV ends up in slots P + base .. P + base + len - 1.  Raises
    AttentionWaitError (nothing accepted, no KV moved, the flag cleared) when an
    attention call of the step gave up its bounded wait."""
    if graph and offset == 0 and size == 0:
        picks = verify_trie_greedy(model, cache, tree, P, base)   # raises if an attention wait gave up
    else:
        logits = verify_trie(model, cache, tree, P, base, graph=graph)
        ws = model.attn_ws_used   # the workspace of the forward just run (eager or replayed)
        # the attention's timeout flag travels with the picks: one device-to-host copy
        vals = torch.cat([greedy_token(logits, offset, size), status_word(ws).to(torch.int64)]).tolist()
        picks = vals[:-1]
        raise_if_gave_up(vals[-1], ws)   # before the walk: nothing is committed
    path, acc, rec = walk(tree, first, cap, eos, lambda a, ch: picks[ch])
    cache.compact(P + base, path)
    return acc, rec, path
