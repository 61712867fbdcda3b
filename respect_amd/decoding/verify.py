"""One forward pass that verifies every node of a trie (respect/decoding/verify.py:12-46).

Node i is written to cache slot P + base + i (its physical slot) while its
rotary position follows its depth (P + base + depth, its logical position);
the mask opens the prompt and the ``base`` committed tokens to every node and
each node to its ancestors.  The mask and the depths are built on the GPU
from the parent array (rspx_trie_mask) instead of a host-built dense mask.
"""
from __future__ import annotations

import torch

from .. import _lib
from ..candidates.trie import Trie


def node_slots(base: int, n: int, step: int = 32) -> int:
    """Node-segment width of a call: committed + trie slots, padded to ``step``."""
    return max(step, -(-(base + n) // step) * step)


def trie_mask(tree: Trie, base: int, NN: int, device, rows: int | None = None,
              out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(msk [rows, NN] uint8, depth [N] int32) on the GPU; rows past N open slot 0 only."""
    N = len(tree.nodes)
    rows = N if rows is None else rows
    parent = torch.from_numpy(tree.parents).to(device)
    msk = out if out is not None else torch.empty((rows, NN), dtype=torch.uint8, device=device)
    depth = torch.empty(N, dtype=torch.int32, device=device)
    rc = _lib.lib().rspx_trie_mask(parent.data_ptr(), N, base, rows, NN, msk.data_ptr(), msk.stride(0),
                                   depth.data_ptr(), _lib.stream_ptr(torch.device(device)))
    _lib.check("rspx_trie_mask", rc)
    return msk, depth


@torch.no_grad()
def verify_trie(model, cache, tree: Trie, P: int, base: int, graph: bool = False) -> torch.Tensor:
    """fp32 logits [N, V] of every trie node.  ``graph``: replay a captured
    forward (rows padded to a multiple of 64, node segment to a multiple of 64)
    whose mask, slots and positions are made on the device (rspx_step_inputs);
    the node segment width never changes a row's result."""
    dev = model.device
    N = len(tree.nodes)
    if graph:
        T = max(64, -(-N // 64) * 64)
        NN = node_slots(base, N, 64)
        gf = model.graphed(cache, P, T, NN)
        return gf.run(N, base, tree.tokens, tree.parents)[:N]
    ids = torch.from_numpy(tree.tokens).to(dev)
    start = P + base
    slots = torch.arange(start, start + N, dtype=torch.int32, device=dev)
    NN = node_slots(base, N)
    if P + NN > cache.cap:
        raise ValueError("KV cache too small for the trie")
    msk, depth = trie_mask(tree, base, NN, dev)
    return model.forward(ids, slots, depth.to(torch.int64) + start, cache, P, msk, NN)


@torch.no_grad()
def verify_trie_greedy(model, cache, tree: Trie, P: int, base: int) -> list[int]:
    """The greedy token (whole vocabulary) of every trie node from one replayed
    forward whose argmax is taken inside the graph; only the N choices come
    back to the host."""
    N = len(tree.nodes)
    T = max(64, -(-N // 64) * 64)
    gf = model.graphed(cache, P, T, node_slots(base, N, 64))
    gf.run(N, base, tree.tokens, tree.parents)
    return gf.greedy(N)
