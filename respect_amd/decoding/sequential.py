"""Token-by-token greedy decoding (respect/decoding/sequential.py:17-42): the
reference a verification step must reproduce bit for bit."""
from __future__ import annotations

import torch

from ..kernels.attention import raise_if_gave_up, status_word
from .acceptance import greedy_token
from .verify import node_slots


@torch.no_grad()
def forward_token(model, cache, token: int, P: int, c: int, graph: bool = False) -> torch.Tensor:
    """Feed ``token`` at node-segment index ``c`` (cache slot P + c, position
    P + c); it sees the prompt and node slots [0, c].  Returns fp32 logits [1, V].
    ``graph``: replay a captured forward (node segment padded to 64)."""
    dev = model.device
    if c < 0 or P + c >= cache.cap:
        raise ValueError(f"forward_token: slot {P + c} outside the cache's {cache.cap} slots")
    if graph:  # a one-node trie after c committed slots: slot P + c, position P + c, slots [0, c] open
        NN = node_slots(c, 1, 64)
        return model.graphed(cache, P, 1, NN).run(1, c, [token], [-1])
    slot = torch.tensor([P + c], dtype=torch.int32, device=dev)
    ids = torch.tensor([token], device=dev)
    NN = node_slots(c, 1)
    msk = (torch.arange(NN, device=dev) <= c).to(torch.uint8)[None]
    return model.forward(ids, slot, slot.to(torch.int64), cache, P, msk, NN)


@torch.no_grad()
def next_token(model, cache, token: int, P: int, c: int) -> int:
    """forward_token(graph=True) followed by the greedy choice (whole
    vocabulary), the argmax taken inside the captured forward."""
    gf = model.graphed(cache, P, 1, node_slots(c, 1, 64))
    gf.run(1, c, [token], [-1])
    return gf.greedy(1)[0]


@torch.no_grad()
def sequential(model, cache, token: int, P: int, base: int, eos: int, offset: int, size: int,
               max_tokens: int) -> list[int]:
    """Generate from ``token`` (already chosen) until EOS or ``max_tokens``, one
    forward per token; ``base`` committed tokens precede it.  Returns the fed
    tokens, ``token`` first."""
    out, c = [], base
    while len(out) < max_tokens:
        out.append(token)
        logits = forward_token(model, cache, token, P, c)
        c += 1
        if token == eos:
            break
        # the attention's timeout flag comes back with the choice (one copy)
        ws = model.attn_ws_used
        token, flag = torch.cat([greedy_token(logits, offset, size), status_word(ws).to(torch.int64)]).tolist()
        raise_if_gave_up(flag, ws)
    return out
