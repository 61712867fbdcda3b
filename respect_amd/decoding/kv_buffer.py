"""Fixed-capacity KV cache of the decoder (respect/decoding/kv_buffer.py:44-104).

One bf16 tensor [HK, capacity, D] per layer for K and for V, allocated once.
Slots [0, P) hold the prompt; slot P + i holds the i-th token after it
(committed tokens first, then the trie nodes of a verification call).
``compact`` moves the accepted path's KV to consecutive slots after the
committed ones, all layers and heads in one launch (rspx_kv_compact).
"""
from __future__ import annotations

import torch

from .. import _lib


class KVCache:
    def __init__(self, layers: int, kv_heads: int, head_dim: int, capacity: int, device="cuda"):
        self.layers, self.HK, self.D, self.cap = layers, kv_heads, head_dim, capacity
        shape = (kv_heads, capacity, head_dim)
        self.k = [torch.zeros(shape, dtype=torch.bfloat16, device=device) for _ in range(layers)]
        self.v = [torch.zeros(shape, dtype=torch.bfloat16, device=device) for _ in range(layers)]
        ptrs = [t.data_ptr() for pair in zip(self.k, self.v) for t in pair]
        self.bases = torch.tensor(ptrs, dtype=torch.int64, device=device)
        self.device = torch.device(device)

    def compact(self, start: int, slots, stream=None) -> None:
        """Move slots ``start + s`` (s in ``slots``, increasing) to ``start, start + 1, ...``
        in every layer (kv_buffer.py:93-104 compact)."""
        slots = list(slots)
        if not slots or slots == list(range(len(slots))):
            return
        src = torch.tensor([start + s for s in slots], dtype=torch.int32).to(self.device, non_blocking=True)
        k0 = self.k[0]
        rc = _lib.lib().rspx_kv_compact(self.bases.data_ptr(), 2 * self.layers, self.HK, self.D, k0.stride(0),
                                        k0.stride(1), self.cap, start, src.data_ptr(), len(slots),
                                        stream if stream is not None else _lib.stream_ptr(self.device))
        _lib.check("rspx_kv_compact", rc)
