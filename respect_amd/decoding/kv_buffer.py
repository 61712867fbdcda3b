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
        # source slots of a compaction: pinned staging + device copy (at most 128 moves)
        self._src_host = torch.zeros(self.COMPACT_MAX, dtype=torch.int32).pin_memory()
        self._src = torch.zeros(self.COMPACT_MAX, dtype=torch.int32, device=device)
        self._src_copied = torch.cuda.Event()

    COMPACT_MAX = 128   # rows rspx_kv_compact moves per call

    def compact(self, start: int, slots) -> None:
        """Move slots ``start + s`` (s in ``slots``, increasing) to ``start, start + 1, ...``
        in every layer (kv_buffer.py:93-104 compact), on the current stream."""
        slots = list(slots)
        if not slots or slots == list(range(len(slots))):
            return
        n = len(slots)
        if n > self.COMPACT_MAX:
            raise ValueError(f"compact: at most {self.COMPACT_MAX} slots per call")
        self._src_copied.synchronize()   # the previous upload is done with the pinned buffer
        self._src_host.numpy()[:n] = [start + s for s in slots]
        self._src[:n].copy_(self._src_host[:n], non_blocking=True)
        self._src_copied.record()
        k0 = self.k[0]
        rc = _lib.lib().rspx_kv_compact(self.bases.data_ptr(), 2 * self.layers, self.HK, self.D, k0.stride(0),
                                        k0.stride(1), self.cap, start, self._src.data_ptr(), n,
                                        _lib.stream_ptr(self.device))
        _lib.check("rspx_kv_compact", rc)
