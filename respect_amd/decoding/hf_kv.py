"""Fixed-capacity KV buffer for a Hugging Face decoder (transformers 5.x).

The interface of respect/decoding/kv_buffer.py:20-104 -- ``WindowLayer``,
``WindowCache``, ``FixedKVBuffer`` (allocate / write_prefill / window / fit /
view) and ``compact(cache, prompt_len, base, slots)`` -- on the cache API of the
transformers in this image.  One buffer holds the Prefill KV followed by
``max(capacities)`` free slots, allocated once; a window exposes its first
``prompt_len + capacity`` slots to a forward pass, and new keys are written in
place at given slots.

API drift from the reference's transformers 4.57: the decoder layers of 5.x
call ``Cache.update(key, value, layer_idx)`` without ``cache_position``, so the
slots a forward writes are given to the window beforehand
(``WindowCache.set_positions``); a ``cache_position`` passed in the update's
keyword arguments, as 4.57 does, still wins.  ``compact`` moves the accepted
path's KV of every layer with one rspx_kv_compact launch instead of an
index_select / index_copy_ pair per layer and tensor.
"""
from __future__ import annotations

from typing import Any

import torch
from transformers import cache_utils
from transformers.cache_utils import DynamicCache, DynamicLayer

from .. import _lib


class WindowLayer(cache_utils.StaticLayer):
    """One layer of the shared buffer, exposing only its first ``window`` slots."""

    def __init__(self, base_k: torch.Tensor, base_v: torch.Tensor, window: int, owner: "WindowCache | None" = None):
        super().__init__(max_cache_len=window)
        self._base_k, self._base_v, self._window = base_k, base_v, window
        self.owner = owner
        self.keys = base_k[:, :, :window, :]
        self.values = base_v[:, :, :window, :]
        self.batch_size, self.num_heads, _, self.k_head_dim = base_k.shape
        self.v_head_dim = base_v.shape[-1]
        self.dtype, self.device = base_k.dtype, base_k.device
        self.is_initialized = True

    def update(self, key_states, value_states, *args, **kwargs):
        ck = kwargs.get("cache_kwargs") or (args[0] if args and isinstance(args[0], dict) else None)
        position = ck.get("cache_position") if ck else None
        if position is None:
            position = self.owner.positions if self.owner is not None else None
        if position is None:
            raise RuntimeError("WindowLayer.update: no slots given (WindowCache.set_positions)")
        self.keys.index_copy_(2, position, key_states)
        self.values.index_copy_(2, position, value_states)
        return self.keys, self.values

    def get_seq_length(self) -> int:
        return self._window

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        return self._window, 0


class WindowCache(cache_utils.Cache):
    def __init__(self, layers: list[WindowLayer]) -> None:
        super().__init__(layers=layers)
        self.positions: torch.Tensor | None = None
        for layer in layers:
            layer.owner = self

    def set_positions(self, positions: torch.Tensor) -> None:
        """Slots (1-D long tensor on the cache's device) the next forward writes."""
        self.positions = positions


class FixedKVBuffer:
    def __init__(self, prompt_len: int, capacities: tuple[int, ...]) -> None:
        self.PL = prompt_len
        self.caps = sorted(capacities)
        self.base_k: list[torch.Tensor] = []
        self.base_v: list[torch.Tensor] = []
        self.caches: dict[int, WindowCache] = {}

    def allocate(self, template: Any) -> None:
        """Allocate once, shaped after a Prefill cache (``.layers[i].keys``). Later calls are no-ops."""
        if self.base_k:
            return
        C = self.PL + self.caps[-1]
        for layer in template.layers:
            k = layer.keys
            shape = (k.shape[0], k.shape[1], C, k.shape[3])
            self.base_k.append(torch.zeros(shape, dtype=k.dtype, device=k.device))
            self.base_v.append(torch.zeros(shape, dtype=k.dtype, device=k.device))
        for cap in self.caps:
            self.caches[cap] = WindowCache(
                [WindowLayer(bk, bv, self.PL + cap) for bk, bv in zip(self.base_k, self.base_v)])

    def write_prefill(self, prefill_cache: Any) -> None:
        """Copy the Prefill KV into the head of the buffer (once per frame)."""
        PL = self.PL
        for i, layer in enumerate(prefill_cache.layers):
            self.base_k[i][:, :, :PL, :].copy_(layer.keys[..., :PL, :])
            self.base_v[i][:, :, :PL, :].copy_(layer.values[..., :PL, :])

    def window(self, capacity: int) -> WindowCache:
        return self.caches[capacity]

    def fit(self, n: int) -> int:
        """Smallest capacity that holds ``n`` slots."""
        return next(c for c in self.caps if c >= n)

    def view(self, length: int) -> DynamicCache:
        """A cache that sees the first ``length`` slots without copying."""
        c = DynamicCache()
        c.layers = []
        for bk, bv in zip(self.base_k, self.base_v):
            layer = DynamicLayer()
            layer.keys = bk[:, :, :length, :]
            layer.values = bv[:, :, :length, :]
            layer.dtype, layer.device, layer.is_initialized = bk.dtype, bk.device, True
            c.layers.append(layer)
        return c


def compact(cache: Any, prompt_len: int, base: int, slots: list[int]) -> None:
    """Move the KV of the accepted path to consecutive slots starting at ``prompt_len + base``
    (kv_buffer.py:93-104), every layer's K and V in one launch.  Slots must increase (a
    root-to-node path in a trie whose parents precede their children)."""
    slots = list(slots)
    if not slots or slots == list(range(len(slots))):
        return
    if any(b <= a for a, b in zip(slots, slots[1:])):
        raise ValueError("compact: slots must increase")
    layers = cache.layers
    k0 = layers[0].keys
    if k0.dtype != torch.bfloat16 or k0.shape[0] != 1:
        raise TypeError("compact: bf16 caches of batch 1 only")
    tensors = [t for layer in layers for t in (layer.keys, layer.values)]
    for t in tensors:
        if t.shape != k0.shape or t.stride() != k0.stride() or t.device != k0.device:
            raise ValueError("compact: every layer's K and V must share shape and strides")
    dev = k0.device
    _, HK, cap, D = k0.shape
    start = prompt_len + base
    bases = torch.tensor([t.data_ptr() for t in tensors], dtype=torch.int64).to(dev)
    src = torch.tensor([start + s for s in slots], dtype=torch.int32).to(dev)
    rc = _lib.lib().rspx_kv_compact(bases.data_ptr(), len(tensors), HK, D, k0.stride(1), k0.stride(2), cap, start,
                                    src.data_ptr(), len(slots), _lib.stream_ptr(dev))
    _lib.check("rspx_kv_compact", rc)
