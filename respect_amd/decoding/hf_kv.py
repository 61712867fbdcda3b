"""Fixed-capacity KV storage for a Hugging Face decoder (transformers 5.x).

Interface kept from respect/decoding/kv_buffer.py:20-104 (the names callers
use): ``WindowLayer(base_k, base_v, window)``, ``WindowCache(layers)``,
``FixedKVBuffer(prompt_len, capacities)`` with ``PL``, ``caps``, ``base_k``,
``base_v``, ``allocate``, ``write_prefill``, ``window``, ``fit``, ``view``, and
``compact(cache, prompt_len, base, slots)``.

Layout: one device allocation, the *arena*, ``[layers, 2 (K, V), batch, kv
heads, prompt_len + max(capacities), head_dim]``, made once from the shapes of
a Prefill cache.  Slot ``prompt_len + i`` of a layer holds the i-th token after
the prompt.  ``base_k[i]`` / ``base_v[i]`` are views of layer i's K and V
planes; a window of capacity c is a cache whose layers see slots
``[0, prompt_len + c)`` of those planes.  Every K and V plane has the same
shape and strides, so ``compact`` moves the accepted path of all layers in
one rspx_kv_compact launch.

transformers 5.x calls ``Cache.update(key, value, layer_idx)`` without a
``cache_position``; the slots the next forward writes are therefore given to
the window first (``WindowCache.set_positions``).  A ``cache_position`` in the
update's cache kwargs (the 4.57 calling convention) takes precedence.
"""
from __future__ import annotations

import bisect
from typing import Any, Sequence

import torch
from transformers import cache_utils
from transformers.cache_utils import DynamicCache, DynamicLayer

from .. import _lib


def _planes_match(k: torch.Tensor, v: torch.Tensor) -> None:
    if k.dim() != 4 or k.shape != v.shape or k.dtype != v.dtype or k.device != v.device:
        raise ValueError(f"K/V planes must be equal 4-D tensors, got {tuple(k.shape)} and {tuple(v.shape)}")


class WindowLayer(cache_utils.StaticLayer):
    """A Hugging Face cache layer over slots [0, window) of one layer's K/V planes.

    Writes go in place to the slots named by the owning ``WindowCache``
    (``set_positions``) or by ``cache_kwargs["cache_position"]``; reads see the
    whole window.  The planes themselves belong to the caller (usually a
    ``FixedKVBuffer``), so any number of windows may share them.
    """

    def __init__(self, base_k: torch.Tensor, base_v: torch.Tensor, window: int,
                 owner: "WindowCache | None" = None) -> None:
        _planes_match(base_k, base_v)
        if not 0 < window <= base_k.shape[2]:
            raise ValueError(f"window {window} outside the planes' {base_k.shape[2]} slots")
        super().__init__(max_cache_len=window)
        self._base_k, self._base_v, self._window = base_k, base_v, int(window)
        self.keys = base_k.narrow(2, 0, window)
        self.values = base_v.narrow(2, 0, window)
        b, hk, _, d = base_k.shape
        # attribute names transformers' StaticLayer reads
        self.batch_size, self.num_heads, self.k_head_dim, self.v_head_dim = b, hk, d, d
        self.dtype, self.device = base_k.dtype, base_k.device
        self.is_initialized = True
        self.owner = owner

    def _target_slots(self, args: tuple, kwargs: dict) -> torch.Tensor:
        ck = kwargs.get("cache_kwargs")
        if ck is None:
            ck = next((a for a in args if isinstance(a, dict)), None)
        slots = None if ck is None else ck.get("cache_position")
        if slots is None and self.owner is not None:
            slots = self.owner.positions
        if slots is None:
            raise RuntimeError("WindowLayer.update: no target slots (call WindowCache.set_positions first)")
        return slots

    def update(self, key_states, value_states, *args, **kwargs):
        slots = self._target_slots(args, kwargs)
        self.keys.index_copy_(2, slots, key_states)
        self.values.index_copy_(2, slots, value_states)
        return self.keys, self.values

    def get_seq_length(self) -> int:
        return self._window

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        return self._window, 0


class WindowCache(cache_utils.Cache):
    """A Hugging Face cache made of ``WindowLayer`` s that share one slot list."""

    def __init__(self, layers: list[WindowLayer]) -> None:
        super().__init__(layers=layers)
        self.positions: torch.Tensor | None = None
        for layer in layers:
            layer.owner = self

    def set_positions(self, positions: torch.Tensor) -> None:
        """Slots (1-D long tensor on the cache's device) that the next forward writes."""
        self.positions = positions


class FixedKVBuffer:
    """All layers' KV in one arena allocated once; windows of fixed capacities over it."""

    def __init__(self, prompt_len: int, capacities: Sequence[int]) -> None:
        caps = sorted({int(c) for c in capacities})
        if prompt_len < 0 or not caps or caps[0] <= 0:
            raise ValueError(f"FixedKVBuffer: prompt_len {prompt_len}, capacities {list(capacities)}")
        self.PL = int(prompt_len)
        self.caps = caps
        self.arena: torch.Tensor | None = None
        self._windows: dict[int, WindowCache] = {}

    @property
    def slots(self) -> int:
        """Slots per layer: the prompt plus the largest capacity."""
        return self.PL + self.caps[-1]

    @property
    def base_k(self) -> list[torch.Tensor]:
        return [] if self.arena is None else list(self.arena[:, 0].unbind(0))

    @property
    def base_v(self) -> list[torch.Tensor]:
        return [] if self.arena is None else list(self.arena[:, 1].unbind(0))

    def allocate(self, template: Any) -> None:
        """Create the arena from a Prefill cache's layer shapes (``.layers[i].keys``);
        a no-op once the arena exists."""
        if self.arena is not None:
            return
        first = template.layers[0].keys
        for layer in template.layers:
            if layer.keys.shape[:2] != first.shape[:2] or layer.keys.shape[3] != first.shape[3]:
                raise ValueError("FixedKVBuffer.allocate: layers with different KV shapes")
        b, hk, _, d = first.shape
        self.arena = torch.zeros((len(template.layers), 2, b, hk, self.slots, d), dtype=first.dtype,
                                 device=first.device)
        self._windows.clear()

    def write_prefill(self, prefill_cache: Any) -> None:
        """Copy the Prefill KV into slots [0, PL) of every layer (once per frame)."""
        if self.arena is None:
            raise RuntimeError("FixedKVBuffer.write_prefill before allocate")
        n = self.PL
        for plane, layer in zip(self.arena, prefill_cache.layers):
            plane[0, :, :, :n].copy_(layer.keys[:, :, :n])
            plane[1, :, :, :n].copy_(layer.values[:, :, :n])

    def window(self, capacity: int) -> WindowCache:
        """The cache that sees slots [0, PL + capacity); built on first use."""
        if capacity not in self.caps:
            raise KeyError(f"capacity {capacity} is not one of {self.caps}")
        if self.arena is None:
            raise RuntimeError("FixedKVBuffer.window before allocate")
        cache = self._windows.get(capacity)
        if cache is None:
            n = self.PL + capacity
            cache = WindowCache([WindowLayer(plane[0], plane[1], n) for plane in self.arena])
            self._windows[capacity] = cache
        return cache

    def fit(self, n: int) -> int:
        """Smallest capacity that holds ``n`` slots after the prompt."""
        i = bisect.bisect_left(self.caps, n)
        if i == len(self.caps):
            raise ValueError(f"no capacity holds {n} slots (largest {self.caps[-1]})")
        return self.caps[i]

    def view(self, length: int) -> DynamicCache:
        """A DynamicCache over slots [0, length) of every layer, sharing the arena."""
        if self.arena is None or not 0 <= length <= self.slots:
            raise ValueError(f"FixedKVBuffer.view({length})")
        cache = DynamicCache()
        cache.layers = []
        for plane in self.arena:
            layer = DynamicLayer()
            layer.keys, layer.values = plane[0].narrow(2, 0, length), plane[1].narrow(2, 0, length)
            layer.dtype, layer.device, layer.is_initialized = plane.dtype, plane.device, True
            cache.layers.append(layer)
        return cache


def compact(cache: Any, prompt_len: int, base: int, slots: list[int]) -> None:
    """Gather the accepted path's KV (node slots ``slots`` after ``prompt_len + base``) into
    consecutive slots from ``prompt_len + base`` in every layer (kv_buffer.py:93-104), with
    one rspx_kv_compact launch for all layers' K and V.  ``slots`` must increase, as a
    root-to-node path of a trie whose parents precede their children does."""
    slots = [int(s) for s in slots]
    if slots == list(range(len(slots))):
        return                      # empty, or already in place
    if any(b <= a for a, b in zip(slots, slots[1:])):
        raise ValueError("compact: slots must increase")
    planes = [t for layer in cache.layers for t in (layer.keys, layer.values)]
    ref = planes[0]
    if ref.dtype != torch.bfloat16 or ref.shape[0] != 1:
        raise TypeError("compact: bf16 caches of batch 1 only")
    if any(t.shape != ref.shape or t.stride() != ref.stride() or t.device != ref.device for t in planes):
        raise ValueError("compact: every layer's K and V must share shape and strides")
    _, hk, cap, d = ref.shape
    start = prompt_len + base
    if start + slots[-1] >= cap:
        raise ValueError(f"compact: slot {start + slots[-1]} outside the cache's {cap} slots")
    dev = ref.device
    ptrs = torch.tensor([t.data_ptr() for t in planes], dtype=torch.int64).to(dev)
    src = torch.tensor([start + s for s in slots], dtype=torch.int32).to(dev)
    rc = _lib.lib().rspx_kv_compact(ptrs.data_ptr(), len(planes), hk, d, ref.stride(1), ref.stride(2), cap, start,
                                    src.data_ptr(), len(slots), _lib.stream_ptr(dev))
    _lib.check("rspx_kv_compact", rc)
