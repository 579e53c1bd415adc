"""Preallocated per-layer KV stores (lazykv/cache.py:20-100): the dense layers' cache and the
one-layer scratch that the layer-major prefill reuses for every selecting layer.

A layer's KV lives in one zeroed [1, kv_heads, max_len, head_dim] pair allocated on its first
update; `update` appends and returns views of the filled prefix only, so attention never scans
unused rows (lazykv/cache.py:1-9,34-54). Batch size 1 only, as in the reference.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from transformers.cache_utils import Cache, CacheLayerMixin


@dataclass
class Decoded:
    """What a selector's `select` returns here (TieredCache, QuestView): the finished attention of
    the step, not a key set. out [1, n_q, 1, d] in the model dtype, lse [1, n_q] float32 (natural log)."""

    out: torch.Tensor
    lse: torch.Tensor


@dataclass
class CacheStats:
    """Where a cache's KV lives (lazykv/cache.py:105-115): bytes resident in VRAM, bytes held only
    in host memory, and the VRAM allocated for KV."""

    seq_len: int
    gpu_resident_kv_bytes: int
    host_kv_bytes: int
    gpu_allocated_kv_bytes: int

    @property
    def gpu_residency_fraction(self) -> float:
        total = self.gpu_resident_kv_bytes + self.host_kv_bytes
        return 1.0 if total == 0 else self.gpu_resident_kv_bytes / total


class PreallocatedLayer(CacheLayerMixin):
    """One layer's KV in a preallocated tensor pair (lazykv/cache.py:20-70)."""

    def __init__(self, max_len: int, **kwargs: object) -> None:
        super().__init__()
        self.max_len = max_len
        self.length = 0

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        b, h, _, d = key_states.shape
        if b != 1:
            raise ValueError("batch size 1 only")
        self.dtype, self.device = key_states.dtype, key_states.device
        # Zeroed once: rows past `length` are never read, but a zeroed pool cannot hold NaN.
        self.keys = torch.zeros((1, h, self.max_len, d), dtype=key_states.dtype, device=key_states.device)
        self.values = torch.zeros((1, value_states.shape[1], self.max_len, value_states.shape[3]), dtype=value_states.dtype, device=value_states.device)
        self.is_initialized = True

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args: object, **kwargs: object) -> tuple[torch.Tensor, torch.Tensor]:
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        end = self.length + key_states.shape[-2]
        if end > self.max_len:
            raise RuntimeError(f"KV cache overflow: {end} > max_len {self.max_len}")
        self.keys[:, :, self.length : end].copy_(key_states)
        self.values[:, :, self.length : end].copy_(value_states)
        self.length = end
        return self.keys[:, :, :end], self.values[:, :, :end]

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        return self.length + query_length, 0

    def get_seq_length(self) -> int:
        return self.length

    def get_max_length(self) -> int:
        return self.max_len

    def reset(self) -> None:
        self.length = 0

    def truncate(self, length: int) -> None:
        if not 0 <= length <= self.length:
            raise ValueError(f"cannot truncate length {self.length} to {length}")
        self.length = length

    def resident_bytes(self) -> int:
        """KV bytes of the filled prefix (lazykv/cache.py:73-77)."""
        if not self.is_initialized:
            return 0
        per_token = self.keys[0, :, 0].numel() * self.keys.element_size() + self.values[0, :, 0].numel() * self.values.element_size()
        return per_token * self.length


class FullGPUCache(Cache):
    """Every layer's KV resident on the GPU, preallocated (lazykv/cache.py:72-80)."""

    def __init__(self, num_layers: int, max_len: int) -> None:
        super().__init__(layers=[PreallocatedLayer(max_len) for _ in range(num_layers)])
        self.max_len = max_len

    def truncate(self, length: int) -> None:
        for layer in self.layers:
            layer.truncate(length)

    def stats(self) -> CacheStats:
        """Everything resident (lazykv/cache.py:91-102)."""
        layers = [layer for layer in self.layers if isinstance(layer, PreallocatedLayer)]
        resident = sum(layer.resident_bytes() for layer in layers)
        allocated = sum(layer.keys.numel() * layer.keys.element_size() + layer.values.numel() * layer.values.element_size()
                        for layer in layers if layer.is_initialized)
        return CacheStats(seq_len=layers[0].get_seq_length() if layers else 0, gpu_resident_kv_bytes=resident, host_kv_bytes=0,
                          gpu_allocated_kv_bytes=allocated)

    @classmethod
    def from_kv(cls, layers: list[tuple[torch.Tensor, torch.Tensor]], max_len: int) -> FullGPUCache:
        """A cache holding copies of per-layer prompt KV [1, h, L, d]."""
        full = cls(len(layers), max_len)
        for store, (k, v) in zip(full.layers, layers):
            store.update(k, v)
        return full
