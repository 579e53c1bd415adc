"""Dense KV stores on the GPU: the layers that attend densely, and the prefill's one-layer scratch.

The transformers `Cache` surface of the reference's dense store (`FullGPUCache`, its per-layer
`PreallocatedLayer` and `CacheStats`, lazykv/cache.py:20-115) is kept, because `TieredCache`,
`QuestView` and the snapshot reader take one. The storage is laid out for this library:

* A layer's keys and values share one slab `[2, 1, h, capacity, d]` in HBM (`keys` is slab[0],
  `values` slab[1]): one allocation per layer, made the first time the layer sees KV, so a layer
  that never stores anything here (a tiered layer built by the layer-major prefill) holds no VRAM.
* `update` appends along the token axis and returns views of the filled prefix `[1, h, n, d]`,
  rows `d` elements apart: exactly the dense layout `kernels.dense_source` describes, so the decode
  kernel reads this store in place.
* The slab is zero-filled once. The HIP kernels never read rows past the live length, but a
  consumer that masks unused rows by adding -inf would turn uninitialised NaN into NaN.

Batch size 1, as in the reference.
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


@dataclass(frozen=True)
class CacheStats:
    """Where a cache's KV sits (the reference's `CacheStats`, lazykv/cache.py:105-115): bytes held
    in VRAM, bytes held only in host memory, and the VRAM reserved for KV."""

    seq_len: int
    gpu_resident_kv_bytes: int
    host_kv_bytes: int
    gpu_allocated_kv_bytes: int

    @property
    def gpu_residency_fraction(self) -> float:
        held = self.gpu_resident_kv_bytes + self.host_kv_bytes
        return self.gpu_resident_kv_bytes / held if held else 1.0


class DenseLayer(CacheLayerMixin):
    """One layer's KV in a single preallocated slab (the reference's `PreallocatedLayer`)."""

    def __init__(self, max_len: int, **kwargs: object) -> None:
        super().__init__()
        if max_len <= 0:
            raise ValueError(f"a dense layer needs a positive capacity, got {max_len}")
        self.max_len = max_len
        self.length = 0
        self.slab: torch.Tensor | None = None

    # -- storage ----------------------------------------------------------------------------------

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        if key_states.shape[0] != 1 or key_states.shape != value_states.shape:
            raise ValueError(f"dense layers hold batch-1 KV with matching key/value shapes, got {tuple(key_states.shape)} / {tuple(value_states.shape)}")
        _, h, _, d = key_states.shape
        self.slab = torch.zeros((2, 1, h, self.max_len, d), dtype=key_states.dtype, device=key_states.device)
        self.keys, self.values = self.slab[0], self.slab[1]
        self.dtype, self.device = key_states.dtype, key_states.device
        self.is_initialized = True

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args: object, **kwargs: object) -> tuple[torch.Tensor, torch.Tensor]:
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        a = self.length
        b = a + key_states.shape[-2]
        if b > self.max_len:
            raise RuntimeError(f"dense layer full: appending {b - a} tokens to {a} exceeds its {self.max_len}-token capacity")
        self.keys[:, :, a:b].copy_(key_states)
        self.values[:, :, a:b].copy_(value_states)
        self.length = b
        return self.keys[:, :, :b], self.values[:, :, :b]

    def _set_length(self, n: int) -> None:
        if n < 0 or n > self.length:
            raise ValueError(f"a dense layer of {self.length} tokens cannot be cut to {n}")
        self.length = n

    def reset(self) -> None:
        """Forget every token; the slab is kept (only the live prefix is ever read)."""
        self.length = 0

    def truncate(self, length: int) -> None:
        """Forget the tokens past `length`, so one prefill can be decoded from more than once."""
        self._set_length(length)

    # -- transformers plumbing --------------------------------------------------------------------

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        return self.length + query_length, 0

    def get_seq_length(self) -> int:
        return self.length

    def get_max_length(self) -> int:
        return self.max_len

    # -- accounting -------------------------------------------------------------------------------

    def _token_bytes(self) -> int:
        if self.slab is None:
            return 0
        _, _, h, _, d = self.slab.shape
        return 2 * h * d * self.slab.element_size()

    def resident_bytes(self) -> int:
        """VRAM bytes of the live tokens' keys and values."""
        return self._token_bytes() * self.length

    def allocated_bytes(self) -> int:
        return self._token_bytes() * self.max_len


PreallocatedLayer = DenseLayer  # the reference's name for the per-layer store (lazykv/cache.py:20)


class FullGPUCache(Cache):
    """Every layer's KV held densely in VRAM (the reference's rung 1, lazykv/cache.py:80-102)."""

    def __init__(self, num_layers: int, max_len: int) -> None:
        super().__init__(layers=[DenseLayer(max_len) for _ in range(num_layers)])
        self.max_len = max_len

    def truncate(self, length: int) -> None:
        for layer in self.layers:
            layer.truncate(length)

    def stats(self) -> CacheStats:
        dense = [layer for layer in self.layers if isinstance(layer, DenseLayer)]
        return CacheStats(
            seq_len=dense[0].get_seq_length() if dense else 0,
            gpu_resident_kv_bytes=sum(layer.resident_bytes() for layer in dense),
            host_kv_bytes=0,
            gpu_allocated_kv_bytes=sum(layer.allocated_bytes() for layer in dense),
        )

    @classmethod
    def from_kv(cls, layers: list[tuple[torch.Tensor, torch.Tensor]], max_len: int) -> FullGPUCache:
        """A cache holding copies of per-layer prompt KV [1, h, L, d]."""
        cache = cls(len(layers), max_len)
        for dense, (k, v) in zip(cache.layers, layers):
            dense.update(k, v)
        return cache
