"""Layer-major prefill straight into the host tier (lazykv/tiered_prefill.py:70-129).

The prompt runs through one decoder layer at a time, every chunk of it, before the next layer
starts (lazykv/tiered_prefill.py:1-26). Only that layer's KV is on the GPU, in one scratch store
reused by every selecting layer. When the layer finishes, `TieredLayer` turns its KV into the
tier with one kernel per layer: each full block is stored into the mapped host pool (model-dtype
bytes, or the int8 record for `quant="int8"`) and its key min/max is written, over the
dequantised keys for an int8 tier, in the same pass. The prompt's full KV is never resident in
VRAM, and each KV byte crosses PCIe once, device to host.

Bit identity with the chunk-major path: every layer sees the same chunk boundaries, inputs and
KV prefix that a chunk-major prefill into a full cache gives it, so the KV, the records and the
last logits are the same bits (lazykv/tiered_prefill.py:22-26).
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Any

import torch
from transformers.cache_utils import Cache

from lazykv_amd.cache import FullGPUCache, PreallocatedLayer
from lazykv_amd.selection import QUEST_DENSE_LAYERS
from lazykv_amd.tiered import TieredCache, TieredLayer


class _OneLayerCache(Cache):
    """Routes each layer's update: dense layers to `full`, the selecting layer being run to `scratch`
    (lazykv/tiered_prefill.py:44-55)."""

    def __init__(self, full: FullGPUCache, scratch: PreallocatedLayer, dense_layers: int) -> None:
        super().__init__(layers=full.layers)
        self.full, self.scratch, self.dense_layers = full, scratch, dense_layers

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int, *args: object, **kwargs: object) -> tuple[torch.Tensor, torch.Tensor]:
        store = self.full.layers[layer_idx] if layer_idx < self.dense_layers else self.scratch
        return store.update(key_states, value_states)


@dataclass
class TieredPrefillResult:
    """lazykv/tiered_prefill.py:58-67."""

    last_logits: torch.Tensor  # [vocab] float32, on the GPU
    cache: TieredCache
    full: FullGPUCache  # the dense layers' store
    wall_s: float
    chunks: int
    boundary_s: float  # device time of the tier builds (store + metadata kernels), summed over layers
    layer_s: list[float] = field(default_factory=list)  # wall time per decoder layer, boundary included
    boundary_layer_s: list[float] = field(default_factory=list)  # device time of each selecting layer's tier build


@torch.inference_mode()
def tiered_prefill(
    model: Any,
    input_ids: torch.Tensor,
    chunk_size: int,
    k_blocks: int,
    block_size: int,
    capacity_tokens: int,
    dense_layers: int = QUEST_DENSE_LAYERS,
    host_pools: list[torch.Tensor] | None = None,
    n_slots: int | None = None,
    quant: str | None = None,
    **cache_kwargs: Any,
) -> TieredPrefillResult:
    """Prefill `input_ids` layer by layer and return a decode-ready TieredCache
    (lazykv/tiered_prefill.py:70-129). `cache_kwargs` (fetch, exact, rank_dtype) go to the tiers and
    the cache."""
    inner = model.model
    layers = inner.layers
    dev = next(model.parameters()).device
    ids = input_ids.to(dev).view(1, -1)
    n = ids.shape[1]
    if n > capacity_tokens:
        raise ValueError(f"prompt of {n} tokens exceeds capacity {capacity_tokens}")
    if chunk_size <= 0:
        raise ValueError("chunk_size must be positive")
    tier_kw = {key: cache_kwargs[key] for key in ("fetch", "exact", "rank_dtype") if key in cache_kwargs}
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    # Dense layers keep growing during decode, so their stores are sized for the full capacity; the
    # full cache allocates a layer on its first update, so the selecting layers' entries stay empty.
    full = FullGPUCache(len(layers), capacity_tokens)
    scratch = PreallocatedLayer(n)
    router = _OneLayerCache(full, scratch, dense_layers)
    bounds = [(s, min(n, s + chunk_size)) for s in range(0, n, chunk_size)]
    hidden = inner.embed_tokens(ids)
    rope = []
    for s, e in bounds:
        pos = torch.arange(s, e, device=dev).unsqueeze(0)
        rope.append((pos, inner.rotary_emb(hidden[:, s:e], position_ids=pos)))
    tiers: dict[int, TieredLayer] = {}
    layer_s: list[float] = []
    events: list[tuple[torch.cuda.Event, torch.cuda.Event]] = []
    for i, layer in enumerate(layers):
        tl = time.perf_counter()
        scratch.reset()
        for (s, e), (pos, pe) in zip(bounds, rope):
            # In place: chunk c's output is never an input to another chunk of this layer.
            hidden[:, s:e] = layer(hidden[:, s:e], attention_mask=None, position_ids=pos, past_key_values=router, use_cache=True, position_embeddings=pe)
        if i >= dense_layers:
            host = None if host_pools is None else host_pools[i - dense_layers]
            b0, b1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            b0.record()
            tiers[i] = TieredLayer(scratch.keys[:, :, :n], scratch.values[:, :, :n], k_blocks, block_size, capacity_tokens, host, n_slots, quant=quant, **tier_kw)
            b1.record()
            events.append((b0, b1))
        torch.cuda.synchronize(dev)
        layer_s.append(time.perf_counter() - tl)
    del scratch, router
    # As LlamaForCausalLM with logits_to_keep=1: the norm over the last chunk, its last row projected.
    s, e = bounds[-1]
    logits = model.lm_head(inner.norm(hidden[:, s:e])[:, -1:])
    last = logits[0, -1].float()
    del hidden
    cache = TieredCache(full, k_blocks, block_size, capacity_tokens, model=model, dense_layers=dense_layers, n_slots=n_slots, quant=quant, tiers=tiers, **cache_kwargs)
    torch.cuda.synchronize(dev)
    boundary = [a.elapsed_time(b) / 1e3 for a, b in events]
    return TieredPrefillResult(last, cache, full, time.perf_counter() - t0, len(bounds), sum(boundary), layer_s, boundary)
