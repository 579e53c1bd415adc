"""Layer-major prefill that streams each layer's KV into the host tier while the layer still runs.

The reference's layer-major prefill (lazykv/tiered_prefill.py:70-129) runs the whole prompt
through one decoder layer before the next, so only one selecting layer's KV is ever on the GPU;
when a layer ends it hands that KV to the tier in one go. Here the tier build is spread over the
layer instead. A layer's KV grows chunk by chunk in one HBM scratch, and the blocks a chunk
completes are final the moment that chunk's forward has written them: later chunks of the same
layer only read them. So after each chunk the tier seals its newly completed blocks -- one
`store_blocks` launch writing the int8 record or model-dtype copy into the mapped host pool, and
the key min/max metadata -- on a second stream, where those PCIe writes overlap the next chunk's
matrix work. When the layer ends, only the last chunk's blocks, the sink and the current block
remain. The compute stream waits for the tier stream once per layer, before the scratch is
overwritten by the next selecting layer.

What is the same as the reference, and why: every layer sees the same chunk boundaries, inputs and
KV prefix that a chunk-major prefill into a full cache gives it, so the KV, the records, the
metadata and the last logits equal the chunk-major path's bits (lazykv/tiered_prefill.py:22-26);
layers below `dense_layers` keep their KV in the dense store, sized for the whole capacity since
decode appends to them.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Any

import torch
from transformers.cache_utils import Cache

from lazykv_amd.cache import DenseLayer, FullGPUCache
from lazykv_amd.selection import QUEST_DENSE_LAYERS
from lazykv_amd.tiered import TieredCache, TieredLayer

_TIER_KW = ("fetch", "exact", "rank_dtype")  # cache arguments that also shape each layer's tier


@dataclass
class TieredPrefillResult:
    """The prefill's product and its timing (the reference's fields, lazykv/tiered_prefill.py:58-67,
    plus the per-layer tier-build device time)."""

    last_logits: torch.Tensor  # [vocab] float32, on the GPU
    cache: TieredCache
    full: FullGPUCache  # the dense layers' store
    wall_s: float
    chunks: int
    boundary_s: float  # device time of every tier-build launch, summed over layers
    layer_s: list[float] = field(default_factory=list)  # wall time per decoder layer
    boundary_layer_s: list[float] = field(default_factory=list)  # tier-build device time per selecting layer


class _StreamingTierCache(Cache):
    """The `past_key_values` the decoder layers see during the prefill: dense layers append to the
    full cache; the selecting layer in flight appends to the scratch, and every full block a chunk
    completes is sealed into that layer's tier on the tier stream right away."""

    def __init__(self, full: FullGPUCache, dense_layers: int, tier_stream: torch.cuda.Stream) -> None:
        super().__init__(layers=full.layers)
        self.full = full
        self.dense_layers = dense_layers
        self.tier_stream = tier_stream
        self.scratch: DenseLayer | None = None
        self.tier: TieredLayer | None = None
        self.sealed = 0  # blocks of the layer in flight handed to the tier
        self.timings: list[tuple[torch.cuda.Event, torch.cuda.Event]] = []

    def begin_layer(self, scratch: DenseLayer, tier: TieredLayer) -> None:
        # The scratch rows are about to be overwritten: every seal still reading them must be done.
        torch.cuda.current_stream().wait_stream(self.tier_stream)
        scratch.reset()
        self.scratch, self.tier, self.sealed = scratch, tier, 0
        self.timings = []

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int, *args: object, **kwargs: object) -> tuple[torch.Tensor, torch.Tensor]:
        if layer_idx < self.dense_layers:
            return self.full.layers[layer_idx].update(key_states, value_states)
        assert self.scratch is not None and self.tier is not None
        k, v = self.scratch.update(key_states, value_states)
        self._seal_completed(self.scratch.get_seq_length() // self.tier.bs)
        return k, v

    def _seal_completed(self, complete: int) -> None:
        """Seal blocks [sealed, complete) on the tier stream, after the writes that produced them."""
        n = complete - self.sealed
        if n <= 0:
            return
        assert self.scratch is not None and self.tier is not None
        self.tier_stream.wait_stream(torch.cuda.current_stream())
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(self.tier_stream):
            t0.record()
            self.tier.seal_prompt_blocks(self.scratch.keys, self.scratch.values, self.sealed, n)
            t1.record()
        self.timings.append((t0, t1))
        self.sealed = complete

    def end_layer(self) -> None:
        """The layer's last tokens: the sink slot and the current block, on the compute stream."""
        assert self.scratch is not None and self.tier is not None
        n = self.scratch.get_seq_length()
        live_k = self.scratch.keys[:, :, :n]
        live_v = self.scratch.values[:, :, :n]
        torch.cuda.current_stream().wait_stream(self.tier_stream)
        self.tier.close_prompt(live_k, live_v)

    def get_seq_length(self, layer_idx: int = 0) -> int:
        if layer_idx < self.dense_layers:
            return self.full.layers[layer_idx].get_seq_length()
        return self.scratch.get_seq_length() if self.scratch is not None else 0


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
    """Prefill `input_ids` layer by layer into a decode-ready TieredCache (the reference's
    signature, lazykv/tiered_prefill.py:70-82). `cache_kwargs` (fetch, exact, rank_dtype, ...) go
    to the cache, and the ones that shape a tier to each layer's tier as well."""
    backbone = model.model
    device = next(model.parameters()).device
    prompt = input_ids.to(device).reshape(1, -1)
    n = prompt.shape[1]
    if n > capacity_tokens:
        raise ValueError(f"prompt of {n} tokens exceeds capacity {capacity_tokens}")
    if chunk_size <= 0:
        raise ValueError(f"chunk_size must be positive, got {chunk_size}")
    tier_kw = {key: value for key, value in cache_kwargs.items() if key in _TIER_KW}
    tier_kw.setdefault("fetch", "runs")  # the layers are read the way the cache will read them: its default
    torch.cuda.synchronize(device)
    start = time.perf_counter()

    spans = [(a, min(n, a + chunk_size)) for a in range(0, n, chunk_size)]
    embedded = backbone.embed_tokens(prompt)
    # Rotary tables for the whole prompt at once: each angle is inv_freq * position, a single
    # product, so slicing them per chunk gives the chunk-major path's values exactly.
    positions = torch.arange(n, device=device).unsqueeze(0)
    cos, sin = backbone.rotary_emb(embedded, position_ids=positions)
    states = [embedded[:, a:b] for a, b in spans]  # per-chunk hidden states, replaced layer by layer
    chunk_rope = [((positions[:, a:b]), (cos[:, a:b], sin[:, a:b])) for a, b in spans]

    full = FullGPUCache(len(backbone.layers), capacity_tokens)
    scratch = DenseLayer(n)
    tier_stream = torch.cuda.Stream(device)
    router = _StreamingTierCache(full, dense_layers, tier_stream)
    tiers: dict[int, TieredLayer] = {}
    layer_wall: list[float] = []
    build_events: list[list[tuple[torch.cuda.Event, torch.cuda.Event]]] = []
    for i, layer in enumerate(backbone.layers):
        t_layer = time.perf_counter()
        selecting = i >= dense_layers
        if selecting:
            attn = layer.self_attn
            h = attn.config.num_key_value_heads
            host = host_pools[i - dense_layers] if host_pools is not None else None
            tiers[i] = TieredLayer.opened(h, attn.head_dim, n, k_blocks, block_size, capacity_tokens, device, embedded.dtype, host, n_slots, quant=quant, **tier_kw)
            router.begin_layer(scratch, tiers[i])
        for c, (pos, rope) in enumerate(chunk_rope):
            states[c] = layer(states[c], attention_mask=None, position_ids=pos, past_key_values=router, use_cache=True, position_embeddings=rope)
        if selecting:
            router.end_layer()
            build_events.append(router.timings)
        torch.cuda.synchronize(device)
        layer_wall.append(time.perf_counter() - t_layer)
    router.scratch = None
    del scratch

    # The causal LM's head with logits_to_keep=1: the final norm over the last chunk, its last row projected.
    logits = model.lm_head(backbone.norm(states[-1])[:, -1:])
    last = logits[0, -1].float()
    del states, embedded
    cache = TieredCache(full, k_blocks, block_size, capacity_tokens, model=model, dense_layers=dense_layers, n_slots=n_slots, quant=quant, tiers=tiers, **cache_kwargs)
    torch.cuda.synchronize(device)
    per_layer = [sum(a.elapsed_time(b) for a, b in events) / 1e3 for events in build_events]
    return TieredPrefillResult(last, cache, full, time.perf_counter() - start, len(spans), sum(per_layer), layer_wall, per_layer)
