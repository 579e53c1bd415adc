"""Session snapshots of a tiered cache, in the reference's file format (lazykv/snapshot.py:16-20).

A sealed block never changes once it is in the host pool, so a snapshot is the pool as it is, plus
what is still only on the GPU (the dense layers' KV, each tiered layer's unsealed tail) and the
logits for the next token.

File layout (lazykv/snapshot.py:16-20,67-114): an 8-byte little-endian header length, a JSON
header, zero padding to ALIGN, then sections each starting at a multiple of ALIGN -- the
next-token logits (float32), then per layer either `L{i}.kv` [2, h, L, d] (a dense layer) or
`L{i}.blocks`, the host pool's own [B, h, 2, bs, d] bytes, and `L{i}.tail` [h, 2, fill, d] (a
tiered layer). Offsets in the header are relative to the first section. The same magic string and
layout as the reference, so either side reads the other's files.

Restore ("store", lazykv/snapshot.py:219-231): each tiered layer's sealed blocks are read straight
into its mapped host pool; the GPU then reads the pool in place to rebuild the block metadata
(`TieredLayer.from_store`), so no KV byte crosses the link twice. ("boundary" instead copies the
layer to the GPU and builds the tier as the prefill boundary does, lazykv/snapshot.py:232-239.)
"""

from __future__ import annotations

import json
import os
import time
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, BinaryIO

import torch

from lazykv_amd.cache import FullGPUCache
from lazykv_amd.pinned import pinned_empty
from lazykv_amd.tiered import TieredCache, TieredLayer

MAGIC = "lazykv-snapshot-1"
ALIGN = 4096
_DTYPES = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def _pad(n: int) -> int:
    return -(-n // ALIGN) * ALIGN


def _bytes(t: torch.Tensor) -> memoryview:
    """A CPU tensor's bytes (bfloat16 has no numpy dtype, so through a uint8 view)."""
    t = t.contiguous()
    return memoryview(t.view(torch.uint8).reshape(-1).numpy())


@dataclass
class SaveStats:
    bytes_written: int
    seconds: float  # fsync included


@dataclass
class RestoreStats:
    bytes_read: int
    read_s: float
    rebuild_s: float  # everything but the reads: H2D, metadata, slots, dense layers, the final sync
    sections: dict[str, float] = field(default_factory=dict)


def save(cache: TieredCache, next_logits: torch.Tensor, path: Path) -> SaveStats:
    """Write `cache` at its current position and the logits for its next token (lazykv/snapshot.py:67-114)."""
    if cache.quant is not None:
        raise ValueError("snapshots of the int8 tier are not supported")
    t0 = time.perf_counter()
    torch.cuda.synchronize()
    tiers = cache.tiers
    any_tier = next(iter(tiers.values()))
    length = any_tier.length
    sections: list[tuple[str, torch.Tensor]] = [("logits", next_logits.float().cpu())]
    layers: list[dict[str, Any]] = []
    for i in range(len(cache.full.layers)):
        if i in tiers:
            t = tiers[i]
            if t.length != length:
                raise RuntimeError("tiered layers disagree on length")
            blocks = t.host[: t.n_sealed] if t.host is not None else t.store[: t.n_sealed].cpu()
            sections.append((f"L{i}.blocks", blocks))
            sections.append((f"L{i}.tail", t.pool[t.tail_slot, :, :, : t.fill].cpu()))  # [h, 2, fill, d]
            layers.append({"kind": "tier", "n_sealed": t.n_sealed, "fill": t.fill})
        else:
            src = cache.full.layers[i]
            if src.get_seq_length() != length:
                raise RuntimeError(f"dense layer {i} has length {src.get_seq_length()}, the tier {length}")
            sections.append((f"L{i}.kv", torch.stack([src.keys[0, :, :length], src.values[0, :, :length]]).cpu()))  # [2, h, L, d]
            layers.append({"kind": "dense"})
    offsets, cursor = {}, 0
    for name, t in sections:
        offsets[name] = [cursor, t.numel() * t.element_size()]
        cursor += _pad(offsets[name][1])
    header = {
        "magic": MAGIC, "length": length, "block_size": cache.block_size, "dense_layers": cache.dense_layers,
        "heads": any_tier.h, "head_dim": any_tier.d, "dtype": str(any_tier.pool.dtype).removeprefix("torch."),
        "vocab": int(next_logits.numel()), "layers": layers, "sections": offsets,
    }
    head = json.dumps(header).encode()
    base = _pad(len(head) + 8)
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    with path.open("wb") as f:
        f.write(len(head).to_bytes(8, "little") + head)
        f.write(b"\0" * (base - len(head) - 8))
        for _, t in sections:
            n = f.write(_bytes(t))
            f.write(b"\0" * (_pad(n) - n))
        f.flush()
        os.fsync(f.fileno())
    return SaveStats(base + cursor, time.perf_counter() - t0)


def read_header(path: Path) -> tuple[dict[str, Any], int]:
    """(header, byte offset of the first section); ValueError for a file that is not a snapshot."""
    with Path(path).open("rb") as f:
        raw = f.read(8)
        n = int.from_bytes(raw, "little") if len(raw) == 8 else -1
        try:
            header = json.loads(f.read(n)) if 0 < n < (1 << 30) else None
        except ValueError:
            header = None
    if not isinstance(header, dict) or header.get("magic") != MAGIC:
        raise ValueError(f"{path} is not a LazyKV snapshot")
    return header, _pad(n + 8)


def _read_into(f: BinaryIO, offset: int, out: torch.Tensor) -> None:
    f.seek(offset)
    view = _bytes(out)  # `out` is contiguous: this aliases its memory
    got = f.readinto(view)
    if got != len(view):
        raise EOFError(f"short read: {got} of {len(view)} bytes at offset {offset}")


def restore(
    path: Path,
    k_blocks: int,
    capacity_tokens: int,
    num_layers: int,
    model: Any = None,
    host_pools: list[torch.Tensor] | None = None,
    n_slots: int | None = None,
    fetch: str = "zerocopy",
    rebuild: str = "store",
    **tier_kwargs: Any,
) -> tuple[TieredCache, torch.Tensor, RestoreStats]:
    """A TieredCache at the snapshot's position and the logits for its next token
    (lazykv/snapshot.py:184-278). `tier_kwargs` (exact, rank_dtype) go to the tiers and the cache."""
    if rebuild not in ("store", "boundary"):
        raise ValueError(f"unknown rebuild {rebuild!r}")
    header, base = read_header(path)
    dt = _DTYPES[header["dtype"]]
    h, d, bs, length = header["heads"], header["head_dim"], header["block_size"], header["length"]
    if len(header["layers"]) != num_layers:
        raise ValueError(f"snapshot has {len(header['layers'])} layers, the model {num_layers}")
    if length > capacity_tokens:
        raise ValueError(f"snapshot of {length} tokens exceeds capacity {capacity_tokens}")
    sec = header["sections"]
    stats = RestoreStats(0, 0.0, 0.0)
    full = FullGPUCache(num_layers, capacity_tokens)
    tiers: dict[int, TieredLayer] = {}
    dense = 0
    dev = torch.device("cuda", torch.cuda.current_device())
    layer_kw = {key: tier_kwargs[key] for key in ("exact", "rank_dtype") if key in tier_kwargs}
    with Path(path).open("rb", buffering=0) as f:

        def load(name: str, shape: tuple[int, ...], dtype: torch.dtype, into: torch.Tensor | None = None) -> torch.Tensor:
            out = torch.empty(shape, dtype=dtype) if into is None else into
            if out.numel() * out.element_size() != sec[name][1]:
                raise ValueError(f"section {name} holds {sec[name][1]} bytes, expected {out.numel() * out.element_size()}")
            t0 = time.perf_counter()
            _read_into(f, base + sec[name][0], out)
            stats.read_s += time.perf_counter() - t0
            stats.bytes_read += sec[name][1]
            return out

        logits = load("logits", (header["vocab"],), torch.float32).to(dev)
        for i, spec in enumerate(header["layers"]):
            if spec["kind"] == "dense":
                kv = load(f"L{i}.kv", (2, h, length, d), dt)
                t0 = time.perf_counter()
                g = kv.to(dev)
                full.layers[i].update(g[0:1], g[1:2])
                stats.rebuild_s += time.perf_counter() - t0
                dense += 1
                continue
            n, fill = spec["n_sealed"], spec["fill"]
            host = None if host_pools is None else host_pools[i - header["dense_layers"]]
            if rebuild == "store":
                t0 = time.perf_counter()
                if host is None:
                    host = pinned_empty((-(-capacity_tokens // bs), h, 2, bs, d), dt)
                stats.rebuild_s += time.perf_counter() - t0
                load(f"L{i}.blocks", (n, h, 2, bs, d), dt, into=host[:n])
                tail = load(f"L{i}.tail", (h, 2, fill, d), dt)
                t0 = time.perf_counter()
                tiers[i] = TieredLayer.from_store(host, n, tail, k_blocks, bs, capacity_tokens, dev, n_slots, fetch=fetch, **layer_kw)
                stats.rebuild_s += time.perf_counter() - t0
                continue
            blocks = load(f"L{i}.blocks", (n, h, 2, bs, d), dt)
            tail = load(f"L{i}.tail", (h, 2, fill, d), dt)
            t0 = time.perf_counter()
            g = blocks.to(dev).permute(1, 2, 0, 3, 4).reshape(h, 2, n * bs, d)  # [h, 2, B*bs, d]
            kv = torch.cat([g, tail.to(dev)], dim=2)
            tiers[i] = TieredLayer(kv[None, :, 0], kv[None, :, 1], k_blocks, bs, capacity_tokens, host, n_slots, fetch=fetch, **layer_kw)
            del g, kv
            stats.rebuild_s += time.perf_counter() - t0
    if dense != header["dense_layers"]:
        raise ValueError("snapshot's dense layer count disagrees with its header")
    t0 = time.perf_counter()
    cache = TieredCache(full, k_blocks, bs, capacity_tokens, model=model, dense_layers=dense, n_slots=n_slots, fetch=fetch, tiers=tiers, **tier_kwargs)
    torch.cuda.synchronize()
    stats.rebuild_s += time.perf_counter() - t0
    return cache, logits, stats
