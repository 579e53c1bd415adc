"""Session snapshots of a tiered cache in the reference's on-disk format (lazykv/snapshot.py:16-20).

A sealed block never changes once it is in the host pool, so a snapshot is the pool's bytes as they
are, plus what lives only on the GPU -- the dense layers' KV and each tiered layer's unsealed tail
-- and the logits for the next token.

Format (kept byte-compatible with the reference, so either side reads the other's files): an
8-byte little-endian header length, the JSON header (magic "lazykv-snapshot-1", length,
block_size, dense_layers, heads, head_dim, dtype, vocab, per-layer kinds, and `sections`: name ->
[offset, bytes] relative to the first section), zero padding to ALIGN = 4096, then the sections,
each starting on a multiple of ALIGN: `logits` (float32), then per layer `L{i}.kv` [2, h, L, d]
for a dense layer, or `L{i}.blocks` (the host pool's own [B, h, 2, bs, d] bytes) and `L{i}.tail`
[h, 2, fill, d] for a tiered one.

I/O here is positioned: the file is sized once (the gaps read back as zeros, the padding the
format asks for), each section is written with `os.pwrite` straight from its memory -- the mapped
pinned host pool needs no staging copy -- and restore reads each section with `os.preadv` straight
into its destination, the blocks into the layer's mapped host pool. With `rebuild="store"` the GPU
then rebuilds that layer's metadata by reading the pool in place (`TieredLayer.from_store`) while
the host reads the next layer; `rebuild="boundary"` instead hands the layer's dense KV to the tier
constructor, as a prefill's boundary would (lazykv/snapshot.py:219-239).
"""

from __future__ import annotations

import json
import os
import time
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any

import torch

from lazykv_amd.cache import FullGPUCache
from lazykv_amd.pinned import pinned_empty
from lazykv_amd.tiered import TieredCache, TieredLayer

MAGIC = "lazykv-snapshot-1"
ALIGN = 4096
_HEADER_MAX = 1 << 30  # a header length beyond this is not a snapshot
_DTYPE_NAMES = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32"}
_NAMED_DTYPES = {name: dt for dt, name in _DTYPE_NAMES.items()}


def _pad(n: int) -> int:
    """`n` rounded up to the section alignment."""
    return (n + ALIGN - 1) // ALIGN * ALIGN


def _raw(t: torch.Tensor) -> memoryview:
    """The bytes of a contiguous CPU tensor, aliased (bfloat16 has no numpy type: via uint8)."""
    if not t.is_contiguous():
        raise ValueError("snapshot sections are contiguous tensors")
    return memoryview(t.view(torch.uint8).reshape(-1).numpy())


@dataclass
class SaveStats:
    bytes_written: int
    seconds: float  # until the file is on disk (fsync included)


@dataclass
class RestoreStats:
    bytes_read: int
    read_s: float
    rebuild_s: float  # everything but the reads: the GPU rebuild, dense layers, the final sync
    sections: dict[str, float] = field(default_factory=dict)


class _Sections:
    """Section names, sizes and aligned offsets, in file order."""

    def __init__(self) -> None:
        self.order: list[tuple[str, torch.Tensor]] = []
        self.table: dict[str, list[int]] = {}
        self.end = 0

    def add(self, name: str, t: torch.Tensor) -> None:
        n = t.numel() * t.element_size()
        self.table[name] = [self.end, n]
        self.order.append((name, t))
        self.end += _pad(n)


def save(cache: TieredCache, next_logits: torch.Tensor, path: Path) -> SaveStats:
    """Write `cache` at its current position and the logits for its next token
    (lazykv/snapshot.py:67-114). The int8 tier is refused, as in the reference."""
    if cache.quant is not None:
        raise ValueError("snapshots hold model-dtype pairs; the int8 tier is not supported")
    t0 = time.perf_counter()
    torch.cuda.synchronize()
    tiers = cache.tiers
    probe = next(iter(tiers.values()))
    length = probe.length
    sec = _Sections()
    sec.add("logits", next_logits.detach().float().cpu().contiguous())
    kinds: list[dict[str, Any]] = []
    for i, layer in enumerate(cache.full.layers):
        t = tiers.get(i)
        if t is None:
            if layer.get_seq_length() != length:
                raise RuntimeError(f"dense layer {i} holds {layer.get_seq_length()} tokens, the tiers {length}")
            kv = torch.stack([layer.keys[0, :, :length], layer.values[0, :, :length]]).cpu()  # [2, h, L, d]
            sec.add(f"L{i}.kv", kv)
            kinds.append({"kind": "dense"})
            continue
        if t.length != length:
            raise RuntimeError(f"tiered layer {i} holds {t.length} tokens, layer {next(iter(tiers))} {length}")
        # The pool is mapped host memory: written from where it lies. An HBM store is copied down.
        blocks = t.host[: t.n_sealed] if t.host is not None else t.store[: t.n_sealed].cpu()
        sec.add(f"L{i}.blocks", blocks)
        sec.add(f"L{i}.tail", t.pool[1, :, :, : t.fill].cpu().contiguous())
        kinds.append({"kind": "tier", "n_sealed": t.n_sealed, "fill": t.fill})
    header = {
        "magic": MAGIC, "length": length, "block_size": cache.block_size, "dense_layers": cache.dense_layers,
        "heads": probe.h, "head_dim": probe.d, "dtype": _DTYPE_NAMES[probe.dtype],
        "vocab": int(next_logits.numel()), "layers": kinds, "sections": sec.table,
    }
    text = json.dumps(header).encode()
    base = _pad(8 + len(text))
    total = base + sec.end
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    fd = os.open(path, os.O_WRONLY | os.O_CREAT | os.O_TRUNC, 0o644)
    try:
        os.ftruncate(fd, total)  # every byte not written below reads back as zero
        _pwrite_all(fd, memoryview(len(text).to_bytes(8, "little") + text), 0)
        for name, t in sec.order:
            _pwrite_all(fd, _raw(t), base + sec.table[name][0])
        os.fsync(fd)
    finally:
        os.close(fd)
    return SaveStats(total, time.perf_counter() - t0)


def _pwrite_all(fd: int, data: memoryview, offset: int) -> None:
    done = 0
    while done < len(data):
        done += os.pwrite(fd, data[done:], offset + done)


def _pread_into(fd: int, dst: memoryview, offset: int) -> None:
    done = 0
    while done < len(dst):
        got = os.preadv(fd, [dst[done:]], offset + done)
        if got <= 0:
            raise EOFError(f"snapshot ends early: {done} of {len(dst)} bytes at offset {offset}")
        done += got


def read_header(path: Path) -> tuple[dict[str, Any], int]:
    """(header, byte offset of the first section); ValueError for a file that is not a snapshot."""
    with Path(path).open("rb") as f:
        prefix = f.read(8)
        size = int.from_bytes(prefix, "little") if len(prefix) == 8 else 0
        header: Any = None
        if 0 < size < _HEADER_MAX:
            try:
                header = json.loads(f.read(size))
            except (ValueError, UnicodeDecodeError):
                header = None
    if not isinstance(header, dict) or header.get("magic") != MAGIC:
        raise ValueError(f"{path} is not a LazyKV snapshot")
    return header, _pad(8 + size)


def restore(
    path: Path,
    k_blocks: int,
    capacity_tokens: int,
    num_layers: int,
    model: Any = None,
    host_pools: list[torch.Tensor] | None = None,
    n_slots: int | None = None,
    fetch: str = "gather",
    stages: Any = None,
    unbuffered: bool = False,
    rebuild: str = "store",
    **tier_kwargs: Any,
) -> tuple[TieredCache, torch.Tensor, RestoreStats]:
    """A TieredCache at the snapshot's position and the logits for its next token
    (lazykv/snapshot.py:184-278), with the reference's arguments and defaults. `fetch`, `n_slots`
    and `stages` mean what they mean to TieredCache. `unbuffered=True` reads from the disk rather
    than the page cache, what a session resumed long after its save pays: the reference opens the
    file unbuffered (Windows only); here the file's cached pages are written back and dropped
    (fdatasync, then POSIX_FADV_DONTNEED) before the reads. `tier_kwargs` (exact, rank_dtype) go to
    the tiers and the cache."""
    if rebuild not in ("store", "boundary"):
        raise ValueError(f"rebuild must be 'store' or 'boundary', got {rebuild!r}")
    if unbuffered and not hasattr(os, "posix_fadvise"):
        raise NotImplementedError("the unbuffered read needs posix_fadvise")
    header, base = read_header(path)
    dtype = _NAMED_DTYPES[header["dtype"]]
    h, d, bs, length = header["heads"], header["head_dim"], header["block_size"], header["length"]
    specs = header["layers"]
    if len(specs) != num_layers:
        raise ValueError(f"the snapshot has {len(specs)} layers, the model {num_layers}")
    if length > capacity_tokens:
        raise ValueError(f"the snapshot's {length} tokens exceed capacity {capacity_tokens}")
    if sum(s["kind"] == "dense" for s in specs) != header["dense_layers"]:
        raise ValueError("the snapshot's dense layer count disagrees with its header")
    table = header["sections"]
    stats = RestoreStats(0, 0.0, 0.0)
    device = torch.device("cuda", torch.cuda.current_device())
    layer_kw = {key: tier_kwargs[key] for key in ("exact", "rank_dtype") if key in tier_kwargs}
    cap_blocks = -(-capacity_tokens // bs)
    full = FullGPUCache(num_layers, capacity_tokens)
    tiers: dict[int, TieredLayer] = {}
    fd = os.open(path, os.O_RDONLY)
    if unbuffered:
        os.fdatasync(fd)  # dirty pages cannot be dropped
        os.posix_fadvise(fd, 0, 0, os.POSIX_FADV_DONTNEED)

    def section(name: str, out: torch.Tensor) -> torch.Tensor:
        """Read section `name` into the contiguous CPU tensor `out` (pinned pools included)."""
        want = out.numel() * out.element_size()
        if table[name][1] != want:
            raise ValueError(f"section {name} holds {table[name][1]} bytes where {want} are expected")
        r0 = time.perf_counter()
        _pread_into(fd, _raw(out), base + table[name][0])
        dt = time.perf_counter() - r0
        stats.read_s += dt
        stats.sections[name] = dt
        stats.bytes_read += want
        return out

    try:
        logits = section("logits", torch.empty(header["vocab"], dtype=torch.float32)).to(device)
        tiered_seen = 0
        for i, spec in enumerate(specs):
            if spec["kind"] == "dense":
                kv = section(f"L{i}.kv", torch.empty((2, h, length, d), dtype=dtype))
                g0 = time.perf_counter()
                on_gpu = kv.to(device)
                full.layers[i].update(on_gpu[0:1], on_gpu[1:2])
                stats.rebuild_s += time.perf_counter() - g0
                continue
            n, fill = spec["n_sealed"], spec["fill"]
            pool = host_pools[tiered_seen] if host_pools is not None else None
            tiered_seen += 1
            if rebuild == "store":
                if pool is None:
                    pool = pinned_empty((cap_blocks, h, 2, bs, d), dtype)
                section(f"L{i}.blocks", pool[:n])
                tail = section(f"L{i}.tail", torch.empty((h, 2, fill, d), dtype=dtype)).to(device)
                g0 = time.perf_counter()
                tiers[i] = TieredLayer.from_store(pool, n, tail, k_blocks, bs, capacity_tokens, device, n_slots, fetch=fetch, **layer_kw)
                stats.rebuild_s += time.perf_counter() - g0
            else:
                blocks = section(f"L{i}.blocks", torch.empty((n, h, 2, bs, d), dtype=dtype))
                tail = section(f"L{i}.tail", torch.empty((h, 2, fill, d), dtype=dtype))
                g0 = time.perf_counter()
                # [n, h, 2, bs, d] -> per head and side, the tokens in order: [2, h, n*bs + fill, d]
                seq = blocks.to(device).permute(2, 1, 0, 3, 4).reshape(2, h, n * bs, d)
                kv = torch.cat([seq, tail.to(device).permute(1, 0, 2, 3)], dim=2)
                tiers[i] = TieredLayer(kv[0:1], kv[1:2], k_blocks, bs, capacity_tokens, pool, n_slots, fetch=fetch, **layer_kw)
                stats.rebuild_s += time.perf_counter() - g0
    finally:
        os.close(fd)
    g0 = time.perf_counter()
    cache = TieredCache(full, k_blocks, bs, capacity_tokens, model=model, dense_layers=header["dense_layers"], n_slots=n_slots, fetch=fetch, stages=stages,
                        tiers=tiers, **tier_kwargs)
    torch.cuda.synchronize()
    stats.rebuild_s += time.perf_counter() - g0
    return cache, logits, stats
