"""The attention seam: the decode kernel behind the reference's registered attention function.

Mirrors lazykv/attention.py:139-182 (`lazykv_attention_forward`, registered as "lazykv_sdpa" with
transformers' AttentionInterface, :269-290). For a decode token of a selecting layer, the
selector (`TieredCache.select`) returns the finished attention of the step -- bound, top-K,
sparse attention and, for the exact tier, the LSE merge, all on the device -- which short-circuits
`attend`. Dense decode (`select` returns None) runs the same kernel over the whole cache.

`attend` keeps the reference's signature (:97-136). Its decode case (q_len == 1) is the HIP
kernel. Chunked prefill (q_len > 1) is not on this path: it is handed to torch's
scaled_dot_product_attention with the reference's lower-right causal alignment.
"""

from __future__ import annotations

import math
import time
from dataclasses import dataclass

import torch

from lazykv_amd import kernels

IMPLEMENTATION_NAME = "lazykv_sdpa"
DENSE_BLOCK = 16  # block granularity the dense decode walks the cache in
STRATEGIES = ("hip",)  # the decode kernel; the reference's are cuDNN / SDPA backends (:44)
_STRATEGY = {"name": "hip", "bucket": 0}


def attend(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, scaling: float | None, strategy: str = "hip", bucket: int = 0, mask: torch.Tensor | None = None) -> torch.Tensor:
    """Exact attention of `query` [1, n_q, q_len, d] over all of `key`/`value` [1, kv, L, d].

    Decode (q_len 1) runs the HIP decode kernel over the L tokens (whole blocks from the cache
    plus a partial last block). `mask`, if given, must be the current-block mask of
    lazykv/selection.py:65-69; the kernel needs only its count of live positions.
    """
    del strategy, bucket
    q_len, kv_len, d = query.shape[-2], key.shape[-2], query.shape[-1]
    scale = scaling if scaling is not None else d**-0.5
    if q_len > 1:
        from torch.nn.attention.bias import causal_lower_right

        return torch.nn.functional.scaled_dot_product_attention(query, key, value, attn_mask=causal_lower_right(q_len, kv_len), scale=scale, enable_gqa=True)
    live = kv_len
    if mask is not None:
        live = int((mask.reshape(-1) == 0).sum().item())  # host sync: the seam's fallback only
    out, _ = dense_decode(query, key[:, :, :live], value[:, :, :live], scale)
    return out


def dense_decode(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, scale: float) -> tuple[torch.Tensor, torch.Tensor]:
    """Decode attention over a dense cache view [1, kv, L, d]: out [1, n_q, 1, d], lse [1, n_q]."""
    n_q, d = query.shape[1], query.shape[-1]
    n_kv, length = key.shape[1], key.shape[2]
    full, tail = divmod(length, DENSE_BLOCK)
    src = kernels.dense_source(key, value, DENSE_BLOCK)
    src.n_blocks = full + (1 if tail else 0)
    out, lse = kernels.sparse_decode(
        query.reshape(n_q, d), n_kv=n_kv, block_size=DENSE_BLOCK, scale=scale, rem=src, rem_range=(0, full),
        cur=src if tail else None, cur_block=full if tail else -1, fill=tail, attend_selected=False,
    )
    return out.view(1, n_q, 1, d), lse.view(1, n_q)


def lazykv_attention_forward(
    module: torch.nn.Module,
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    attention_mask: torch.Tensor | None,
    dropout: float = 0.0,
    scaling: float | None = None,
    **kwargs: object,
) -> tuple[torch.Tensor, None]:
    """transformers attention function (lazykv/attention.py:139-182). Returns ([1, q_len, n_q, d], None)."""
    if attention_mask is not None:
        raise RuntimeError("lazykv attention owns causality; a mask should never be passed")
    if query.shape[0] != 1:
        raise RuntimeError("batch size 1 only")
    selector = kwargs.get("lazykv_selector")
    out = None
    if selector is not None:
        decoded = selector.select(int(getattr(module, "layer_idx")), query, key, value, scaling)
        if decoded is not None:
            out = decoded.out
    if out is None:
        out = attend(query, key, value, scaling)
    return out.transpose(1, 2).contiguous(), None


@dataclass
class KernelCheck:
    """One strategy's startup verification (lazykv/attention.py:186-194)."""

    strategy: str
    ok: bool
    max_rel_err_decode: float | None
    max_rel_err_prefill: float | None
    seconds_decode_growing_median: float | None
    seconds_decode_growing_max: float | None
    error: str | None = None


def _reference(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, scaling: float) -> torch.Tensor:
    """Float32 explicit attention with lower-right causal masking: the ground truth (:196-207)."""
    q, k, v = query.float(), key.float(), value.float()
    groups = q.shape[1] // k.shape[1]
    k = k.repeat_interleave(groups, dim=1)
    v = v.repeat_interleave(groups, dim=1)
    scores = (q @ k.transpose(-1, -2).contiguous()) * scaling
    q_len, kv_len = q.shape[-2], k.shape[-2]
    q_pos = torch.arange(kv_len - q_len, kv_len, device=q.device)[:, None]
    k_pos = torch.arange(kv_len, device=q.device)[None, :]
    scores = scores.masked_fill(k_pos > q_pos, float("-inf"))
    return torch.softmax(scores, dim=-1) @ v


def _rel_err(got: torch.Tensor, ref: torch.Tensor) -> float:
    return ((got.float() - ref).abs().max() / ref.abs().max()).item()


def _check_one(strategy: str, n_q: int, n_kv: int, head_dim: int, dtype: torch.dtype, probe_ctx: int, steps: int, tolerance: float) -> KernelCheck:
    """Decode and chunked prefill against the float32 truth, with spare storage past the live
    length as a preallocated cache has, then decode speed as the length grows by one per step
    (lazykv/attention.py:214-245)."""
    gen = torch.Generator(device="cuda").manual_seed(0)
    scaling = head_dim**-0.5

    def rand(*shape: int) -> torch.Tensor:
        return torch.randn(*shape, device="cuda", dtype=dtype, generator=gen)

    try:
        store_k, store_v = rand(1, n_kv, 1024, head_dim), rand(1, n_kv, 1024, head_dim)
        live = 509
        k, v = store_k[:, :, :live], store_v[:, :, :live]
        pq, dq = rand(1, n_q, 64, head_dim), rand(1, n_q, 1, head_dim)
        err_p = _rel_err(attend(pq, k, v, scaling, strategy), _reference(pq, k, v, scaling))
        err_d = _rel_err(attend(dq, k, v, scaling, strategy), _reference(dq, k, v, scaling))
        big_k, big_v = rand(1, n_kv, probe_ctx + steps, head_dim), rand(1, n_kv, probe_ctx + steps, head_dim)
        times = []
        for i in range(steps):
            length = probe_ctx + i
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            attend(dq, big_k[:, :, :length], big_v[:, :, :length], scaling, strategy)
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t0)
    except (RuntimeError, ValueError) as exc:
        return KernelCheck(strategy, False, None, None, None, None, str(exc).splitlines()[0])
    ok = math.isfinite(err_p) and math.isfinite(err_d) and max(err_p, err_d) <= tolerance
    steady = sorted(times[1:])
    return KernelCheck(strategy, ok, err_d, err_p, steady[len(steady) // 2], max(times))


def verify_strategies(n_q_heads: int, n_kv_heads: int, head_dim: int, dtype: torch.dtype = torch.bfloat16, tolerance: float = 1e-2,
                      probe_ctx: int = 16_000, steps: int = 24, candidates: tuple[str, ...] = STRATEGIES) -> list[KernelCheck]:
    """Correctness (decode + chunked prefill vs float32) and growing-length decode speed (:248-266)."""
    out = []
    for name in candidates:
        if name not in STRATEGIES:
            out.append(KernelCheck(name, False, None, None, None, None, f"unknown strategy {name!r}: this build has {STRATEGIES}"))
            continue
        out.append(_check_one(name, n_q_heads, n_kv_heads, head_dim, dtype, probe_ctx, steps, tolerance))
    return out


def install(strategy: str | None = None, n_q_heads: int | None = None, n_kv_heads: int | None = None, head_dim: int | None = None,
            bucket: int = 0) -> tuple[str, list[KernelCheck]]:
    """Register the attention function with transformers under IMPLEMENTATION_NAME and pin the
    strategy (lazykv/attention.py:269-290). Given the model's head counts and head_dim, the
    decode kernel is verified first against the float32 truth; a strategy that fails (or that
    this build does not have) is a hard error, never a silent fallback."""
    from transformers import AttentionInterface

    checks: list[KernelCheck] = []
    chosen = strategy or "hip"
    if n_q_heads is not None and n_kv_heads is not None and head_dim is not None:
        checks = verify_strategies(n_q_heads, n_kv_heads, head_dim, candidates=(chosen,))
        if not checks[0].ok:
            raise RuntimeError(f"attention strategy {chosen!r} failed verification: {checks[0]}")
    elif chosen not in STRATEGIES:
        raise RuntimeError(f"unknown attention strategy {chosen!r}: this build has {STRATEGIES}")
    _STRATEGY["name"], _STRATEGY["bucket"] = chosen, bucket
    AttentionInterface.register(IMPLEMENTATION_NAME, lazykv_attention_forward)
    return chosen, checks


def current_strategy() -> tuple[str, int]:
    return _STRATEGY["name"], _STRATEGY["bucket"]
