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
from collections.abc import Callable
from dataclasses import dataclass, replace

import torch

from lazykv_amd import kernels

IMPLEMENTATION_NAME = "lazykv_sdpa"
DEFAULT_BUCKET = 1024  # the reference's bucket default (:42); the decode kernel has no use for one
DENSE_BLOCK = 16  # block granularity the dense decode walks the cache in
# The reference's names pick a cuDNN or SDPA backend (lazykv/attention.py:44,104-113). This library
# has one decode implementation, the HIP kernel, so every one of those names selects it: a caller
# that installs "cudnn_bucketed" (as the reference's fixtures and generate.py do) registers the HIP
# path and has it verified. "hip" names it directly.
REFERENCE_STRATEGIES = ("cudnn_bucketed", "cudnn", "efficient", "math")
STRATEGIES = ("hip",) + REFERENCE_STRATEGIES
_STRATEGY = {"name": "hip", "bucket": DEFAULT_BUCKET}


def _known(strategy: str) -> None:
    if strategy not in STRATEGIES:
        raise ValueError(f"unknown attention strategy {strategy!r}; this library has {STRATEGIES}")


def attend(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, scaling: float | None, strategy: str = "hip", bucket: int = DEFAULT_BUCKET, mask: torch.Tensor | None = None) -> torch.Tensor:
    """Exact attention of `query` [1, n_q, q_len, d] over all of `key`/`value` [1, kv, L, d].

    Decode (q_len 1) runs the HIP decode kernel over the L tokens (whole blocks from the cache
    plus a partial last block). `mask`, if given, must be the current-block mask of
    lazykv/selection.py:65-69; the kernel needs only its count of live positions. Every name in
    STRATEGIES selects this path; another name is a ValueError, as in the reference (:113). `bucket`
    is accepted for the reference's signature: the kernel reads exactly the live prefix, so there is
    no plan to keep stable across lengths and nothing to pad.
    """
    _known(strategy)
    del bucket
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
    """The start-up verification of one strategy (the reference's record, lazykv/attention.py:186-194)."""

    strategy: str
    ok: bool
    max_rel_err_decode: float | None
    max_rel_err_prefill: float | None
    seconds_decode_growing_median: float | None
    seconds_decode_growing_max: float | None
    error: str | None = None


def _truth(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, scaling: float) -> torch.Tensor:
    """Causal GQA attention in float64 on the host: query [1, n_q, q_len, d] at the last q_len
    positions of key/value [1, kv, L, d]. Returns float64 [1, n_q, q_len, d] on the host."""
    q = query.detach().double().cpu()[0]
    k = key.detach().double().cpu()[0]
    v = value.detach().double().cpu()[0]
    n_q, q_len, _ = q.shape
    n_kv, length, _ = k.shape
    group = n_q // n_kv
    out = torch.empty_like(q)
    for head in range(n_q):
        kh, vh = k[head // group], v[head // group]
        logits = (q[head] @ kh.T) * scaling  # [q_len, L]
        # Query row r sits at position L - q_len + r and sees keys 0 .. that position.
        visible = torch.arange(length)[None, :] <= (length - q_len + torch.arange(q_len))[:, None]
        logits = logits.masked_fill(~visible, float("-inf"))
        out[head] = torch.softmax(logits, dim=-1) @ vh
    return out.unsqueeze(0)


def _worst_rel(got: torch.Tensor, want: torch.Tensor) -> float:
    """Largest absolute deviation relative to the largest output magnitude."""
    g = got.detach().double().cpu()
    return float((g - want).abs().max() / want.abs().max().clamp_min(1e-30))


def _verify_hip(n_q: int, n_kv: int, head_dim: int, dtype: torch.dtype, probe_ctx: int, steps: int, tolerance: float) -> KernelCheck:
    """The HIP decode and the chunked-prefill path against the float64 truth, over a preallocated
    store whose rows past the live length hold large values (they must not be read), at live lengths
    that end inside a block and on a block boundary; then the decode's device time, by events, as the
    length grows one token per call from `probe_ctx`."""
    rng = torch.Generator(device="cuda").manual_seed(1234)
    scaling = head_dim**-0.5
    spare = 48
    try:
        worst_d, worst_p = 0.0, 0.0
        for live in (DENSE_BLOCK - 1, 8 * DENSE_BLOCK, 8 * DENSE_BLOCK + 5, 600):
            store = torch.randn((2, 1, n_kv, live + spare, head_dim), device="cuda", dtype=dtype, generator=rng)
            store[:, :, :, live:] = 1e4
            k, v = store[0, :, :, :live], store[1, :, :, :live]
            for q_len in (1, 33):
                if q_len > live:
                    continue
                q = torch.randn((1, n_q, q_len, head_dim), device="cuda", dtype=dtype, generator=rng)
                err = _worst_rel(attend(q, k, v, scaling), _truth(q, k, v, scaling))
                if q_len == 1:
                    worst_d = max(worst_d, err)
                else:
                    worst_p = max(worst_p, err)
        growing = torch.randn((2, 1, n_kv, probe_ctx + steps, head_dim), device="cuda", dtype=dtype, generator=rng)
        q = torch.randn((1, n_q, 1, head_dim), device="cuda", dtype=dtype, generator=rng)
        marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        for i, (e0, e1) in enumerate(marks):
            e0.record()
            attend(q, growing[0, :, :, : probe_ctx + i], growing[1, :, :, : probe_ctx + i], scaling)
            e1.record()
        torch.cuda.synchronize()
        took = sorted(e0.elapsed_time(e1) / 1e3 for e0, e1 in marks)
    except (RuntimeError, ValueError) as exc:
        return KernelCheck("hip", False, None, None, None, None, str(exc).splitlines()[0])
    ok = math.isfinite(worst_d) and math.isfinite(worst_p) and max(worst_d, worst_p) <= tolerance
    return KernelCheck("hip", ok, worst_d, worst_p, took[len(took) // 2], took[-1])


def verify_strategies(n_q_heads: int, n_kv_heads: int, head_dim: int, dtype: torch.dtype = torch.bfloat16, tolerance: float = 1e-2,
                      probe_ctx: int = 16_000, steps: int = 24, candidates: tuple[str, ...] = STRATEGIES) -> list[KernelCheck]:
    """Correctness of decode and chunked prefill, and growing-length decode speed, for each
    candidate strategy (the reference's entry point, lazykv/attention.py:248-266). The names in
    STRATEGIES all select the HIP kernel, which is checked once and reported under each of them; a
    name this library does not have fails its check instead of raising."""
    checks = []
    measured: KernelCheck | None = None
    for name in candidates:
        if name not in STRATEGIES:
            checks.append(KernelCheck(name, False, None, None, None, None, f"unknown strategy {name!r}: this library has {STRATEGIES}"))
            continue
        if measured is None:
            measured = _verify_hip(n_q_heads, n_kv_heads, head_dim, dtype, probe_ctx, steps, tolerance)
        checks.append(replace(measured, strategy=name))
    return checks


def install(strategy: str | None = None, n_q_heads: int | None = None, n_kv_heads: int | None = None, head_dim: int | None = None,
            bucket: int = DEFAULT_BUCKET) -> tuple[str, list[KernelCheck]]:
    """Register the attention function with transformers under IMPLEMENTATION_NAME and pin the
    strategy (lazykv/attention.py:269-290). Given the model's head counts and head_dim, the decode
    kernel and the chunked-prefill path are verified first against a float64 truth. A named strategy
    that fails (or that this library does not have) is a hard error, never a silent fallback.
    `strategy=None` picks the fastest strategy that verifies; every name is the same HIP kernel, so
    that is "hip"."""
    from transformers import AttentionInterface

    checks: list[KernelCheck] = []
    if strategy is not None and strategy not in STRATEGIES:
        # The reference's refusal of a name it did not verify: a RuntimeError (:282-284).
        raise RuntimeError(f"requested attention strategy {strategy!r} is unknown: this library has {STRATEGIES}")
    chosen = strategy or "hip"
    if n_q_heads is not None and n_kv_heads is not None and head_dim is not None:
        checks = verify_strategies(n_q_heads, n_kv_heads, head_dim, candidates=(chosen,))
        if not checks[0].ok:
            what = "no attention strategy passed verification" if strategy is None else f"requested attention strategy {chosen!r} failed verification"
            raise RuntimeError(f"{what}: {checks[0]}")
    _STRATEGY["name"], _STRATEGY["bucket"] = chosen, bucket
    AttentionInterface.register(IMPLEMENTATION_NAME, lazykv_attention_forward)
    return chosen, checks


def set_strategy_for_test(strategy: str) -> Callable[[], None]:
    """Pin `strategy` for a test or cross-check and register the attention function; returns the
    function that restores the previous strategy (lazykv/attention.py:301-310)."""
    from transformers import AttentionInterface

    _known(strategy)
    previous = _STRATEGY["name"]
    _STRATEGY["name"] = strategy
    AttentionInterface.register(IMPLEMENTATION_NAME, lazykv_attention_forward)

    def restore() -> None:
        _STRATEGY["name"] = previous

    return restore


def current_strategy() -> tuple[str, int]:
    return _STRATEGY["name"], _STRATEGY["bucket"]
