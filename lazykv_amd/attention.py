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

import torch

from lazykv_amd import kernels

IMPLEMENTATION_NAME = "lazykv_sdpa"
DENSE_BLOCK = 16  # block granularity the dense decode walks the cache in


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


def install() -> str:
    """Register the attention function with transformers under IMPLEMENTATION_NAME (:269-290)."""
    from transformers import AttentionInterface

    AttentionInterface.register(IMPLEMENTATION_NAME, lazykv_attention_forward)
    return IMPLEMENTATION_NAME
