"""Exact attention over a tiered cache: partial attention and the log-sum-exp merge, on the GPU.

Mirrors lazykv/exact.py's module functions. `merge_lse` (:69-85) is the `lkv_merge_lse` kernel.
`partial_attention` is `cpu_partial_attention` (:88-127) with the same arguments and results:
attention of a query over every block of a per-head KV store except the excluded ones, returning
the output and its LSE (an all-excluded head gives lse = -inf and a zero output). The reference
runs it on the CPU over a float32 mirror; here it is the decode kernel's remainder pass, run where
the KV lives (HBM or mapped host memory, in any model dtype).
"""

from __future__ import annotations

import numpy as np
import torch

from lazykv_amd import kernels

NEG_INF = float("-inf")


def merge_lse(out_a: torch.Tensor, lse_a: torch.Tensor, out_b: torch.Tensor, lse_b: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Combine two partial softmax attentions into the attention over their union (:69-85).

    `out_*` [..., d] are already normalised; `lse_*` [...] are their log-sum-exps. Exact for
    disjoint key sets; a partial with lse = -inf contributes nothing.
    """
    return kernels.merge_lse(out_a, lse_a, out_b, lse_b)


def partial_attention(
    keys: torch.Tensor,
    values: torch.Tensor,
    query: torch.Tensor,
    scaling: float,
    block_size: int,
    excluded: np.ndarray | torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Exact attention of `query` over `keys`/`values`, with whole blocks excluded per KV head (:88-127).

    `keys`/`values` are [kv_heads, n_blocks * block_size, head_dim] (rows contiguous per head);
    `query` is [kv_heads, groups, head_dim]; `excluded` is [kv_heads, e] block indices. Returns the
    output [kv_heads, groups, head_dim] and its LSE [kv_heads, groups], both float32.
    """
    h, total, d = keys.shape
    if total % block_size:
        raise ValueError(f"{total} tokens are not whole blocks of {block_size}")
    n_blocks = total // block_size
    groups = query.shape[1]
    ex = torch.as_tensor(np.asarray(excluded) if not isinstance(excluded, torch.Tensor) else excluded)
    if ex.ndim != 2 or ex.shape[0] != h:
        raise ValueError(f"excluded must be [{h}, e], got {tuple(ex.shape)}")
    idx = ex.to(device=keys.device, dtype=torch.int32).contiguous() if ex.shape[1] else None
    src = kernels.dense_source(keys, values, block_size)
    out, lse = kernels.sparse_decode(
        query.reshape(h * groups, d), n_kv=h, block_size=block_size, scale=scaling, idx=idx, attend_selected=False,
        rem=src, rem_range=(0, n_blocks), out_dtype=torch.float32,
    )
    return out.view(h, groups, d), lse.view(h, groups)


# The reference's name for the cold partial (lazykv/exact.py:88-127). It runs on the GPU here, so
# its tensors must be GPU tensors (or pinned host pools); CPU tensors are refused, not computed.
cpu_partial_attention = partial_attention
