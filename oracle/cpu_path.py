"""The reference's decode step for one selecting layer, on the CPU, for the `cpu_baseline` leg.

TEST/BASELINE INFRASTRUCTURE ONLY (see `oracle/__init__.py`): bench.py times it beside the GPU
kernels; the product never calls it.

It keeps the reference's algorithm and op order, in torch CPU ops:

1. `quest_bound` + `topk` + 1 on the candidate metadata (lazykv/selection.py:38-62, ranked in
   float32 as `dtype=torch.float32` does; call site lazykv/tiered.py:500);
2. the zero-copy gather: flat (block * h + head) ids, `index_select` from the host pool viewed as
   [blocks * h, 2, bs, d], then `cat(sink, selected, current)` (lazykv/tiered.py:501-507);
3. explicit attention over the gathered set with the current block masked past `fill`
   (lazykv/attention.py:196-207's float32 form, lazykv/selection.py:65-69's mask), and its
   log-sum-exp (lazykv/exact.py:276-288), in float32 as the reference's CPU pass computes.
"""

from __future__ import annotations

import torch


def decode_layer(
    query: torch.Tensor,
    kmin: torch.Tensor,
    kmax: torch.Tensor,
    n_full: int,
    k: int,
    host_pool: torch.Tensor,
    sink: torch.Tensor,
    current: torch.Tensor,
    fill: int,
    scale: float,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """query [n_q, d]; kmin/kmax [1, h, cap, d]; host_pool [cap, h, 2, bs, d]; sink/current [h, 2, bs, d].

    Returns (out [n_q, d] float32, lse [n_q] float32, chosen block ids [h, k]).
    """
    h, d = kmin.shape[1], kmin.shape[-1]
    bs = host_pool.shape[3]
    n_q = query.shape[0]
    g = n_q // h
    # 1. bound + top-K (selection.py:46-53 with dtype=float32, :62; +1 at tiered.py:500)
    q = query.float().view(1, h, g, d)
    qp = q.clamp_min(0)
    mn = kmin[:, :, 1:n_full].float()
    mx = kmax[:, :, 1:n_full].float()
    bound = (qp @ mx.transpose(-1, -2)) + ((q - qp) @ mn.transpose(-1, -2))
    top = bound.amax(dim=2).topk(k, dim=-1).indices + 1  # [1, h, K]
    # 2. gather (tiered.py:501-507)
    flat = (top[0] * h + torch.arange(h)[:, None]).reshape(-1)
    sel = host_pool.view(-1, 2, bs, d).index_select(0, flat).view(h, k, 2, bs, d)
    keys = torch.cat([sink[:, None, 0], sel[:, :, 0], current[:, None, 0]], dim=1).view(h, (k + 2) * bs, d)
    values = torch.cat([sink[:, None, 1], sel[:, :, 1], current[:, None, 1]], dim=1).view(h, (k + 2) * bs, d)
    # 3. attention + LSE over the gathered set (attention.py:196-207, exact.py:276-288)
    total = (k + 2) * bs
    mask = torch.zeros(total)
    mask[total - bs + fill :] = float("-inf")
    scores = (q[0] @ keys.float().transpose(-1, -2)) * scale + mask  # [h, g, total]
    lse = torch.logsumexp(scores, dim=-1)
    out = torch.softmax(scores, dim=-1) @ values.float()
    return out.reshape(n_q, d), lse.reshape(n_q), top[0]
