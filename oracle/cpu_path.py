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

The other workloads' CPU paths follow the same rule: `decode_layer_int8` (the int8 tier: gather
records, `unpack`, attend), `exact_layer` (the exact tier: the gathered partial plus the batched,
masked CPU partial over the float32 mirror, merged by log-sum-exp), `hybrid_layer` (the hybrid
residency tier: rank, admit the missed blocks into the least recently used slots, gather from the
slots, attend) and `tier_build_layer` (the int8 boundary: `pack`, `unpack`, key min/max).
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


def _rank(query: torch.Tensor, kmin: torch.Tensor, kmax: torch.Tensor, n_full: int, k: int) -> tuple[torch.Tensor, int, int, int]:
    """Quest's bound over candidates 1..n_full-1 and each head's top k, in descending bound order
    (lazykv/selection.py:46-62 ranked in float32, +1 at lazykv/tiered.py:386)."""
    h, d = kmin.shape[1], kmin.shape[-1]
    g = query.shape[0] // h
    q = query.float().view(1, h, g, d)
    qp = q.clamp_min(0)
    bound = (qp @ kmax[:, :, 1:n_full].float().transpose(-1, -2)) + ((q - qp) @ kmin[:, :, 1:n_full].float().transpose(-1, -2))
    return bound.amax(dim=2).topk(k, dim=-1).indices[0] + 1, h, g, d


def _attend(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, bs: int, fill: int, scale: float) -> tuple[torch.Tensor, torch.Tensor]:
    """Explicit float32 attention with its LSE over [h, total, d], the last block masked past fill."""
    total = keys.shape[1]
    mask = torch.zeros(total)
    mask[total - bs + fill :] = float("-inf")
    scores = (q @ keys.float().transpose(-1, -2)) * scale + mask
    return torch.softmax(scores, dim=-1) @ values.float(), torch.logsumexp(scores, dim=-1)


def hybrid_layer(
    query: torch.Tensor,
    kmin: torch.Tensor,
    kmax: torch.Tensor,
    n_full: int,
    k: int,
    host_pool: torch.Tensor,
    slot_pool: torch.Tensor,
    residency: tuple,
    step: int,
    sink: torch.Tensor,
    current: torch.Tensor,
    fill: int,
    scale: float,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """One decode step of the hybrid residency tier (rung 6), in the reference's order: rank
    (lazykv/tiered.py:383-387), admit the missed (head, block) pairs into the least recently used
    slots the choice does not hit, copying them from the host pool (:389-449; an int8 record is
    widened on arrival, :428-432), then gather sink, the chosen blocks from their slots in rank
    order and the current block (:450-470), and attend.

    host_pool [cap, h, 2, bs, d] (or int8 records [cap, h, P]); slot_pool [n_slots, h, 2, bs, d];
    residency = (block_slot, slot_block, last_used) as `reference.residency_state` builds them,
    updated in place by `reference.residency_step`. Returns (out [n_q, d], lse [n_q], chosen [h, k]).
    """
    from oracle.reference import LOC_MISS, residency_step

    top, h, g, d = _rank(query, kmin, kmax, n_full, k)
    bs = sink.shape[2]
    chosen = top.numpy()
    loc = residency_step(*residency, chosen, step)
    heads = torch.arange(h)[:, None].expand(h, k)
    miss = torch.from_numpy((loc & LOC_MISS) != 0)
    slot = torch.from_numpy(loc & ~LOC_MISS)
    if bool(miss.any()):
        src = (top[miss] * h + heads[miss]).reshape(-1)
        dst = (slot[miss] * h + heads[miss]).reshape(-1)
        flat = host_pool.reshape(host_pool.shape[0] * h, -1)
        arrived = flat.index_select(0, src)
        if host_pool.dtype == torch.uint8:
            arrived = unpack_records(arrived, bs, d, slot_pool.dtype)
        slot_pool.view(-1, 2, bs, d).index_copy_(0, dst, arrived.view(-1, 2, bs, d))
    sel = slot_pool.view(-1, 2, bs, d).index_select(0, (slot * h + heads).reshape(-1)).view(h, k, 2, bs, d)
    keys = torch.cat([sink[:, None, 0], sel[:, :, 0], current[:, None, 0]], dim=1).view(h, (k + 2) * bs, d)
    values = torch.cat([sink[:, None, 1], sel[:, :, 1], current[:, None, 1]], dim=1).view(h, (k + 2) * bs, d)
    out, lse = _attend(query.float().view(h, g, d), keys, values, bs, fill, scale)
    return out.reshape(-1, d), lse.reshape(-1), top


# -- int8 tier, exact split and the tier build: the reference's torch ops on CPU tensors ------------


def unpack_records(records: torch.Tensor, bs: int, d: int, dtype: torch.dtype) -> torch.Tensor:
    """lazykv/quant.py:90-105 in torch CPU ops: uint8 [m, P] -> [m, 2, bs, d] in `dtype`."""
    n = bs * d
    o1, o2, o3, o4, o5 = n, 2 * n, 2 * n + 2 * d, 2 * n + 4 * d, 2 * n + 4 * d + 2 * bs
    kq = records[:, :o1].view(torch.int8).unflatten(1, (bs, d))
    vq = records[:, o1:o2].view(torch.int8).unflatten(1, (bs, d))
    ks, kz = records[:, o2:o3].view(torch.float16), records[:, o3:o4].view(torch.float16)
    vs, vz = records[:, o4:o5].view(torch.float16), records[:, o5:].view(torch.float16)
    k = (kq.float() + 128) * ks.float().unsqueeze(1) + kz.float().unsqueeze(1)
    v = (vq.float() + 128) * vs.float().unsqueeze(2) + vz.float().unsqueeze(2)
    return torch.stack([k, v], dim=1).to(dtype)


def pack_pairs(pairs: torch.Tensor) -> torch.Tensor:
    """lazykv/quant.py:59-87 in torch CPU ops: [m, 2, bs, d] -> uint8 [m, P]."""
    levels = 255.0

    def affine(x: torch.Tensor, dim: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        mn = x.amin(dim=dim, keepdim=True).float()
        mx = x.amax(dim=dim, keepdim=True).float()
        scale = ((mx - mn) / levels).clamp_min(torch.finfo(torch.float32).tiny)
        q = ((x.float() - mn) / scale).round_().clamp_(0, levels).sub_(128).to(torch.int8)
        return q, scale.squeeze(dim).to(torch.float16), mn.squeeze(dim).to(torch.float16)

    kq, ks, kz = affine(pairs[:, 0], 1)
    vq, vs, vz = affine(pairs[:, 1], 2)
    parts = [kq.flatten(1), vq.flatten(1), ks, kz, vs, vz]
    return torch.cat([p.contiguous().view(torch.uint8) for p in parts], dim=1)


def tier_build_layer(keys: torch.Tensor, values: torch.Tensor, bs: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The int8 tier's boundary for one layer (lazykv/tiered.py:187-197): pack every full block,
    unpack it again and take the per-channel key min/max of the dequantised keys.

    keys/values [h, n, d] -> records [blocks, h, P], kmin/kmax [h, blocks, d]."""
    h, n, d = keys.shape
    nb = n // bs
    pairs = torch.stack([keys[:, : nb * bs], values[:, : nb * bs]], dim=1).view(h, 2, nb, bs, d).permute(2, 0, 1, 3, 4).reshape(nb * h, 2, bs, d)
    records = pack_pairs(pairs)
    deq_keys = unpack_records(records, bs, d, keys.dtype)[:, 0].view(nb, h, bs, d)
    return records.view(nb, h, -1), deq_keys.amin(dim=2).transpose(0, 1), deq_keys.amax(dim=2).transpose(0, 1)


def decode_layer_int8(
    query: torch.Tensor,
    kmin: torch.Tensor,
    kmax: torch.Tensor,
    n_full: int,
    k: int,
    records: torch.Tensor,
    sink: torch.Tensor,
    current: torch.Tensor,
    fill: int,
    scale: float,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """`decode_layer` over an int8 tier: the selected records are gathered and dequantised
    (lazykv/tiered.py:430-449 gather, quant.py:90-105 unpack) before attention.
    records [cap, h, P]; sink/current exact [h, 2, bs, d]."""
    h, d = kmin.shape[1], kmin.shape[-1]
    bs = sink.shape[2]
    n_q = query.shape[0]
    g = n_q // h
    q = query.float().view(1, h, g, d)
    qp = q.clamp_min(0)
    mn = kmin[:, :, 1:n_full].float()
    mx = kmax[:, :, 1:n_full].float()
    bound = (qp @ mx.transpose(-1, -2)) + ((q - qp) @ mn.transpose(-1, -2))
    top = bound.amax(dim=2).topk(k, dim=-1).indices + 1
    flat = (top[0] * h + torch.arange(h)[:, None]).reshape(-1)
    sel = unpack_records(records.view(-1, records.shape[-1]).index_select(0, flat), bs, d, sink.dtype).view(h, k, 2, bs, d)
    keys = torch.cat([sink[:, None, 0], sel[:, :, 0], current[:, None, 0]], dim=1).view(h, (k + 2) * bs, d)
    values = torch.cat([sink[:, None, 1], sel[:, :, 1], current[:, None, 1]], dim=1).view(h, (k + 2) * bs, d)
    total = (k + 2) * bs
    mask = torch.zeros(total)
    mask[total - bs + fill :] = float("-inf")
    scores = (q[0] @ keys.float().transpose(-1, -2)) * scale + mask
    lse = torch.logsumexp(scores, dim=-1)
    out = torch.softmax(scores, dim=-1) @ values.float()
    return out.reshape(n_q, d), lse.reshape(n_q), top[0]


def exact_layer(
    query: torch.Tensor,
    kmin: torch.Tensor,
    kmax: torch.Tensor,
    n_full: int,
    k: int,
    pool: torch.Tensor,
    mirror_k: torch.Tensor,
    mirror_v: torch.Tensor,
    current: torch.Tensor,
    fill: int,
    scale: float,
) -> tuple[torch.Tensor, torch.Tensor]:
    """The exact tier's decode step (lazykv/exact.py:225-264): `decode_layer` over the gathered set,
    then the CPU partial over every sealed block not gathered (cpu_partial_attention, :88-127,
    one batched GEMM with the excluded blocks masked to -inf before the row max) from the float32
    mirror [h, n_full * bs, d], merged by log-sum-exp (:69-85)."""
    h, d = kmin.shape[1], kmin.shape[-1]
    bs = pool.shape[3]
    g = query.shape[0] // h
    out_a, lse_a, top = decode_layer(query, kmin, kmax, n_full, k, pool, pool[0], current, fill, scale)
    excluded = torch.cat([torch.zeros((h, 1), dtype=top.dtype), top], dim=1)  # sink + chosen
    q = query.float().view(h, g, d)
    scores = torch.matmul(q, mirror_k.transpose(1, 2)) * scale  # [h, g, n_full * bs]
    rows = torch.arange(h).repeat_interleave(excluded.shape[1])
    scores.view(h, g, n_full, bs)[rows, :, excluded.reshape(-1)] = float("-inf")
    m = scores.amax(dim=-1, keepdim=True)
    p = (scores - m).exp()
    norm = p.sum(dim=-1, keepdim=True)
    out_b = torch.matmul(p / norm, mirror_v)
    lse_b = (m + norm.log()).squeeze(-1)
    la, lb = lse_a.view(h, g), lse_b
    lse = torch.logaddexp(la, lb)
    out = (la - lse).exp().unsqueeze(-1) * out_a.view(h, g, d) + (lb - lse).exp().unsqueeze(-1) * out_b
    return out.reshape(-1, d), lse.reshape(-1)
