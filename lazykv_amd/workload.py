"""Seeded synthetic decode workloads (the benchmark and parity-test inputs).

Per layer l, following the workload definition of the tiered decode benchmarks:

* per-channel scales s_K[h, c], s_V[h, c] ~ U[0.5, 2]        (seed 1000 + l)
* K = N(0, 1) * s_K, V = N(0, 1) * s_V, shape [h, T, d]         (seed 2000 + l)
* q ~ N(0, 1), shape [n_q, d]                                   (seed 3000 + l)
* one needle block b* ~ U{1 .. N-2}                             (seed 4000 + l): for every KV head
  h, K[h, b*bs:(b*+1)bs] = 4 q^ + N(0, 0.1), q^ the query of the group's first head normalised
  to unit per-element RMS (|q^|^2 = d). (With a unit-norm q^ the needle's Quest bound, about
  4|q| + 18 at d = 128, would sit far below the 6.25%-budget threshold of N(0,1)-scaled blocks,
  about 237, and could never be selected.)

Sequence state: T = N * bs tokens under lazy sealing, so blocks 0..N-2 are sealed, block N-1 is
the current block with fill = bs, the candidates are blocks 1..N-2.

Draws use torch's CPU generator for small shapes (bit-reproducible anywhere) and the device
generator for large ones (`device="cuda"`), which is how the 16 GiB benchmark state is built in
seconds; both are seeded the same way.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class LayerDraw:
    keys: torch.Tensor  # [h, T, d]
    values: torch.Tensor  # [h, T, d]
    query: torch.Tensor  # [n_q, d]
    needle: int


def draw_layer(layer: int, n_q: int, n_kv: int, head_dim: int, tokens: int, block_size: int, dtype: torch.dtype, device: str | torch.device = "cpu", needle: bool = True) -> LayerDraw:
    dev = torch.device(device)
    g = n_q // n_kv

    def gen(seed: int) -> torch.Generator:
        return torch.Generator(device=dev).manual_seed(seed)

    g1 = gen(1000 + layer)
    s_k = torch.rand((n_kv, 1, head_dim), generator=g1, device=dev) * 1.5 + 0.5
    s_v = torch.rand((n_kv, 1, head_dim), generator=g1, device=dev) * 1.5 + 0.5
    g2 = gen(2000 + layer)
    keys = torch.randn((n_kv, tokens, head_dim), generator=g2, device=dev).mul_(s_k)
    values = torch.randn((n_kv, tokens, head_dim), generator=g2, device=dev).mul_(s_v)
    q = torch.randn((n_q, head_dim), generator=gen(3000 + layer), device=dev)
    n_blocks = tokens // block_size
    b_star = -1
    if needle and n_blocks >= 3:
        g4 = gen(4000 + layer)
        b_star = int(torch.randint(1, n_blocks - 1, (1,), generator=g4, device=dev).item())
        lead = q[0::g]  # first query head of each group, [n_kv, d]
        unit = lead / lead.pow(2).mean(dim=-1, keepdim=True).sqrt()
        noise = torch.randn((n_kv, block_size, head_dim), generator=g4, device=dev) * 0.1
        keys[:, b_star * block_size : (b_star + 1) * block_size] = 4.0 * unit[:, None, :] + noise
    return LayerDraw(keys.to(dtype), values.to(dtype), q.to(dtype), b_star)


def to_pool(keys: torch.Tensor, values: torch.Tensor, block_size: int) -> torch.Tensor:
    """[h, T, d] keys/values -> the tier's pair layout [T/bs, h, 2, bs, d] (lazykv/tiered.py:163-164)."""
    h, t, d = keys.shape
    n = t // block_size
    pairs = torch.stack([keys[:, : n * block_size], values[:, : n * block_size]], dim=1)  # [h, 2, T, d]
    return pairs.view(h, 2, n, block_size, d).permute(2, 0, 1, 3, 4).contiguous()
