"""The timed CPU baseline (oracle/cpu_path.py) computes what the reference computes (CPU).

bench.py times these torch CPU functions beside the kernels; the comparison is only fair if they
are the reference's algorithm. Each is checked here against the float64 / bit-level oracle
(oracle/reference.py) on small seeded inputs: selected sets under the near-tie rule, attention
within 1e-4 (float32 against float64), int8 records bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import cpu_path as C
from oracle import reference as R

H, G, D, BS = 4, 4, 64, 16


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _state(seed: int, n_full: int, fill: int, dtype: torch.dtype = torch.bfloat16):  # noqa: ANN202
    """Keys/values [h, (n_full + 1) * bs, d] with a per-channel key scale, the host pool
    [cap, h, 2, bs, d], the metadata [1, h, cap, d] of blocks 0..n_full-1 and a query [n_q, d]."""
    gen = torch.Generator().manual_seed(seed)
    n = (n_full + 1) * BS
    keys = (torch.randn((H, n, D), generator=gen) * (0.5 + 1.5 * torch.rand((H, 1, D), generator=gen))).to(dtype)
    values = torch.randn((H, n, D), generator=gen).to(dtype)
    pool = torch.stack([keys, values], dim=1).view(H, 2, n_full + 1, BS, D).permute(2, 0, 1, 3, 4).contiguous()
    kmin_np, kmax_np = R.block_minmax(keys[:, : n_full * BS].double().numpy(), BS)
    kmin = torch.zeros((1, H, n_full + 1, D), dtype=dtype)
    kmax = torch.zeros_like(kmin)
    kmin[0, :, :n_full] = torch.from_numpy(kmin_np).to(dtype)
    kmax[0, :, :n_full] = torch.from_numpy(kmax_np).to(dtype)
    query = torch.randn((H * G, D), generator=gen).to(dtype)
    return keys, values, pool, kmin, kmax, query


def _check_selection(top: torch.Tensor, query: torch.Tensor, kmin: torch.Tensor, kmax: torch.Tensor, n_full: int, k: int) -> None:
    bound = R.quest_bound(query.double().numpy(), kmin[0, :, 1:n_full].double().numpy(), kmax[0, :, 1:n_full].double().numpy())
    for j in range(H):
        ok, _ = R.selection_ok(top[j].numpy() - 1, bound[j], k, abs_err=1e-4)
        assert ok, j


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_cpu_pack_and_unpack_are_the_oracles_bytes(dt: torch.dtype) -> None:
    gen = torch.Generator().manual_seed(7)
    pairs = (torch.randn((12, 2, BS, D), generator=gen) * 3).to(dt)
    pairs[0, 0] = 1.5  # a constant key group
    pairs[1, 1, :, 5] = 40.0  # a value outlier
    name = "f16" if dt == torch.float16 else "bf16"
    rec = C.pack_pairs(pairs)
    assert np.array_equal(rec.numpy(), R.pack(_bits(pairs), name))
    assert np.array_equal(_bits(C.unpack_records(rec, BS, D, dt)), R.unpack(rec.numpy(), BS, D, name))


def test_cpu_tier_build_writes_the_oracles_records_and_dequantised_metadata() -> None:
    keys, values, *_ = _state(1, 10, 5, torch.float16)
    rec, kmin, kmax = C.tier_build_layer(keys, values, BS)
    nb = keys.shape[1] // BS
    pairs = torch.stack([keys[:, : nb * BS], values[:, : nb * BS]], dim=1).view(H, 2, nb, BS, D).permute(2, 0, 1, 3, 4)
    assert np.array_equal(rec.numpy(), R.pack(_bits(pairs), "f16"))
    deq = R.to_f32(R.unpack(rec.numpy().reshape(nb * H, -1), BS, D, "f16"), "f16").reshape(nb, H, 2, BS, D)[:, :, 0]
    assert np.array_equal(kmin.float().numpy(), deq.min(axis=2).transpose(1, 0, 2))
    assert np.array_equal(kmax.float().numpy(), deq.max(axis=2).transpose(1, 0, 2))


@pytest.mark.parametrize("fill", [1, 9, BS])
def test_cpu_decode_layer_is_the_oracles_decode(fill: int) -> None:
    n_full, k = 40, 8
    keys, values, pool, kmin, kmax, query = _state(2 + fill, n_full, fill)
    out, lse, top = C.decode_layer(query, kmin, kmax, n_full, k, pool, pool[0], pool[n_full], fill, D**-0.5)
    _check_selection(top, query, kmin, kmax, n_full, k)
    pf = pool.double().numpy()
    ks, vs = R.gathered_tokens(lambda j, b: (pf[b, j, 0], pf[b, j, 1]), H, top.numpy(), 0, n_full, fill, BS)
    want_o, want_l = R.attend_tokens(query.double().numpy(), ks, vs, D**-0.5)
    assert np.abs(out.numpy() - want_o).max() < 1e-4
    assert np.abs(lse.numpy() - want_l).max() < 1e-4


def test_cpu_decode_layer_int8_attends_the_dequantised_blocks() -> None:
    n_full, k, fill = 30, 6, 11
    keys, values, pool, _, _, query = _state(5, n_full, fill, torch.float16)
    rec, kmin_h, kmax_h = C.tier_build_layer(keys, values, BS)  # metadata of the dequantised keys
    kmin, kmax = kmin_h[None], kmax_h[None]
    out, lse, top = C.decode_layer_int8(query, kmin, kmax, n_full, k, rec, pool[0], pool[n_full], fill, D**-0.5)
    _check_selection(top, query, kmin, kmax, n_full, k)
    deq = R.to_f32(R.unpack(rec.numpy().reshape(-1, rec.shape[-1]), BS, D, "f16"), "f16").reshape(rec.shape[0], H, 2, BS, D).astype(np.float64)
    exact = pool.double().numpy()

    def bkv(j: int, b: int):  # noqa: ANN202
        src = exact if b in (0, n_full) else deq
        return src[b, j, 0], src[b, j, 1]

    ks, vs = R.gathered_tokens(bkv, H, top.numpy(), 0, n_full, fill, BS)
    want_o, want_l = R.attend_tokens(query.double().numpy(), ks, vs, D**-0.5)
    assert np.abs(out.numpy() - want_o).max() < 1e-4
    assert np.abs(lse.numpy() - want_l).max() < 1e-4


def test_cpu_exact_layer_is_full_attention() -> None:
    n_full, k, fill = 25, 5, 7
    keys, values, pool, kmin, kmax, query = _state(6, n_full, fill)
    mirror_k = keys[:, : n_full * BS].float()
    mirror_v = values[:, : n_full * BS].float()
    out, lse = C.exact_layer(query, kmin, kmax, n_full, k, pool, mirror_k, mirror_v, pool[n_full], fill, D**-0.5)
    live = n_full * BS + fill
    ks = [keys[j, :live].double().numpy() for j in range(H)]
    vs = [values[j, :live].double().numpy() for j in range(H)]
    want_o, want_l = R.attend_tokens(query.double().numpy(), ks, vs, D**-0.5)
    assert np.abs(out.numpy() - want_o).max() < 1e-4
    assert np.abs(lse.numpy() - want_l).max() < 1e-4


@pytest.mark.parametrize("int8", [False, True])
def test_cpu_hybrid_layer_decodes_like_the_zero_copy_path(int8: bool) -> None:
    """Over a drifting query sequence, the hybrid step attends exactly what the zero-copy step
    attends (the same blocks, read from slots that hold the host pool's pairs, or the records
    dequantised), so out, LSE and the chosen ids are equal bit for bit; after each step every
    resident slot holds its block, and the slots the step names are the chosen blocks'."""
    n_full, k, fill, steps = 40, 6, 9, 8
    keys, values, pool, kmin, kmax, query = _state(11, n_full, fill)
    host = C.pack_pairs(pool.reshape(-1, 2, BS, D)).view(pool.shape[0], H, -1) if int8 else pool
    widened = C.unpack_records(host.reshape(-1, host.shape[-1]), BS, D, pool.dtype).view(pool.shape) if int8 else pool
    sink, cur = widened[0], widened[n_full]
    slots = torch.zeros((k, H, 2, BS, D), dtype=pool.dtype)
    res = R.residency_state(H, k, pool.shape[0])
    gen = torch.Generator().manual_seed(3)
    misses = []
    for t in range(steps):
        q = (query.float() + 0.5 * torch.randn(query.shape, generator=gen)).to(query.dtype)
        before = res[0].copy()
        out, lse, top = C.hybrid_layer(q, kmin, kmax, n_full, k, host, slots, res, t, sink, cur, fill, D**-0.5)
        zc = (C.decode_layer_int8 if int8 else C.decode_layer)(q, kmin, kmax, n_full, k, host, sink, cur, fill, D**-0.5)
        assert torch.equal(out, zc[0]) and torch.equal(lse, zc[1]) and torch.equal(top, zc[2]), t
        block_slot, slot_block, last_used = res
        for j in range(H):
            for s in range(k):
                b = int(slot_block[j, s])
                if b >= 0:
                    assert torch.equal(slots[s, j], widened[b, j]), (t, j, s)
            assert sorted(block_slot[j, top[j].numpy()].tolist()) == list(range(k))  # k slots hold exactly the choice
            assert (last_used[j] == t).all()
        misses.append(int((np.take_along_axis(before, top.numpy(), axis=1) < 0).sum()))
    assert misses[0] == H * k and 0 < sum(misses[1:]) < (steps - 1) * H * k  # some hits, some misses
