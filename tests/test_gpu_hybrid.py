"""Device-side hybrid residency on the GPU: over a drifting sequence of decode steps, the hybrid
decode's output and LSE equal the zero-copy decode's bit for bit, its residency tables equal the
oracle's (oracle.reference.residency_step), and every slot holds an exact copy of its block (for
an int8 host tier: the block's dequantised rows, as lkv_unpack_int8 writes them)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference as R

pytestmark = pytest.mark.gpu


def _layer(seed: int, h: int, g: int, n: int, bs: int, d: int, dt: torch.dtype):  # noqa: ANN202
    from lazykv_amd import kernels
    from lazykv_amd.pinned import pinned_empty
    from lazykv_amd.workload import draw_layer, to_pool

    w = draw_layer(seed, h * g, h, d, n * bs, bs, dt)
    pool = to_pool(w.keys, w.values, bs).cuda()
    kmin = torch.zeros((1, h, n, d), dtype=dt, device="cuda")
    kmax = torch.zeros_like(kmin)
    kernels.store_blocks(kernels.dense_source(w.keys.cuda(), w.values.cuda(), bs), n_kv=h, head_dim=d, block_size=bs, first_block=0, n_blocks=n - 1, kmin=kmin, kmax=kmax)
    host = pinned_empty(tuple(pool.shape), dt)
    host.copy_(pool)
    return w, pool, host, kmin, kmax


@pytest.mark.parametrize(
    ("h", "g", "n", "bs", "d", "k", "dt", "fill", "quant", "spare"),
    [
        (8, 4, 300, 16, 128, 32, torch.bfloat16, 16, None, 0),
        (4, 4, 200, 16, 64, 24, torch.float16, 5, None, 0),
        (2, 8, 150, 32, 128, 40, torch.bfloat16, 19, None, 0),
        (8, 4, 300, 16, 128, 32, torch.bfloat16, 16, "int8", 0),
        (4, 4, 200, 16, 64, 24, torch.float16, 5, "int8", 0),
        (4, 4, 120, 20, 64, 16, torch.float16, 7, "int8", 0),  # a 4-row tail chunk per pair
        (2, 8, 100, 64, 128, 20, torch.bfloat16, 50, "int8", 0),
        (4, 2, 160, 8, 128, 30, torch.bfloat16, 8, None, 0),
        (8, 4, 300, 16, 128, 32, torch.bfloat16, 16, None, 32),  # spare slots: twice the selection
        (4, 4, 200, 16, 64, 24, torch.float16, 5, "int8", 7),
        (2, 4, 400, 16, 64, 100, torch.bfloat16, 11, None, 1000),  # 1,100 slots: several per thread of the residency launch
    ],
)
def test_hybrid_decode_is_the_zero_copy_decode(h: int, g: int, n: int, bs: int, d: int, k: int, dt: torch.dtype, fill: int, quant: str | None, spare: int) -> None:
    from lazykv_amd import kernels
    from lazykv_amd.pinned import pinned_empty

    w, pool, host, kmin, kmax = _layer(n + k, h, g, n, bs, d, dt)
    hsrc = kernels.pool_source(host)
    expect = pool  # what each slot must hold: the block's rows as a decode reads them
    if quant == "int8":
        recs = kernels.pack_int8(pool.reshape(n * h, 2, bs, d))
        expect = kernels.unpack_int8(recs, bs, d, dt).reshape(n, h, 2, bs, d)
        host = pinned_empty((n, h, recs.shape[1]), torch.uint8)
        host.copy_(recs.reshape(n, h, -1))
        hsrc = kernels.record_source(host, dt)
    n_slots = k + spare
    res = kernels.Residency.allocate(k, h, n, bs, d, dt, torch.device("cuda"), n_slots=n_slots)
    bs_ref, sb_ref, lu_ref = R.residency_state(h, n_slots, n)
    slots_src = pool[[0, n - 1]].contiguous()
    ss = kernels.pool_source(slots_src)
    gen = torch.Generator().manual_seed(5)
    q0 = w.query.float()
    hits = 0
    for step in range(12):
        q = (q0 + 0.35 * torch.randn(q0.shape, generator=gen)).to(dt).cuda()
        idx = kernels.bound_topk(q, kmin, kmax, k, cand_offset=1, n_cand=n - 2)
        common = dict(n_kv=h, block_size=bs, scale=d**-0.5, idx=idx, sink=ss, sink_block=0, cur=ss, cur_block=1, fill=fill, out_dtype=torch.float32)
        out_z, lse_z = kernels.sparse_decode(q, sel=hsrc, **common)
        out_h, lse_h = kernels.hybrid_decode(q, host=hsrc, res=res, **common)
        torch.cuda.synchronize()
        assert torch.equal(out_h, out_z) and torch.equal(lse_h, lse_z), step
        chosen = idx.cpu().numpy().astype(np.int64)
        prev = bs_ref.copy()
        R.residency_step(bs_ref, sb_ref, lu_ref, chosen, step)
        assert np.array_equal(res.block_slot.cpu().numpy(), bs_ref), step
        assert np.array_equal(res.slot_block.cpu().numpy(), sb_ref), step
        assert np.array_equal(res.order.cpu().numpy(), R.slot_order(lu_ref)), step
        hits += int((np.take_along_axis(prev, chosen, axis=1) >= 0).sum())
        # every occupied slot holds an exact copy of the block the table names
        for j in range(h):
            held = np.flatnonzero(sb_ref[j] >= 0)
            assert torch.equal(res.slots[torch.from_numpy(held).cuda(), j], expect[torch.from_numpy(sb_ref[j, held]).cuda(), j])
    assert hits > 0  # the drift keeps part of each selection resident
    if spare:
        assert (sb_ref >= 0).sum() > h * k  # spare slots keep blocks the current selection does not name


@pytest.mark.parametrize(("dt", "d", "u", "scale_bits"), [(torch.float16, 64, 145, 0x01C4), (torch.bfloat16, 128, 185, 0x0989)])
def test_int8_miss_fill_rounds_like_the_reference(dt: torch.dtype, d: int, u: int, scale_bits: int) -> None:
    """Records planted so that one key channel and one value token dequantise to u * s + 8 just
    above a tie of the model dtype: quant.py:103-105 rounds to float32 first, which lands on the
    tie and rounds to 8. The decode's in-register dequantisation (here: the hybrid miss fill, whose
    slot rows are those values) and lkv_unpack_int8 must both give the oracle's rows bit for bit,
    8 at every planted element; the hybrid output equals the zero-copy output."""
    from lazykv_amd import kernels
    from lazykv_amd.pinned import pinned_empty

    h, g, n, bs, k, c0, t0 = 2, 4, 40, 16, 8, 5, 3
    name = "f16" if dt == torch.float16 else "bf16"
    w, pool, _, _, _ = _layer(11, h, g, n, bs, d, dt)
    recs = kernels.pack_int8(pool.reshape(n * h, 2, bs, d)).cpu().numpy()
    o1, o2, o3, o4, o5 = R.record_offsets(bs, d)
    code = u ^ 0x80  # the int8 code u - 128, as a byte
    recs[:, [t * d + c0 for t in range(bs)]] = code  # key channel c0 of every token
    recs[:, o1 + t0 * d : o1 + (t0 + 1) * d] = code  # every channel of value token t0
    for at, val in ((o2 + 2 * c0, scale_bits), (o3 + 2 * c0, 0x4800), (o4 + 2 * t0, scale_bits), (o5 + 2 * t0, 0x4800)):
        recs[:, at : at + 2] = np.array([val], dtype="<u2").view(np.uint8)  # float16, little-endian; 0x4800 = 8.0
    recs_np = np.ascontiguousarray(recs)
    want = torch.from_numpy(R.unpack(recs_np, bs, d, name).view(np.int16)).view(dt).reshape(n, h, 2, bs, d)
    assert torch.all(want[:, :, 0, :, c0] == 8.0) and torch.all(want[:, :, 1, t0, :] == 8.0)
    recs_gpu = torch.from_numpy(recs_np).cuda()
    assert torch.equal(kernels.unpack_int8(recs_gpu, bs, d, dt).cpu().view(torch.int16), want.reshape(n * h, 2, bs, d).view(torch.int16))
    host = pinned_empty((n, h, recs_np.shape[1]), torch.uint8)
    host.copy_(torch.from_numpy(recs_np).reshape(n, h, -1))
    hsrc = kernels.record_source(host, dt)
    res = kernels.Residency.allocate(k, h, n, bs, d, dt, torch.device("cuda"))
    ss = kernels.pool_source(pool[[0, n - 1]].contiguous())
    idx = torch.arange(2, 2 + 3 * k, 3, dtype=torch.int32).repeat(h, 1).cuda()
    q = w.query.cuda()
    common = dict(n_kv=h, block_size=bs, scale=d**-0.5, idx=idx, sink=ss, sink_block=0, cur=ss, cur_block=1, fill=9, out_dtype=torch.float32)
    out_z, lse_z = kernels.sparse_decode(q, sel=hsrc, **common)
    out_h, lse_h = kernels.hybrid_decode(q, host=hsrc, res=res, **common)
    torch.cuda.synchronize()
    assert torch.equal(out_h, out_z) and torch.equal(lse_h, lse_z)
    sb = res.slot_block.cpu()
    assert sorted(sb[0].tolist()) == idx[0].cpu().tolist()
    for j in range(h):
        got = res.slots[:, j].cpu()
        assert torch.equal(got.view(torch.int16), want[sb[j].long(), j].view(torch.int16)), j
        assert torch.all(got[:, 0, :, c0] == 8.0) and torch.all(got[:, 1, t0, :] == 8.0), j


@pytest.mark.parametrize(
    ("h", "g", "n", "bs", "d", "k", "dt", "quant", "mode", "spare", "exact"),
    [
        (8, 4, 300, 16, 128, 32, torch.bfloat16, None, "f32", 0, False),
        (4, 4, 200, 16, 64, 24, torch.float16, "int8", "f32", 0, False),
        (2, 8, 150, 32, 128, 40, torch.bfloat16, None, "model", 0, False),
        (8, 4, 1200, 16, 64, 200, torch.float16, "int8", "model", 0, False),
        (2, 4, 8194, 16, 64, 512, torch.bfloat16, None, "f32", 0, False),  # 8,192 candidates: the largest selected in the residency launch
        (2, 4, 8300, 16, 64, 512, torch.bfloat16, None, "f32", 0, False),  # beyond: the selection takes its own launch
        (8, 4, 300, 16, 128, 32, torch.bfloat16, None, "f32", 16, False),  # spare slots
        (4, 4, 200, 16, 64, 24, torch.float16, "int8", "f32", 24, True),  # spare slots and an exact remainder
        (8, 4, 300, 16, 128, 32, torch.bfloat16, None, "model", 0, True),  # the exact remainder over k slots
        (2, 4, 8300, 16, 64, 512, torch.bfloat16, None, "f32", 0, True),  # the remainder after the selection's own launch
    ],
)
def test_one_call_hybrid_step_is_bound_topk_then_hybrid_decode(h: int, g: int, n: int, bs: int, d: int, k: int, dt: torch.dtype, quant: str | None, mode: str,
                                                                spare: int, exact: bool) -> None:
    """lkv_select_hybrid_decode against lkv_bound_topk + lkv_hybrid_decode from the same empty
    tables over a drifting sequence: the same ids, tables, use order, slot contents, output and LSE,
    bit for bit, at every step. With `exact`, both attend the remainder (every other sealed block,
    from the host tier), and the two-call output equals lkv_sparse_decode's over the host tier."""
    from lazykv_amd import kernels
    from lazykv_amd.pinned import pinned_empty

    w, pool, host, kmin, kmax = _layer(n + k + 1, h, g, n, bs, d, dt)
    hsrc = kernels.pool_source(host)
    if quant == "int8":
        recs = kernels.pack_int8(pool.reshape(n * h, 2, bs, d))
        host = pinned_empty((n, h, recs.shape[1]), torch.uint8)
        host.copy_(recs.reshape(n, h, -1))
        hsrc = kernels.record_source(host, dt)
    rank = kernels._lib.RANK_F32 if mode == "f32" else kernels._lib.RANK_MODEL
    dev = torch.device("cuda")
    res_a = kernels.Residency.allocate(k, h, n, bs, d, dt, dev, n_slots=k + spare)
    res_b = kernels.Residency.allocate(k, h, n, bs, d, dt, dev, n_slots=k + spare)
    ss = kernels.pool_source(pool[[0, n - 1]].contiguous())
    common = dict(block_size=bs, scale=d**-0.5, sink=ss, sink_block=0, cur=ss, cur_block=1, fill=bs - 3, out_dtype=torch.float32)
    if exact:
        common.update(rem=hsrc, rem_range=(1, n - 1))
    gen = torch.Generator().manual_seed(9)
    q0 = w.query.float()
    idx_b = torch.empty((h, k), dtype=torch.int32, device="cuda")
    for step in range(6):
        q = (q0 + 0.3 * torch.randn(q0.shape, generator=gen)).to(dt).cuda()
        idx_a = kernels.bound_topk(q, kmin, kmax, k, cand_offset=1, n_cand=n - 2, rank_mode=rank)
        out_a, lse_a = kernels.hybrid_decode(q, n_kv=h, host=hsrc, res=res_a, idx=idx_a, **common)
        out_b, lse_b = kernels.select_hybrid_decode(q, kmin, kmax, k, cand_offset=1, n_cand=n - 2, host=hsrc, res=res_b, rank_mode=rank, out_idx=idx_b, **common)
        if exact:
            out_z, lse_z = kernels.sparse_decode(q, n_kv=h, sel=hsrc, idx=idx_a, **common)
        torch.cuda.synchronize()
        assert torch.equal(idx_b, idx_a), step
        assert torch.equal(out_b, out_a) and torch.equal(lse_b, lse_a), step
        assert torch.equal(res_b.block_slot, res_a.block_slot) and torch.equal(res_b.slot_block, res_a.slot_block), step
        assert torch.equal(res_b.order, res_a.order), step
        assert torch.equal(res_b.slots, res_a.slots), step
        if exact:
            assert torch.equal(out_a, out_z) and torch.equal(lse_a, lse_z), step
    assert (res_b.block_slot >= 0).any()


@pytest.mark.parametrize(("tables", "spare"), [("zeros", 0), ("garbage", 0), ("zeros", 5), ("garbage", 5)])
def test_hybrid_decode_survives_tables_that_disagree(tables: str, spare: int) -> None:
    """Tables filled with zeros instead of -1, or with out-of-range and contradictory entries, and
    a use order that is not a permutation of the slots: a hit needs block_slot and slot_block to
    agree and a bad order is read as ascending slots, so every step still equals the zero-copy
    decode, and after it the selected blocks are resident with consistent tables and the order is a
    permutation again. (A pair of entries that agree is a residency claim, which no table check can
    tell from a true one.)"""
    from lazykv_amd import kernels

    h, g, n, bs, d, k = 4, 4, 120, 16, 64, 16
    n_slots = k + spare
    w, pool, host, kmin, kmax = _layer(5, h, g, n, bs, d, torch.float16)
    res = kernels.Residency.allocate(k, h, n, bs, d, torch.float16, torch.device("cuda"), n_slots=n_slots)
    gen = torch.Generator().manual_seed(9)
    if tables == "zeros":
        res.block_slot.zero_()
        res.slot_block.zero_()
        res.order.zero_()
    else:  # out-of-range and contradictory entries; no pair that agrees (that would be a residency claim)
        bsl = torch.randint(-9, n_slots + 9, (h, n), generator=gen, dtype=torch.int32)
        sbl = torch.randint(-9, n + 9, (h, n_slots), generator=gen, dtype=torch.int32)
        for j in range(h):
            for s_ in range(n_slots):
                b = int(sbl[j, s_])
                if 0 <= b < n and int(bsl[j, b]) == s_:
                    sbl[j, s_] = -5
        res.block_slot.copy_(bsl.cuda())
        res.slot_block.copy_(sbl.cuda())
        res.order.copy_(torch.randint(-3, n_slots + 3, (h, n_slots), generator=gen, dtype=torch.int32).cuda())
    res.slots.normal_()  # slot contents that no table entry may be trusted to describe
    ss = kernels.pool_source(pool[[0, n - 1]].contiguous())
    hsrc = kernels.pool_source(host)
    q0 = w.query.float()
    for step in range(4):
        q = (q0 + 0.3 * torch.randn(q0.shape, generator=gen)).to(torch.float16).cuda()
        idx = kernels.bound_topk(q, kmin, kmax, k, cand_offset=1, n_cand=n - 2)
        common = dict(n_kv=h, block_size=bs, scale=d**-0.5, idx=idx, sink=ss, sink_block=0, cur=ss, cur_block=1, fill=5, out_dtype=torch.float32)
        out_z, lse_z = kernels.sparse_decode(q, sel=hsrc, **common)
        out_h, lse_h = kernels.hybrid_decode(q, host=hsrc, res=res, **common)
        torch.cuda.synchronize()
        assert torch.equal(out_h, out_z) and torch.equal(lse_h, lse_z), step
        bsl, sbl = res.block_slot.cpu(), res.slot_block.cpu()
        for j in range(h):
            for b in idx[j].cpu().tolist():
                s_ = int(bsl[j, b])
                assert 0 <= s_ < n_slots and int(sbl[j, s_]) == b, (step, j, b)
                assert torch.equal(res.slots[s_, j], pool[b, j].cuda())
            assert sorted(res.order[j].cpu().tolist()) == list(range(n_slots)), (step, j)


def test_hybrid_decode_refuses_what_it_cannot_hold() -> None:
    from lazykv_amd import kernels

    h, g, n, bs, d, k = 2, 4, 60, 16, 64, 8
    w, pool, host, kmin, kmax = _layer(1, h, g, n, bs, d, torch.float16)
    idx = kernels.bound_topk(w.query.cuda(), kmin, kmax, k, cand_offset=1, n_cand=n - 2)
    wrong = kernels.Residency.allocate(k - 1, h, n, bs, d, torch.float16, torch.device("cuda"))  # fewer slots than selected blocks
    with pytest.raises(ValueError, match="slots"):
        kernels.hybrid_decode(w.query.cuda(), n_kv=h, block_size=bs, scale=d**-0.5, host=kernels.pool_source(host), res=wrong, idx=idx)
    common = dict(cand_offset=1, block_size=bs, scale=d**-0.5, host=kernels.pool_source(host))
    with pytest.raises(ValueError, match="slots"):
        kernels.select_hybrid_decode(w.query.cuda(), kmin, kmax, k, n_cand=n - 2, res=wrong, **common)
    spare = kernels.Residency.allocate(k, h, n, bs, d, torch.float16, torch.device("cuda"), n_slots=k + 4)
    unordered = kernels.Residency(spare.slots, spare.block_slot, spare.slot_block, None)  # spare slots need the use order
    with pytest.raises(ValueError, match="use order"):
        kernels.select_hybrid_decode(w.query.cuda(), kmin, kmax, k, n_cand=n - 2, res=unordered, **common)
    too_many = kernels.Residency.allocate(k, h, n, bs, d, torch.float16, torch.device("cuda"), n_slots=5000)  # past the 4,096-slot limit
    with pytest.raises(ValueError, match="limit"):
        kernels.select_hybrid_decode(w.query.cuda(), kmin, kmax, k, n_cand=n - 2, res=too_many, **common)
    right = kernels.Residency.allocate(k, h, n, bs, d, torch.float16, torch.device("cuda"))
    with pytest.raises(ValueError, match="candidates"):
        kernels.select_hybrid_decode(w.query.cuda(), kmin, kmax, k, n_cand=n, res=right, **common)  # past the metadata
    with pytest.raises(ValueError, match="k="):
        kernels.select_hybrid_decode(w.query.cuda(), kmin, kmax, n, n_cand=n - 2, res=right, **common)  # more than the candidates
    short = kernels.Residency(right.slots, right.block_slot[:, : n - 5].contiguous(), right.slot_block, right.order)
    with pytest.raises(ValueError, match="residency table"):
        kernels.select_hybrid_decode(w.query.cuda(), kmin, kmax, k, n_cand=n - 2, res=short, **common)


def test_hybrid_cache_decodes_like_the_zero_copy_cache() -> None:
    """A transformers Llama stack decoding 40 tokens through seals: the hybrid tier's
    log-probabilities equal the zero-copy tier's bit for bit."""
    import copy

    from transformers import LlamaConfig, LlamaForCausalLM

    from lazykv_amd.attention import IMPLEMENTATION_NAME, install
    from lazykv_amd.tiered_prefill import tiered_prefill

    install()
    torch.manual_seed(0)
    cfg = LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=4, num_attention_heads=4, num_key_value_heads=2, head_dim=64, vocab_size=512, max_position_embeddings=4096)
    with torch.device("cuda"):
        model = LlamaForCausalLM(copy.deepcopy(cfg))
    model.set_attn_implementation(IMPLEMENTATION_NAME)
    model = model.to(dtype=torch.float16).eval()
    gen = torch.Generator(device="cuda").manual_seed(7)
    ids = torch.randint(0, cfg.vocab_size, (1, 140), device="cuda", generator=gen)
    caches = {}
    for fetch in ("zerocopy", "hybrid"):
        got = tiered_prefill(model, ids[:, :100], 32, 3, 16, 512, dense_layers=1, fetch=fetch)
        rows = [torch.log_softmax(got.last_logits, -1)]
        with torch.inference_mode():
            for t in range(100, 140):
                out = model(input_ids=ids[:, t : t + 1], past_key_values=got.cache, use_cache=True, **got.cache.model_kwargs())
                rows.append(torch.log_softmax(out.logits[0, -1].float(), -1))
        caches[fetch] = (torch.stack(rows), got.cache)
    assert torch.equal(caches["zerocopy"][0], caches["hybrid"][0])
    tier = caches["hybrid"][1].tiers[1]
    assert tier.res is not None and (tier.res.block_slot >= 0).any()
