"""The tier's decode path end to end on the GPU (TieredLayer / TieredCache / ExactTieredCache),
against the oracle: boundary stores, metadata, selection, seals through decode, the exact split,
graph capture and the reference's refusals."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference as R

pytestmark = pytest.mark.gpu

TOL = 2e-3
H, G, D, BS = 8, 4, 128, 16


def _f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _prompt(seed: int, length: int, dtype=torch.bfloat16):
    gen = torch.Generator().manual_seed(seed)
    s = torch.rand((1, H, 1, D), generator=gen) * 1.5 + 0.5
    keys = (torch.randn((1, H, length, D), generator=gen) * s).to(dtype)
    values = torch.randn((1, H, length, D), generator=gen).to(dtype)
    return keys, values, gen


class _Shadow:
    """The oracle's copy of a layer's token sequence, with the tier's storage rules.

    Sealed blocks are stored exactly (bf16 tier) or as int8 records (int8 tier); the sink and the
    current block are always exact (lazykv/tiered.py:200-205).
    """

    def __init__(self, keys: torch.Tensor, values: torch.Tensor, quant: str | None, bs: int = BS) -> None:
        self.bs = bs
        self.k = list(_f64(keys[0]).transpose(1, 0, 2))  # per token [h, d]
        self.v = list(_f64(values[0]).transpose(1, 0, 2))
        self.kb = list(_bits(keys[0]).transpose(1, 0, 2))
        self.vb = list(_bits(values[0]).transpose(1, 0, 2))
        self.quant = quant

    def append(self, k: torch.Tensor, v: torch.Tensor) -> None:
        self.k.append(_f64(k[0, :, 0]))
        self.v.append(_f64(v[0, :, 0]))
        self.kb.append(_bits(k[0, :, 0]))
        self.vb.append(_bits(v[0, :, 0]))

    def block(self, b: int, sealed: bool) -> tuple[np.ndarray, np.ndarray]:
        """[h, bs, d] keys and values of block b as the tier stores it."""
        bs = self.bs
        k = np.stack(self.k[b * bs : (b + 1) * bs], axis=1)
        v = np.stack(self.v[b * bs : (b + 1) * bs], axis=1)
        if self.quant == "int8" and sealed and b > 0:
            kb = np.stack(self.kb[b * bs : (b + 1) * bs], axis=1)
            vb = np.stack(self.vb[b * bs : (b + 1) * bs], axis=1)
            pairs = np.stack([kb, vb], axis=1)  # [h, 2, bs, d]
            deq = R.to_f32(R.unpack(R.pack(pairs, "bf16"), bs, D, "bf16"), "bf16").reshape(H, 2, bs, D).astype(np.float64)
            return deq[:, 0], deq[:, 1]
        return k, v

    def meta(self, n_sealed: int) -> tuple[np.ndarray, np.ndarray]:
        ks = np.stack([self.block(b, True)[0] for b in range(n_sealed)], axis=1)  # [h, n, bs, d]
        return ks.min(axis=2), ks.max(axis=2)


def _check_step(layer, shadow: _Shadow, q: torch.Tensor, exact_store: bool = False) -> None:
    BS = shadow.bs  # noqa: N806 -- the layer's block size
    n_sealed, fill = layer.candidates()
    idx = layer.rank(q.view(1, -1, 1, D))
    out32 = torch.empty((H * G, D), dtype=torch.float32, device="cuda")
    lse = torch.empty((H * G,), dtype=torch.float32, device="cuda")
    layer.decode(q, D**-0.5, idx=idx, out=out32, lse=lse)
    torch.cuda.synchronize()
    # selection against the oracle's bound over the metadata the tier should hold
    if exact_store:
        ks = np.stack([np.stack(shadow.k[b * BS : (b + 1) * BS], axis=1) for b in range(n_sealed)], axis=1)
        mn, mx = ks.min(axis=2), ks.max(axis=2)
    else:
        mn, mx = shadow.meta(n_sealed)
    bound = R.quest_bound(_f64(q), mn[:, 1:], mx[:, 1:])
    chosen = idx.cpu().numpy()
    err = float(np.abs(_f64(q)).max() * np.maximum(np.abs(mn), np.abs(mx)).sum(-1).max()) * 2.0**-19
    for j in range(H):
        ok, _ = R.selection_ok(chosen[j] - 1, bound[j], layer.k, abs_err=err)
        assert ok, (j, n_sealed)
    # attention over sink + chosen + current[:fill], as the tier stores them

    def bkv(j: int, b: int):
        if b == n_sealed:  # current block, exact
            k = np.stack(shadow.k[b * BS : b * BS + fill], axis=1)[j]
            v = np.stack(shadow.v[b * BS : b * BS + fill], axis=1)[j]
            pad = BS - fill
            return np.concatenate([k, np.zeros((pad, D))]), np.concatenate([v, np.zeros((pad, D))])
        k, v = shadow.block(b, sealed=not exact_store)
        return k[j], v[j]

    ks, vs = R.gathered_tokens(bkv, H, chosen, 0, n_sealed, fill, BS)
    want_o, want_l = R.attend_tokens(_f64(q), ks, vs, D**-0.5)
    assert np.abs(out32.cpu().numpy() - want_o).max() < TOL
    assert np.abs(lse.cpu().numpy() - want_l).max() < TOL


def test_boundary_stores_every_full_block_with_exact_metadata() -> None:
    from lazykv_amd.tiered import TieredLayer
    from lazykv_amd.workload import to_pool

    keys, values, _ = _prompt(1, 1000)  # 62 full blocks + 8 tokens
    layer = TieredLayer(keys.cuda(), values.cuda(), 8, BS, 2048)
    torch.cuda.synchronize()
    assert layer.candidates() == (62, 8) and layer.length == 1000
    pool = to_pool(keys[0], values[0], BS)
    assert torch.equal(layer.host[:62], pool[:62])
    mn, mx = R.block_minmax(_f64(keys[0, :, : 62 * BS]), BS)
    assert np.array_equal(_f64(layer.kmin[0, :, :62]), mn) and np.array_equal(_f64(layer.kmax[0, :, :62]), mx)
    assert torch.equal(layer.pool[0].cpu(), pool[0])
    assert torch.equal(layer.pool[1, :, 0, :8].cpu(), keys[0, :, 992:1000])
    assert layer.host_bytes() == 62 * H * 2 * BS * D * 2


@pytest.mark.parametrize(("fetch", "quant"), [("zerocopy", None), ("zerocopy", "int8"), ("resident", None), ("hybrid", None), ("hybrid", "int8")])
def test_decode_through_seals_matches_the_oracle(fetch: str, quant: str | None) -> None:
    """Each step appends a token (sealing every 16), ranks and decodes; every step is checked."""
    from lazykv_amd.tiered import TieredLayer

    keys, values, gen = _prompt(2, 1000)
    layer = TieredLayer(keys.cuda(), values.cuda(), 8, BS, 2048, quant=quant, fetch=fetch)
    shadow = _Shadow(keys, values, quant)
    for step in range(40):
        k = torch.randn((1, H, 1, D), generator=gen).to(torch.bfloat16)
        v = torch.randn((1, H, 1, D), generator=gen).to(torch.bfloat16)
        layer.append(k.cuda(), v.cuda())
        shadow.append(k, v)
        q = torch.randn((H * G, D), generator=gen).to(torch.bfloat16)
        if step % 4 == 3 or step in (0, 8, 9):
            _check_step(layer, shadow, q.cuda())
    assert layer.candidates() == (64, 16)  # 1040 tokens, sealed lazily when tokens 1009 and 1025 arrived


@pytest.mark.parametrize(("bs", "fetch", "quant"), [(128, "zerocopy", None), (128, "hybrid", "int8"), (256, "resident", None), (256, "zerocopy", "int8")])
def test_decode_through_seals_at_large_block_sizes(bs: int, fetch: str, quant: str | None) -> None:
    """Blocks of 128 and 256 tokens (the reference sweeps 16-256): the prompt ends 3 tokens short
    of a block, so the appends seal it; every step is checked against the oracle."""
    from lazykv_amd.tiered import TieredLayer

    keys, values, gen = _prompt(20 + bs, 6 * bs - 3)
    layer = TieredLayer(keys.cuda(), values.cuda(), 2, bs, 12 * bs, quant=quant, fetch=fetch)
    shadow = _Shadow(keys, values, quant, bs)
    for step in range(8):
        k = torch.randn((1, H, 1, D), generator=gen).to(torch.bfloat16)
        v = torch.randn((1, H, 1, D), generator=gen).to(torch.bfloat16)
        layer.append(k.cuda(), v.cuda())
        shadow.append(k, v)
        q = torch.randn((H * G, D), generator=gen).to(torch.bfloat16)
        _check_step(layer, shadow, q.cuda())
    assert layer.candidates() == (6, 5)  # 6 bs + 5 tokens: the sixth block sealed when token 6 bs + 1 arrived


@pytest.mark.parametrize("quant", [None, "int8"])
def test_exact_cache_reconstructs_full_attention(quant: str | None) -> None:
    """Selected blocks from HBM + every other sealed block from the host tier = full attention."""
    from lazykv_amd.tiered import ExactTieredCache

    keys, values, gen = _prompt(3, 1200)
    cache = ExactTieredCache([(keys.cuda(), values.cuda()), (keys.cuda(), values.cuda())], 10, BS, 2048, dense_layers=1, quant=quant, fetch="resident")
    shadow = _Shadow(keys, values, quant)
    for _ in range(3):
        k = torch.randn((1, H, 1, D), generator=gen).to(torch.bfloat16)
        v = torch.randn((1, H, 1, D), generator=gen).to(torch.bfloat16)
        cache.update(k.cuda(), v.cuda(), 1)
        shadow.append(k, v)
    q = torch.randn((1, H * G, 1, D), generator=gen).to(torch.bfloat16)
    assert cache.select(0, q.cuda()) is None  # dense layer
    dec = cache.select(1, q.cuda())
    torch.cuda.synchronize()
    tier = cache.tiers[1]
    n_sealed, fill = tier.candidates()
    idx = tier.rank(q.cuda()).cpu().numpy()
    ks, vs = [], []
    for j in range(H):
        sel = set(idx[j].tolist())
        kk, vv = [], []
        for b in range(n_sealed):
            k_b, v_b = shadow.block(b, sealed=(b > 0 and b not in sel))
            kk.append(k_b[j])
            vv.append(v_b[j])
        cur_k = np.stack(shadow.k[n_sealed * BS :], axis=1)[j]
        cur_v = np.stack(shadow.v[n_sealed * BS :], axis=1)[j]
        ks.append(np.concatenate(kk + [cur_k]))
        vs.append(np.concatenate(vv + [cur_v]))
    want_o, want_l = R.attend_tokens(_f64(q[0, :, 0]), ks, vs, D**-0.5)
    got = dec.out.float().cpu().numpy()[0, :, 0]
    assert (np.abs(got - want_o) <= TOL + np.abs(want_o) * 2.0**-8).all()  # output rounded to bf16
    assert np.abs(dec.lse.cpu().numpy()[0] - want_l).max() < TOL
    if quant is None:  # bf16 host tier: exactly full attention over the original tokens
        full_o, _ = R.attend_tokens(_f64(q[0, :, 0]), [np.stack(shadow.k, axis=1)[j] for j in range(H)], [np.stack(shadow.v, axis=1)[j] for j in range(H)], D**-0.5)
        assert np.abs(want_o - full_o).max() < 1e-9
    assert cache.counters.remainder_pairs == H * (n_sealed - 1 - 10)


def test_cache_routes_layers_and_counts_like_the_reference() -> None:
    from lazykv_amd.tiered import TieredCache

    keys, values, gen = _prompt(4, 700)
    cache = TieredCache([(keys.cuda(), values.cuda())] * 3, 6, BS, 1024, dense_layers=1, fetch="zerocopy")
    assert sorted(cache.tiers) == [1, 2] and cache.get_seq_length(1) == 700 and cache.get_seq_length(0) == 700
    k = torch.randn((1, H, 1, D), generator=gen).to(torch.bfloat16).cuda()
    cache.update(k, k, 1)
    assert cache.get_seq_length(1) == 701 and cache.model_kwargs() == {"lazykv_selector": cache}
    q = torch.randn((1, H * G, 1, D), generator=gen).to(torch.bfloat16).cuda()
    dec = cache.select(1, q)
    assert dec.out.shape == (1, H * G, 1, D) and dec.lse.shape == (1, H * G)
    assert cache.select(1, q.expand(1, H * G, 2, D)) is None  # multi-token forwards are not selected
    c = cache.counters
    assert c.selections == 1 and c.selected_pairs == H * 6 and c.zerocopy_bytes == H * 6 * 2 * BS * D * 2


def test_refusals_match_the_reference() -> None:
    """lazykv/tiered.py:245-252,269-270,566-577, lazykv/exact.py:165-176, and
    tests/test_tiered_int8.py:142-143."""
    from lazykv_amd.tiered import ExactTieredCache, TieredCache, TieredLayer, allocate_host_pools

    keys, values, _ = _prompt(5, 300)
    kc, vc = keys.cuda(), values.cuda()
    with pytest.raises(ValueError, match="covers all"):
        TieredLayer(kc, vc, 17, BS, 512)
    with pytest.raises(ValueError, match="needs the model"):
        TieredCache([(kc, vc)] * 2, 4, BS, 512, dense_layers=1, prefetch=True)
    with pytest.raises(ValueError, match="zero-copy"):
        TieredCache([(kc, vc)] * 2, 4, BS, 512, model=object(), dense_layers=1, fetch="zerocopy", prefetch=True)
    with pytest.raises(ValueError, match="zero-copy"):
        TieredCache([(kc, vc)] * 2, 4, BS, 512, dense_layers=1, fetch="zerocopy", record_selection=True)
    with pytest.raises(ValueError, match="outside this path"):
        TieredCache([(kc, vc)] * 2, 4, BS, 512, dense_layers=1, fetch="gather", record_selection=True)
    with pytest.raises(ValueError, match="needs fetch='gather'"):
        TieredCache([(kc, vc)] * 2, 4, BS, 512, dense_layers=1, fetch="runs", quant="int8")
    with pytest.raises(ValueError, match="unknown fetch mode"):
        TieredCache([(kc, vc)] * 2, 4, BS, 512, dense_layers=1, fetch="staged")
    with pytest.raises(ValueError, match="cannot hold a selection"):
        TieredLayer(kc, vc, 4, BS, 512, n_slots=3, fetch="gather")
    with pytest.raises(ValueError, match="zero-copy"):
        ExactTieredCache([(kc, vc)] * 2, 4, BS, 512, dense_layers=1, fetch="zerocopy")
    with pytest.raises(ValueError, match="prefetch"):
        ExactTieredCache([(kc, vc)] * 2, 4, BS, 512, dense_layers=1, prefetch=True)
    wrong = allocate_host_pools(1, H, D, BS, 512)  # a bf16 pool handed to an int8 tier
    with pytest.raises(ValueError, match="host pool must be pinned"):
        TieredLayer(kc, vc, 4, BS, 512, host=wrong[0], quant="int8")
    with pytest.raises(ValueError, match="unknown tier precision"):
        TieredLayer(kc, vc, 4, BS, 512, quant="int4")


def test_graph_replays_equal_the_eager_step() -> None:
    """The per-layer step (bound, select, decode, merge) captured in a HIP graph: every replay,
    with unrelated eager work and synchronisations between replays, equals the eager result."""
    from lazykv_amd import kernels
    from lazykv_amd.tiered import TieredLayer

    keys, values, gen = _prompt(6, 2003)
    layer = TieredLayer(keys.cuda(), values.cuda(), 16, BS, 4096)
    q = torch.randn((H * G, D), generator=gen).to(torch.bfloat16).cuda()
    idx = torch.empty((H, 16), dtype=torch.int32, device="cuda")
    out = torch.empty((H * G, D), dtype=torch.float32, device="cuda")
    lse = torch.empty((H * G,), dtype=torch.float32, device="cuda")
    ws1, ws2 = kernels.Workspace(), kernels.Workspace()
    n_sealed, fill = layer.candidates()
    rank = kernels.PreparedBoundTopk(q, layer.kmin, layer.kmax, 16, cand_offset=1, n_cand=n_sealed - 1, out_idx=idx, ws=ws1)
    dec = kernels.PreparedDecode(q, n_kv=H, block_size=BS, scale=D**-0.5, sel=layer._host_src, idx=idx, sink=layer._pool_src, sink_block=0,
                                 cur=layer._pool_src, cur_block=1, fill=fill, out=out, lse=lse, ws=ws2)
    rank()
    dec()
    torch.cuda.synchronize()
    ref_o, ref_l, ref_i = out.clone(), lse.clone(), idx.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rank()
        dec()
    noise = torch.randn((1 << 20,), device="cuda")
    for i in range(5):
        out.zero_()
        idx.zero_()
        noise.mul_(1.0001).add_(float(i))  # unrelated eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(idx, ref_i) and torch.equal(out, ref_o) and torch.equal(lse, ref_l), i


@pytest.mark.parametrize("fetch", ["zerocopy", "hybrid", "resident"])
def test_decode_steps_never_synchronise_with_the_host(fetch: str) -> None:
    """Selection, decode, append and seal run with torch's sync debug mode set to raise: no step
    waits on the GPU from the host (the reference's rank() copies ids to the host, :387)."""
    from lazykv_amd.tiered import TieredCache

    keys, values, gen = _prompt(8, 700)  # 43 full blocks + 12 tokens: a seal within 4 steps
    cache = TieredCache([(keys.cuda(), values.cuda())] * 2, 8, BS, 1024, dense_layers=0, fetch=fetch)
    q = torch.randn((1, H * G, 1, D), generator=gen).to(torch.bfloat16).cuda()
    kv = torch.randn((1, H, 1, D), generator=gen).to(torch.bfloat16).cuda()
    seals = cache.counters.seals
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        for _ in range(6):
            for layer in (0, 1):
                cache.update(kv, kv, layer)
                decoded = cache.select(layer, q, scaling=D**-0.5)
                assert decoded is not None
    finally:
        torch.cuda.set_sync_debug_mode(0)
    torch.cuda.synchronize()
    assert cache.counters.seals > seals
    assert torch.isfinite(decoded.out.float()).all()
