"""QuestView (rung 5, lazykv/selection.py:90-183) and the caches' byte accounting on the GPU.

QuestView selects over a dense cache resident in HBM: one step is checked against the oracle
(the selected set under the near-tie rule, output and LSE within 2e-3), and a decode through a
transformers Llama stack must equal the resident tier's bit for bit, since both attend the same
blocks of the same values with the same kernels. `stats()` follows lazykv/cache.py:91-115 and
lazykv/tiered.py:841-857.
"""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch

from oracle import reference as R

pytestmark = pytest.mark.gpu

H, G, D, BS = 4, 4, 64, 16


def _kv(seed: int, n: int, dtype: torch.dtype = torch.float16) -> tuple[torch.Tensor, torch.Tensor]:
    gen = torch.Generator().manual_seed(seed)
    scale = 0.5 + 1.5 * torch.rand((1, H, 1, D), generator=gen)
    keys = (torch.randn((1, H, n, D), generator=gen) * scale).to(dtype)
    values = torch.randn((1, H, n, D), generator=gen).to(dtype)
    return keys, values


def test_questview_select_matches_the_oracle() -> None:
    from lazykv_amd.cache import FullGPUCache
    from lazykv_amd.selection import QuestView

    n, k = 63 * BS + 9, 8  # 63 full blocks, a current block of 9 tokens
    keys, values = _kv(1, n)
    full = FullGPUCache.from_kv([(keys.cuda(), values.cuda())], 1024)
    view = QuestView(full, k, BS, dense_layers=0, bound_dtype=torch.float32)
    q = torch.randn((1, H * G, 1, D), generator=torch.Generator().manual_seed(2)).to(torch.float16)
    got = view.select(0, q.cuda())
    torch.cuda.synchronize()
    assert got is not None and view.counters.selections == 1
    chosen = view._idx.cpu().numpy()  # [h, k] ascending block ids
    kf = keys[0].double().numpy()
    kmin, kmax = R.block_minmax(kf[:, : 63 * BS], BS)  # [h, 63, d]
    bound = R.quest_bound(q[0, :, 0].double().numpy(), kmin[:, 1:63], kmax[:, 1:63])  # candidates 1..62
    for j in range(H):
        ok, _ = R.selection_ok(chosen[j] - 1, bound[j], k, abs_err=1e-3)
        assert ok, j
    pf = torch.stack([keys[0], values[0]], dim=1).double().numpy()  # [h, 2, n, d]

    def bkv(j: int, b: int):  # noqa: ANN202
        return pf[j, 0, b * BS : (b + 1) * BS], pf[j, 1, b * BS : (b + 1) * BS]

    ks, vs = R.gathered_tokens(bkv, H, chosen, 0, 63, 9, BS)
    want_o, want_l = R.attend_tokens(q[0, :, 0].double().numpy(), ks, vs, D**-0.5)
    # float16 output: 2e-3 plus one float16 rounding step of the largest output.
    tol = 2e-3 + float(np.abs(want_o).max()) * 2.0**-10
    assert np.abs(got.out.float().cpu().numpy().reshape(H * G, D) - want_o).max() < tol
    assert np.abs(got.lse.cpu().numpy().reshape(-1) - want_l).max() < 2e-3


def test_questview_attends_densely_where_the_reference_does() -> None:
    from lazykv_amd.cache import FullGPUCache
    from lazykv_amd.selection import QuestView

    keys, values = _kv(3, 20 * BS + 4)
    full = FullGPUCache.from_kv([(keys.cuda(), values.cuda())] * 2, 512)
    q = torch.randn((1, H * G, 1, D)).to(torch.float16).cuda()
    view = QuestView(full, 8, BS, dense_layers=1)
    assert view.select(0, q) is None  # a dense layer
    assert view.select(1, torch.randn((1, H * G, 3, D)).to(torch.float16).cuda()) is None  # not a decode step
    assert QuestView(full, 19, BS, dense_layers=0).select(1, q) is None  # the budget covers blocks 1..19
    assert QuestView(full, 18, BS, dense_layers=0).select(1, q) is not None
    assert view.stats() == full.stats() and view.attended_tokens() == 10 * BS
    assert view.policy_name == "quest" and QuestView(full, 8, BS, bound_dtype=torch.float32).policy_name == "quest_float32"


def test_questview_decodes_like_the_resident_tier() -> None:
    """A Llama stack decoding 40 tokens (two blocks complete on the way): QuestView over the dense
    cache and the resident tier over its HBM store give the same log-probabilities bit for bit."""
    from transformers import LlamaConfig, LlamaForCausalLM

    from lazykv_amd.attention import IMPLEMENTATION_NAME, install
    from lazykv_amd.cache import FullGPUCache
    from lazykv_amd.selection import QuestView
    from lazykv_amd.tiered import TieredCache

    install()
    torch.manual_seed(0)
    cfg = LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=3, num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                      vocab_size=512, max_position_embeddings=4096)
    with torch.device("cuda"):
        model = LlamaForCausalLM(copy.deepcopy(cfg))
    model.set_attn_implementation(IMPLEMENTATION_NAME)
    model = model.to(dtype=torch.float16).eval()
    ids = torch.randint(0, cfg.vocab_size, (1, 190), device="cuda", generator=torch.Generator(device="cuda").manual_seed(5))
    prompt = 150
    full = FullGPUCache(cfg.num_hidden_layers, 512)
    with torch.inference_mode():
        first = model(input_ids=ids[:, :prompt], past_key_values=full, use_cache=True).logits[0, -1].float()
    kv = [(layer.keys[:, :, :prompt].clone(), layer.values[:, :, :prompt].clone()) for layer in full.layers]
    caches = {
        "quest": QuestView(full, 3, BS, dense_layers=1, bound_dtype=torch.float32),
        "resident": TieredCache(FullGPUCache.from_kv(kv, 512), 3, BS, 512, dense_layers=1, fetch="resident"),
    }
    rows = {}
    for name, cache in caches.items():
        out = [torch.log_softmax(first, -1)]
        with torch.inference_mode():
            for t in range(prompt, 190):
                logits = model(input_ids=ids[:, t : t + 1], past_key_values=cache, use_cache=True, **cache.model_kwargs()).logits[0, -1]
                out.append(torch.log_softmax(logits.float(), -1))
        rows[name] = torch.stack(out)
    assert caches["quest"].counters.selections == 2 * 40  # two selecting layers, every step
    assert torch.equal(rows["quest"], rows["resident"])


def test_zerocopy_and_hybrid_tiers_decode_like_questview() -> None:
    """After lazykv/tests/test_tiered.py:190-217: the zero-copy tier reads the selected blocks of
    the pinned pool in place (VRAM holds only the sink and the current block), over 40 decode
    steps that cross two seals, and so does the hybrid tier through its HBM slots. Both make the
    same number of selections as QuestView over the dense cache and give the same log-probabilities
    within 2e-2; the zero-copy byte count is the selected pairs times the pair size. Bit identity
    is not asked: a host source is cut into fewer, longer runs per workgroup than an HBM one, so
    the partials are combined in another order."""
    from transformers import LlamaConfig, LlamaForCausalLM

    from lazykv_amd.attention import IMPLEMENTATION_NAME, install
    from lazykv_amd.cache import FullGPUCache
    from lazykv_amd.selection import QuestView
    from lazykv_amd.tiered import TieredCache

    install()
    torch.manual_seed(0)
    cfg = LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=3, num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                      vocab_size=512, max_position_embeddings=4096)
    with torch.device("cuda"):
        model = LlamaForCausalLM(copy.deepcopy(cfg))
    model.set_attn_implementation(IMPLEMENTATION_NAME)
    model = model.to(dtype=torch.float16).eval()
    ids = torch.randint(0, cfg.vocab_size, (1, 190), device="cuda", generator=torch.Generator(device="cuda").manual_seed(5))
    prompt = 150
    full = FullGPUCache(cfg.num_hidden_layers, 512)
    with torch.inference_mode():
        first = model(input_ids=ids[:, :prompt], past_key_values=full, use_cache=True).logits[0, -1].float()
    kv = [(layer.keys[:, :, :prompt].clone(), layer.values[:, :, :prompt].clone()) for layer in full.layers]
    caches = {
        "quest": QuestView(full, 3, BS, dense_layers=1, bound_dtype=torch.float32),
        "zerocopy": TieredCache(FullGPUCache.from_kv(kv, 512), 3, BS, 512, dense_layers=1, fetch="zerocopy"),
        "hybrid": TieredCache(FullGPUCache.from_kv(kv, 512), 3, BS, 512, dense_layers=1, fetch="hybrid"),
    }
    rows = {}
    for name, cache in caches.items():
        out = [torch.log_softmax(first, -1)]
        with torch.inference_mode():
            for t in range(prompt, 190):
                logits = model(input_ids=ids[:, t : t + 1], past_key_values=cache, use_cache=True, **cache.model_kwargs()).logits[0, -1]
                out.append(torch.log_softmax(logits.float(), -1))
        rows[name] = torch.stack(out)
    assert torch.isfinite(rows["quest"]).all()
    for name in ("zerocopy", "hybrid"):
        c = caches[name].counters
        assert c.selections == caches["quest"].counters.selections == 2 * 40, name
        assert c.seals == 2 * 2, name  # blocks 9 and 10 seal in both selecting layers
        assert (rows[name] - rows["quest"]).abs().max().item() < 2e-2, name
    zc = caches["zerocopy"]
    c = zc.counters
    pair = next(iter(zc.tiers.values())).pair_bytes
    assert c.zerocopy_bytes == c.selected_pairs * pair > 0
    for t in zc.tiers.values():
        assert t.n_slots == 0 and t.pool.shape[0] == 2  # VRAM: the sink and the current block


@pytest.mark.parametrize(("fetch", "quant"), [("zerocopy", None), ("zerocopy", "int8"), ("resident", None), ("hybrid", None)])
def test_tier_stats_count_what_vram_does_not_hold(fetch: str, quant: str | None) -> None:
    from lazykv_amd.quant import packed_pair_bytes
    from lazykv_amd.tiered import TieredCache

    keys, values = _kv(4, 40 * BS + 5)
    cache = TieredCache([(keys.cuda(), values.cuda())] * 2, 8, BS, 1024, dense_layers=1, fetch=fetch, quant=quant)
    tier = cache.tiers[1]
    logical = 2 * BS * D * 2
    stored = packed_pair_bytes(BS, D) if quant else logical
    st = cache.stats()
    dense = H * (40 * BS + 5) * D * 2 * 2  # layer 0's keys and values
    if fetch == "resident":
        assert st.host_kv_bytes == 0
    else:
        # Every sealed block but the sink, less those a hybrid tier's slots were seeded with (the k
        # most recent, lazykv/tiered.py:165-168).
        seeded = min(8, tier.n_sealed - 1) if fetch == "hybrid" else 0
        assert st.host_kv_bytes == H * (tier.n_sealed - 1 - seeded) * stored
        assert cache.host_logical_bytes() * stored == st.host_kv_bytes * logical
    assert st.gpu_resident_kv_bytes == dense + tier.gpu_bytes() + tier.metadata_bytes()
    assert cache.host_pinned_bytes() == (0 if tier.host is None else tier.host.numel() * tier.host.element_size())
    if fetch == "hybrid":  # after a step, the k selected blocks of each head are in HBM slots
        q = torch.randn((1, H * G, 1, D)).to(torch.float16).cuda()
        assert cache.select(1, q) is not None
        assert cache.stats().host_kv_bytes == H * (tier.n_sealed - 1 - 8) * stored
