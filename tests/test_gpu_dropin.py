"""The reference's callers, with their own arguments, against this library's tier.

Every cache here is built with exactly the keyword set a reference caller passes: `build_cache`
(lazykv/sweep.py:178-187) for the zero-copy tier, rung 6 with and without spare slots
(`n_slots_for`, lazykv/sweep.py:120-125), the int8 tier (fetch="gather") and rung 9
(`mirrors`, `threads`); and `snapshot.restore` as lazykv/snapshot.py:184-196,275 and
tests/test_snapshot.py:56-67 call it (`fetch="gather"`, `stages`, `unbuffered`). The attention
seam is registered as the reference's fixtures register it: install("cudnn_bucketed", ...,
bucket=64) (tests/test_tiered.py:25).

Each decodes 20 tokens of a Llama stack, crossing a seal, and is held to the existing bars:
- the zero-copy tier against QuestView over the dense cache: log-probabilities within 2e-2;
- the rung-6 fetches against the zero-copy tier over the same tokens: bit for bit (the device
  hybrid reads each pair from its slot or in place, and folds it exactly as the zero-copy read);
- the int8 "gather" tier against the int8 zero-copy tier: bit for bit;
- rung 9 against dense attention over the whole cache: log-probabilities within 2e-2;
- a restored session against the saved one: bit for bit.
"""

from __future__ import annotations

import copy

import pytest
import torch

pytestmark = pytest.mark.gpu

BS = 16
K = 3
PROMPT = 150  # 9 full blocks and 6 tokens; decode crosses the seal of block 9 at token 160
STEPS = 20
CAP = 512


@pytest.fixture(scope="module")
def tiny():  # noqa: ANN201
    from transformers import LlamaConfig, LlamaForCausalLM

    from lazykv_amd.attention import IMPLEMENTATION_NAME, current_strategy, install

    torch.manual_seed(0)
    cfg = LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=4, num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                      vocab_size=512, max_position_embeddings=4096)
    chosen, checks = install("cudnn_bucketed", cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, bucket=64)
    assert chosen == "cudnn_bucketed" and len(checks) == 1 and checks[0].ok, checks
    assert current_strategy() == ("cudnn_bucketed", 64)
    with torch.device("cuda"):
        model = LlamaForCausalLM(copy.deepcopy(cfg))
    model.set_attn_implementation(IMPLEMENTATION_NAME)
    model = model.to(dtype=torch.float16).eval()
    ids = torch.randint(0, cfg.vocab_size, (1, PROMPT + STEPS), device="cuda", generator=torch.Generator(device="cuda").manual_seed(5))
    return cfg, model, ids


@torch.inference_mode()
def _prefilled(model, ids):  # noqa: ANN001, ANN202
    """A full cache after the prompt, as build_cache receives it, and the first next-token logits."""
    from lazykv_amd.cache import FullGPUCache

    full = FullGPUCache(model.config.num_hidden_layers, CAP)
    logits = model(input_ids=ids[:, :PROMPT], past_key_values=full, use_cache=True).logits[0, -1].float()
    return full, logits


@torch.inference_mode()
def _decode(model, cache, ids, first_logits) -> torch.Tensor:  # noqa: ANN001
    rows = [torch.log_softmax(first_logits, -1)]
    for t in range(PROMPT, PROMPT + STEPS - 1):
        kwargs = cache.model_kwargs() if hasattr(cache, "model_kwargs") else {}  # a plain full cache has no selector
        out = model(input_ids=ids[:, t : t + 1], past_key_values=cache, use_cache=True, **kwargs)
        rows.append(torch.log_softmax(out.logits[0, -1].float(), -1))
    return torch.stack(rows)


def _build(kind, full, k, block_size, model, quant, fetch, n_slots, exact=False):  # noqa: ANN001, ANN202
    """lazykv/sweep.py:178-187, argument for argument, with host=None (no preallocated pools) and
    instrument=False."""
    extra = {"mirrors": None, "threads": 8} if exact else {}
    return kind(
        full, k, block_size, full.max_len, model=model, prefetch=False,
        host_pools=None, instrument=False, n_slots=n_slots,
        fetch=fetch, stages=None, quant=quant, **extra,
    )


def test_sweep_keyword_sets_build_and_decode(tiny) -> None:  # noqa: ANN001
    from lazykv_amd.selection import QuestView
    from lazykv_amd.tiered import ExactTieredCache, TieredCache

    cfg, model, ids = tiny
    rows, caches = {}, {}

    def run(name, make) -> None:  # noqa: ANN001
        full, logits = _prefilled(model, ids)
        caches[name] = make(full)
        rows[name] = _decode(model, caches[name], ids, logits)

    # build_cache leaves dense_layers at its default, Quest's first two layers (lazykv/selection.py:35).
    run("quest", lambda full: QuestView(full, K, BS, bound_dtype=torch.float32))
    run("zerocopy", lambda full: _build(TieredCache, full, K, BS, model, None, "zerocopy", 0))
    run("runs", lambda full: _build(TieredCache, full, K, BS, model, None, "runs", K))  # spare 0
    run("gather_spare", lambda full: _build(TieredCache, full, K, BS, model, None, "gather", 2 * K))  # spare 1.0
    run("int8_gather", lambda full: _build(TieredCache, full, K, BS, model, "int8", "gather", K))
    run("int8_zerocopy", lambda full: TieredCache(full, K, BS, full.max_len, model=model, fetch="zerocopy", quant="int8"))
    run("exact", lambda full: _build(ExactTieredCache, full, K, BS, model, None, "runs", K, exact=True))
    run("dense", lambda full: full)

    assert (rows["zerocopy"] - rows["quest"]).abs().max().item() < 2e-2
    assert torch.equal(rows["runs"], rows["zerocopy"])
    assert torch.equal(rows["gather_spare"], rows["zerocopy"])
    assert torch.equal(rows["int8_gather"], rows["int8_zerocopy"])
    assert (rows["exact"] - rows["dense"]).abs().max().item() < 2e-2
    assert (rows["exact"] - rows["zerocopy"]).abs().max().item() > 0  # the exact tier attends more than the selection

    # What build_cache's callers read back (lazykv/sweep.py:222-238).
    for name in ("zerocopy", "runs", "gather_spare", "int8_gather", "exact"):
        cache = caches[name]
        facts = cache.counters_dict()
        for key in ("host_select_s", "hit_pairs", "fetched_pairs", "thrash_pairs", "zerocopy_bytes", "seals", "fetched_pairs_per_step"):
            assert key in facts, (name, key)
        assert cache.k_blocks == K and cache.block_size == BS and cache.dense_layers == 2
        assert cache.stats().host_kv_bytes >= 0 and cache.host_logical_bytes() >= 0
        assert cache.counters.selections == (cfg.num_hidden_layers - 2) * (STEPS - 1), name
        assert cache.counters.seals == cfg.num_hidden_layers - 2, name  # block 9 seals once per selecting layer
    assert caches["zerocopy"].n_slots == 0 and caches["runs"].n_slots == K and caches["gather_spare"].n_slots == 2 * K
    assert caches["runs"].policy_name == "tiered_sync" and caches["int8_gather"].policy_name == "tiered_int8"
    ex = caches["exact"].exact_counters_dict()
    assert ex["merges"] == (cfg.num_hidden_layers - 2) * (STEPS - 1) and ex["threads"] == 8 and ex["mirror_bytes"] == 0
    # Spare slots keep blocks the last selection did not name; exactly K slots hold exactly it.
    for layer, tier in caches["gather_spare"].tiers.items():
        held = (tier.res.slot_block >= 0).sum(dim=1)
        assert (held > K).all(), layer
    for layer, tier in caches["runs"].tiers.items():
        assert ((tier.res.slot_block >= 0).sum(dim=1) == K).all(), layer


@pytest.mark.parametrize("unbuffered", [False, True])
@pytest.mark.parametrize("rebuild", ["store", "boundary"])
def test_restore_with_the_reference_callers_arguments(tiny, tmp_path, unbuffered: bool, rebuild: str) -> None:  # noqa: ANN001
    """tests/test_snapshot.py:56-67: a rung-6 session ("gather") saved mid-decode and restored with
    restore(path, K, CAP, n_layers, model=model, fetch="gather", unbuffered=..., rebuild=...)
    continues bit for bit; the restored tiers' slots are seeded with the most recent blocks, as the
    reference's from_store seeds them."""
    from lazykv_amd import snapshot
    from lazykv_amd.tiered import TieredCache

    cfg, model, ids = tiny
    full, logits = _prefilled(model, ids)
    cache = TieredCache(full, K, BS, CAP, model=model, dense_layers=1, fetch="gather")
    mid = 7
    with torch.inference_mode():
        for t in range(PROMPT, PROMPT + mid):
            logits = model(input_ids=ids[:, t : t + 1], past_key_values=cache, use_cache=True, **cache.model_kwargs()).logits[0, -1].float()
    path = tmp_path / "session.lkv"
    snapshot.save(cache, logits, path)
    restored, logits2, stats = snapshot.restore(path, K, CAP, cfg.num_hidden_layers, model=model, fetch="gather", stages=None,
                                                unbuffered=unbuffered, rebuild=rebuild)
    assert torch.equal(logits, logits2) and stats.bytes_read > 0
    for tier in restored.tiers.values():
        assert tier.res is not None and tier.n_slots == K
        seeded = min(K, tier.n_sealed - 1)
        want = torch.arange(tier.n_sealed - seeded, tier.n_sealed, dtype=torch.int32, device="cuda")
        assert torch.equal(tier.res.slot_block[:, :seeded], want.expand(tier.h, -1))
        # the seeded slots hold the blocks' pairs exactly
        assert torch.equal(tier.res.slots[:seeded].cpu(), tier.host[tier.n_sealed - seeded : tier.n_sealed])
    a, b = [], []
    with torch.inference_mode():
        for t in range(PROMPT + mid, PROMPT + STEPS):
            tok = ids[:, t : t + 1]
            a.append(torch.log_softmax(model(input_ids=tok, past_key_values=cache, use_cache=True, **cache.model_kwargs()).logits[0, -1].float(), -1))
            b.append(torch.log_softmax(model(input_ids=tok, past_key_values=restored, use_cache=True, **restored.model_kwargs()).logits[0, -1].float(), -1))
    assert torch.equal(torch.stack(a), torch.stack(b))


def test_seeded_int8_slots_hold_the_dequantised_records(tiny) -> None:  # noqa: ANN001
    """An int8 "gather" tier seeds its slots with the most recent blocks as the decode reads them:
    the records dequantised (the reference seeds from the dequantised keys, lazykv/tiered.py:176-194),
    which the oracle's unpack reproduces bit for bit."""
    import numpy as np

    from lazykv_amd.tiered import TieredCache
    from oracle import reference as R

    cfg, model, ids = tiny
    full, _ = _prefilled(model, ids)
    cache = TieredCache(full, K, BS, CAP, model=model, dense_layers=1, fetch="gather", quant="int8", n_slots=K + 2)
    torch.cuda.synchronize()
    for tier in cache.tiers.values():
        seeded = min(tier.n_slots, tier.n_sealed - 1)
        first = tier.n_sealed - seeded
        recs = tier.host[first : tier.n_sealed].numpy().reshape(seeded * tier.h, -1)
        want = R.unpack(recs, BS, tier.d, "f16").reshape(seeded, tier.h, 2, BS, tier.d)
        got = tier.res.slots[:seeded].cpu().view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(got, want)
        order = tier.res.order.cpu().numpy()
        # the empty slots come first in the use order, then the seeded ones
        assert order[0].tolist() == list(range(seeded, tier.n_slots)) + list(range(seeded))
