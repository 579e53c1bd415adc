"""Multi-token forwards through the tier (row a14), after the reference's tests/test_multiturn.py:146-200
and lazykv/tiered.py:316-351,649-663: a user's turn attends densely to the layer's whole KV and then
enters the tier exactly as token-by-token appends would; a session fed turns this way decodes like
QuestView over the dense cache."""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch

from oracle import reference as R

pytestmark = pytest.mark.gpu

H, D = 2, 64


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _kv(seed: int, length: int, dtype: torch.dtype) -> torch.Tensor:
    gen = torch.Generator().manual_seed(seed)
    return (torch.randn((2, 1, H, length, D), generator=gen) * 1.5).to(dtype).cuda()


@pytest.mark.parametrize("pieces", [[1], [5, 3], [8], [13, 8, 1, 20], [3, 64, 2], [40]])
@pytest.mark.parametrize(("fetch", "quant"), [("zerocopy", None), ("zerocopy", "int8"), ("resident", None), ("hybrid", None)])
def test_extend_leaves_the_same_state_as_appending_token_by_token(pieces: list[int], fetch: str, quant: str | None) -> None:
    """tests/test_multiturn.py:184-200: records, metadata, the current block, the counters and the
    HBM store equal, bit for bit, those of a tier fed the same tokens one `append` at a time."""
    from lazykv_amd.tiered import TierCounters, TieredLayer

    bs, prompt = 8, 45
    kv = _kv(2, prompt + sum(pieces), torch.bfloat16)
    a = TieredLayer(kv[0, :, :, :prompt], kv[1, :, :, :prompt], 3, bs, 256, quant=quant, fetch=fetch)
    b = TieredLayer(kv[0, :, :, :prompt], kv[1, :, :, :prompt], 3, bs, 256, quant=quant, fetch=fetch)
    ca, cb = TierCounters(), TierCounters()
    pos = prompt
    for m in pieces:
        a.extend(kv[0, :, :, pos : pos + m], kv[1, :, :, pos : pos + m], ca)
        for j in range(pos, pos + m):
            b.append(kv[0, :, :, j : j + 1], kv[1, :, :, j : j + 1], cb)
        pos += m
    torch.cuda.synchronize()
    assert (a.n_sealed, a.fill, a.length) == (b.n_sealed, b.fill, b.length) == (a.n_sealed, a.fill, pos)
    assert 1 <= a.fill <= bs and a.n_sealed * bs + a.fill == pos  # lazy sealing: the last block stays current
    if a.host is not None:
        assert torch.equal(a.host[: a.n_sealed], b.host[: b.n_sealed])
    if a.store is not None:
        assert torch.equal(a.store[: a.n_sealed], b.store[: b.n_sealed])
    assert torch.equal(a.kmin[:, :, : a.n_sealed], b.kmin[:, :, : b.n_sealed])
    assert torch.equal(a.kmax[:, :, : a.n_sealed], b.kmax[:, :, : b.n_sealed])
    assert torch.equal(a.pool[1, :, :, : a.fill], b.pool[1, :, :, : b.fill])
    assert (ca.seals, ca.seal_bytes) == (cb.seals, cb.seal_bytes)
    # And against the oracle: every sealed block is the stored form of the tokens in order.
    n = a.n_sealed
    pairs = np.stack([_bits(kv[0, 0, :, : n * bs]).reshape(H, n, bs, D), _bits(kv[1, 0, :, : n * bs]).reshape(H, n, bs, D)], axis=2).transpose(1, 0, 2, 3, 4)
    if quant == "int8":
        assert np.array_equal(a.host[:n].numpy(), R.pack(pairs, "bf16"))
    elif a.host is not None:
        assert np.array_equal(a.host[:n].view(torch.int16).numpy().view(np.uint16), pairs)


@pytest.mark.parametrize(("fetch", "quant"), [("zerocopy", None), ("zerocopy", "int8"), ("resident", None), ("hybrid", None)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_dense_kv_is_the_layers_whole_kv_then_the_new_tokens(fetch: str, quant: str | None, dtype: torch.dtype) -> None:
    """lazykv/tiered.py:334-351: sealed blocks (read in place from the host pool, or from the HBM
    store), the current block's tokens, then the forward's own KV, in token order. A model-dtype tier
    returns the original bits; an int8 tier returns the records dequantised as quant.py unpacks them
    (the reference refuses dense ingestion there), except block 0, the exact sink."""
    from lazykv_amd.tiered import DenseScratch, TieredLayer

    bs, prompt, new = 16, 16 * 37 + 9, 23
    kv = _kv(3, prompt + new, dtype)
    layer = TieredLayer(kv[0, :, :, :prompt], kv[1, :, :, :prompt], 4, bs, 1024, quant=quant, fetch=fetch)
    scratch = DenseScratch()
    k, v, moved = layer.dense_kv(kv[0, :, :, prompt:], kv[1, :, :, prompt:], scratch)
    torch.cuda.synchronize()
    assert k.shape == v.shape == (1, H, prompt + new, D)
    n = layer.n_sealed
    assert moved == (0 if fetch == "resident" else n * H * layer.pair_bytes)
    want_k, want_v = _bits(kv[0, 0]), _bits(kv[1, 0])  # [h, L, d]
    if quant == "int8":
        tag = "bf16" if dtype == torch.bfloat16 else "f16"
        pairs = np.stack([want_k[:, : n * bs].reshape(H, n, bs, D), want_v[:, : n * bs].reshape(H, n, bs, D)], axis=2).transpose(1, 0, 2, 3, 4)
        deq = R.unpack(R.pack(pairs, tag).reshape(n * H, -1), bs, D, tag).reshape(n, H, 2, bs, D)  # model-dtype bits
        want_k = want_k.copy()
        want_v = want_v.copy()
        want_k[:, bs : n * bs] = deq[1:, :, 0].transpose(1, 0, 2, 3).reshape(H, (n - 1) * bs, D)
        want_v[:, bs : n * bs] = deq[1:, :, 1].transpose(1, 0, 2, 3).reshape(H, (n - 1) * bs, D)
    assert np.array_equal(_bits(k[0]), want_k)
    assert np.array_equal(_bits(v[0]), want_v)
    # A second, shorter call reuses the scratch and returns exactly its own length.
    k2, _, _ = layer.dense_kv(kv[0, :, :, prompt : prompt + 1], kv[1, :, :, prompt : prompt + 1], scratch)
    assert k2.shape[2] == prompt + 1 and k2.data_ptr() == k.data_ptr()


@pytest.fixture(scope="module")
def tiny():  # noqa: ANN201
    from transformers import LlamaConfig, LlamaForCausalLM

    from lazykv_amd.attention import IMPLEMENTATION_NAME, install

    install()
    torch.manual_seed(0)
    cfg = LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=3, num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                      vocab_size=512, max_position_embeddings=4096)
    with torch.device("cuda"):
        model = LlamaForCausalLM(copy.deepcopy(cfg))
    model.set_attn_implementation(IMPLEMENTATION_NAME)
    return cfg, model.to(dtype=torch.float16).eval()


def _session(model, cache, first_logits, ids, turns, answer, turn_chunk):  # noqa: ANN001, ANN202
    """Teacher-forced multi-turn session: each turn's tokens in forwards of at most `turn_chunk`
    tokens, then `answer` decode steps. Returns the log-probabilities of every decode step."""
    rows = [torch.log_softmax(first_logits, -1)]
    pos = 0
    with torch.inference_mode():
        for n_turn in turns:
            for a in range(0, n_turn, turn_chunk):
                b = min(n_turn, a + turn_chunk)
                out = model(input_ids=ids[:, pos + a : pos + b], past_key_values=cache, use_cache=True, **cache.model_kwargs())
            rows.append(torch.log_softmax(out.logits[0, -1].float(), -1))
            pos += n_turn
            for _ in range(answer):
                out = model(input_ids=ids[:, pos : pos + 1], past_key_values=cache, use_cache=True, **cache.model_kwargs())
                rows.append(torch.log_softmax(out.logits[0, -1].float(), -1))
                pos += 1
    return torch.stack(rows), pos


@pytest.mark.parametrize("turn_chunk", [16, 4096])  # 16: a turn spans several forwards and seals blocks mid-turn
@pytest.mark.parametrize("fetch", ["resident", "zerocopy", "hybrid"])
def test_tier_ingests_turns_densely_like_questview(tiny, turn_chunk: int, fetch: str) -> None:  # noqa: ANN001
    """tests/test_multiturn.py:146-179: turns of 30, 17 and 41 tokens, each followed by 6 decode
    steps. Against QuestView over the dense cache (float32 ranking on both sides): the tier ends up
    holding the dense cache's KV bit for bit, and the log-probabilities are equal bit for bit for the
    HBM-resident tier, within 2e-2 for the tiers that read the host pool (a host source is cut into
    fewer partials per head, so sums run in another order)."""
    from lazykv_amd.cache import FullGPUCache
    from lazykv_amd.selection import QuestView
    from lazykv_amd.tiered import TieredCache

    cfg, model = tiny
    prompt, turns, answer, bs, k = 100, [30, 17, 41], 6, 8, 3
    ids = torch.randint(0, cfg.vocab_size, (1, prompt + sum(turns) + answer * len(turns)), device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(11))
    full = FullGPUCache(cfg.num_hidden_layers, 512)
    with torch.inference_mode():
        first = model(input_ids=ids[:, :prompt], past_key_values=full, use_cache=True).logits[0, -1].float()
    kv = [(layer.keys[:, :, :prompt].clone(), layer.values[:, :, :prompt].clone()) for layer in full.layers]
    quest = QuestView(full, k, bs, dense_layers=1, bound_dtype=torch.float32)
    ref, end = _session(model, quest, first, ids[:, prompt:], turns, answer, turn_chunk)
    tier = TieredCache(FullGPUCache.from_kv(kv, 512), k, bs, 512, dense_layers=1, fetch=fetch)
    got, _ = _session(model, tier, first, ids[:, prompt:], turns, answer, turn_chunk)
    torch.cuda.synchronize()
    assert torch.isfinite(ref).all()
    if fetch == "resident":
        assert torch.equal(got, ref)
    else:
        assert (got - ref).abs().max().item() < 2e-2
    n = prompt + end
    assert tier.get_seq_length(1) == full.layers[1].get_seq_length() == n
    for i, t in tier.tiers.items():
        b = t.n_sealed
        held = t.store[:b] if t.store is not None else t.host[:b].cuda()
        host_k = held[:, :, 0].permute(1, 0, 2, 3).reshape(1, t.h, b * t.bs, t.d)
        keys = torch.cat([host_k, t.pool[1, :, 0, : t.fill].unsqueeze(0)], dim=2)
        assert torch.equal(keys, full.layers[i].keys[:, :, :n]), i
    c = tier.counters
    # A one-token forward (a turn's 17 = 16 + 1 split) is an ordinary decode step, as in the reference.
    dense = sum(min(turn_chunk, f - o) for f in turns for o in range(0, f, turn_chunk) if f - o > 1)
    assert c.ingest_tokens == dense * (cfg.num_hidden_layers - 1)
    assert c.ingest_forwards == sum(1 for f in turns for o in range(0, f, turn_chunk) if f - o > 1) * (cfg.num_hidden_layers - 1)
    assert (c.ingest_h2d_bytes > 0) == (fetch != "resident")


def test_int8_tier_ingests_turns_and_keeps_decoding(tiny) -> None:  # noqa: ANN001
    """The int8 tier, which the reference refuses for dense ingestion: a turn attends over the
    dequantised sealed blocks, the tier ends up in the state per-token appends give, and decode after
    it stays close to QuestView over the exact cache (the int8 rounding is all that differs)."""
    from lazykv_amd.cache import FullGPUCache
    from lazykv_amd.selection import QuestView
    from lazykv_amd.tiered import TieredCache

    cfg, model = tiny
    prompt, turns, answer, bs, k = 100, [30, 41], 4, 8, 3
    ids = torch.randint(0, cfg.vocab_size, (1, prompt + sum(turns) + answer * len(turns)), device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(12))
    full = FullGPUCache(cfg.num_hidden_layers, 512)
    with torch.inference_mode():
        first = model(input_ids=ids[:, :prompt], past_key_values=full, use_cache=True).logits[0, -1].float()
    kv = [(layer.keys[:, :, :prompt].clone(), layer.values[:, :, :prompt].clone()) for layer in full.layers]
    quest = QuestView(full, k, bs, dense_layers=1, bound_dtype=torch.float32)
    ref, _ = _session(model, quest, first, ids[:, prompt:], turns, answer, 4096)
    tier = TieredCache(FullGPUCache.from_kv(kv, 512), k, bs, 512, dense_layers=1, quant="int8", fetch="zerocopy")
    got, _ = _session(model, tier, first, ids[:, prompt:], turns, answer, 4096)
    assert torch.isfinite(got).all()
    assert (got - ref).abs().max().item() < 0.25
    assert tier.counters.ingest_forwards == len(turns) * (cfg.num_hidden_layers - 1)
