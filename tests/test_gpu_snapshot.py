"""Snapshots on the GPU (lazykv/snapshot.py), after the reference's tests/test_snapshot.py:45-115:
a session saved mid-decode and restored continues bit-identically, the restored tier equals the
saved one, and the int8 tier is refused."""

from __future__ import annotations

import copy

import pytest
import torch

pytestmark = pytest.mark.gpu

BS = 16
PROMPT = 100  # 6 full blocks and 4 tokens in the current block
K = 3
CAP = 512


@pytest.fixture(scope="module")
def tiny():  # noqa: ANN201
    from transformers import LlamaConfig, LlamaForCausalLM

    from lazykv_amd.attention import IMPLEMENTATION_NAME, install

    install()
    torch.manual_seed(0)
    cfg = LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=4, num_attention_heads=4, num_key_value_heads=2, head_dim=64, vocab_size=512, max_position_embeddings=4096)
    with torch.device("cuda"):
        model = LlamaForCausalLM(copy.deepcopy(cfg))
    model.set_attn_implementation(IMPLEMENTATION_NAME)
    return cfg, model.to(dtype=torch.float16).eval()


def _ids(cfg):  # noqa: ANN001, ANN202
    gen = torch.Generator(device="cuda").manual_seed(7)
    return torch.randint(0, cfg.vocab_size, (1, PROMPT + 60), device="cuda", generator=gen)


@torch.inference_mode()
def _step(model, cache, tok):  # noqa: ANN001, ANN202
    out = model(input_ids=tok, past_key_values=cache, use_cache=True, **cache.model_kwargs())
    return out.logits[0, -1].float()


@pytest.mark.parametrize("mid", [0, 9, 30])
@pytest.mark.parametrize("rebuild", ["store", "boundary"])
def test_restored_session_continues_bit_identically(tiny, tmp_path, mid: int, rebuild: str) -> None:  # noqa: ANN001
    from lazykv_amd import snapshot
    from lazykv_amd.tiered_prefill import tiered_prefill

    cfg, model = tiny
    ids = _ids(cfg)
    got = tiered_prefill(model, ids[:, :PROMPT], 32, K, BS, CAP, dense_layers=1, fetch="zerocopy")
    cache, logits = got.cache, got.last_logits
    for t in range(mid):
        logits = _step(model, cache, ids[:, PROMPT + t : PROMPT + t + 1])
    path = tmp_path / "session.lkv"
    stats = snapshot.save(cache, logits, path)
    assert stats.bytes_written == path.stat().st_size and stats.bytes_written % snapshot.ALIGN == 0
    header, base = snapshot.read_header(path)
    assert header["length"] == PROMPT + mid and base % snapshot.ALIGN == 0
    restored, logits2, rstats = snapshot.restore(path, K, CAP, cfg.num_hidden_layers, fetch="zerocopy", rebuild=rebuild)
    assert rstats.bytes_read > 0
    assert torch.equal(logits, logits2)
    for i, t in cache.tiers.items():
        r = restored.tiers[i]
        if rebuild == "store" or t.fill < BS:
            assert (r.n_sealed, r.fill, r.length) == (t.n_sealed, t.fill, t.length)
        assert torch.equal(r.host[: r.n_sealed], t.host[: t.n_sealed])
        assert torch.equal(r.kmin[:, :, : r.n_sealed], t.kmin[:, :, : t.n_sealed])
        assert torch.equal(r.kmax[:, :, : r.n_sealed], t.kmax[:, :, : t.n_sealed])
        assert torch.equal(r.pool[0], t.pool[0])
        assert torch.equal(r.pool[1, :, :, : t.fill], t.pool[1, :, :, : t.fill])
    assert torch.equal(restored.full.layers[0].keys[:, :, : PROMPT + mid], cache.full.layers[0].keys[:, :, : PROMPT + mid])
    # Both sessions continue through seals with the same log-probabilities, bit for bit.
    a, b = [], []
    for t in range(mid, mid + 24):
        tok = ids[:, PROMPT + t : PROMPT + t + 1]
        a.append(torch.log_softmax(_step(model, cache, tok), -1))
        b.append(torch.log_softmax(_step(model, restored, tok), -1))
    assert torch.equal(torch.stack(a), torch.stack(b))


def test_snapshot_refuses_the_int8_tier(tiny, tmp_path) -> None:  # noqa: ANN001
    from lazykv_amd import snapshot
    from lazykv_amd.tiered_prefill import tiered_prefill

    cfg, model = tiny
    got = tiered_prefill(model, _ids(cfg)[:, :PROMPT], 32, K, BS, CAP, dense_layers=1, quant="int8", fetch="zerocopy")
    with pytest.raises(ValueError, match="int8"):
        snapshot.save(got.cache, got.last_logits, tmp_path / "x.lkv")
