"""Layer-major tiered prefill on the GPU (lazykv/tiered_prefill.py:70-129), after the reference's
tests/test_tiered_prefill.py:48-100: the tier it writes is the one quant.py (or the plain copy)
makes of the chunk-major prefill's KV, bit for bit, and decoding after it gives the same
log-probabilities as decoding after the chunk-major path."""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch

from oracle import reference as R

pytestmark = pytest.mark.gpu

BS = 16
PROMPT = 100  # a partial last chunk and a partial current block (6 full blocks, fill 4)
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
    return torch.randint(0, cfg.vocab_size, (1, PROMPT + 40), device="cuda", generator=gen)


@torch.inference_mode()
def _chunk_major(model, cfg, ids, chunk: int):  # noqa: ANN001, ANN202
    """The path the layer-major prefill replaces: chunk by chunk through every layer into a full cache."""
    from lazykv_amd.cache import FullGPUCache

    full = FullGPUCache(cfg.num_hidden_layers, CAP)
    out = None
    for s in range(0, ids.shape[1], chunk):
        out = model(input_ids=ids[:, s : s + chunk], past_key_values=full, use_cache=True, logits_to_keep=1)
    return out.logits[0, -1].float(), full


@torch.inference_mode()
def _teacher_forced(model, cache, first_logits, cont):  # noqa: ANN001, ANN202
    rows = [torch.log_softmax(first_logits, -1)]
    for t in range(cont.shape[1]):
        out = model(input_ids=cont[:, t : t + 1], past_key_values=cache, use_cache=True, **cache.model_kwargs())
        rows.append(torch.log_softmax(out.logits[0, -1].float(), -1))
    return torch.stack(rows)


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("chunk", [32, 100, 128])
@pytest.mark.parametrize("quant", [None, "int8"])
def test_layer_major_prefill_writes_the_reference_tier(tiny, chunk: int, quant: str | None) -> None:  # noqa: ANN001
    from lazykv_amd.tiered import TieredCache
    from lazykv_amd.tiered_prefill import tiered_prefill

    cfg, model = tiny
    ids = _ids(cfg)
    ref_logits, full = _chunk_major(model, cfg, ids[:, :PROMPT], chunk)
    got = tiered_prefill(model, ids[:, :PROMPT], chunk, K, BS, CAP, dense_layers=1, quant=quant, fetch="zerocopy")
    assert got.chunks == -(-PROMPT // chunk)
    assert torch.equal(got.last_logits, ref_logits)
    nb, fill = divmod(PROMPT, BS)
    d = cfg.head_dim
    for i, t in got.cache.tiers.items():
        assert (t.n_sealed, t.fill, t.length) == (nb, fill, PROMPT)
        kb = _bits(full.layers[i].keys[0, :, :PROMPT])  # [h, n, d] float16 bits
        vb = _bits(full.layers[i].values[0, :, :PROMPT])
        h = kb.shape[0]
        pairs = np.stack([kb[:, : nb * BS].reshape(h, nb, BS, d), vb[:, : nb * BS].reshape(h, nb, BS, d)], axis=2)  # [h, nb, 2, bs, d]
        pairs = pairs.transpose(1, 0, 2, 3, 4)  # [nb, h, 2, bs, d], the host pool's layout
        host = t.host[:nb].numpy()
        if quant == "int8":
            want = R.pack(pairs, "f16")
            assert np.array_equal(host, want)
            keys = R.to_f32(R.unpack(want.reshape(nb * h, -1), BS, d, "f16"), "f16").reshape(nb, h, 2, BS, d)[:, :, 0]
        else:
            assert np.array_equal(host.view(np.uint16), pairs)
            keys = R.to_f32(pairs[:, :, 0], "f16")
        kmin = R.from_f32(keys.min(axis=2), "f16").transpose(1, 0, 2)  # [h, nb, d]
        kmax = R.from_f32(keys.max(axis=2), "f16").transpose(1, 0, 2)
        assert np.array_equal(_bits(t.kmin[0, :, :nb]), kmin)
        assert np.array_equal(_bits(t.kmax[0, :, :nb]), kmax)
        # Sink and current block stay exact in the GPU slots.
        assert np.array_equal(_bits(t.pool[0, :, 0]), kb[:, :BS])
        assert np.array_equal(_bits(t.pool[0, :, 1]), vb[:, :BS])
        assert np.array_equal(_bits(t.pool[1, :, 0, :fill]), kb[:, nb * BS :])
        assert np.array_equal(_bits(t.pool[1, :, 1, :fill]), vb[:, nb * BS :])
    assert torch.equal(got.full.layers[0].keys[:, :, :PROMPT], full.layers[0].keys[:, :, :PROMPT])
    # Decode after it, through seals: the same log-probabilities as the chunk-major path's tier.
    ref = TieredCache(full, K, BS, CAP, dense_layers=1, quant=quant, fetch="zerocopy")
    cont = ids[:, PROMPT : PROMPT + 40]
    a = _teacher_forced(model, ref, ref_logits, cont)
    b = _teacher_forced(model, got.cache, got.last_logits, cont)
    assert torch.isfinite(a).all()
    assert torch.equal(a, b)
    assert got.cache.counters.boundary_d2h_bytes == ref.counters.boundary_d2h_bytes
    assert got.cache.counters.seals == ref.counters.seals > 0


def test_selecting_layers_never_allocate_in_the_full_cache(tiny) -> None:  # noqa: ANN001
    from lazykv_amd.tiered_prefill import tiered_prefill

    cfg, model = tiny
    got = tiered_prefill(model, _ids(cfg)[:, :PROMPT], 32, K, BS, CAP, dense_layers=1, fetch="zerocopy")
    assert got.full.layers[0].is_initialized and got.full.layers[0].get_seq_length() == PROMPT
    assert not any(layer.is_initialized for layer in got.full.layers[1:])
    assert len(got.layer_s) == cfg.num_hidden_layers
    assert len(got.boundary_layer_s) == cfg.num_hidden_layers - 1


def test_prompt_longer_than_capacity_is_refused(tiny) -> None:  # noqa: ANN001
    from lazykv_amd.tiered_prefill import tiered_prefill

    cfg, model = tiny
    with pytest.raises(ValueError, match="exceeds capacity"):
        tiered_prefill(model, _ids(cfg)[:, :PROMPT], 32, K, BS, capacity_tokens=64, dense_layers=1, fetch="zerocopy")


@torch.inference_mode()
def test_layer_major_prefill_32k_1b_shape_writes_quant_py_records() -> None:
    """The 1B-shaped prefill at its real size: 16 layers (hidden 2048, 32/8 heads, d 64), float16
    weights ~ N(0, 0.02) with unit RMSNorm gains, a 32,768-token prompt uniform over 128,256 ids,
    every layer's KV straight into the int8 host tier. In every layer, every one of the 16,384
    (block, head) records equals quant.py's pack of the chunk-major prefill's KV (the oracle's C
    restatement, pinned to quant.py's own golden vectors), and every metadata row the min/max of
    the keys that pack's records unpack to."""
    from transformers import LlamaConfig, LlamaForCausalLM

    from lazykv_amd.attention import IMPLEMENTATION_NAME, install
    from lazykv_amd.cache import FullGPUCache
    from lazykv_amd.tiered_prefill import tiered_prefill

    install()
    n, chunk, bs, d, k = 32768, 4096, 16, 64, 512
    cfg = LlamaConfig(hidden_size=2048, intermediate_size=8192, num_hidden_layers=16, num_attention_heads=32, num_key_value_heads=8, head_dim=d,
                      vocab_size=128256, max_position_embeddings=131072, rope_theta=500000.0, tie_word_embeddings=True)
    torch.manual_seed(0)
    with torch.device("cuda"):
        model = LlamaForCausalLM(cfg)
    model.set_attn_implementation(IMPLEMENTATION_NAME)
    model = model.to(dtype=torch.float16).eval()
    gen = torch.Generator(device="cuda").manual_seed(0)
    ids = torch.randint(0, cfg.vocab_size, (1, n), device="cuda", generator=gen)
    got = tiered_prefill(model, ids, chunk, k, bs, n + 64, dense_layers=0, quant="int8", fetch="zerocopy")
    full = FullGPUCache(cfg.num_hidden_layers, n)
    out = None
    for s in range(0, n, chunk):
        out = model(input_ids=ids[:, s : s + chunk], past_key_values=full, use_cache=True, logits_to_keep=1)
    # Both sides project the same last row onto the 128,256-entry vocabulary. The BLAS library does
    # not promise run-to-run identical bits for that single-row product: after a long test session
    # the two results once differed by one float16 step. So the logits are compared within four
    # float16 steps of the largest; the tier's records below are compared bit for bit.
    want_logits = out.logits[0, -1].float()
    assert (got.last_logits - want_logits).abs().max().item() <= 4 * 2.0**-10 * max(1.0, want_logits.abs().max().item())
    assert not any(layer.is_initialized for layer in got.full.layers)
    from oracle import quant_c

    nb = n // bs
    h = cfg.num_key_value_heads
    for i, t in got.cache.tiers.items():
        assert (t.n_sealed, t.fill) == (nb, 0)
        kb = _bits(full.layers[i].keys[0, :, :n]).reshape(h, nb, bs, d)  # float16 bits
        vb = _bits(full.layers[i].values[0, :, :n]).reshape(h, nb, bs, d)
        pairs = np.stack([kb, vb], axis=2).transpose(1, 0, 2, 3, 4).reshape(nb * h, 2, bs, d)  # the host pool's order
        want = quant_c.pack(pairs, "f16")  # [nb * h, P]
        assert np.array_equal(t.host[:nb].numpy().reshape(nb * h, -1), want), f"layer {i}: records"
        keys = R.to_f32(quant_c.unpack(want, bs, d, "f16")[:, 0], "f16").reshape(nb, h, bs, d)
        assert np.array_equal(_bits(t.kmin[0, :, :nb]), R.from_f32(keys.min(axis=2), "f16").transpose(1, 0, 2)), f"layer {i}: kmin"
        assert np.array_equal(_bits(t.kmax[0, :, :nb]), R.from_f32(keys.max(axis=2), "f16").transpose(1, 0, 2)), f"layer {i}: kmax"
        print(f"layer {i}: {nb * h} records and metadata rows equal the oracle", flush=True)
    print(f"tiered prefill 32K x 16 layers: wall {got.wall_s:.3f} s, tier builds {got.boundary_s * 1e3:.2f} ms in all")
