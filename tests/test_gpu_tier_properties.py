"""Properties of the host tier that the reference's own tests state, restated for the tiered cache here (GPU):
exact-size pinning outside torch's caching host allocator (tests/test_pinned.py:12-40), the int8
host pool narrowing by exactly the record width and the sink staying exact
(tests/test_tiered_int8.py:27-99), `pack` keeping the leading axes (tests/test_quant.py:29-34), and
an int8 tier changing the decode, finitely and not wildly (tests/test_tiered_int8.py:114-135)."""

from __future__ import annotations

import copy

import pytest
import torch

pytestmark = pytest.mark.gpu

H, D, BS = 4, 64, 16


def _host_allocated() -> int:
    return torch.cuda.host_memory_stats().get("allocated_bytes.current", 0)


def test_pinned_empty_is_pinned_at_exactly_its_size_without_the_caching_allocator() -> None:
    from lazykv_amd.pinned import device_view, pinned_empty

    before = _host_allocated()
    t = pinned_empty((3, 5 * 2**20 + 7), torch.uint8)  # not a power of two
    assert t.is_pinned()
    assert t.untyped_storage().nbytes() == 3 * (5 * 2**20 + 7)
    assert _host_allocated() == before  # not rounded up by torch's caching host allocator
    t.random_(0, 255)
    d = torch.empty_like(t, device="cuda")
    d.copy_(t, non_blocking=True)
    torch.cuda.synchronize()
    assert torch.equal(d.cpu(), t)
    assert torch.equal(device_view(t)[1, -64:].cpu(), t[1, -64:])  # the device alias reads the same bytes


@pytest.mark.parametrize("quant", [None, "int8"])
def test_host_pools_use_exact_size_pinning(quant: str | None) -> None:
    from lazykv_amd.quant import packed_pair_bytes
    from lazykv_amd.tiered import allocate_host_pools

    before = _host_allocated()
    pools = allocate_host_pools(2, heads=2, head_dim=16, block_size=8, capacity_tokens=100, quant=quant)
    assert all(p.is_pinned() for p in pools)
    blocks = -(-100 // 8)
    want = blocks * 2 * (packed_pair_bytes(8, 16) if quant else 2 * 8 * 16 * 2)
    assert all(p.untyped_storage().nbytes() == want for p in pools)
    assert _host_allocated() == before


def _prompt(seed: int, n: int) -> tuple[torch.Tensor, torch.Tensor]:
    gen = torch.Generator().manual_seed(seed)
    keys = torch.randn((1, H, n, D), generator=gen).to(torch.float16)
    values = torch.randn((1, H, n, D), generator=gen).to(torch.float16)
    return keys, values


def test_the_int8_host_pool_narrows_by_exactly_the_record_width_and_the_sink_stays_exact() -> None:
    from lazykv_amd.quant import packed_pair_bytes
    from lazykv_amd.tiered import TieredLayer

    keys, values = _prompt(1, 40 * BS + 5)
    exact = TieredLayer(keys.cuda(), values.cuda(), 8, BS, 1024)
    narrow = TieredLayer(keys.cuda(), values.cuda(), 8, BS, 1024, quant="int8")
    torch.cuda.synchronize()
    assert exact.n_sealed == narrow.n_sealed == 40
    assert narrow.host_bytes() * (2 * BS * D * 2) == exact.host_bytes() * packed_pair_bytes(BS, D)
    # Block 0 never leaves HBM, so it is not narrowed (lazykv/tiered.py:200-202).
    assert torch.equal(narrow.pool[0, :, 0].cpu(), keys[0, :, :BS])
    assert torch.equal(narrow.pool[0, :, 1].cpu(), values[0, :, :BS])


def test_pack_keeps_the_leading_axes() -> None:
    from lazykv_amd.quant import pack, packed_pair_bytes, unpack

    x = torch.randn((3, 5, 2, BS, D), dtype=torch.float16, device="cuda")
    rec = pack(x)
    assert rec.shape == (3, 5, packed_pair_bytes(BS, D)) and rec.dtype == torch.uint8
    back = unpack(rec.reshape(15, -1), BS, D, torch.float16).reshape(x.shape)
    level = (x.float().amax(dim=3, keepdim=True) - x.float().amin(dim=3, keepdim=True)) / 255  # key groups: per channel
    assert ((back[:, :, 0].float() - x[:, :, 0].float()).abs() <= level[:, :, 0] + 2e-3).all()


def test_int8_decode_differs_from_the_exact_tier_but_not_wildly() -> None:
    """A transformers Llama stack decoding 40 tokens: the int8 tier moves the logits, finitely,
    by a small fraction of their spread on average (where a different block gets selected the
    move can be larger; the reference bounds it by the spread)."""
    from transformers import LlamaConfig, LlamaForCausalLM

    from lazykv_amd.attention import IMPLEMENTATION_NAME, install
    from lazykv_amd.tiered_prefill import tiered_prefill

    install()
    torch.manual_seed(0)
    cfg = LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=4, num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                      vocab_size=512, max_position_embeddings=4096)
    with torch.device("cuda"):
        model = LlamaForCausalLM(copy.deepcopy(cfg))
    model.set_attn_implementation(IMPLEMENTATION_NAME)
    model = model.to(dtype=torch.float16).eval()
    gen = torch.Generator(device="cuda").manual_seed(11)
    ids = torch.randint(0, cfg.vocab_size, (1, 200), device="cuda", generator=gen)
    logits = {}
    for quant in (None, "int8"):
        got = tiered_prefill(model, ids[:, :160], 32, 3, BS, 512, dense_layers=1, quant=quant, fetch="zerocopy")
        rows = [got.last_logits.float()]
        with torch.inference_mode():
            for t in range(160, 200):
                out = model(input_ids=ids[:, t : t + 1], past_key_values=got.cache, use_cache=True, **got.cache.model_kwargs())
                rows.append(out.logits[0, -1].float())
        logits[quant] = torch.stack(rows)
    ref, got = logits[None], logits["int8"]
    assert torch.isfinite(got).all()
    assert not torch.equal(got, ref)  # the tier does quantise
    diff, spread = (got - ref).abs(), ref.std()
    assert diff.mean() < 0.02 * spread
    assert diff.max() < spread
