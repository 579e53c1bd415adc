"""Pinning the oracle (CPU): golden vectors, the reference tests' known answers, closed forms, brute force.

Every check here is chosen so that a plausible mistake in the restatement (a dropped term, a
swapped operand, a wrong rounding rule, an off-by-one in a mask) fails it.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest

from oracle import quant_c
from oracle import reference as R

GOLDEN = Path(__file__).resolve().parent / "golden" / "quant_vectors.npz"


def _cases():
    g = np.load(GOLDEN)
    out = []
    for key in sorted(k[: -len("_in")] for k in g.files if k.endswith("_in")):
        dt, bs, d = key.split("_")
        out.append((key, dt, int(bs[2:]), int(d[1:])))
    return out


# -- int8 records: golden vectors written by the reference's own quant.py -----------------------


@pytest.mark.parametrize(("key", "dt", "bs", "d"), _cases())
def test_numpy_pack_unpack_match_the_reference_bytes(key: str, dt: str, bs: int, d: int) -> None:
    g = np.load(GOLDEN)
    x = g[f"{key}_in"]
    assert np.array_equal(R.pack(x, dt), g[f"{key}_packed"])
    assert np.array_equal(R.unpack(g[f"{key}_packed"], bs, d, dt), g[f"{key}_unpacked"])


@pytest.mark.parametrize(("key", "dt", "bs", "d"), _cases())
def test_c_pack_unpack_match_the_reference_bytes(key: str, dt: str, bs: int, d: int) -> None:
    g = np.load(GOLDEN)
    assert np.array_equal(quant_c.pack(g[f"{key}_in"], dt), g[f"{key}_packed"])
    assert np.array_equal(quant_c.unpack(g[f"{key}_packed"], bs, d, dt), g[f"{key}_unpacked"])


def test_record_width_formula_matches_the_reference_fixture() -> None:
    g = np.load(GOLDEN)
    for bs, d, p in g["packed_pair_bytes"]:
        assert R.packed_pair_bytes(int(bs), int(d)) == p
    # The record sizes of the workloads' geometries: P(16,64), P(16,128).
    assert R.packed_pair_bytes(16, 64) == 2368 and R.packed_pair_bytes(16, 128) == 4672


def test_record_is_half_a_bf16_pair_plus_scales() -> None:
    """tests/test_quant.py:21-27 of the reference, at its BS=D=64 geometry."""
    width, payload = R.packed_pair_bytes(64, 64), 2 * 64 * 64
    assert width == payload + 2 * 2 * (64 + 64)
    assert 0.5 < width / (payload * 2) < 0.55


def _bf16(x: np.ndarray) -> np.ndarray:
    return R.from_f32(x.astype(np.float32), "bf16")


def test_roundtrip_error_is_within_one_level() -> None:
    """tests/test_quant.py:36-47: one level of the group's range, plus the scale's and output's rounding."""
    rng = np.random.default_rng(0)
    x = _bf16(rng.standard_normal((4, 2, 64, 64)) * 3)
    back = R.to_f32(R.unpack(R.pack(x, "bf16"), 64, 64, "bf16"), "bf16").reshape(x.shape)
    xf = R.to_f32(x, "bf16")
    k_range = (xf[:, 0].max(1) - xf[:, 0].min(1))[:, None, :]
    v_range = (xf[:, 1].max(2) - xf[:, 1].min(2))[:, :, None]
    level = np.stack([np.broadcast_to(k_range, xf[:, 0].shape), np.broadcast_to(v_range, xf[:, 1].shape)], axis=1) / 255
    assert (np.abs(back - xf) <= level + np.abs(back) * 2**-7 + 1e-6).all()


def test_key_channel_outlier_does_not_degrade_its_neighbours() -> None:
    """tests/test_quant.py:49-57: keys are per channel, so a x500 channel keeps to itself."""
    rng = np.random.default_rng(0)
    xf = rng.standard_normal((1, 2, 64, 64)).astype(np.float32)
    xf[0, 0, :, 0] *= 500
    x = _bf16(xf)
    back = R.to_f32(R.unpack(R.pack(x, "bf16"), 64, 64, "bf16"), "bf16").reshape(x.shape)
    quiet = np.abs(back[0, 0, :, 1:] - R.to_f32(x, "bf16")[0, 0, :, 1:]).max()
    assert quiet < 0.05


def test_constant_group_is_exact() -> None:
    """tests/test_quant.py:59-63: a zero range clamps the scale to float32 tiny and round-trips exactly."""
    x = _bf16(np.full((2, 2, 64, 64), 3.5))
    assert np.array_equal(R.unpack(R.pack(x, "bf16"), 64, 64, "bf16").reshape(x.shape), x)


def test_quantiser_rounds_half_to_even() -> None:
    """min 0, max 255 => scale exactly 1.0, so x.5 quotients exercise the rounding rule."""
    bs, d = 16, 64
    x = np.zeros((1, 2, bs, d), dtype=np.float32)
    col = np.arange(bs, dtype=np.float32) + 0.5
    col[0], col[1] = 0.0, 255.0
    x[0, 0, :, 0] = col
    rec = R.pack(R.from_f32(x, "f16"), "f16")
    kq = rec[0, : bs * d].view(np.int8).reshape(bs, d)[:, 0].astype(int) + 128
    want = [0, 255] + [round(float(v)) for v in col[2:]]  # Python's round() is half-to-even
    assert list(kq) == want
    assert kq[2] == 2 and kq[3] == 4  # 2.5 -> 2, 3.5 -> 4


@pytest.mark.parametrize(("dt", "u", "scale_bits", "single"), [("f16", 145, 0x01C4, 8.0078125), ("bf16", 185, 0x0989, 8.0625)])
def test_unpack_rounds_to_float32_before_the_model_dtype(dt: str, u: int, scale_bits: int, single: float) -> None:
    """quant.py:103-105 dequantises in float32 and then casts. With code u (q = u - 128), the
    scale s given and zero 8, the exact u * s + 8 lies just above a tie of the model dtype between
    8 and `single`; float32 rounding lands on the tie, which then rounds to the even 8. A
    dequantisation that rounds once (float64, or one fused rounding into the model dtype) gives
    `single` instead."""
    from fractions import Fraction

    bs, d = 4, 8
    s = np.array([scale_bits], dtype=np.uint16).view(np.float16)[0]
    exact = Fraction(u) * Fraction(float(s)) + 8
    tie = (Fraction(8) + Fraction(single)) / 2
    assert tie < exact < tie + Fraction(1, 2**20)  # above the tie by less than half a float32 ulp at 8
    o1, o2, o3, o4, o5 = R.record_offsets(bs, d)
    rec = np.zeros((1, R.packed_pair_bytes(bs, d)), dtype=np.uint8)
    rec[0, :o2] = u ^ 0x80  # the int8 code u - 128
    rec[0, o2:o3] = np.full(d, scale_bits, dtype=np.uint16).view(np.uint8)
    rec[0, o3:o4] = np.full(d, 0x4800, dtype=np.uint16).view(np.uint8)  # float16 8.0
    rec[0, o4:o5] = np.full(bs, scale_bits, dtype=np.uint16).view(np.uint8)
    rec[0, o5:] = np.full(bs, 0x4800, dtype=np.uint16).view(np.uint8)
    assert np.all(R.unpack_f32(rec, bs, d) == np.float32(float(tie)))
    assert np.all(R.to_f32(R.unpack(rec, bs, d, dt), dt) == 8.0)
    assert np.all(quant_c.unpack(rec, bs, d, dt) == R.unpack(rec, bs, d, dt))


def test_rejects_bad_widths_and_pairs() -> None:
    """tests/test_quant.py:66-73."""
    with pytest.raises(ValueError, match="packed_pair_bytes"):
        R.unpack(np.zeros((2, 7), dtype=np.uint8), 64, 64, "bf16")
    with pytest.raises(ValueError, match="KV pair"):
        R.pack(np.zeros((3, 3, 64, 64), dtype=np.uint16), "bf16")


def test_bf16_rounding_is_nearest_even() -> None:
    vals = np.array([1.0 + 2**-8, 1.0 + 3 * 2**-8, -(1.0 + 2**-8), np.nan], dtype=np.float32)
    got = R.from_f32(vals, "bf16")
    assert got[0] == 0x3F80 and got[1] == 0x3F82 and got[2] == 0xBF80 and got[3] == 0x7FC0


# -- selection -----------------------------------------------------------------------------------


def _meta(rng, h=2, n=10, bs=8, d=16):
    keys = rng.standard_normal((h, n * bs, d))
    kmin, kmax = R.block_minmax(keys, bs)
    return keys, kmin, kmax


def test_bound_matches_quests_definition() -> None:
    """q+.M + q-.m equals sum_i max(q_i m_i, q_i M_i): a sign or operand swap breaks this."""
    rng = np.random.default_rng(3)
    _, kmin, kmax = _meta(rng)
    q = rng.standard_normal((8, 16))
    assert np.allclose(R.quest_bound(q, kmin, kmax), R.quest_bound_bruteforce(q, kmin, kmax), atol=1e-12)
    # and the float32 variant agrees to float32 accuracy
    assert np.allclose(R.quest_bound(q, kmin, kmax, "f32"), R.quest_bound_bruteforce(q, kmin, kmax), atol=1e-4)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_model_dtype_bound_rounds_where_torch_does(dt: str) -> None:
    """The `dtype=None` bound of lazykv/selection.py:47-52 is two model-dtype matrix products
    (float32 sums, rounded to the model dtype) and a model-dtype add. torch's own bf16 / fp16
    kernels evaluate that expression here, on inputs that are multiples of 1/8, so every float32
    sum is exact and only the rounding points can differ: the oracle's "model" bound must equal
    it bit for bit, and a single rounding of a + b must not."""
    import torch

    tdt = {"bf16": torch.bfloat16, "f16": torch.float16}[dt]
    rng = np.random.default_rng(7)
    h, g, n, d = 2, 4, 300, 32
    q = rng.integers(-40, 41, (h * g, d)) / 8.0
    lo = rng.integers(-40, 41, (h, n, d)) / 8.0
    hi = lo + rng.integers(0, 41, (h, n, d)) / 8.0
    tq = torch.tensor(q, dtype=tdt).view(1, h, g, d)
    qp = tq.clamp_min(0)
    tmin, tmax = torch.tensor(lo, dtype=tdt).view(1, h, n, d), torch.tensor(hi, dtype=tdt).view(1, h, n, d)
    want = ((qp @ tmax.transpose(-1, -2)) + ((tq - qp) @ tmin.transpose(-1, -2))).amax(dim=2)[0].float().numpy()
    assert np.array_equal(R.quest_bound(q, lo, hi, "model", dt), want)
    once = R.round_to(R.quest_bound(q, lo, hi, "f32"), dt)
    assert not np.array_equal(once, want)


def test_bound_dominates_every_dot_product_in_its_block() -> None:
    """tests/test_selection.py:47-56."""
    rng = np.random.default_rng(4)
    keys, kmin, kmax = _meta(rng)
    q = rng.standard_normal((8, 16))
    bound = R.quest_bound(q, kmin, kmax)
    g = 4
    for h in range(2):
        s = q[h * g : (h + 1) * g] @ keys[h].T  # [g, n*bs]
        exact = s.reshape(g, 10, 8).max(-1).max(0)
        assert (bound[h] >= exact - 1e-9).all()


def test_float32_bound_breaks_the_bf16_tie() -> None:
    """tests/test_selection.py:121-133: 256+1 vs 256+0.5 tie in bf16, not in float32."""
    q = np.ones((1, 2))
    kmax = np.array([[[256.0, 0.5], [256.0, 1.0]]])
    kmin = kmax.copy()
    model = R.quest_bound(q, kmin, kmax, "model", "bf16")
    assert model[0, 0] == model[0, 1]
    b32 = R.quest_bound(q, kmin, kmax, "f32")
    assert b32[0, 1] > b32[0, 0]
    assert R.top_blocks(b32, 1)[0, 0] == 1


def test_top_blocks_is_a_descending_sort_with_low_id_ties() -> None:
    bound = np.array([[0.5, 3.0, 1.0, 3.0, -2.0, 2.0]])
    assert R.top_blocks(bound, 3).tolist() == [[1, 3, 5]]
    rng = np.random.default_rng(5)
    b = rng.standard_normal((3, 50))
    top = R.top_blocks(b, 7)
    for h in range(3):
        assert top[h].tolist() == list(np.argsort(-b[h], kind="stable")[:7])


def test_selection_ok_accepts_only_near_tie_swaps() -> None:
    b = np.array([5.0, 4.0, 3.0, 3.0 - 1e-7, 1.0])
    assert R.selection_ok(np.array([0, 1, 2]), b, 3) == (True, True)
    assert R.selection_ok(np.array([0, 1, 3]), b, 3)[0]  # the near-tie swap
    assert not R.selection_ok(np.array([0, 1, 4]), b, 3)[0]  # a real miss
    assert not R.selection_ok(np.array([0, 0, 1]), b, 3)[0]  # duplicates
    assert R.selection_ok(np.array([2, 1, 0]), np.array([5.0, 4.0, 3.0, 1.0]), 3) == (True, False)


def test_blocks_for_budget_leaves_room_for_sink_and_current() -> None:
    """tests/test_selection.py:38-44, plus the workloads' budgets (510 at 6.25% of 131,072 / 16)."""
    for frac in (0.75, 0.25, 0.0625):
        k = R.blocks_for_budget(frac, 32768, 64)
        assert (k + 2) * 64 <= frac * 32768
    assert R.blocks_for_budget(0.0625, 131072, 16) == 510
    assert R.blocks_for_budget(0.25, 32768, 16) == 510


def test_current_block_mask_hides_the_unfilled_tail() -> None:
    """tests/test_selection.py:98: 5 live tokens of the current block of 8, K=3."""
    m = R.current_block_mask(5 * 8, 8, 5)
    assert (m[: 4 * 8 + 5] == 0).all() and np.isinf(m[4 * 8 + 5 :]).all()


def test_candidates_follow_lazy_sealing() -> None:
    assert R.candidates(131072, 16) == (8191, 16)
    assert R.candidates(101, 8) == (12, 5)


# -- attention, merge, partial ------------------------------------------------------------------


def _brute_softmax(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float) -> tuple[np.ndarray, float]:
    s = [float(np.dot(q, k[t])) * scale for t in range(k.shape[0])]
    mx = max(s)
    w = [math.exp(x - mx) for x in s]
    den = sum(w)
    out = sum(w[t] * v[t] for t in range(k.shape[0])) / den
    return out, mx + math.log(den)


def test_attend_tokens_matches_a_scalar_softmax_loop() -> None:
    rng = np.random.default_rng(6)
    q = rng.standard_normal((4, 8))
    keys = [rng.standard_normal((11, 8)), rng.standard_normal((5, 8))]
    values = [rng.standard_normal((11, 8)), rng.standard_normal((5, 8))]
    out, lse = R.attend_tokens(q, keys, values, 0.3)
    for i in range(4):
        o, l = _brute_softmax(q[i], keys[i // 2], values[i // 2], 0.3)
        assert np.allclose(out[i], o, atol=1e-12) and abs(lse[i] - l) < 1e-12


def test_gathered_tokens_order_and_fill() -> None:
    bs, d = 4, 2
    store = np.arange(6 * bs * d, dtype=float).reshape(6, bs, d)

    def block_kv(h, b):
        return store[b] + 1000 * h, -store[b]

    ks, vs = R.gathered_tokens(block_kv, 2, np.array([[3, 1], [2, 4]]), 0, 5, 3, bs)
    assert ks[0].shape == (4 * 3 + 3, d)
    assert np.array_equal(ks[0][:4], store[0]) and np.array_equal(ks[0][4:8], store[3])
    assert np.array_equal(ks[1][8:12], store[4] + 1000) and np.array_equal(ks[1][12:], store[5][:3] + 1000)


def test_merge_is_the_lse_weighting() -> None:
    """tests/test_exact.py:72-84."""
    merged, lse = R.merge_lse(np.array([[1.0, 0.0]]), np.array([2.0]), np.array([[0.0, 1.0]]), np.array([0.0]))
    wa = math.exp(2.0 - float(np.logaddexp(2.0, 0.0)))
    assert merged[0, 0] == pytest.approx(wa) and merged[0, 0] > merged[0, 1]
    assert float(lse[0]) == pytest.approx(float(np.logaddexp(2.0, 0.0)))


def test_merging_two_halves_reconstructs_the_whole() -> None:
    """tests/test_exact.py:32-49, against the float64 brute force."""
    rng = np.random.default_rng(0)
    h, groups, n_blocks, d, bs = 3, 2, 6, 16, 8
    keys = rng.standard_normal((h, n_blocks * bs, d))
    values = rng.standard_normal((h, n_blocks * bs, d))
    query = rng.standard_normal((h, groups, d))
    first = np.tile(np.arange(0, 2), (h, 1))
    second = np.tile(np.arange(2, n_blocks), (h, 1))
    oa, la = R.partial_attention(keys, values, query, d**-0.5, bs, second)
    ob, lb = R.partial_attention(keys, values, query, d**-0.5, bs, first)
    merged, _ = R.merge_lse(oa, la, ob, lb)
    for j in range(h):
        for gi in range(groups):
            o, _ = _brute_softmax(query[j, gi], keys[j], values[j], d**-0.5)
            assert np.allclose(merged[j, gi], o, atol=1e-10)


def test_empty_partial_contributes_nothing() -> None:
    """tests/test_exact.py:52-69."""
    rng = np.random.default_rng(1)
    h, groups, n_blocks, d, bs = 2, 2, 4, 8, 8
    keys, values = rng.standard_normal((h, n_blocks * bs, d)), rng.standard_normal((h, n_blocks * bs, d))
    query = rng.standard_normal((h, groups, d))
    everything = np.tile(np.arange(n_blocks), (h, 1))
    eo, el = R.partial_attention(keys, values, query, d**-0.5, bs, everything)
    assert np.isneginf(el).all() and np.isfinite(eo).all() and (eo == 0).all()
    fo, fl = R.partial_attention(keys, values, query, d**-0.5, bs, np.empty((h, 0), dtype=np.int64))
    merged, lse = R.merge_lse(fo, fl, eo, el)
    assert np.allclose(merged, fo, atol=1e-12) and np.allclose(lse, fl)
    both, lse2 = R.merge_lse(eo, el, eo, el)
    assert np.isneginf(lse2).all() and (both == 0).all()


def test_excluding_a_block_removes_exactly_that_block() -> None:
    """tests/test_exact.py:87-101."""
    rng = np.random.default_rng(2)
    h, groups, n_blocks, d, bs = 3, 1, 5, 8, 8
    keys, values = rng.standard_normal((h, n_blocks * bs, d)), rng.standard_normal((h, n_blocks * bs, d))
    query = rng.standard_normal((h, groups, d))
    excluded = np.array([[2], [4], [4]])
    out, _ = R.partial_attention(keys, values, query, d**-0.5, bs, excluded)
    for j, drop in enumerate(excluded[:, 0]):
        keep = [t for t in range(n_blocks * bs) if not (drop * bs <= t < (drop + 1) * bs)]
        o, _ = _brute_softmax(query[j, 0], keys[j, keep], values[j, keep], d**-0.5)
        assert np.allclose(out[j, 0], o, atol=1e-10)


# -- hybrid residency ---------------------------------------------------------------------------------


def _lru_reference(steps: list[np.ndarray], n_slots: int, seeded: list[int]) -> list[list[int]]:
    """The reference's residency for one head, written over plain lists (lazykv/tiered.py:274-287
    seeding, :389-418 admit, :450-452 gather): slot s holds slot_block[s]; a seeded slot was last
    used at -1 and an empty one at -2; victims are the least recently used slots outside the chosen
    set, ties to the lower slot, handed to the misses in the order the step lists them. Returns
    slot_block after each step."""
    slot_block = list(seeded) + [-1] * (n_slots - len(seeded))
    last_used = [-1] * len(seeded) + [-2] * (n_slots - len(seeded))
    out = []
    for step, chosen in enumerate(steps):
        where = {b: s for s, b in enumerate(slot_block) if b >= 0}
        keep = {where[b] for b in chosen.tolist() if b in where}
        misses = [b for b in chosen.tolist() if b not in where]
        free = sorted((s for s in range(n_slots) if s not in keep), key=lambda s: (last_used[s], s))
        for b, s in zip(misses, free):
            slot_block[s] = b
        for b in chosen.tolist():
            last_used[slot_block.index(b)] = step
        out.append(list(slot_block))
    return out


@pytest.mark.parametrize(("k", "spare", "seed"), [(8, 0, 0), (8, 0, 8), (8, 3, 0), (8, 8, 5), (5, 11, 16)])
def test_residency_step_keeps_hits_and_evicts_the_least_recently_used(k: int, spare: int, seed: int) -> None:
    rng = np.random.default_rng(3 + k + spare + seed)
    h, n = 3, 60
    n_slots = k + spare
    seed = min(seed, n_slots)
    first = n - 2 - seed  # the most recent candidate blocks, as a prompt of n - 1 sealed blocks seeds them
    block_slot, slot_block, last_used = R.residency_state(h, n_slots, n, first, seed)
    seqs: list[list[np.ndarray]] = [[] for _ in range(h)]
    chosen = np.stack([np.sort(rng.choice(n, k, replace=False)) for _ in range(h)])
    for step in range(40):
        nxt = []
        for j in range(h):  # drift: each step keeps most of the previous choice
            keep = rng.choice(chosen[j], k - 3, replace=False)
            pool = np.setdiff1d(np.arange(n), keep)
            nxt.append(np.sort(np.concatenate([keep, rng.choice(pool, 3, replace=False)])))
        prev_bs, prev_sb, prev_lu = block_slot.copy(), slot_block.copy(), last_used.copy()
        chosen = np.stack(nxt)
        loc = R.residency_step(block_slot, slot_block, last_used, chosen, step)
        for j in range(h):
            seqs[j].append(chosen[j])
            resident = set(slot_block[j][slot_block[j] >= 0].tolist())
            assert set(chosen[j].tolist()) <= resident
            for s in range(n_slots):  # the two tables agree
                if slot_block[j, s] >= 0:
                    assert block_slot[j, slot_block[j, s]] == s
            assert (block_slot[j] >= 0).sum() == len(resident)
            hits = [i for i in range(k) if prev_bs[j, chosen[j, i]] >= 0]
            for i in hits:  # a hit keeps its slot and is read from it
                assert loc[j, i] == prev_bs[j, chosen[j, i]] and not loc[j, i] & R.LOC_MISS
            misses = [i for i in range(k) if i not in hits]
            victims = [int(loc[j, i]) & ~R.LOC_MISS for i in misses]  # in the order the step lists the misses
            hit_slots = {int(prev_bs[j, chosen[j, i]]) for i in hits}
            unhit = sorted((s for s in range(n_slots) if s not in hit_slots), key=lambda s: (prev_lu[j, s], s))
            assert victims == unhit[: len(misses)]  # the least recently used, handed out in order
            if spare == 0:
                assert resident == set(chosen[j].tolist())  # k slots: exactly the chosen set
            assert all(prev_sb[j, v] not in chosen[j] for v in victims)
            used = set(hit_slots) | set(victims)
            assert all(last_used[j, s] == step for s in used) and all(last_used[j, s] == prev_lu[j, s] for s in set(range(n_slots)) - used)
            assert np.array_equal(R.slot_order(last_used)[j], sorted(range(n_slots), key=lambda s: (last_used[j, s], s)))
    for j in range(h):
        seeded = list(range(first, first + seed))
        assert _lru_reference(seqs[j], n_slots, seeded)[-1] == slot_block[j].tolist()
