"""numpy restatement of the reference's tiered decode-attention hot path.

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`): the product never imports this module.

Every function cites the reference file:line it restates. Conventions:

* KV in a model dtype is passed as raw bits (`uint16` for "f16"/"bf16") or as float32 ("f32");
  `to_f32` / `from_f32` convert exactly / with round-to-nearest-even.
* Attention, bound and merge truths are computed in float64. The int8 quantiser is restated in
  float32, operation by operation, because its bytes are the parity target.

How each function is pinned (each check lives in `tests/test_oracle.py`):

* `pack` / `unpack`: bit-equality with golden vectors written by the reference's own
  `quant.py` (`tests/golden/make_quant_vectors.py`), plus an independent C restatement
  (`oracle/quant_ref.c`) and the reference tests' invariants (`tests/test_quant.py:21-73`).
* `quest_bound`: brute force of Quest's definition sum_i max(q_i m_i, q_i M_i) (a different
  formula from q+.M + q-.m, so a sign or operand swap fails), the dominance invariant
  (`tests/test_selection.py:47-56`) and the bf16 tie known answer (`tests/test_selection.py:121-133`).
* `top_blocks`: brute-force sort; tie order (lower block id first) is the rule of lkv_bound_topk.
* `block_minmax`, `current_block_mask`, `blocks_for_budget`: closed forms and the reference's
  own known answers (`tests/test_selection.py:38-44,98`).
* `residency_state` / `residency_step` / `slot_order`: invariants that fix them (every chosen
  block is resident after a step, hits keep their slots, the victims are the least recently used
  unhit slots, and with as many slots as chosen blocks exactly the unhit ones), and a separate
  least-recently-used simulation written over plain lists in the reference's own terms
  (lazykv/tiered.py:274-287,389-418,450-452), on random step sequences with and without spare
  slots and with a seeded start.
* `attend` / `partial_attention` / `merge_lse`: float64 brute force over explicit token lists,
  the reference's merge known answer (`tests/test_exact.py:72-84`), the empty-partial rule
  (`tests/test_exact.py:52-69`) and the two-halves reconstruction (`tests/test_exact.py:32-49`).
"""

from __future__ import annotations

import math

import numpy as np

F32_TINY = np.finfo(np.float32).tiny
LEVELS = np.float32(255.0)  # lazykv/quant.py:43 -- 256 levels, 255 intervals
DENSE_LAYERS = 2  # lazykv/selection.py:35


# -- dtype helpers ------------------------------------------------------------------------------


def to_f32(x: np.ndarray, dtype: str) -> np.ndarray:
    """Exact widening of model-dtype bits to float32."""
    if dtype == "f32":
        return np.asarray(x, dtype=np.float32)
    if dtype == "f16":
        return np.asarray(x, dtype=np.uint16).view(np.float16).astype(np.float32)
    if dtype == "bf16":
        return (np.asarray(x, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
    raise ValueError(dtype)


def from_f32(x: np.ndarray, dtype: str) -> np.ndarray:
    """float32 -> model-dtype bits, round to nearest even (torch's `.to(dtype)`)."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "f32":
        return x.copy()
    if dtype == "f16":
        return x.astype(np.float16).view(np.uint16)
    if dtype == "bf16":
        u = x.view(np.uint32).astype(np.uint64)
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        nan = np.isnan(x)
        r[nan] = 0x7FC0
        return r
    raise ValueError(dtype)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """float32 values rounded through a model dtype and widened back."""
    return to_f32(from_f32(x, dtype), dtype)


# -- int8 warm/cold records: lazykv/quant.py ----------------------------------------------------


def packed_pair_bytes(bs: int, d: int) -> int:
    """lazykv/quant.py:46-49: both int8 payloads plus four float16 scale arrays."""
    return 2 * bs * d + 2 * 2 * d + 2 * 2 * bs


def record_offsets(bs: int, d: int) -> tuple[int, int, int, int, int]:
    """lazykv/quant.py:52-56: kq | vq | k scale | k zero | v scale | v zero."""
    n = bs * d
    return n, 2 * n, 2 * n + 2 * d, 2 * n + 4 * d, 2 * n + 4 * d + 2 * bs


def _affine(x: np.ndarray, axis: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """lazykv/quant.py:59-70 on float32 `x` [n, bs, d]: q int8, scale f16, zero f16."""
    mn = x.min(axis=axis, keepdims=True)
    mx = x.max(axis=axis, keepdims=True)
    scale = np.maximum((mx - mn) / LEVELS, np.float32(F32_TINY))
    q = np.clip(np.rint((x - mn) / scale), np.float32(0), LEVELS) - np.float32(128)
    return q.astype(np.int8), scale.squeeze(axis).astype(np.float16), mn.squeeze(axis).astype(np.float16)


def pack(pairs: np.ndarray, dtype: str) -> np.ndarray:
    """lazykv/quant.py:73-87: `[..., 2, bs, d]` model-dtype bits -> uint8 records `[..., P]`."""
    *lead, two, bs, d = pairs.shape
    if two != 2:
        raise ValueError("expected a [..., 2, block_size, head_dim] KV pair")
    x = to_f32(pairs.reshape(-1, 2, bs, d), dtype)
    kq, ks, kz = _affine(x[:, 0], axis=1)  # keys: per channel, range over tokens
    vq, vs, vz = _affine(x[:, 1], axis=2)  # values: per token, range over head_dim
    m = x.shape[0]
    parts = [kq.reshape(m, -1), vq.reshape(m, -1), ks, kz, vs, vz]
    rec = np.concatenate([np.ascontiguousarray(p).view(np.uint8).reshape(m, -1) for p in parts], axis=1)
    return rec.reshape(*lead, rec.shape[-1])


def unpack_f32(rec: np.ndarray, bs: int, d: int) -> np.ndarray:
    """lazykv/quant.py:90-105 up to the final cast: float32 `[m, 2, bs, d]`."""
    if rec.ndim != 2 or rec.shape[1] != packed_pair_bytes(bs, d):
        raise ValueError("expected uint8 records of packed_pair_bytes width")
    o1, o2, o3, o4, o5 = record_offsets(bs, d)
    rec = np.ascontiguousarray(rec)
    kq = rec[:, :o1].view(np.int8).reshape(-1, bs, d).astype(np.float32)
    vq = rec[:, o1:o2].view(np.int8).reshape(-1, bs, d).astype(np.float32)
    ks = np.ascontiguousarray(rec[:, o2:o3]).view(np.float16).astype(np.float32)
    kz = np.ascontiguousarray(rec[:, o3:o4]).view(np.float16).astype(np.float32)
    vs = np.ascontiguousarray(rec[:, o4:o5]).view(np.float16).astype(np.float32)
    vz = np.ascontiguousarray(rec[:, o5:]).view(np.float16).astype(np.float32)
    # Separate multiply and add, both rounded to float32: no fused multiply-add.
    k = (kq + np.float32(128)) * ks[:, None, :]
    k = k + kz[:, None, :]
    v = (vq + np.float32(128)) * vs[:, :, None]
    v = v + vz[:, :, None]
    return np.stack([k, v], axis=1)


def unpack(rec: np.ndarray, bs: int, d: int, dtype: str) -> np.ndarray:
    """lazykv/quant.py:90-105: records -> `[m, 2, bs, d]` model-dtype bits."""
    return from_f32(unpack_f32(rec, bs, d), dtype)


# -- selection: lazykv/selection.py -------------------------------------------------------------


def quest_bound(q: np.ndarray, kmin: np.ndarray, kmax: np.ndarray, precision: str = "f64", model_dtype: str = "bf16") -> np.ndarray:
    """lazykv/selection.py:38-53: Quest bound per KV head and candidate block, max over the group.

    `q` [H_q, d], `kmin`/`kmax` [H_kv, C, d] (float values). `precision`:
    "f64" the truth; "f32" float32 products and sum (the `dtype=torch.float32` variant);
    "model" both products and their sum rounded to `model_dtype` (the `dtype=None` variant's
    rounding points). Returns [H_kv, C].
    """
    h_kv, _, d = kmin.shape
    g = q.shape[0] // h_kv
    ft = np.float64 if precision == "f64" else np.float32
    qq = np.asarray(q, dtype=ft).reshape(h_kv, g, d)
    qp = np.maximum(qq, 0)
    qn = qq - qp
    a = qp @ np.asarray(kmax, dtype=ft).transpose(0, 2, 1)
    b = qn @ np.asarray(kmin, dtype=ft).transpose(0, 2, 1)
    if precision == "model":
        bound = round_to(round_to(a, model_dtype) + round_to(b, model_dtype), model_dtype)
    else:
        bound = a + b
    return bound.max(axis=1)


def quest_bound_bruteforce(q: np.ndarray, kmin: np.ndarray, kmax: np.ndarray) -> np.ndarray:
    """Quest's own definition, U = sum_i max(q_i m_i, q_i M_i), max over the group, in float64."""
    h_kv, c, d = kmin.shape
    g = q.shape[0] // h_kv
    out = np.empty((h_kv, c))
    for h in range(h_kv):
        qh = q[h * g : (h + 1) * g].astype(np.float64)
        lo = qh[:, None, :] * kmin[h].astype(np.float64)[None]
        hi = qh[:, None, :] * kmax[h].astype(np.float64)[None]
        out[h] = np.maximum(lo, hi).sum(-1).max(0)
    return out


def top_blocks(bound: np.ndarray, k: int) -> np.ndarray:
    """lazykv/selection.py:56-62: the k highest bounds per head, descending; ties by lower id.

    Returns candidate-relative indices [H_kv, k] (callers add the candidate offset, 1, as
    lazykv/tiered.py:386,500 do).
    """
    h_kv, c = bound.shape
    if k > c:
        raise ValueError("k exceeds the candidate count")
    out = np.empty((h_kv, k), dtype=np.int64)
    ids = np.arange(c)
    for h in range(h_kv):
        order = np.lexsort((ids, -bound[h]))
        out[h] = order[:k]
    return out


def selection_ok(got: np.ndarray, bound: np.ndarray, k: int, abs_err: float = 0.0, rel: float = 1e-5) -> tuple[bool, bool]:
    """Accept a kernel's selected set for one head against the float64 `bound` row.

    The near-tie rule: with b_K the K-th largest bound, tol = rel*max(1,|b_K|) + abs_err (the
    float32 accumulation error bound of the kernel's dot products). Every block with a bound
    above b_K + tol must be chosen, and every chosen block must have a bound of at least
    b_K - tol, with exactly K distinct ids. Returns (ok, was_near_tie).
    """
    got = np.asarray(got)
    if got.size != k or np.unique(got).size != k or got.min() < 0 or got.max() >= bound.size:
        return False, False
    srt = np.sort(bound)[::-1]
    bk = srt[k - 1]
    tol = rel * max(1.0, abs(bk)) + abs_err
    near = k < bound.size and (bk - srt[k]) <= tol
    required = np.flatnonzero(bound > bk + tol)
    if not np.isin(required, got).all():
        return False, near
    return bool((bound[got] >= bk - tol).all()), near


def current_block_mask(total: int, block_size: int, fill: int) -> np.ndarray:
    """lazykv/selection.py:65-69: additive 0/-inf mask hiding the current block's unfilled tail."""
    mask = np.zeros(total, dtype=np.float32)
    mask[total - block_size + fill :] = -np.inf
    return mask


def blocks_for_budget(fraction: float, total_tokens: int, block_size: int) -> int:
    """lazykv/selection.py:72-74: sink + K + current within the budget."""
    return max(1, math.floor(fraction * total_tokens / block_size) - 2)


def candidates(length: int, block_size: int) -> tuple[int, int]:
    """(n_sealed, fill) under lazy sealing (lazykv/tiered.py:306-314,379-381; selection.py:153-155)."""
    n_full, fill = divmod(length, block_size)
    if fill == 0:
        n_full, fill = n_full - 1, block_size
    return n_full, fill


def block_minmax(keys: np.ndarray, block_size: int) -> tuple[np.ndarray, np.ndarray]:
    """Per-block, per-channel key min/max (lazykv/tiered.py:173-175, selection.py:142-144).

    `keys` [H_kv, n*bs, d] float values -> (kmin, kmax) [H_kv, n, d].
    """
    h, t, d = keys.shape
    b = keys.reshape(h, t // block_size, block_size, d)
    return b.min(axis=2), b.max(axis=2)


# -- attention: lazykv/attention.py, lazykv/exact.py --------------------------------------------


def attend_tokens(q: np.ndarray, keys: list[np.ndarray], values: list[np.ndarray], scale: float) -> tuple[np.ndarray, np.ndarray]:
    """Softmax attention per KV head over an explicit token list, GQA query head i -> KV head i // g.

    The float64 form of `attend` + `_gpu_lse` (lazykv/attention.py:97-136,196-207;
    lazykv/exact.py:276-288). `keys[h]`/`values[h]` [n_h, d]. Returns out [H_q, d], lse [H_q];
    an empty set gives lse = -inf and a zero output (lazykv/exact.py:117-126).
    """
    h_kv = len(keys)
    g = q.shape[0] // h_kv
    d = q.shape[1]
    out = np.zeros((q.shape[0], d))
    lse = np.full(q.shape[0], -np.inf)
    for h in range(h_kv):
        k = np.asarray(keys[h], dtype=np.float64)
        v = np.asarray(values[h], dtype=np.float64)
        if k.shape[0] == 0:
            continue
        s = (q[h * g : (h + 1) * g].astype(np.float64) @ k.T) * scale  # [g, n]
        m = s.max(axis=1, keepdims=True)
        p = np.exp(s - m)
        den = p.sum(axis=1, keepdims=True)
        out[h * g : (h + 1) * g] = (p / den) @ v
        lse[h * g : (h + 1) * g] = (m + np.log(den)).ravel()
    return out, lse


def gathered_tokens(block_kv, h_kv: int, chosen: np.ndarray, sink: int, current: int, fill: int, bs: int) -> tuple[list, list]:
    """The key/value sequence a selecting layer attends to, per KV head.

    Sink, then the chosen blocks in the given order, then the current block's first `fill`
    tokens (lazykv/tiered.py:466-474,503-510; selection.py:164-179). `block_kv(h, b)` returns
    float arrays (k [bs, d], v [bs, d]); `chosen` [H_kv, K] are block ids.
    """
    ks, vs = [], []
    for h in range(h_kv):
        kk, vv = [], []
        for b in [sink, *chosen[h].tolist()]:
            k, v = block_kv(h, b)
            kk.append(k)
            vv.append(v)
        if fill > 0:
            k, v = block_kv(h, current)
            kk.append(k[:fill])
            vv.append(v[:fill])
        ks.append(np.concatenate(kk) if kk else np.zeros((0, bs)))
        vs.append(np.concatenate(vv) if vv else np.zeros((0, bs)))
    return ks, vs


def merge_lse(out_a: np.ndarray, lse_a: np.ndarray, out_b: np.ndarray, lse_b: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """lazykv/exact.py:69-85: exact two-partial merge; an empty partial (lse -inf) adds nothing."""
    lse = np.logaddexp(lse_a, lse_b)
    finite = np.isfinite(lse)
    safe = np.where(finite, lse, 0.0)
    with np.errstate(invalid="ignore", over="ignore"):
        wa = np.where(finite, np.exp(lse_a - safe), 0.0)
        wb = np.where(finite, np.exp(lse_b - safe), 0.0)
    return wa[..., None] * out_a + wb[..., None] * out_b, lse


def partial_attention(keys: np.ndarray, values: np.ndarray, query: np.ndarray, scaling: float, block_size: int, excluded: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """lazykv/exact.py:88-127 in float64: attention over every block except `excluded` per head.

    `keys`/`values` [h, n*bs, d]; `query` [h, g, d]; `excluded` [h, e] block ids. Excluded
    columns are -inf before the row max; an all-excluded head gives lse -inf and a zero output.
    """
    h, total, _ = keys.shape
    n_blocks = total // block_size
    scores = np.einsum("hgd,htd->hgt", query.astype(np.float64), keys.astype(np.float64)) * scaling
    sv = scores.reshape(h, query.shape[1], n_blocks, block_size)
    for j in range(h):
        sv[j, :, excluded[j]] = -np.inf
    m = scores.max(axis=-1, keepdims=True)
    empty = np.isneginf(m)
    p = np.exp(scores - np.where(empty, 0.0, m))
    p[np.broadcast_to(empty, p.shape)] = 0.0
    norm = p.sum(axis=-1, keepdims=True)
    out = (p / np.maximum(norm, np.finfo(np.float64).tiny)) @ values.astype(np.float64)
    with np.errstate(divide="ignore"):
        lse = np.where(empty, -np.inf, m + np.log(norm)).squeeze(-1)
    return out, lse


# -- hybrid residency (device-side rung 6): which selected blocks sit in the HBM slots ------------

LOC_MISS = 0x40000000


def residency_state(h: int, n_slots: int, cap_blocks: int, first: int = 0, seed: int = 0) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """A hybrid tier's residency when its prompt closes (lazykv/tiered.py:165-168,274-287): slots
    0..seed-1 of every head hold blocks first..first+seed-1 and were last used at -1; the other slots
    are empty, last used at -2, so they are taken first. Returns block_slot [h, cap] (slot or -1),
    slot_block [h, n_slots] (block or -1) and last_used [h, n_slots]. Slots are numbered from 0 here;
    the reference numbers them 1..n_slots after the sink."""
    block_slot = np.full((h, cap_blocks), -1, dtype=np.int64)
    slot_block = np.full((h, n_slots), -1, dtype=np.int64)
    last_used = np.full((h, n_slots), -2, dtype=np.int64)
    if seed:
        slot_block[:, :seed] = np.arange(first, first + seed)
        block_slot[:, first : first + seed] = np.arange(seed)
        last_used[:, :seed] = -1
    return block_slot, slot_block, last_used


def residency_step(block_slot: np.ndarray, slot_block: np.ndarray, last_used: np.ndarray, chosen: np.ndarray, step: int) -> np.ndarray:
    """One decode step of the hybrid tier's residency, per KV head, over n_slots >= k slots:
    lazykv/tiered.py:389-418 (admit) followed by the last-use update of gather (:450-452).

    The chosen blocks already in a slot keep it. The victims are the slots the choice does not hit,
    least recently used first (a stable sort of last_used, so ties go to the lower slot), as many as
    there are missed blocks, which take them in the order `chosen` lists them. Every slot the step
    uses, hit or victim, is then last used at `step`. Updates block_slot [h, cap], slot_block
    [h, n_slots] and last_used [h, n_slots] in place and returns loc [h, k]: the slot of a hit, or
    LOC_MISS | slot for a miss read from the host and copied into that slot.
    """
    h, k = chosen.shape
    n_slots = slot_block.shape[1]
    loc = np.empty((h, k), dtype=np.int64)
    for j in range(h):
        row = chosen[j]
        slots = block_slot[j, row]
        miss = slots < 0
        keep = np.zeros(n_slots, dtype=bool)
        keep[slots[~miss]] = True
        free = np.flatnonzero(~keep)
        victims = free[np.argsort(last_used[j, free], kind="stable")[: int(miss.sum())]]
        want = row[miss]
        old = slot_block[j, victims]
        block_slot[j, old[old >= 0]] = -1
        slot_block[j, victims] = want
        block_slot[j, want] = victims
        loc[j, ~miss] = slots[~miss]
        loc[j, miss] = LOC_MISS | victims
        last_used[j, block_slot[j, row]] = step
    return loc


def slot_order(last_used: np.ndarray) -> np.ndarray:
    """Each head's slots from least to most recently used, ties to the lower slot: the order in
    which the reference's stable sort offers them as victims (lazykv/tiered.py:412)."""
    return np.argsort(last_used, axis=1, kind="stable")