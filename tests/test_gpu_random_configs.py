"""Seeded random decode configurations against the float64 oracle (GPU).

Each case draws the number of KV heads, the group size, head_dim, block size, budget, current-block
fill, model dtype, where the selected blocks live (HBM or mapped host memory), whether they are
int8 records, and whether an exact remainder partial is added (from HBM or host memory, model
dtype or int8). The kernels then take every launch shape and instance in combinations the
hand-picked cases do not: 4- and 8-wave workgroups, the matrix-core and vector instances, one to
three pairs per step, chunked and short blocks. Bars as elsewhere: float32 output and LSE within
2e-3 of the float64 oracle. A second sweep draws bound + top-K calls (candidate counts on both
sides of the in-register limit, offsets, sorted and ascending output): the float32 bounds within
the accumulation error bound of the float64 ones, the selected sets under the near-tie rule. A
third draws hybrid residency configurations over drifting steps: bit-identical to the zero-copy
decode, tables and use order equal to the oracle's.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference as R

pytestmark = pytest.mark.gpu

TOL = 2e-3
N_CASES = 64


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _case(seed: int) -> dict:
    rng = np.random.default_rng(1000 + seed)
    d = int(rng.choice([64, 128]))
    bs = int(rng.choice([4, 8, 16, 16, 16, 20, 32, 64, 128, 256]))
    n = int(rng.integers(8, max(9, 4096 // bs)))
    return {
        "h": int(rng.choice([1, 2, 3, 4, 8])),
        "g": int(rng.choice([1, 2, 4, 4, 8])),
        "d": d,
        "bs": bs,
        "n": n,
        "k": int(rng.integers(1, n - 1)),
        "fill": int(rng.integers(1, bs + 1)),
        "dt": [torch.float16, torch.bfloat16][int(rng.integers(0, 2))],
        "sel_where": str(rng.choice(["hbm", "hbm", "host"])),
        "sel_int8": bool(rng.random() < 0.3),
        "rem": str(rng.choice(["none", "none", "hbm", "host"])),
        "rem_int8": bool(rng.random() < 0.5),
    }


def _place(t: torch.Tensor, where: str) -> torch.Tensor:
    from lazykv_amd.pinned import pinned_empty

    out = pinned_empty(tuple(t.shape), t.dtype) if where == "host" else torch.empty(tuple(t.shape), dtype=t.dtype, device="cuda")
    out.copy_(t)
    return out


@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_decode_configuration_matches_the_oracle(seed: int) -> None:
    from lazykv_amd import kernels
    from lazykv_amd.quant import packed_pair_bytes
    from lazykv_amd.workload import draw_layer, to_pool

    c = _case(seed)
    h, g, d, bs, n, k, fill, dt = c["h"], c["g"], c["d"], c["bs"], c["n"], c["k"], c["fill"], c["dt"]
    name = "bf16" if dt == torch.bfloat16 else "f16"
    print(f"case {seed}: {c}", flush=True)
    w = draw_layer(seed, h * g, h, d, n * bs, bs, dt)
    pool = to_pool(w.keys, w.values, bs)  # [n, h, 2, bs, d]
    exact = pool.double().numpy()
    recs = R.pack(_bits(pool), name)  # [n, h, P]
    deq = R.to_f32(R.unpack(recs.reshape(n * h, -1), bs, d, name), name).reshape(n, h, 2, bs, d).astype(np.float64)

    def source(int8: bool, where: str):  # noqa: ANN202
        if int8:
            store = _place(torch.from_numpy(recs).view(torch.uint8).reshape(n, h, packed_pair_bytes(bs, d)), where)
            return kernels.record_source(store, dt), deq, store
        store = _place(pool, where)
        return kernels.pool_source(store), exact, store

    sel, sel_vals, keep_sel = source(c["sel_int8"], c["sel_where"])
    slots = pool[[0, n - 1]].contiguous().cuda()  # sink and current in the model dtype, in HBM
    ss = kernels.pool_source(slots)
    gen = torch.Generator().manual_seed(seed)
    chosen = torch.stack([torch.randperm(n - 2, generator=gen)[:k] + 1 for _ in range(h)]).to(torch.int32)
    extra: dict = {}
    rem_vals = None
    keep_rem = None
    if c["rem"] != "none":
        rem, rem_vals, keep_rem = source(c["rem_int8"], c["rem"])
        extra = {"rem": rem, "rem_range": (1, n - 1)}
    out, lse = kernels.sparse_decode(w.query.cuda(), n_kv=h, block_size=bs, scale=d**-0.5, sel=sel, idx=chosen.cuda(), sink=ss, sink_block=0, cur=ss,
                                     cur_block=1, fill=fill, out_dtype=torch.float32, **extra)
    torch.cuda.synchronize()
    del keep_sel, keep_rem
    q = w.query.double().numpy()
    ks, vs = [], []
    for j in range(h):
        picked = set(chosen[j].tolist())
        kk, vv = [exact[0, j, 0]], [exact[0, j, 1]]
        for b in range(1, n - 1):
            if b in picked:
                kk.append(sel_vals[b, j, 0])
                vv.append(sel_vals[b, j, 1])
            elif rem_vals is not None:
                kk.append(rem_vals[b, j, 0])
                vv.append(rem_vals[b, j, 1])
        kk.append(exact[n - 1, j, 0, :fill])
        vv.append(exact[n - 1, j, 1, :fill])
        ks.append(np.concatenate(kk))
        vs.append(np.concatenate(vv))
    want_o, want_l = R.attend_tokens(q, ks, vs, d**-0.5)
    assert np.abs(out.cpu().numpy() - want_o).max() < TOL, c
    assert np.abs(lse.cpu().numpy() - want_l).max() < TOL, c


def _sel_case(seed: int) -> dict:
    rng = np.random.default_rng(5000 + seed)
    n = int(rng.choice([5, 64, 500, 2046, 4094, 8190, 12288, 12289, 20000]))
    h = int(rng.choice([1, 2, 3, 4, 8]))
    if h * n > 60000:
        h = max(1, 60000 // n)
    sorted_ = bool(rng.random() < 0.3)
    return {
        "d": int(rng.choice([64, 128])),
        "h": h,
        "g": int(rng.choice([1, 2, 4, 8])),
        "n": n,
        "offset": int(rng.integers(0, 3)),
        "k": int(rng.integers(1, min(n, 2048 if sorted_ else 4096) + 1)),
        "sorted": sorted_,
        "dt": [torch.float16, torch.bfloat16][int(rng.integers(0, 2))],
    }


@pytest.mark.parametrize("seed", range(32))
def test_random_selection_matches_the_oracle(seed: int) -> None:
    """Bound + top-K over random metadata: up to 20,000 candidates per head (past the 12,288 that
    one workgroup holds in registers), offsets, unsorted (ascending ids) and sorted (descending
    bound, lower id first on ties) output."""
    from lazykv_amd import kernels

    c = _sel_case(seed)
    d, h, g, n, off, k, dt = c["d"], c["h"], c["g"], c["n"], c["offset"], c["k"], c["dt"]
    print(f"selection case {seed}: {c}", flush=True)
    gen = torch.Generator().manual_seed(seed)
    cap = off + n + 1
    centre = torch.randn((1, h, cap, d), generator=gen) * (torch.rand((1, h, 1, d), generator=gen) * 1.5 + 0.5)
    kmin = (centre - torch.rand((1, h, cap, d), generator=gen)).to(dt)
    kmax = (centre + torch.rand((1, h, cap, d), generator=gen)).to(dt)
    q = torch.randn((h * g, d), generator=gen).to(dt)
    bounds = torch.empty((h, n), dtype=torch.float32, device="cuda")
    idx = kernels.bound_topk(q.cuda(), kmin.cuda(), kmax.cuda(), k, cand_offset=off, n_cand=n, sorted_=c["sorted"], out_bound=bounds)
    torch.cuda.synchronize()
    qf = q.double().numpy()
    lo, hi = kmin[0, :, off : off + n].double().numpy(), kmax[0, :, off : off + n].double().numpy()
    want = R.quest_bound(qf, lo, hi)
    err = float(np.abs(qf).max() * np.maximum(np.abs(lo), np.abs(hi)).sum(-1).max()) * 2.0**-19
    got_b = bounds.cpu().numpy()
    assert np.abs(got_b - want).max() <= err
    top = idx.cpu().numpy() - off
    for j in range(h):
        ok, _ = R.selection_ok(top[j], want[j], k, abs_err=err)
        assert ok, (j, c)
        if c["sorted"]:
            b = got_b[j][top[j]]
            assert (np.diff(b) <= 0).all() and all(top[j][i] < top[j][i + 1] for i in range(k - 1) if b[i] == b[i + 1]), c
        else:
            assert (np.diff(top[j]) > 0).all(), c


@pytest.mark.parametrize("seed", range(24))
def test_random_block_store_matches_the_oracle(seed: int) -> None:
    """store_blocks over random ranges: metadata only, a copy into the pool layout, or int8 records
    (HBM or mapped host memory), bs 4-256. Copies and records bit for bit (quant.py's pack), the
    metadata the exact min/max of the keys as stored (dequantised for records), and nothing outside
    the range touched."""
    from lazykv_amd import kernels
    from lazykv_amd.pinned import pinned_empty
    from lazykv_amd.quant import packed_pair_bytes

    rng = np.random.default_rng(9000 + seed)
    d = int(rng.choice([64, 128]))
    bs = int(rng.choice([4, 8, 16, 16, 20, 32, 64, 128, 256]))
    h = int(rng.integers(1, 9))
    n = int(rng.integers(2, max(3, 2048 // bs)))
    first = int(rng.integers(0, n))
    count = int(rng.integers(1, n - first + 1))
    dt = [torch.float16, torch.bfloat16][int(rng.integers(0, 2))]
    mode = str(rng.choice(["meta", "copy", "int8"]))
    where = str(rng.choice(["hbm", "host"]))
    name = "bf16" if dt == torch.bfloat16 else "f16"
    print(f"store case {seed}: d={d} bs={bs} h={h} n={n} first={first} count={count} {dt} {mode} {where}", flush=True)
    gen = torch.Generator().manual_seed(seed)
    keys = (torch.randn((1, h, n * bs, d), generator=gen) * (torch.rand((1, h, 1, d), generator=gen) * 3 + 0.1)).to(dt)
    values = torch.randn((1, h, n * bs, d), generator=gen).to(dt)
    pairs = torch.stack([keys[0], values[0]], dim=1).view(h, 2, n, bs, d).permute(2, 0, 1, 3, 4).contiguous()  # [n, h, 2, bs, d]
    kmin = torch.zeros((1, h, n, d), dtype=dt, device="cuda")
    kmax = torch.zeros_like(kmin)

    def alloc(shape, dtype):  # noqa: ANN001, ANN202
        t = pinned_empty(shape, dtype) if where == "host" else torch.empty(shape, dtype=dtype, device="cuda")
        t.zero_()
        return t

    dst, store = None, None
    if mode == "copy":
        store = alloc((n, h, 2, bs, d), dt)
        dst = kernels.pool_source(store)
    elif mode == "int8":
        store = alloc((n, h, packed_pair_bytes(bs, d)), torch.uint8)
        dst = kernels.record_source(store, dt)
    kernels.store_blocks(kernels.dense_source(keys.cuda(), values.cuda(), bs), dst=dst, n_kv=h, head_dim=d, block_size=bs, first_block=first, n_blocks=count,
                         kmin=kmin, kmax=kmax)
    torch.cuda.synchronize()
    rng_b = slice(first, first + count)
    if mode == "int8":
        want = R.pack(_bits(pairs[rng_b]), name)
        got = store.cpu().numpy()
        assert np.array_equal(got[rng_b], want)
        assert not got[:first].any() and not got[first + count :].any()
        stored_keys = R.to_f32(R.unpack(want.reshape(count * h, -1), bs, d, name), name).reshape(count, h, 2, bs, d)[:, :, 0].astype(np.float64)
    else:
        if mode == "copy":
            got = store.cpu()
            assert torch.equal(got[rng_b], pairs[rng_b])
            assert not got[:first].any() and not got[first + count :].any()
        stored_keys = pairs[rng_b][:, :, 0].double().numpy()
    mn = kmin[0].cpu().double().numpy().transpose(1, 0, 2)  # [n, h, d]
    mx = kmax[0].cpu().double().numpy().transpose(1, 0, 2)
    assert np.array_equal(mn[rng_b], stored_keys.min(axis=2)) and np.array_equal(mx[rng_b], stored_keys.max(axis=2))
    assert not mn[:first].any() and not mn[first + count :].any()


N_HYBRID = 24


def _hybrid_case(seed: int) -> dict:
    rng = np.random.default_rng(5000 + seed)
    bs = int(rng.choice([4, 8, 16, 16, 16, 32, 64]))
    n = int(rng.integers(24, max(25, 2048 // bs)))
    k = int(rng.integers(1, min(n - 2, 600)))
    return {
        "h": int(rng.choice([1, 2, 4, 8])),
        "g": int(rng.choice([1, 2, 4, 8])),
        "d": int(rng.choice([64, 128])),
        "bs": bs,
        "n": n,
        "k": k,
        "spare": int(rng.choice([0, 0, int(rng.integers(1, k + 2))])),
        "fill": int(rng.integers(1, bs + 1)),
        "dt": [torch.float16, torch.bfloat16][int(rng.integers(0, 2))],
        "int8": bool(rng.random() < 0.4),
    }


@pytest.mark.parametrize("seed", range(N_HYBRID))
def test_random_hybrid_configuration_is_the_zero_copy_decode(seed: int) -> None:
    """Seeded random hybrid configurations (KV heads, group size, head_dim, block size -- the
    pipelined item loop for model-dtype pools of blocks up to 16 tokens, the one-pair loop
    otherwise --, budget, spare slots, dtype, bf16/f16 pairs or int8 records) over five drifting
    steps: output and LSE equal the zero-copy decode's bit for bit, the tables and use order equal
    the oracle's, and every occupied slot holds its block as a decode reads it."""
    from lazykv_amd import kernels
    from lazykv_amd.pinned import pinned_empty
    from lazykv_amd.workload import draw_layer, to_pool

    c = _hybrid_case(seed)
    h, g, d, bs, n, k, dt = c["h"], c["g"], c["d"], c["bs"], c["n"], c["k"], c["dt"]
    print(f"hybrid case {seed}: {c}", flush=True)
    w = draw_layer(seed, h * g, h, d, n * bs, bs, dt)
    pool = to_pool(w.keys, w.values, bs).cuda()
    kmin = torch.zeros((1, h, n, d), dtype=dt, device="cuda")
    kmax = torch.zeros_like(kmin)
    kernels.store_blocks(kernels.dense_source(w.keys.cuda(), w.values.cuda(), bs), n_kv=h, head_dim=d, block_size=bs, first_block=0, n_blocks=n - 1,
                         kmin=kmin, kmax=kmax)
    expect = pool
    if c["int8"]:
        recs = kernels.pack_int8(pool.reshape(n * h, 2, bs, d))
        expect = kernels.unpack_int8(recs, bs, d, dt).reshape(n, h, 2, bs, d)
        host = pinned_empty((n, h, recs.shape[1]), torch.uint8)
        host.copy_(recs.reshape(n, h, -1))
        hsrc = kernels.record_source(host, dt)
    else:
        host = pinned_empty(tuple(pool.shape), dt)
        host.copy_(pool)
        hsrc = kernels.pool_source(host)
    n_slots = k + c["spare"]
    res = kernels.Residency.allocate(k, h, n, bs, d, dt, torch.device("cuda"), n_slots=n_slots)
    tb, ts, tl = R.residency_state(h, n_slots, n)
    ss = kernels.pool_source(pool[[0, n - 1]].contiguous())
    gen = torch.Generator().manual_seed(seed)
    q0 = w.query.float()
    for step in range(5):
        q = (q0 + 0.35 * torch.randn(q0.shape, generator=gen)).to(dt).cuda()
        idx = kernels.bound_topk(q, kmin, kmax, k, cand_offset=1, n_cand=n - 2)
        common = dict(n_kv=h, block_size=bs, scale=d**-0.5, idx=idx, sink=ss, sink_block=0, cur=ss, cur_block=1, fill=c["fill"], out_dtype=torch.float32)
        out_z, lse_z = kernels.sparse_decode(q, sel=hsrc, **common)
        out_h, lse_h = kernels.hybrid_decode(q, host=hsrc, res=res, **common)
        torch.cuda.synchronize()
        assert torch.equal(out_h, out_z) and torch.equal(lse_h, lse_z), step
        R.residency_step(tb, ts, tl, idx.cpu().numpy().astype(np.int64), step)
        assert np.array_equal(res.block_slot.cpu().numpy(), tb), step
        assert np.array_equal(res.slot_block.cpu().numpy(), ts), step
        assert np.array_equal(res.order.cpu().numpy(), R.slot_order(tl)), step
        for j in range(h):
            held = np.flatnonzero(ts[j] >= 0)
            assert torch.equal(res.slots[torch.from_numpy(held).cuda(), j], expect[torch.from_numpy(ts[j, held]).cuda(), j]), (step, j)
