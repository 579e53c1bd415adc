"""The one-call decode step (lkv_select_decode: the bound kernel, then the top K chosen inside the
decode launch up to 8,192 candidates per head, or by its own launch beyond) against the
two-entry-point path (lkv_bound_topk, then lkv_sparse_decode) and against the oracle: the selected
ids are identical, the outputs equal bit for bit (the same plan and partials), and both match the
float64 oracle within the 2e-3 bar (lazykv/selection.py:38-62, lazykv/attention.py:97-136)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference as R

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _layer(seed: int, h: int, g: int, n: int, bs: int, d: int, dt: torch.dtype):
    """A layer as the tier holds it: pool [n, h, 2, bs, d] (block n - 1 is the current one) and the
    metadata of blocks 0..n-1 [1, h, n, d]."""
    from lazykv_amd.workload import draw_layer, to_pool

    w = draw_layer(seed, h * g, h, d, n * bs, bs, dt)
    pool = to_pool(w.keys, w.values, bs)
    blocks = w.keys.view(h, n, bs, d)  # exact per-channel extremes, representable in the model dtype
    kmin = blocks.amin(dim=2)[None].cuda()
    kmax = blocks.amax(dim=2)[None].cuda()
    return w, pool, kmin, kmax


CASES = [
    # (KV heads, group, blocks, block size, head dim, k, fill, dtype, where the selected pairs live)
    (8, 4, 8192, 16, 128, 512, 16, torch.bfloat16, "host"),  # the 128K-token 8B-shaped layer, zero-copy
    (8, 4, 8192, 16, 128, 512, 16, torch.bfloat16, "hbm"),
    (8, 4, 2048, 16, 64, 512, 16, torch.float16, "hbm"),  # the 32K-token 1B-shaped layer
    (8, 4, 4096, 16, 64, 1024, 16, torch.float16, "int8-hbm"),  # the 64K-token int8 tier
    (8, 4, 300, 16, 128, 64, 5, torch.bfloat16, "int8-host"),
    (2, 8, 500, 16, 128, 37, 9, torch.bfloat16, "hbm"),
    (4, 2, 130, 32, 64, 100, 1, torch.float16, "host"),
    (1, 4, 700, 16, 64, 3, 16, torch.bfloat16, "hbm"),
    (4, 1, 60, 64, 128, 58, 60, torch.float16, "hbm"),  # every candidate selected
    (2, 4, 2050, 16, 64, 300, 3, torch.float16, "hbm"),  # 2,048 candidates: the most in 2,048 key slots
    (2, 4, 2051, 16, 64, 300, 3, torch.float16, "hbm"),  # 2,049: 4,096 key slots
    (2, 4, 4098, 16, 128, 300, 3, torch.bfloat16, "host"),  # 4,096: the most a host launch selects inside itself
    (2, 4, 4099, 16, 128, 300, 3, torch.bfloat16, "host"),  # 4,097 from host memory: the top-K in its own launch
    (2, 4, 4098, 16, 64, 300, 3, torch.bfloat16, "hbm"),  # 4,096 candidates: the most in 4,096 key slots
    (2, 4, 4099, 16, 64, 300, 3, torch.bfloat16, "hbm"),  # 4,097: 8,192 key slots
    (2, 4, 8194, 16, 64, 600, 3, torch.float16, "hbm"),  # 8,192: the most selected inside the decode launch
    (1, 8, 8195, 16, 64, 600, 3, torch.float16, "hbm"),  # 8,193: the top-K in its own launch
    (1, 8, 20002, 16, 64, 700, 12, torch.float16, "host"),  # 20,000: the streaming top-K
]


@pytest.mark.parametrize(("h", "g", "n", "bs", "d", "k", "fill", "dt", "where"), CASES)
def test_select_decode_equals_the_two_launch_path_and_the_oracle(h: int, g: int, n: int, bs: int, d: int, k: int, fill: int, dt: torch.dtype, where: str) -> None:
    _check_one_call(h, g, n, bs, d, k, fill, dt, where)


# Launches whose decode instance is not a matrix-core one over HBM pairs: a float32 query takes the
# 8-wave vector instance, which has no selecting form, so the one-call step selects in its own
# launch and then decodes as the two-call path does; int8 records at head_dim 128 with a group of 4
# take the 4-wave instance over the HBM plan, which selects inside the launch only up to 16 keys per
# thread of its 256 (4,096 candidates).
CASES_OTHER_INSTANCES = [
    (8, 4, 2048, 16, 64, 512, 16, torch.float16, "hbm", True),
    (8, 4, 8192, 16, 128, 512, 16, torch.bfloat16, "hbm", True),
    (2, 2, 700, 16, 128, 50, 7, torch.bfloat16, "hbm", True),
    (4, 4, 4098, 16, 128, 300, 9, torch.bfloat16, "int8-hbm", False),  # 4,096 candidates: inside, 16 keys per thread
    (4, 4, 4102, 16, 128, 300, 9, torch.bfloat16, "int8-hbm", False),  # 4,100: the selection's own launch
]


@pytest.mark.parametrize(("h", "g", "n", "bs", "d", "k", "fill", "dt", "where", "q_f32"), CASES_OTHER_INSTANCES)
def test_select_decode_equals_the_two_launch_path_on_other_instances(h: int, g: int, n: int, bs: int, d: int, k: int, fill: int, dt: torch.dtype,
                                                                      where: str, q_f32: bool) -> None:
    _check_one_call(h, g, n, bs, d, k, fill, dt, where, q_f32=q_f32)


def _check_one_call(h: int, g: int, n: int, bs: int, d: int, k: int, fill: int, dt: torch.dtype, where: str, q_f32: bool = False) -> None:
    """lkv_select_decode against lkv_bound_topk + lkv_sparse_decode on one layer: the same ids, the
    same output bits, and both within the bar of the float64 oracle."""
    from lazykv_amd import kernels
    from lazykv_amd.pinned import pinned_empty
    from lazykv_amd.quant import packed_pair_bytes

    print(f"fused decode case: h={h} g={g} n={n} bs={bs} d={d} k={k} fill={fill} {dt} {where} q_f32={q_f32}", flush=True)
    w, pool, kmin, kmax = _layer(n * 7 + d + k, h, g, n, bs, d, dt)
    n_cand = n - 2  # blocks 1 .. n - 2; block n - 1 is the current block
    tag = "bf16" if dt == torch.bfloat16 else "f16"
    if where.startswith("int8"):
        recs = R.pack(_bits(pool), tag)
        store = pinned_empty((n, h, packed_pair_bytes(bs, d)), torch.uint8) if where.endswith("host") else torch.empty((n, h, packed_pair_bytes(bs, d)), dtype=torch.uint8, device="cuda")
        store.copy_(torch.from_numpy(recs))
        sel = kernels.record_source(store, dt)
        deq_bits = R.unpack(recs.reshape(n * h, -1), bs, d, tag).reshape(n, h, 2, bs, d)

        def stored(b, j):
            x = R.to_f32(deq_bits[b, j], tag).astype(np.float64)
            return x[0], x[1]
    else:
        store = pinned_empty(tuple(pool.shape), dt) if where == "host" else pool.cuda()
        if where == "host":
            store.copy_(pool)
        sel = kernels.pool_source(store)

        def stored(b, j):
            x = _f64(pool[b, j])
            return x[0], x[1]
    slots = pool[[0, n - 1]].contiguous().cuda()
    ss = kernels.pool_source(slots)
    q = w.query.float().cuda() if q_f32 else w.query.cuda()
    scale = d**-0.5
    common = dict(block_size=bs, scale=scale, sel=sel, sink=ss, sink_block=0, cur=ss, cur_block=1, fill=fill)
    idx_f = torch.full((h, k), -1, dtype=torch.int32, device="cuda")
    ws = kernels.Workspace()
    out_f, lse_f = kernels.select_decode(q, kmin, kmax, k, cand_offset=1, n_cand=n_cand, out_idx=idx_f, out_dtype=torch.float32, ws=ws, **common)
    idx_2 = kernels.bound_topk(q, kmin, kmax, k, cand_offset=1, n_cand=n_cand, ws=ws)
    out_2, lse_2 = kernels.sparse_decode(q, n_kv=h, idx=idx_2, out_dtype=torch.float32, ws=ws, **common)
    # Once more on the same workspace, after the two-call path used it.
    out_g, lse_g = kernels.select_decode(q, kmin, kmax, k, cand_offset=1, n_cand=n_cand, out_dtype=torch.float32, ws=ws, **common)
    torch.cuda.synchronize()
    assert torch.equal(idx_f, idx_2)
    assert torch.equal(out_f, out_2) and torch.equal(lse_f, lse_2)
    assert torch.equal(out_g, out_f) and torch.equal(lse_g, lse_f)
    # The oracle: the selected set (near-tie rule) and the attention over it.
    bound = R.quest_bound(_f64(w.query), _f64(kmin[0, :, 1 : n - 1]), _f64(kmax[0, :, 1 : n - 1]))
    chosen = idx_f.cpu().numpy()
    for j in range(h):
        assert (np.diff(chosen[j]) > 0).all(), j  # ascending, distinct
        ok, _ = R.selection_ok(chosen[j] - 1, bound[j], k, abs_err=1e-3)
        assert ok, j

    def bkv(j, b):
        if b in (0, n - 1):  # sink and current block stay in the model dtype
            x = _f64(pool[b, j])
            return x[0], x[1]
        return stored(b, j)

    ks, vs = R.gathered_tokens(bkv, h, chosen, 0, n - 1, fill, bs)
    want_o, want_l = R.attend_tokens(_f64(w.query), ks, vs, scale)
    assert np.abs(out_f.cpu().numpy() - want_o).max() < TOL
    assert np.abs(lse_f.cpu().numpy() - want_l).max() < TOL


def test_fused_step_replays_in_a_graph_like_the_eager_call() -> None:
    """The one-call step captured in a HIP graph (bound kernel, the decode launch choosing the top K,
    the merge launch): every replay, with unrelated eager work and synchronisations between replays,
    equals the eager result bit for bit."""
    from lazykv_amd import kernels

    h, g, n, bs, d, k = 8, 4, 1030, 16, 128, 128
    w, pool, kmin, kmax = _layer(99, h, g, n, bs, d, torch.bfloat16)
    store = pool.cuda()
    src = kernels.pool_source(store)
    ss = kernels.pool_source(pool[[0, n - 1]].contiguous().cuda())
    q = w.query.cuda()
    out = torch.empty((h * g, d), dtype=torch.float32, device="cuda")
    lse = torch.empty((h * g,), dtype=torch.float32, device="cuda")
    step = kernels.PreparedSelectDecode(q, kmin, kmax, k, cand_offset=1, n_cand=n - 2, block_size=bs, scale=d**-0.5, sel=src, sink=ss, sink_block=0,
                                        cur=ss, cur_block=1, fill=7, out=out, lse=lse, ws=kernels.Workspace())
    step()
    torch.cuda.synchronize()
    want_o, want_l = out.clone(), lse.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()
    for rep in range(5):
        out.zero_()
        lse.zero_()
        noise = torch.randn(1 << 20, device="cuda").sum()  # unrelated eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(noise)
        assert torch.equal(out, want_o) and torch.equal(lse, want_l), rep


def test_tier_takes_the_fused_launch_and_agrees_with_rank_then_decode() -> None:
    """TieredCache.select decodes through lkv_select_decode (one call per selecting layer); its
    output equals rank() + decode(idx) (the two-entry-point path) bit for bit."""
    from lazykv_amd.tiered import TieredCache

    h, g, d, bs, k = 8, 4, 128, 16, 24
    gen = torch.Generator().manual_seed(5)
    keys = (torch.randn((1, h, 700, d), generator=gen) * 1.3).to(torch.bfloat16).cuda()
    values = torch.randn((1, h, 700, d), generator=gen).to(torch.bfloat16).cuda()
    for fetch in ("zerocopy", "resident"):
        cache = TieredCache([(keys, values)] * 2, k, bs, 1024, dense_layers=1, fetch=fetch)
        tier = cache.tiers[1]
        assert tier.fused_select()
        q = torch.randn((1, h * g, 1, d), generator=gen).to(torch.bfloat16).cuda()
        dec = cache.select(1, q)
        idx = tier.rank(q)
        out2, lse2 = tier.decode(q, None, idx=idx)
        torch.cuda.synchronize()
        assert torch.equal(dec.out.view(h * g, d), out2) and torch.equal(dec.lse.view(-1), lse2), fetch


def test_select_decode_refuses_what_it_cannot_do() -> None:
    from lazykv_amd import kernels

    h, d, bs = 2, 64, 16
    kmin = torch.zeros((1, h, 300, d), dtype=torch.float16, device="cuda")
    pool = torch.zeros((4, h, 2, bs, d), dtype=torch.float16, device="cuda")
    src = kernels.pool_source(pool)
    q = torch.zeros((h * 4, d), dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):  # nothing selected
        kernels.select_decode(q, kmin, kmin, 0, cand_offset=1, n_cand=100, block_size=bs, scale=0.1, sel=src)
    with pytest.raises(ValueError):  # more selected than there are candidates
        kernels.select_decode(q, kmin, kmin, 101, cand_offset=1, n_cand=100, block_size=bs, scale=0.1, sel=src)
    with pytest.raises(ValueError):  # candidates past the metadata
        kernels.select_decode(q, kmin, kmin, 10, cand_offset=1, n_cand=300, block_size=bs, scale=0.1, sel=src)


def _designed_bounds(kind: str, n: int, rng: np.random.Generator) -> np.ndarray:
    """Bounds that exercise each exit of the in-workgroup selection (as bfloat16 values)."""
    if kind == "all equal":  # one value: ties only, taken in index order
        b = np.full(n, 1.5)
    elif kind == "three values":  # the threshold value repeated hundreds of times
        b = rng.choice([0.5, 1.0, 2.0], size=n)
    elif kind == "outlier and a dense cluster":
        # One huge bound stretches the first pass's range so wide that the cluster of every other
        # bound falls into one bin holding far more keys than threads: a second pass is needed,
        # whose boundary bin is then ranked directly among heavy ties.
        b = 1.0 + rng.integers(0, 8, size=n) / 128.0
        b[n // 3] = 3.0e38
    elif kind == "distinct":  # every bound different: the boundary bin is taken whole or ranked
        b = rng.permutation(n).astype(np.float64) / 8.0 - n / 16.0
    else:  # "negative and zero": signs and a zero mix in the order-preserving keys
        b = rng.choice([-2.0, -0.0, 0.0, 0.25], size=n)
    return b


DESIGNED = [
    ("all equal", 2, 4, 1000, 300),
    ("three values", 2, 4, 4094, 1024),
    ("outlier and a dense cluster", 1, 4, 4094, 1500),
    ("distinct", 2, 4, 2046, 512),
    ("negative and zero", 2, 4, 3000, 1100),
    ("three values", 1, 8, 4096, 4096),  # every candidate selected
    ("outlier and a dense cluster", 2, 4, 8000, 2500),  # 8,192 key slots
    ("distinct", 1, 4, 8190, 512),
]


@pytest.mark.parametrize(("kind", "h", "g", "n_cand", "k"), DESIGNED)
def test_selection_inside_the_decode_launch_on_designed_bounds(kind: str, h: int, g: int, n_cand: int, k: int) -> None:
    """With a one-hot query every bound is exactly one metadata value, so the selected set is known
    exactly: the k largest, ties towards the lower id. The one-call path, the two-call path (its
    own selection kernel) and that set agree id for id, and the outputs bit for bit."""
    from lazykv_amd import kernels

    print(f"designed bounds: {kind} h={h} g={g} n_cand={n_cand} k={k}", flush=True)
    rng = np.random.default_rng(n_cand + k)
    bs, d, n = 16, 64, n_cand + 2
    dt = torch.bfloat16
    b = _designed_bounds(kind, n_cand, rng)
    kmax = torch.zeros((1, h, n, d), dtype=dt)
    for j in range(h):
        kmax[0, j, 1 : n - 1, 0] = torch.from_numpy(b).to(dt)
    exact = kmax[0, :, 1 : n - 1, 0].float().numpy().astype(np.float64)  # the bounds the kernels see
    kmin = kmax.clone()
    q = torch.zeros((h * g, d), dtype=dt)
    q[:, 0] = 1.0  # bound = sum_d max(q kmax, q kmin) = kmax[..., 0]
    pool = (torch.randn((n, h, 2, bs, d), generator=torch.Generator().manual_seed(k)) * 0.5).to(dt)
    store, kmin, kmax, q = pool.cuda(), kmin.cuda(), kmax.cuda(), q.cuda()
    sel = kernels.pool_source(store)
    common = dict(block_size=bs, scale=d**-0.5, sel=sel, sink=sel, sink_block=0, cur=sel, cur_block=n - 1, fill=bs)
    ws = kernels.Workspace()
    idx_f = torch.full((h, k), -1, dtype=torch.int32, device="cuda")
    out_f, lse_f = kernels.select_decode(q, kmin, kmax, k, cand_offset=1, n_cand=n_cand, out_idx=idx_f, out_dtype=torch.float32, ws=ws, **common)
    idx_2 = kernels.bound_topk(q, kmin, kmax, k, cand_offset=1, n_cand=n_cand, ws=ws)
    out_2, lse_2 = kernels.sparse_decode(q, n_kv=h, idx=idx_2, out_dtype=torch.float32, ws=ws, **common)
    torch.cuda.synchronize()
    for j in range(h):
        order = np.lexsort((np.arange(n_cand), -exact[j]))  # bound descending, then id ascending
        want = np.sort(order[:k]) + 1
        assert np.array_equal(idx_f[j].cpu().numpy(), want), (kind, j)
    assert torch.equal(idx_f, idx_2)
    assert torch.equal(out_f, out_2) and torch.equal(lse_f, lse_2)
