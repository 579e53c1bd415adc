"""Kernel parity on the GPU, through the C ABI, against the oracle.

Integer and byte work (int8 records, block ids, metadata) must be bit-exact; attention output and
LSE (float32 accumulation) must be within 2e-3 max-abs of the float64 oracle on the same inputs.
Selected sets must equal the oracle's top-K except where the K-th and (K+1)-th bounds are a near
tie (oracle.reference.selection_ok).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import reference as R

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "quant_vectors.npz"
TOL = 2e-3
DT = {"f16": torch.float16, "bf16": torch.bfloat16}


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def _from_bits(bits: np.ndarray, dt: str) -> torch.Tensor:
    return torch.from_numpy(bits.astype(np.uint16).view(np.int16)).view(DT[dt])


# -- int8 records ----------------------------------------------------------------------------------


def _golden_cases():
    g = np.load(GOLDEN)
    out = []
    for key in sorted(k[: -len("_in")] for k in g.files if k.endswith("_in")):
        dt, bs, d = key.split("_")
        if int(d[1:]) in (64, 128):
            out.append((key, dt, int(bs[2:]), int(d[1:])))
    return out


@pytest.mark.parametrize(("key", "dt", "bs", "d"), _golden_cases())
def test_pack_and_unpack_reproduce_the_reference_bytes(key: str, dt: str, bs: int, d: int) -> None:
    from lazykv_amd import quant

    g = np.load(GOLDEN)
    x = _from_bits(g[f"{key}_in"], dt).cuda()
    packed = quant.pack(x)
    assert np.array_equal(packed.cpu().numpy(), g[f"{key}_packed"])
    back = quant.unpack(torch.from_numpy(g[f"{key}_packed"]).cuda(), bs, d, DT[dt])
    assert np.array_equal(_bits(back), g[f"{key}_unpacked"])


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize(("bs", "d"), [(16, 128), (16, 64), (8, 64), (64, 128), (128, 64), (256, 128)])
def test_pack_unpack_bit_exact_on_seeded_data(dt: str, bs: int, d: int) -> None:
    from lazykv_amd import quant

    gen = torch.Generator().manual_seed(bs * 1000 + d)
    scale = torch.rand((1, 2, 1, d), generator=gen) * 1.5 + 0.5
    x = (torch.randn((300, 2, bs, d), generator=gen) * scale).to(DT[dt])
    x[7, 0, :, 5] = 1.25  # a constant key channel
    x[9, 1, 3, :] = -0.5  # a constant value token
    x[11, 0, :, 0] *= 300  # an outlier channel
    packed = quant.pack(x.cuda())
    want = R.pack(_bits(x), dt)
    assert np.array_equal(packed.cpu().numpy(), want)
    back = quant.unpack(packed, bs, d, DT[dt])
    assert np.array_equal(_bits(back), R.unpack(want, bs, d, dt).reshape(_bits(back).shape))
    back32 = quant.unpack(packed, bs, d, torch.float32)
    assert np.array_equal(back32.cpu().numpy(), R.unpack_f32(want, bs, d))


def test_pack_rejects_what_the_reference_rejects() -> None:
    from lazykv_amd import quant

    with pytest.raises(ValueError, match="KV pair"):
        quant.pack(torch.zeros((3, 3, 16, 64), dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(ValueError, match="uint8 records"):
        quant.unpack(torch.zeros((2, 7), dtype=torch.uint8, device="cuda"), 16, 64, torch.bfloat16)


# -- block stores and metadata ---------------------------------------------------------------------


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_store_blocks_copies_pairs_and_writes_exact_metadata(dt: str) -> None:
    from lazykv_amd import kernels

    h, bs, d, n = 4, 16, 128, 37
    gen = torch.Generator().manual_seed(11)
    keys = torch.randn((1, h, n * bs + 5, d), generator=gen).to(DT[dt]).cuda()
    values = torch.randn((1, h, n * bs + 5, d), generator=gen).to(DT[dt]).cuda()
    pool = torch.zeros((n + 3, h, 2, bs, d), dtype=DT[dt], device="cuda")
    kmin = torch.zeros((1, h, n + 3, d), dtype=DT[dt], device="cuda")
    kmax = torch.zeros_like(kmin)
    src = kernels.dense_source(keys, values, bs)
    kernels.store_blocks(src, dst=kernels.pool_source(pool), n_kv=h, head_dim=d, block_size=bs, first_block=2, n_blocks=n - 2, kmin=kmin, kmax=kmax)
    torch.cuda.synchronize()
    want_pool = torch.stack([keys[0, :, : n * bs], values[0, :, : n * bs]], dim=1).view(h, 2, n, bs, d).permute(2, 0, 1, 3, 4)
    assert torch.equal(pool[2:n], want_pool[2:n])
    assert (pool[:2] == 0).all() and (pool[n:] == 0).all()
    mn, mx = R.block_minmax(_f64(keys[0, :, : n * bs]), bs)
    assert np.array_equal(_f64(kmin[0, :, 2:n]), mn[:, 2:n]) and np.array_equal(_f64(kmax[0, :, 2:n]), mx[:, 2:n])
    assert (kmin[0, :, :2] == 0).all()


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_int8_store_writes_records_and_dequantised_metadata(dt: str) -> None:
    from lazykv_amd import kernels
    from lazykv_amd.pinned import pinned_empty
    from lazykv_amd.quant import packed_pair_bytes

    h, bs, d, n = 8, 16, 64, 41
    p = packed_pair_bytes(bs, d)
    gen = torch.Generator().manual_seed(12)
    keys = (torch.randn((1, h, n * bs, d), generator=gen) * 2).to(DT[dt]).cuda()
    values = torch.randn((1, h, n * bs, d), generator=gen).to(DT[dt]).cuda()
    host = pinned_empty((n, h, p), torch.uint8)
    host.zero_()
    kmin = torch.zeros((1, h, n, d), dtype=DT[dt], device="cuda")
    kmax = torch.zeros_like(kmin)
    kernels.store_blocks(kernels.dense_source(keys, values, bs), dst=kernels.record_source(host, DT[dt]), n_kv=h, head_dim=d, block_size=bs, first_block=0, n_blocks=n, kmin=kmin, kmax=kmax)
    torch.cuda.synchronize()
    pairs = torch.stack([keys[0], values[0]], dim=1).view(h, 2, n, bs, d).permute(2, 0, 1, 3, 4).contiguous()
    want = R.pack(_bits(pairs), dt)  # [n, h, P]
    assert np.array_equal(host.numpy(), want)
    deq = R.to_f32(R.unpack(want.reshape(n * h, p), bs, d, dt), dt).reshape(n, h, 2, bs, d)
    assert np.array_equal(_f64(kmin[0]), deq[:, :, 0].min(axis=2).transpose(1, 0, 2))
    assert np.array_equal(_f64(kmax[0]), deq[:, :, 0].max(axis=2).transpose(1, 0, 2))
    # The same metadata rebuilt from the records alone.
    kmin2, kmax2 = torch.zeros_like(kmin), torch.zeros_like(kmax)
    kernels.store_blocks(kernels.record_source(host, DT[dt]), n_kv=h, head_dim=d, block_size=bs, first_block=0, n_blocks=n, kmin=kmin2, kmax=kmax2)
    torch.cuda.synchronize()
    assert torch.equal(kmin2, kmin) and torch.equal(kmax2, kmax)


# -- bound and top-K -------------------------------------------------------------------------------


def _meta_case(seed: int, h: int, n_blocks: int, bs: int, d: int, g: int, dt: torch.dtype):
    gen = torch.Generator().manual_seed(seed)
    s = torch.rand((h, 1, d), generator=gen) * 1.5 + 0.5
    keys = (torch.randn((h, n_blocks * bs, d), generator=gen) * s).to(dt)
    q = torch.randn((h * g, d), generator=gen).to(dt)
    kmin, kmax = R.block_minmax(_f64(keys), bs)
    return q, torch.from_numpy(kmin).to(dt), torch.from_numpy(kmax).to(dt)


def _abs_err(q: np.ndarray, kmin: np.ndarray, kmax: np.ndarray) -> float:
    """A float32 accumulation error bound for the kernel's dot products."""
    mag = np.abs(q).max() * np.maximum(np.abs(kmin), np.abs(kmax)).sum(-1).max()
    return float(mag) * 2.0**-19


@pytest.mark.parametrize(("h", "n", "d", "g", "k"), [(8, 8190, 128, 4, 512), (8, 2046, 64, 4, 512), (2, 300, 128, 8, 17), (4, 100, 64, 1, 100), (3, 97, 128, 2, 1)])
def test_top_blocks_selects_the_oracle_set(h: int, n: int, d: int, g: int, k: int) -> None:
    from lazykv_amd import selection

    q, kmin, kmax = _meta_case(h * n + d, h, n, 16, d, g, torch.bfloat16)
    bound_gpu = selection.quest_bound(q.view(1, -1, 1, d).cuda(), kmin[None].cuda(), kmax[None].cuda(), torch.float32)[0]
    want = R.quest_bound(_f64(q), _f64(kmin), _f64(kmax))
    err = _abs_err(_f64(q), _f64(kmin), _f64(kmax))
    assert np.abs(bound_gpu.cpu().numpy() - want).max() <= err
    top = selection.top_blocks(q.view(1, -1, 1, d).cuda(), kmin[None].cuda(), kmax[None].cuda(), k, torch.float32)[0].cpu().numpy()
    assert top.shape == (h, k)
    for j in range(h):
        ok, _ = R.selection_ok(top[j], want[j], k, abs_err=err)
        assert ok, j
        # descending order of the kernel's own bounds, ties by lower id
        b = bound_gpu[j].cpu().numpy()[top[j]]
        assert (np.diff(b) <= 0).all()


@pytest.mark.parametrize(("d", "g", "dt"), [(128, 4, torch.bfloat16), (64, 4, torch.float16), (128, 8, torch.float16), (64, 1, torch.bfloat16), (128, 2, torch.bfloat16)])
def test_matrix_core_and_vector_bounds_agree_with_the_oracle(d: int, g: int, dt: torch.dtype) -> None:
    """A query in the metadata's dtype is scored on the matrix cores, a float32 query (the same
    values) by the vector kernel: both are the oracle's bound within the float32 accumulation error,
    in both rank modes, and choose the oracle's set under the near-tie rule."""
    from lazykv_amd import kernels

    h, n, k = 4, 1500, 200
    q, kmin, kmax = _meta_case(d * g + n, h, n, 16, d, g, dt)
    want = R.quest_bound(_f64(q), _f64(kmin), _f64(kmax))
    err = _abs_err(_f64(q), _f64(kmin), _f64(kmax))
    full_min = torch.cat([torch.zeros((h, 1, d), dtype=dt), kmin], dim=1)[None].cuda()
    full_max = torch.cat([torch.zeros((h, 1, d), dtype=dt), kmax], dim=1)[None].cuda()
    tag = "bf16" if dt == torch.bfloat16 else "f16"
    for qq in (q.cuda(), q.float().cuda()):  # the matrix cores, then the vector kernel
        for mode in (kernels._lib.RANK_F32, kernels._lib.RANK_MODEL):
            bnd = torch.empty((h, n), dtype=torch.float32, device="cuda")
            kernels.bound_topk(qq, full_min, full_max, 0, cand_offset=1, n_cand=n, out_bound=bnd, rank_mode=mode)
            got = bnd.cpu().numpy().astype(np.float64)
            if mode == kernels._lib.RANK_F32:
                assert np.abs(got - want).max() <= err, (qq.dtype, mode)
            else:
                # Each half-sum rounded to the model dtype, then their sum: a half-sum a few float32
                # ulps away from the oracle's can round one model-dtype ulp the other way, so allow
                # two ulps of the half-sums' magnitude bound.
                model = R.quest_bound(_f64(q), _f64(kmin), _f64(kmax), "model", tag)
                mag = np.abs(_f64(q)).max() * np.maximum(np.abs(_f64(kmin)), np.abs(_f64(kmax))).sum(-1).max()
                tol = mag * (2.0**-6 if dt == torch.bfloat16 else 2.0**-9)
                assert np.abs(got - model).max() <= tol, (qq.dtype, mode)
        idx = kernels.bound_topk(qq, full_min, full_max, k, cand_offset=1, n_cand=n)
        for j in range(h):
            assert R.selection_ok(idx[j].cpu().numpy() - 1, want[j], k, abs_err=err)[0], (qq.dtype, j)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("n", [1, 7, 16, 17, 63, 64, 65, 129])
def test_matrix_core_bound_on_partial_tiles(n: int, d: int) -> None:
    """Candidate counts around the matrix-core kernel's 16-block tiles and 64-block workgroups: a
    tile past the last candidate reads that candidate's row and writes nothing, so every bound is
    the oracle's and the words after the last row keep their sentinel."""
    from lazykv_amd import kernels

    h, g, dt = 3, 4, torch.bfloat16
    q, kmin, kmax = _meta_case(1000 * d + n, h, n, 16, d, g, dt)
    want = R.quest_bound(_f64(q), _f64(kmin), _f64(kmax))
    err = _abs_err(_f64(q), _f64(kmin), _f64(kmax))
    flat = torch.full((h * n + 64,), -7.0, dtype=torch.float32, device="cuda")
    kernels.bound_topk(q.cuda(), kmin[None].cuda(), kmax[None].cuda(), 0, n_cand=n, out_bound=flat[: h * n].view(h, n), rank_mode=kernels._lib.RANK_F32)
    got = flat.cpu().numpy().astype(np.float64)
    assert np.abs(got[: h * n].reshape(h, n) - want).max() <= err
    assert (got[h * n :] == -7.0).all()


@pytest.mark.parametrize(("h", "n", "d", "k", "sorted_"), [(8, 12289, 128, 512, False), (4, 40000, 64, 2048, True), (2, 100000, 64, 4096, False), (1, 70000, 128, 17, True)])
def test_long_context_selection_streams_the_bounds(h: int, n: int, d: int, k: int, sorted_: bool) -> None:
    """More candidates per head than the registers hold: the streaming select gives the oracle's set."""
    from lazykv_amd import selection

    q, kmin, kmax = _meta_case(n + k, h, n, 16, d, 4, torch.bfloat16)
    want = R.quest_bound(_f64(q), _f64(kmin), _f64(kmax))
    err = _abs_err(_f64(q), _f64(kmin), _f64(kmax))
    from lazykv_amd import kernels

    full_min = torch.cat([torch.zeros((h, 1, d), dtype=torch.bfloat16), kmin], dim=1)[None].cuda()
    full_max = torch.cat([torch.zeros((h, 1, d), dtype=torch.bfloat16), kmax], dim=1)[None].cuda()
    idx = kernels.bound_topk(q.cuda(), full_min, full_max, k, cand_offset=1, n_cand=n, sorted_=sorted_)
    got = idx.cpu().numpy() - 1
    for j in range(h):
        assert R.selection_ok(got[j], want[j], k, abs_err=err)[0], j
        assert len(set(got[j].tolist())) == k
        if not sorted_:
            assert (np.diff(got[j]) > 0).all()
    if sorted_:
        b = selection.quest_bound(q.view(1, -1, 1, d).cuda(), full_min, full_max, torch.float32)[0].cpu().numpy()
        for j in range(h):
            assert (np.diff(b[j][got[j] + 1]) <= 0).all()


def test_unsorted_selection_is_ascending_and_offset() -> None:
    from lazykv_amd import kernels

    q, kmin, kmax = _meta_case(5, 8, 1000, 16, 128, 4, torch.bfloat16)
    full_min = torch.cat([torch.zeros((8, 1, 128), dtype=torch.bfloat16), kmin], dim=1)[None].cuda()
    full_max = torch.cat([torch.zeros((8, 1, 128), dtype=torch.bfloat16), kmax], dim=1)[None].cuda()
    idx = kernels.bound_topk(q.cuda(), full_min, full_max, 64, cand_offset=1, n_cand=1000)
    got = idx.cpu().numpy()
    want = R.quest_bound(_f64(q), _f64(kmin), _f64(kmax))
    for j in range(8):
        assert (np.diff(got[j]) > 0).all()
        assert R.selection_ok(got[j] - 1, want[j], 64, abs_err=_abs_err(_f64(q), _f64(kmin), _f64(kmax)))[0]


def test_model_dtype_bound_reproduces_the_bf16_tie() -> None:
    """tests/test_selection.py:121-133: tied in bf16 (dtype=None), broken in float32."""
    from lazykv_amd import selection

    pad = torch.zeros((1, 1, 2, 62), dtype=torch.bfloat16)
    kmax = torch.cat([torch.tensor([[[[256.0, 0.5], [256.0, 1.0]]]], dtype=torch.bfloat16), pad], dim=-1).cuda()
    kmin = kmax.clone()
    q = torch.cat([torch.ones((1, 1, 1, 2)), torch.zeros((1, 1, 1, 62))], dim=-1).to(torch.bfloat16).cuda()
    b = selection.quest_bound(q, kmin, kmax)
    assert b.dtype == torch.bfloat16 and b[0, 0, 0] == b[0, 0, 1]
    b32 = selection.quest_bound(q, kmin, kmax, torch.float32)
    assert b32[0, 0, 1] > b32[0, 0, 0]
    assert selection.top_blocks(q, kmin, kmax, 1, torch.float32)[0, 0, 0].item() == 1
    assert selection.top_blocks(q, kmin, kmax, 1)[0, 0, 0].item() == 0  # the tie goes to the lower id


def test_selecting_every_candidate_and_rejecting_more() -> None:
    from lazykv_amd import selection

    q, kmin, kmax = _meta_case(9, 2, 40, 16, 64, 4, torch.float16)
    top = selection.top_blocks(q.view(1, -1, 1, 64).cuda(), kmin[None].cuda(), kmax[None].cuda(), 40, torch.float32)
    assert sorted(top[0, 0].tolist()) == list(range(40))
    with pytest.raises(ValueError, match="exceeds"):
        selection.top_blocks(q.view(1, -1, 1, 64).cuda(), kmin[None].cuda(), kmax[None].cuda(), 41, torch.float32)


# -- sparse decode --------------------------------------------------------------------------------


def _pool_case(seed: int, h: int, g: int, n_blocks: int, bs: int, d: int, dt: torch.dtype):
    from lazykv_amd.workload import draw_layer, to_pool

    w = draw_layer(seed, h * g, h, d, n_blocks * bs, bs, dt)
    return w, to_pool(w.keys, w.values, bs)  # [n, h, 2, bs, d]


def _oracle_decode(q, pool_f64, chosen, sink, cur, fill, scale, bs, block_kv=None):
    h = pool_f64.shape[1]

    def bkv(j, b):
        return pool_f64[b, j, 0], pool_f64[b, j, 1]

    ks, vs = R.gathered_tokens(block_kv or bkv, h, chosen, sink, cur, fill, bs)
    return R.attend_tokens(_f64(q), ks, vs, scale)


@pytest.mark.parametrize("where", ["hbm", "host"])
@pytest.mark.parametrize(("h", "g", "n", "d", "k", "fill"), [(8, 4, 300, 128, 64, 16), (8, 4, 300, 64, 64, 1), (2, 8, 50, 128, 7, 9), (4, 1, 40, 64, 38, 3), (4, 2, 70, 128, 16, 16)])
def test_sparse_decode_matches_the_oracle(where: str, h: int, g: int, n: int, d: int, k: int, fill: int) -> None:
    from lazykv_amd import kernels
    from lazykv_amd.pinned import pinned_empty

    bs = 16
    w, pool = _pool_case(n + d + k, h, g, n, bs, d, torch.bfloat16)
    if where == "host":
        store = pinned_empty(tuple(pool.shape), pool.dtype)
        store.copy_(pool)
    else:
        store = pool.cuda()
    gen = torch.Generator().manual_seed(3)
    chosen = torch.stack([torch.randperm(n - 2, generator=gen)[:k] + 1 for _ in range(h)]).to(torch.int32)
    src = kernels.pool_source(store)
    scale = d**-0.5
    out, lse = kernels.sparse_decode(w.query.cuda(), n_kv=h, block_size=bs, scale=scale, sel=src, idx=chosen.cuda(), sink=src, sink_block=0, cur=src, cur_block=n - 1, fill=fill, out_dtype=torch.float32)
    out_bf, lse_bf = kernels.sparse_decode(w.query.cuda(), n_kv=h, block_size=bs, scale=scale, sel=src, idx=chosen.cuda(), sink=src, sink_block=0, cur=src, cur_block=n - 1, fill=fill)
    torch.cuda.synchronize()
    want_o, want_l = _oracle_decode(w.query, _f64(pool), chosen.numpy(), 0, n - 1, fill, scale, bs)
    assert np.abs(out.cpu().numpy() - want_o).max() < TOL
    assert np.abs(lse.cpu().numpy() - want_l).max() < TOL
    assert torch.equal(out_bf, out.to(torch.bfloat16)) and torch.equal(lse_bf, lse)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize(("g", "k"), [(4, 6), (4, 254), (4, 262), (4, 510), (4, 518), (4, 1022), (8, 254), (8, 510), (8, 1022)])
def test_merge_folds_any_number_of_partials(d: int, g: int, k: int) -> None:
    """The merge launch over 1, 32, 33, 64, 65 and 128 partials per head (2 KV heads, 4 query heads
    each: the HBM plan splits a head's k + 2 items into runs of 8 over 128 workgroups), across the
    one-wave merge's limits of 32 and 64 partials and into the 512-thread merge beyond; with 8 query
    heads per KV head (the 4-wave plan: at most 64 partials, 32 and 64 here) the G = 8 merges.
    Output and LSE match the oracle, and the model-dtype output is the float32 one rounded."""
    from lazykv_amd import kernels

    h, bs, fill = 2, 16, 11
    n = k + 10
    w, pool = _pool_case(k + d, h, g, n, bs, d, torch.bfloat16)
    gen = torch.Generator().manual_seed(k)
    chosen = torch.stack([torch.randperm(n - 2, generator=gen)[:k] + 1 for _ in range(h)]).to(torch.int32)
    src = kernels.pool_source(pool.cuda())
    scale = d**-0.5
    args = dict(n_kv=h, block_size=bs, scale=scale, sel=src, idx=chosen.cuda(), sink=src, sink_block=0, cur=src, cur_block=n - 1, fill=fill)
    out, lse = kernels.sparse_decode(w.query.cuda(), out_dtype=torch.float32, **args)
    out_bf, lse_bf = kernels.sparse_decode(w.query.cuda(), **args)
    torch.cuda.synchronize()
    want_o, want_l = _oracle_decode(w.query, _f64(pool), chosen.numpy(), 0, n - 1, fill, scale, bs)
    assert np.abs(out.cpu().numpy() - want_o).max() < TOL
    assert np.abs(lse.cpu().numpy() - want_l).max() < TOL
    assert torch.equal(out_bf, out.to(torch.bfloat16)) and torch.equal(lse_bf, lse)


@pytest.mark.parametrize("bs", [32, 64, 128])
def test_host_reads_of_large_blocks_take_the_workgroup_floor_and_match_the_oracle(bs: int) -> None:
    """Selected pairs of 16-64 KiB read from host memory: the read budget alone would give 1-4
    workgroups per KV head, the floor of 64 workgroups gives 8 here (98 items per head). Output and
    LSE match the oracle, and the HBM launch over the same pool gives the same result to float32
    summation order."""
    from lazykv_amd import kernels
    from lazykv_amd.pinned import pinned_empty

    h, g, n, d, k, fill = 8, 4, 120, 128, 96, 5
    w, pool = _pool_case(bs + 11, h, g, n, bs, d, torch.bfloat16)
    store = pinned_empty(tuple(pool.shape), pool.dtype)
    store.copy_(pool)
    gen = torch.Generator().manual_seed(bs)
    chosen = torch.stack([torch.randperm(n - 2, generator=gen)[:k] + 1 for _ in range(h)]).to(torch.int32)
    scale = d**-0.5
    outs = []
    for src in (kernels.pool_source(store), kernels.pool_source(pool.cuda())):
        outs.append(kernels.sparse_decode(w.query.cuda(), n_kv=h, block_size=bs, scale=scale, sel=src, idx=chosen.cuda(), sink=src, sink_block=0, cur=src, cur_block=n - 1, fill=fill, out_dtype=torch.float32))
    torch.cuda.synchronize()
    want_o, want_l = _oracle_decode(w.query, _f64(pool), chosen.numpy(), 0, n - 1, fill, scale, bs)
    for out, lse in outs:
        assert np.abs(out.cpu().numpy() - want_o).max() < TOL
        assert np.abs(lse.cpu().numpy() - want_l).max() < TOL
    assert (outs[0][0] - outs[1][0]).abs().max().item() < 1e-5


@pytest.mark.parametrize(("d", "g", "dt"), [(128, 4, torch.bfloat16), (64, 4, torch.float16), (64, 2, torch.bfloat16), (128, 1, torch.float16)])
def test_matrix_core_and_vector_scoring_agree(d: int, g: int, dt: torch.dtype) -> None:
    """HBM launches score on the matrix cores when the query has the pool's dtype and 16-byte
    aligned rows, and on the vector ALUs otherwise (a float32 query, or rows 2 bytes off): all three
    match the oracle, and each other to float32 summation-order differences."""
    from lazykv_amd import kernels

    h, n, k, bs, fill = 8, 200, 40, 16, 11
    w, pool = _pool_case(d + g, h, g, n, bs, d, dt)
    store = pool.cuda()
    gen = torch.Generator().manual_seed(d * g)
    chosen = torch.stack([torch.randperm(n - 2, generator=gen)[:k] + 1 for _ in range(h)]).to(torch.int32)
    src = kernels.pool_source(store)
    q = w.query.to(dt)
    flat = torch.empty(q.numel() + 1, dtype=dt, device="cuda")
    q_off = flat[1:].view(q.shape)  # rows 2 bytes past a 16-byte boundary
    q_off.copy_(q.cuda())
    assert q_off.data_ptr() % 16 != 0
    runs = {}
    for name, qq in (("mfma", q.cuda()), ("unaligned", q_off), ("float32", q.float().cuda())):
        runs[name] = kernels.sparse_decode(qq, n_kv=h, block_size=bs, scale=d**-0.5, sel=src, idx=chosen.cuda(), sink=src, sink_block=0, cur=src,
                                           cur_block=n - 1, fill=fill, out_dtype=torch.float32)
    torch.cuda.synchronize()
    want_o, want_l = _oracle_decode(q, _f64(pool), chosen.numpy(), 0, n - 1, fill, d**-0.5, bs)
    for name, (out, lse) in runs.items():
        assert np.abs(out.cpu().numpy() - want_o).max() < TOL, name
        assert np.abs(lse.cpu().numpy() - want_l).max() < TOL, name
    o_m, l_m = runs["mfma"]
    for name in ("unaligned", "float32"):
        o_v, l_v = runs[name]
        assert (o_m - o_v).abs().max().item() < 1e-5 and (l_m - l_v).abs().max().item() < 1e-5, name


@pytest.mark.parametrize("where", ["hbm", "host"])
@pytest.mark.parametrize("src_kind", ["f16", "bf16", "f32", "int8/f16", "int8/bf16"])
@pytest.mark.parametrize(("bs", "d", "fill"), [(4, 64, 1), (8, 128, 8), (20, 64, 3), (20, 128, 17), (32, 64, 32), (64, 128, 50), (128, 64, 100), (256, 128, 255)])
def test_sparse_decode_block_sizes_and_dtypes(where: str, src_kind: str, bs: int, d: int, fill: int) -> None:
    """Every block size the kernels take (multiples of 4 up to 256, including chunks shorter than
    16 rows and a 4-row tail chunk at bs 20), partial and full current blocks, each model dtype and
    int8 records (read in place, dequantised in the load), from HBM and from host memory."""
    from lazykv_amd import kernels
    from lazykv_amd.pinned import pinned_empty
    from lazykv_amd.quant import packed_pair_bytes

    h, g, n, k = 4, 4, 60, 12
    int8 = src_kind.startswith("int8")
    dt = src_kind.split("/")[-1]
    tdt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[dt]
    w, pool = _pool_case(bs * 1000 + d + len(src_kind), h, g, n, bs, d, torch.float16 if dt == "f32" else tdt)
    pool = pool.to(tdt)
    gen = torch.Generator().manual_seed(bs + d)
    chosen = torch.stack([torch.randperm(n - 2, generator=gen)[:k] + 1 for _ in range(h)]).to(torch.int32)
    exact = _f64(pool)
    if int8:
        recs = R.pack(_bits(pool), dt)  # [n, h, P]
        store = pinned_empty((n, h, packed_pair_bytes(bs, d)), torch.uint8) if where == "host" else torch.empty((n, h, packed_pair_bytes(bs, d)), dtype=torch.uint8).cuda()
        store.copy_(torch.from_numpy(recs))
        sel = kernels.record_source(store, tdt)
        deq = R.to_f32(R.unpack(recs.reshape(n * h, -1), bs, d, dt), dt).reshape(n, h, 2, bs, d).astype(np.float64)
    else:
        store = pinned_empty(tuple(pool.shape), tdt) if where == "host" else torch.empty(tuple(pool.shape), dtype=tdt).cuda()
        store.copy_(pool)
        sel = kernels.pool_source(store)
        deq = exact
    slots = pool[[0, n - 1]].contiguous().cuda()  # sink and current in the model dtype
    ss = kernels.pool_source(slots)
    out, lse = kernels.sparse_decode(w.query.to(tdt).cuda(), n_kv=h, block_size=bs, scale=d**-0.5, sel=sel, idx=chosen.cuda(), sink=ss, sink_block=0, cur=ss, cur_block=1,
                                     fill=fill, out_dtype=torch.float32)
    torch.cuda.synchronize()

    def bkv(j, b):
        src = exact if b in (0, n - 1) else deq
        return src[b, j, 0], src[b, j, 1]

    want_o, want_l = _oracle_decode(w.query.to(tdt), exact, chosen.numpy(), 0, n - 1, fill, d**-0.5, bs, bkv)
    assert np.abs(out.cpu().numpy() - want_o).max() < TOL
    assert np.abs(lse.cpu().numpy() - want_l).max() < TOL


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_sparse_decode_reads_int8_records_in_place(dt: str) -> None:
    from lazykv_amd import kernels
    from lazykv_amd.pinned import pinned_empty
    from lazykv_amd.quant import packed_pair_bytes

    h, g, n, bs, d, k = 8, 4, 200, 16, 128, 40
    w, pool = _pool_case(77, h, g, n, bs, d, DT[dt])
    recs = R.pack(_bits(pool), dt)  # [n, h, P]
    host = pinned_empty((n, h, packed_pair_bytes(bs, d)), torch.uint8)
    host.copy_(torch.from_numpy(recs))
    slots = pool[[0, n - 1]].contiguous().cuda()  # sink and current stay exact
    gen = torch.Generator().manual_seed(4)
    chosen = torch.stack([torch.randperm(n - 2, generator=gen)[:k] + 1 for _ in range(h)]).to(torch.int32)
    slot_src = kernels.pool_source(slots)
    out, lse = kernels.sparse_decode(w.query.cuda(), n_kv=h, block_size=bs, scale=d**-0.5, sel=kernels.record_source(host, DT[dt]), idx=chosen.cuda(), sink=slot_src, sink_block=0, cur=slot_src, cur_block=1, fill=11, out_dtype=torch.float32)
    torch.cuda.synchronize()
    deq = R.to_f32(R.unpack(recs.reshape(n * h, -1), bs, d, dt), dt).reshape(n, h, 2, bs, d).astype(np.float64)
    exact = _f64(pool)

    def bkv(j, b):
        src = exact if b in (0, n - 1) else deq
        return src[b, j, 0], src[b, j, 1]

    want_o, want_l = _oracle_decode(w.query, exact, chosen.numpy(), 0, n - 1, 11, d**-0.5, bs, bkv)
    assert np.abs(out.cpu().numpy() - want_o).max() < TOL
    assert np.abs(lse.cpu().numpy() - want_l).max() < TOL


@pytest.mark.parametrize("rem_where", ["host", "hbm"])
@pytest.mark.parametrize("rem_kind", ["bf16", "int8"])
@pytest.mark.parametrize("k", [5, 60, 118])
def test_exact_split_reconstructs_full_attention(rem_kind: str, k: int, rem_where: str) -> None:
    """Selected from HBM + remainder from the host tier (or from HBM: the 8-wave kernels, whose
    remainder runs skip the selected ids through a bitmap and take three blocks per softmax step),
    merged in-kernel = attention over everything."""
    from lazykv_amd import kernels
    from lazykv_amd.pinned import pinned_empty
    from lazykv_amd.quant import packed_pair_bytes

    h, g, n, bs, d, fill = 8, 4, 120, 16, 128, 16
    w, pool = _pool_case(k, h, g, n, bs, d, torch.bfloat16)
    dev_pool = pool.cuda()
    if rem_kind == "bf16":
        host = pinned_empty(tuple(pool.shape), pool.dtype) if rem_where == "host" else torch.empty(tuple(pool.shape), dtype=pool.dtype, device="cuda")
        host.copy_(pool)
        rem = kernels.pool_source(host)
        cold = _f64(pool)
    else:
        recs = R.pack(_bits(pool), "bf16")
        shape = (n, h, packed_pair_bytes(bs, d))
        host = pinned_empty(shape, torch.uint8) if rem_where == "host" else torch.empty(shape, dtype=torch.uint8, device="cuda")
        host.copy_(torch.from_numpy(recs))
        rem = kernels.record_source(host, torch.bfloat16)
        cold = R.to_f32(R.unpack(recs.reshape(n * h, -1), bs, d, "bf16"), "bf16").reshape(n, h, 2, bs, d).astype(np.float64)
    gen = torch.Generator().manual_seed(k)
    chosen = torch.stack([torch.randperm(n - 2, generator=gen)[:k] + 1 for _ in range(h)]).to(torch.int32)
    src = kernels.pool_source(dev_pool)
    out, lse = kernels.sparse_decode(w.query.cuda(), n_kv=h, block_size=bs, scale=d**-0.5, sel=src, idx=chosen.cuda(), sink=src, sink_block=0, cur=src, cur_block=n - 1, fill=fill, rem=rem, rem_range=(1, n - 1), out_dtype=torch.float32)
    torch.cuda.synchronize()
    exact = _f64(pool)
    ks, vs = [], []
    for j in range(h):
        sel = set(chosen[j].tolist())
        kk = [exact[0, j, 0]] + [(exact if b in sel else cold)[b, j, 0] for b in range(1, n - 1)] + [exact[n - 1, j, 0, :fill]]
        vv = [exact[0, j, 1]] + [(exact if b in sel else cold)[b, j, 1] for b in range(1, n - 1)] + [exact[n - 1, j, 1, :fill]]
        ks.append(np.concatenate(kk))
        vs.append(np.concatenate(vv))
    want_o, want_l = R.attend_tokens(_f64(w.query), ks, vs, d**-0.5)
    assert np.abs(out.cpu().numpy() - want_o).max() < TOL
    assert np.abs(lse.cpu().numpy() - want_l).max() < TOL


def test_partial_attention_matches_the_oracle_and_handles_empty_sets() -> None:
    from lazykv_amd import exact

    gen = torch.Generator().manual_seed(2)
    h, groups, n_blocks, d, bs = 4, 4, 30, 64, 16
    keys = torch.randn((h, n_blocks * bs, d), generator=gen)
    values = torch.randn((h, n_blocks * bs, d), generator=gen)
    query = torch.randn((h, groups, d), generator=gen)
    excluded = np.stack([np.random.default_rng(j).choice(n_blocks, 7, replace=False) for j in range(h)])
    out, lse = exact.partial_attention(keys.cuda(), values.cuda(), query.cuda(), d**-0.5, bs, excluded)
    want_o, want_l = R.partial_attention(_f64(keys), _f64(values), _f64(query), d**-0.5, bs, excluded)
    assert np.abs(out.cpu().numpy() - want_o).max() < TOL and np.abs(lse.cpu().numpy() - want_l).max() < TOL
    everything = np.tile(np.arange(n_blocks), (h, 1))
    eo, el = exact.partial_attention(keys.cuda(), values.cuda(), query.cuda(), d**-0.5, bs, everything)
    assert torch.isneginf(el).all() and torch.isfinite(eo).all() and (eo == 0).all()
    none = np.empty((h, 0), dtype=np.int64)
    fo, fl = exact.partial_attention(keys.bfloat16().cuda(), values.bfloat16().cuda(), query.cuda(), d**-0.5, bs, none)
    wo, wl = R.partial_attention(_f64(keys.bfloat16()), _f64(values.bfloat16()), _f64(query), d**-0.5, bs, none)
    assert np.abs(fo.cpu().numpy() - wo).max() < TOL and np.abs(fl.cpu().numpy() - wl).max() < TOL
    merged, mlse = exact.merge_lse(fo, fl, eo, el)
    assert torch.allclose(merged, fo, atol=1e-6) and torch.equal(mlse, fl)


def test_merge_lse_known_answer_and_random() -> None:
    """tests/test_exact.py:72-84, then random partials against the oracle."""
    from lazykv_amd import exact

    m, lse = exact.merge_lse(torch.tensor([[1.0, 0.0]]).cuda(), torch.tensor([2.0]).cuda(), torch.tensor([[0.0, 1.0]]).cuda(), torch.tensor([0.0]).cuda())
    wa = float(np.exp(2.0 - np.logaddexp(2.0, 0.0)))
    assert abs(m[0, 0].item() - wa) < 1e-6 and m[0, 0] > m[0, 1]
    assert abs(lse[0].item() - float(np.logaddexp(2.0, 0.0))) < 1e-6
    gen = torch.Generator().manual_seed(1)
    oa, ob = torch.randn((3, 32, 128), generator=gen), torch.randn((3, 32, 128), generator=gen)
    la, lb = torch.randn((3, 32), generator=gen) * 5, torch.randn((3, 32), generator=gen) * 5
    la[0, 0] = float("-inf")
    la[1, 1] = lb[1, 1] = float("-inf")
    got, gl = exact.merge_lse(oa.cuda(), la.cuda(), ob.cuda(), lb.cuda())
    want, wl = R.merge_lse(_f64(oa), _f64(la), _f64(ob), _f64(lb))
    assert np.abs(got.cpu().numpy() - want).max() < 1e-5
    assert np.array_equal(np.isneginf(gl.cpu().numpy()), np.isneginf(wl))
    fin = np.isfinite(wl)
    assert np.abs(gl.cpu().numpy()[fin] - wl[fin]).max() < 1e-5


@pytest.mark.parametrize("length", [16, 100, 1000, 4099])
def test_dense_decode_is_full_attention(length: int) -> None:
    from lazykv_amd import attention

    gen = torch.Generator().manual_seed(length)
    h, g, d = 8, 4, 128
    store = torch.randn((1, h, length + 64, d), generator=gen).to(torch.float16)
    vstore = torch.randn((1, h, length + 64, d), generator=gen).to(torch.float16)
    q = torch.randn((1, h * g, 1, d), generator=gen).to(torch.float16)
    k, v = store[:, :, :length].cuda(), vstore[:, :, :length].cuda()
    out, lse = attention.dense_decode(q.cuda(), k, v, d**-0.5)
    torch.cuda.synchronize()
    want_o, want_l = R.attend_tokens(_f64(q[0, :, 0]), list(_f64(k[0])), list(_f64(v[0])), d**-0.5)
    assert np.abs(out.float().cpu().numpy()[0, :, 0] - want_o).max() < TOL + 2e-3  # output rounded to fp16
    assert np.abs(lse.cpu().numpy()[0] - want_l).max() < TOL


def test_pinned_pool_round_trips_and_the_stream_probe_reads_it() -> None:
    from lazykv_amd import kernels
    from lazykv_amd.pinned import device_address, device_view, pinned_empty

    t = pinned_empty((3, 5 * 2**20 + 16), torch.uint8)
    assert t.is_pinned()
    t.random_(0, 255)
    d = torch.empty_like(t, device="cuda")
    d.copy_(t, non_blocking=True)
    torch.cuda.synchronize()
    assert torch.equal(d.cpu(), t)
    view = device_view(t)
    assert view.is_cuda and torch.equal(view.cpu(), t)
    sink = torch.zeros(64, dtype=torch.int32, device="cuda")
    kernels.stream_read(device_address(t), t.numel(), 64, sink)
    sink_dev = torch.zeros(64, dtype=torch.int32, device="cuda")
    kernels.stream_read(d.data_ptr(), d.numel(), 64, sink_dev)
    torch.cuda.synchronize()
    assert torch.equal(sink, sink_dev) and sink.abs().sum() > 0


def test_install_verifies_the_decode_kernel_and_refuses_unknown_strategies() -> None:
    """install() with the model's head counts checks decode (the HIP kernel, spare storage past the
    live length) and chunked prefill against a float64 truth first (lazykv/attention.py:214-290).
    The reference's strategy names (:44) select the HIP kernel, as the reference's fixtures install
    them (tests/test_tiered.py:25); a name this library does not have is a hard error, and `attend`
    refuses it as the reference's does (:113)."""
    from lazykv_amd import attention

    chosen, checks = attention.install(None, 32, 8, 128)
    assert chosen == "hip" and len(checks) == 1 and checks[0].ok, checks
    assert checks[0].max_rel_err_decode < 1e-2 and checks[0].max_rel_err_prefill < 1e-2
    assert checks[0].seconds_decode_growing_median > 0
    assert attention.current_strategy() == ("hip", attention.DEFAULT_BUCKET)
    chosen, checks = attention.install("hip", 32, 8, 64)
    assert checks[0].ok, checks
    for name in attention.REFERENCE_STRATEGIES:
        chosen, checks = attention.install(name, 32, 8, 64, bucket=64)
        assert chosen == name and checks[0].strategy == name and checks[0].ok, checks
        assert attention.current_strategy() == (name, 64)
    with pytest.raises(RuntimeError, match="unknown"):
        attention.install("flash", 32, 8, 64)
    with pytest.raises(RuntimeError, match="unknown"):
        attention.install("flash")
    q = torch.randn(1, 8, 1, 64, device="cuda", dtype=torch.float16)
    k = torch.randn(1, 2, 32, 64, device="cuda", dtype=torch.float16)
    with pytest.raises(ValueError, match="unknown attention strategy"):
        attention.attend(q, k, k, None, "flash")
    pinned = attention.current_strategy()[0]  # the last name installed above
    restore = attention.set_strategy_for_test("efficient")
    assert attention.current_strategy()[0] == "efficient"
    restore()
    assert attention.current_strategy()[0] == pinned


def test_attention_seam_refuses_a_mask_and_reads_only_the_live_prefix() -> None:
    """After lazykv/tests/test_runtime.py:147-170: the registered attention function refuses an
    external mask (it owns causality), and `attend` over the live prefix of a preallocated store
    whose spare rows hold large values matches the float64 truth within 1e-2 relative, for a decode
    token and for a 17-token chunk. head_dim is 64, the smallest the decode kernel takes (the
    reference's test uses 16). The startup verification passes under every strategy name and fails,
    without raising, for one the library does not have (lazykv/attention.py:248-266)."""
    from lazykv_amd.attention import _truth, attend, lazykv_attention_forward, verify_strategies

    q = torch.randn(1, 8, 1, 64, device="cuda", dtype=torch.float16)
    k = torch.randn(1, 2, 4, 64, device="cuda", dtype=torch.float16)
    with pytest.raises(RuntimeError, match="owns causality"):
        lazykv_attention_forward(torch.nn.Module(), q, k, k, torch.ones(1, 1, 1, 4, device="cuda", dtype=torch.bool))
    gen = torch.Generator(device="cuda").manual_seed(1)
    store_k = torch.randn(1, 2, 256, 64, device="cuda", dtype=torch.float16, generator=gen) * 50
    store_v = torch.randn(1, 2, 256, 64, device="cuda", dtype=torch.float16, generator=gen) * 50
    live = 100
    k, v = store_k[:, :, :live], store_v[:, :, :live]
    for q_len in (1, 17):
        q = torch.randn(1, 8, q_len, 64, device="cuda", dtype=torch.float16, generator=gen)
        ref = _truth(q, k, v, 64**-0.5)
        got = attend(q, k, v, 64**-0.5).double().cpu()
        assert ((got - ref).abs().max() / ref.abs().max()).item() < 1e-2, q_len
    from lazykv_amd.attention import STRATEGIES

    checks = verify_strategies(8, 2, 64, dtype=torch.float16, probe_ctx=2048, steps=4)
    assert [c.strategy for c in checks] == list(STRATEGIES) and all(c.ok for c in checks), checks
    # one kernel behind every name: one measurement, reported under each
    assert len({(c.max_rel_err_decode, c.seconds_decode_growing_median) for c in checks}) == 1
    other = verify_strategies(8, 2, 64, dtype=torch.float16, candidates=("flash",))
    assert not other[0].ok and "unknown strategy" in other[0].error
