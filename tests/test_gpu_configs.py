"""Parity at the real shapes of the tiered decode workloads, one layer each, against the oracle.

Each case draws a seeded layer (lazykv_amd.workload), builds its tier with the store kernel, then
checks: the block metadata bit-exact (exact keys, or the dequantised keys of an int8 tier); every
int8 record bit-exact against the oracle's pack; the selected sets against the
oracle's float64 Quest bound (identical outside near-tie cells) with the planted needle block
selected for every KV head; and the decode output and LSE within 2e-3 of float64 attention over
the set the tier attends.

Workloads (32 query / 8 KV heads, 16-token blocks, lazy sealing: fill 16, candidates 1..N-2):
* 1B-shaped, 32,768 tokens, d 64, float16, K 512, all in HBM;
* 1B-shaped, 65,536 tokens, d 64, float16, K 1,024, sealed blocks as int8 records (HBM or host);
* 8B-shaped, 131,072 tokens, d 128, bfloat16, K 512, read zero-copy from mapped host memory;
* 8B-shaped, 131,072 tokens, d 128, bfloat16, exact split: K of 512 / 2,048 / 4,096 selected
  from HBM, every other sealed block from the int8 host tier, merged by LSE;
* 8B-shaped, 524,288 tokens (32,766 candidates per head: the streaming select), K 2,048, zero-copy.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference as R

pytestmark = pytest.mark.gpu

TOL = 2e-3
N_Q, H, BS = 32, 8, 16
NAMES = {torch.float16: "f16", torch.bfloat16: "bf16"}


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


class _Layer:
    """One drawn layer with its tier: pool [N, h, 2, bs, d] on the GPU, metadata, optional records."""

    def __init__(self, d: int, tokens: int, dtype: torch.dtype, int8: bool, meta_from: str) -> None:
        from lazykv_amd import kernels
        from lazykv_amd.quant import packed_pair_bytes
        from lazykv_amd.workload import draw_layer, to_pool

        self.d, self.dtype, self.dn = d, dtype, NAMES[dtype]
        self.n = tokens // BS
        self.n_sealed, self.fill = self.n - 1, BS
        w = draw_layer(0, N_Q, H, d, tokens, BS, dtype, device="cuda")
        self.q, self.needle = w.query.contiguous(), w.needle
        self.pool = to_pool(w.keys, w.values, BS)
        self.kmin = torch.zeros((1, H, self.n, d), dtype=dtype, device="cuda")
        self.kmax = torch.zeros_like(self.kmin)
        self.records = None
        src = kernels.dense_source(w.keys, w.values, BS)
        if int8:
            self.records = torch.zeros((self.n, H, packed_pair_bytes(BS, d)), dtype=torch.uint8, device="cuda")
            meta = meta_from == "dequantised"
            kernels.store_blocks(src, dst=kernels.record_source(self.records, dtype), n_kv=H, head_dim=d, block_size=BS, first_block=0, n_blocks=self.n_sealed,
                                 kmin=self.kmin if meta else None, kmax=self.kmax if meta else None)
        if self.records is None or meta_from == "exact":
            kernels.store_blocks(src, n_kv=H, head_dim=d, block_size=BS, first_block=0, n_blocks=self.n_sealed, kmin=self.kmin, kmax=self.kmax)
        del w
        torch.cuda.synchronize()
        self.exact = _f32(self.pool)  # [N, h, 2, bs, d], exact widening of the model dtype
        self.deq = None
        if self.records is not None:
            rec = self.records[: self.n_sealed].cpu().numpy()
            self.deq = R.to_f32(R.unpack(rec.reshape(self.n_sealed * H, -1), BS, d, self.dn), self.dn).reshape(self.n_sealed, H, 2, BS, d)

    def check_records(self, chunk: int = 1024) -> None:
        """Every sealed (block, head) record against the C oracle's pack of the same pair's bits."""
        from oracle import quant_c

        for b0 in range(0, self.n_sealed, chunk):
            b1 = min(self.n_sealed, b0 + chunk)
            pairs = _bits(self.pool[b0:b1]).reshape((b1 - b0) * H, 2, BS, self.d)  # the records' (block, head) order
            want = quant_c.pack(pairs, self.dn)
            got = self.records[b0:b1].cpu().numpy().reshape((b1 - b0) * H, -1)
            assert np.array_equal(got, want), f"records of blocks {b0}..{b1 - 1}"

    def check_metadata(self, source: str) -> None:
        keys = (self.deq if source == "dequantised" else self.exact[: self.n_sealed])[:, :, 0]  # [n_sealed, h, bs, d]
        want_min = R.from_f32(keys.min(axis=2), self.dn).transpose(1, 0, 2)
        want_max = R.from_f32(keys.max(axis=2), self.dn).transpose(1, 0, 2)
        assert np.array_equal(_bits(self.kmin[0, :, : self.n_sealed]), want_min)
        assert np.array_equal(_bits(self.kmax[0, :, : self.n_sealed]), want_max)

    def select(self, k: int) -> np.ndarray:
        from lazykv_amd import kernels

        idx = kernels.bound_topk(self.q, self.kmin, self.kmax, k, cand_offset=1, n_cand=self.n_sealed - 1)
        torch.cuda.synchronize()
        chosen = idx.cpu().numpy()
        q = self.q.double().cpu().numpy()
        mn = self.kmin[0, :, 1 : self.n_sealed].double().cpu().numpy()
        mx = self.kmax[0, :, 1 : self.n_sealed].double().cpu().numpy()
        bound = R.quest_bound(q, mn, mx)
        err = float(np.abs(q).max() * np.maximum(np.abs(mn), np.abs(mx)).sum(-1).max()) * 2.0**-19
        for j in range(H):
            ok, _ = R.selection_ok(chosen[j] - 1, bound[j], k, abs_err=err)
            assert ok, j
            assert self.needle in chosen[j], (j, self.needle)
        return idx

    def oracle(self, chosen: np.ndarray, exact_remainder: bool) -> tuple[np.ndarray, np.ndarray]:
        """float64 attention over sink + chosen (+ every other sealed block) + current[:fill]."""
        q = self.q.double().cpu().numpy()
        ks, vs = [], []
        for j in range(H):
            sel = chosen[j]
            if exact_remainder:
                arr = self.deq[:, j].copy()  # [n_sealed, 2, bs, d]: every sealed block, dequantised
                arr[0] = self.exact[0, j]  # the sink is exact
                arr[sel] = self.exact[sel, j]  # the selected blocks are read exactly from HBM
                kk = np.concatenate([arr[:, 0].reshape(-1, self.d), self.exact[self.n_sealed, j, 0, : self.fill]])
                vv = np.concatenate([arr[:, 1].reshape(-1, self.d), self.exact[self.n_sealed, j, 1, : self.fill]])
            else:
                src = self.deq if self.deq is not None else self.exact
                kk = np.concatenate([self.exact[0, j, 0], src[sel, j, 0].reshape(-1, self.d), self.exact[self.n_sealed, j, 0, : self.fill]])
                vv = np.concatenate([self.exact[0, j, 1], src[sel, j, 1].reshape(-1, self.d), self.exact[self.n_sealed, j, 1, : self.fill]])
            ks.append(kk)
            vs.append(vv)
        return R.attend_tokens(q, ks, vs, self.d**-0.5)


def _decode(layer: _Layer, idx: torch.Tensor, sel, rem=None, rem_range=(0, 0)):  # noqa: ANN001, ANN202
    from lazykv_amd import kernels

    slots = layer.pool[[0, layer.n_sealed]].contiguous()
    ss = kernels.pool_source(slots)
    out, lse = kernels.sparse_decode(layer.q, n_kv=H, block_size=BS, scale=layer.d**-0.5, sel=sel, idx=idx, sink=ss, sink_block=0, cur=ss, cur_block=1,
                                     fill=layer.fill, rem=rem, rem_range=rem_range, out_dtype=torch.float32)
    torch.cuda.synchronize()
    return out.cpu().numpy(), lse.cpu().numpy()


def test_hbm_decode_32k_float16_k512() -> None:
    from lazykv_amd import kernels

    layer = _Layer(64, 32768, torch.float16, int8=False, meta_from="exact")
    layer.check_metadata("exact")
    idx = layer.select(512)
    out, lse = _decode(layer, idx, kernels.pool_source(layer.pool))
    want_o, want_l = layer.oracle(idx.cpu().numpy(), exact_remainder=False)
    assert np.abs(out - want_o).max() < TOL
    assert np.abs(lse - want_l).max() < TOL


@pytest.mark.parametrize("where", ["hbm", "host"])
def test_int8_tier_decode_64k_float16_k1024(where: str) -> None:
    from lazykv_amd import kernels
    from lazykv_amd.pinned import pinned_empty

    layer = _Layer(64, 65536, torch.float16, int8=True, meta_from="dequantised")
    layer.check_records()
    layer.check_metadata("dequantised")
    recs = layer.records
    if where == "host":
        recs = pinned_empty(tuple(layer.records.shape), torch.uint8)
        recs.copy_(layer.records)
    idx = layer.select(1024)
    out, lse = _decode(layer, idx, kernels.record_source(recs, torch.float16))
    want_o, want_l = layer.oracle(idx.cpu().numpy(), exact_remainder=False)
    assert np.abs(out - want_o).max() < TOL
    assert np.abs(lse - want_l).max() < TOL


def test_zero_copy_decode_128k_bfloat16_k512() -> None:
    from lazykv_amd import kernels
    from lazykv_amd.pinned import pinned_empty

    layer = _Layer(128, 131072, torch.bfloat16, int8=False, meta_from="exact")
    layer.check_metadata("exact")
    host = pinned_empty(tuple(layer.pool.shape), torch.bfloat16)
    host.copy_(layer.pool)
    idx = layer.select(512)
    out, lse = _decode(layer, idx, kernels.pool_source(host))
    want_o, want_l = layer.oracle(idx.cpu().numpy(), exact_remainder=False)
    assert np.abs(out - want_o).max() < TOL
    assert np.abs(lse - want_l).max() < TOL


@pytest.mark.parametrize("quant", [None, "int8"])
def test_hybrid_residency_128k_bfloat16_k512_is_the_zero_copy_step(quant: str | None) -> None:
    """The hybrid step at the 8B shape (131,072 tokens, K 512 of 8,190, 512 slots per head, bf16
    pairs or int8 records in host memory) over three drifting queries -- the first with empty
    slots, the others with hits and misses -- chooses the zero-copy step's ids and gives its
    output and LSE bit for bit: the decode launch takes the zero-copy plan, and a hit reads from
    its slot exactly what the miss wrote there."""
    from lazykv_amd import kernels
    from lazykv_amd.pinned import pinned_empty

    int8 = quant == "int8"
    layer = _Layer(128, 131072, torch.bfloat16, int8=int8, meta_from="dequantised" if int8 else "exact")
    src = layer.records if int8 else layer.pool
    host = pinned_empty(tuple(src.shape), src.dtype)
    host.copy_(src)
    hs = kernels.record_source(host, torch.bfloat16) if int8 else kernels.pool_source(host)
    res = kernels.Residency.allocate(512, H, layer.n, BS, 128, torch.bfloat16, torch.device("cuda"))
    slots = layer.pool[[0, layer.n_sealed]].contiguous()
    ss = kernels.pool_source(slots)
    common = dict(cand_offset=1, n_cand=layer.n_sealed - 1, block_size=BS, scale=128**-0.5, sink=ss, sink_block=0, cur=ss, cur_block=1, fill=layer.fill,
                  out_dtype=torch.float32)
    gen = torch.Generator(device="cuda").manual_seed(3)
    base = layer.q.float()
    rms = base.pow(2).mean(dim=-1, keepdim=True).sqrt()
    hits = []
    for step in range(3):
        q = (base + 0.25 * rms * torch.randn(base.shape, generator=gen, device="cuda")).to(torch.bfloat16)
        before = res.block_slot.clone()
        ih = torch.empty((H, 512), dtype=torch.int32, device="cuda")
        iz = torch.empty_like(ih)
        oh, lh = kernels.select_hybrid_decode(q, layer.kmin, layer.kmax, 512, host=hs, res=res, out_idx=ih, **common)
        oz, lz = kernels.select_decode(q, layer.kmin, layer.kmax, 512, sel=hs, out_idx=iz, **common)
        torch.cuda.synchronize()
        assert torch.equal(ih, iz), step
        assert torch.equal(oh, oz) and torch.equal(lh, lz), step
        hits.append(int((torch.gather(before, 1, ih.long()) >= 0).sum()))
    assert hits[0] == 0 and all(0 < x < H * 512 for x in hits[1:]), hits


@pytest.fixture(scope="module")
def exact_layer():  # noqa: ANN201
    from lazykv_amd.pinned import pinned_empty

    layer = _Layer(128, 131072, torch.bfloat16, int8=True, meta_from="exact")
    host = pinned_empty(tuple(layer.records.shape), torch.uint8)
    host.copy_(layer.records)
    return layer, host


@pytest.mark.parametrize("k", [512, 2048, 4096])
def test_exact_split_128k_bfloat16(exact_layer, k: int) -> None:  # noqa: ANN001
    """Selected from HBM exactly, the rest from the int8 host tier: the oracle is float64 attention
    over every token with the unselected sealed blocks dequantised. Against float64 dense attention
    over the original values of all 8,192 blocks, the output and LSE must also stay within 2e-3:
    the int8 tier's error and the kernel's together."""
    from lazykv_amd import kernels

    layer, host = exact_layer
    if k == 512:
        layer.check_records()
        layer.check_metadata("exact")
    idx = layer.select(k)
    out, lse = _decode(layer, idx, kernels.pool_source(layer.pool), rem=kernels.record_source(host, torch.bfloat16), rem_range=(1, layer.n_sealed))
    chosen = idx.cpu().numpy()
    want_o, want_l = layer.oracle(chosen, exact_remainder=True)
    assert np.abs(out - want_o).max() < TOL
    assert np.abs(lse - want_l).max() < TOL
    # Against dense attention over the original values.
    q = layer.q.double().cpu().numpy()
    total = layer.n_sealed * BS + layer.fill
    ks = [layer.exact[:, j, 0].reshape(-1, layer.d)[:total] for j in range(H)]
    vs = [layer.exact[:, j, 1].reshape(-1, layer.d)[:total] for j in range(H)]
    dense_o, dense_l = R.attend_tokens(q, ks, vs, layer.d**-0.5)
    dev_o, dev_l = np.abs(out - dense_o).max(), np.abs(lse - dense_l).max()
    print(f"exact split K={k}: max|out - dense| {dev_o:.2e}, max|lse - dense| {dev_l:.2e}")
    # The workload's own bar: full dense attention over all 8,192 blocks within 2e-3.
    assert dev_o < TOL and dev_l < TOL


def test_zero_copy_decode_512k_streams_the_selection() -> None:
    """A context past the register-resident select (32,766 candidates per head): 524,288 tokens,
    bf16 d128, K 2,048, read zero-copy."""
    from lazykv_amd import kernels
    from lazykv_amd.pinned import pinned_empty

    layer = _Layer(128, 524288, torch.bfloat16, int8=False, meta_from="exact")
    host = pinned_empty(tuple(layer.pool.shape), torch.bfloat16)
    host.copy_(layer.pool)
    idx = layer.select(2048)
    out, lse = _decode(layer, idx, kernels.pool_source(host))
    want_o, want_l = layer.oracle(idx.cpu().numpy(), exact_remainder=False)
    assert np.abs(out - want_o).max() < TOL
    assert np.abs(lse - want_l).max() < TOL
