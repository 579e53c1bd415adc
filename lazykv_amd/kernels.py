"""Tensor-level calls into the HIP kernels: validation, layout descriptors, workspaces.

Every function here enqueues work on the current HIP stream of its tensors' device and returns
without synchronising. Shapes are checked on the host before any launch (the kernels assume
them). The reference-facing modules (`selection`, `quant`, `exact`, `attention`, `tiered`) are
built on these.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from lazykv_amd import _lib
from lazykv_amd.pinned import device_address, is_mapped


# -- workspaces -----------------------------------------------------------------------------------


class Workspace:
    """A device scratch buffer (partials, bounds), grown on demand.

    Its contents need no initialisation, so one workspace serves any number of calls issued in
    order on one stream. Growing it allocates a fresh buffer; calls already prepared against the
    old one keep it alive.
    """

    def __init__(self, device: torch.device | str | None = None, nbytes: int = 0) -> None:
        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.buf = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=self.device)

    def get(self, nbytes: int) -> tuple[int, int]:
        if nbytes > self.buf.numel():
            self.buf = torch.zeros(int(nbytes * 1.25) + 256, dtype=torch.uint8, device=self.device)
        return self.buf.data_ptr(), self.buf.numel()


_DEFAULT_WS: dict[tuple[int, int], Workspace] = {}


def default_workspace(device: torch.device) -> Workspace:
    """One workspace per (device, stream), for callers that do not bring their own."""
    dev = torch.device(device)
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    key = (idx, torch.cuda.current_stream(idx).cuda_stream)
    ws = _DEFAULT_WS.get(key)
    if ws is None:
        ws = _DEFAULT_WS[key] = Workspace(torch.device("cuda", idx))
    return ws


# -- layout descriptors ---------------------------------------------------------------------------


def address(t: torch.Tensor) -> int:
    """Device-visible address of a tensor: its own pointer on the GPU, the mapped alias for a pool."""
    if t.is_cuda:
        return t.data_ptr()
    if is_mapped(t):
        return device_address(t)
    raise RuntimeError("tensor is neither on the GPU nor in mapped pinned memory (there is no CPU path)")


@dataclass
class Source:
    """A `lkv_kv_source`: base addresses and strides of one set of KV blocks, plus its keep-alives."""

    k: int
    v: int
    block_stride: int
    head_stride: int
    dtype: int
    deq_dtype: int
    n_blocks: int
    owners: tuple = ()
    flags: int = 0  # _lib.SRC_HOST for blocks in mapped host memory

    def c(self) -> _lib.KVSource:
        return _lib.KVSource(self.k, self.v, self.block_stride, self.head_stride, self.n_blocks, self.dtype, self.deq_dtype, self.flags)


def _location(t: torch.Tensor) -> int:
    return 0 if t.is_cuda else _lib.SRC_HOST


def pool_source(pool: torch.Tensor) -> Source:
    """Blocks of a `[blocks, h, 2, bs, d]` pool (host pool or GPU slot pool, lazykv/tiered.py:261,265)."""
    if pool.ndim != 5 or pool.shape[2] != 2 or not pool.is_contiguous():
        raise ValueError(f"expected a contiguous [blocks, h, 2, bs, d] pool, got {tuple(pool.shape)}")
    _, h, _, bs, d = pool.shape
    base = address(pool)
    es = pool.element_size()
    code = _lib.dtype_code(pool.dtype)
    return Source(base, base + bs * d * es, h * 2 * bs * d, 2 * bs * d, code, code, pool.shape[0], (pool,), _location(pool))


def record_source(records: torch.Tensor, deq_dtype: torch.dtype) -> Source:
    """Blocks of an int8 record pool `[blocks, h, P]` (lazykv/tiered.py:265, quant.py:46-56)."""
    if records.ndim != 3 or records.dtype != torch.uint8 or not records.is_contiguous():
        raise ValueError(f"expected contiguous uint8 records [blocks, h, P], got {tuple(records.shape)} {records.dtype}")
    _, h, p = records.shape
    base = address(records)
    return Source(base, 0, h * p, p, _lib.INT8_RECORD, _lib.dtype_code(deq_dtype), records.shape[0], (records,), _location(records))


def dense_source(keys: torch.Tensor, values: torch.Tensor, block_size: int) -> Source:
    """Blocks of dense per-head KV `[1, h, T, d]` or `[h, T, d]` (a full cache, lazykv/cache.py:35-36;
    the exact tier's float32 mirror, lazykv/exact.py:131-140). Rows must be contiguous and the token
    stride must be head_dim."""
    k = keys[0] if keys.ndim == 4 else keys
    v = values[0] if values.ndim == 4 else values
    if k.ndim != 3 or k.shape != v.shape or k.dtype != v.dtype:
        raise ValueError(f"expected matching [h, T, d] keys/values, got {tuple(keys.shape)} / {tuple(values.shape)}")
    d = k.shape[-1]
    for t in (k, v):
        if t.stride(-1) != 1 or t.stride(-2) != d:
            raise ValueError("dense KV rows must be contiguous with a token stride of head_dim")
    if k.stride(0) != v.stride(0):
        raise ValueError("keys and values must share their head stride")
    code = _lib.dtype_code(k.dtype)
    return Source(address(k), address(v), block_size * d, k.stride(0), code, code, k.shape[1] // block_size, (keys, values), _location(k))


# -- a1 + a2: bound and top-K -----------------------------------------------------------------------


def _meta_layout(kmin: torch.Tensor, kmax: torch.Tensor) -> tuple[int, int, int, int]:
    """(n_kv, n_blocks, head_dim, head_stride) of `[1, h, n, d]` or `[h, n, d]` metadata views."""
    a = kmin[0] if kmin.ndim == 4 else kmin
    b = kmax[0] if kmax.ndim == 4 else kmax
    if a.ndim != 3 or a.shape != b.shape or a.dtype != b.dtype:
        raise ValueError(f"kmin/kmax must be matching [1, h, n, d] tensors, got {tuple(kmin.shape)} / {tuple(kmax.shape)}")
    if a.stride() != b.stride() or a.stride(-1) != 1 or a.stride(-2) != a.shape[-1]:
        raise ValueError("kmin/kmax rows must be contiguous, with equal strides")
    return a.shape[0], a.shape[1], a.shape[2], a.stride(0)


def bound_topk(
    q: torch.Tensor,
    kmin: torch.Tensor,
    kmax: torch.Tensor,
    k: int,
    *,
    cand_offset: int = 0,
    n_cand: int | None = None,
    rank_mode: int = _lib.RANK_F32,
    sorted_: bool = False,
    out_idx: torch.Tensor | None = None,
    out_bound: torch.Tensor | None = None,
    ws: Workspace | None = None,
) -> torch.Tensor | None:
    """Quest bound + top-k over block metadata `[1, h, cap, d]`; candidates are blocks
    cand_offset .. cand_offset + n_cand - 1 (default: all of them).

    Returns int32 block ids `[h, k]` (cand_offset included), ascending, or in descending bound
    order when `sorted_`. `out_bound` `[h, n_cand]` float32 receives the bounds when given.
    """
    _lib.require_cuda(q, kmin, kmax)
    n_kv, cap, d, hs = _meta_layout(kmin, kmax)
    if n_cand is None:
        n_cand = cap - cand_offset
    if cand_offset < 0 or n_cand <= 0 or cand_offset + n_cand > cap:
        raise ValueError(f"candidates {cand_offset}..{cand_offset + (n_cand or 0)} outside {cap} metadata blocks")
    qq = q.reshape(-1, q.shape[-1])
    if qq.shape[-1] != d or qq.shape[0] % n_kv:
        raise ValueError(f"query {tuple(q.shape)} does not match metadata with {n_kv} heads of dim {d}")
    qq = qq.contiguous()
    if k > 0 and out_idx is None:
        out_idx = torch.empty((n_kv, k), dtype=torch.int32, device=q.device)
    if out_idx is not None and (out_idx.dtype != torch.int32 or out_idx.shape[-1] < k or out_idx.stride(-1) != 1):
        raise ValueError("out_idx must be int32 [h, >=k] with contiguous rows")
    if out_bound is not None and (out_bound.dtype != torch.float32 or tuple(out_bound.shape) != (n_kv, n_cand) or not out_bound.is_contiguous()):
        raise ValueError(f"out_bound must be contiguous float32 [{n_kv}, {n_cand}]")
    meta_base = address(kmin[0] if kmin.ndim == 4 else kmin)
    meta_max = address(kmax[0] if kmax.ndim == 4 else kmax)
    ws = ws or default_workspace(q.device)
    ws_ptr, ws_n = ws.get(_lib.lib().lkv_bound_topk_workspace_bytes(n_kv, n_cand, k))
    rc = _lib.lib().lkv_bound_topk(
        _lib.stream_of(q), qq.data_ptr(), _lib.dtype_code(qq.dtype), meta_base, meta_max, _lib.dtype_code(kmin.dtype), hs,
        qq.shape[0], n_kv, d, cand_offset, n_cand, k, rank_mode, _lib.SORTED if sorted_ else 0,
        out_idx.data_ptr() if out_idx is not None else None, out_idx.stride(0) if out_idx is not None else 0,
        out_bound.data_ptr() if out_bound is not None else None, ws_ptr, ws_n,
    )
    _lib.check(rc, "bound_topk")
    return out_idx


# -- a5..a9, a11: sparse decode ---------------------------------------------------------------------


def sparse_decode(
    q: torch.Tensor,
    *,
    n_kv: int,
    block_size: int,
    scale: float,
    sel: Source | None = None,
    idx: torch.Tensor | None = None,
    attend_selected: bool = True,
    sink: Source | None = None,
    sink_block: int = -1,
    cur: Source | None = None,
    cur_block: int = -1,
    fill: int = 0,
    rem: Source | None = None,
    rem_range: tuple[int, int] = (0, 0),
    out: torch.Tensor | None = None,
    out_dtype: torch.dtype | None = None,
    lse: torch.Tensor | None = None,
    ws: Workspace | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Block-sparse GQA decode attention with LSE; see lkv_sparse_decode in include/lazykv_hip.h.

    q `[n_q, d]`; idx int32 `[n_kv, k]` block ids (device). Returns (out `[n_q, d]`, lse `[n_q]` float32).
    """
    _lib.require_cuda(q)
    qq = q.reshape(-1, q.shape[-1]).contiguous()
    n_q, d = qq.shape
    k = 0
    if idx is not None:
        _lib.require_cuda(idx)
        if idx.dtype != torch.int32 or idx.ndim != 2 or idx.shape[0] != n_kv or idx.stride(-1) != 1:
            raise ValueError(f"idx must be int32 [{n_kv}, k] with contiguous rows, got {tuple(idx.shape)} {idx.dtype}")
        k = idx.shape[1]
    out_dtype = out_dtype or (out.dtype if out is not None else qq.dtype)
    if out is None:
        out = torch.empty((n_q, d), dtype=out_dtype, device=q.device)
    if lse is None:
        lse = torch.empty((n_q,), dtype=torch.float32, device=q.device)
    if not out.is_contiguous() or out.numel() != n_q * d or not lse.is_contiguous() or lse.numel() != n_q or lse.dtype != torch.float32:
        raise ValueError("out must be contiguous [n_q, d] and lse contiguous float32 [n_q]")
    desc = _lib.DecodeDesc(n_q, n_kv, d, block_size, float(scale), k, 1 if attend_selected else 0, sink_block, cur_block, fill, rem_range[0], rem_range[1])
    ws = ws or default_workspace(q.device)
    ws_ptr, ws_n = ws.get(_lib.lib().lkv_sparse_decode_workspace_bytes(ctypes.byref(desc)))
    cs = [s.c() if s is not None else None for s in (sel, sink, cur, rem)]
    refs = [ctypes.byref(c) if c is not None else None for c in cs]
    rc = _lib.lib().lkv_sparse_decode(
        _lib.stream_of(qq), ctypes.byref(desc), qq.data_ptr(), _lib.dtype_code(qq.dtype), refs[0],
        idx.data_ptr() if idx is not None else None, idx.stride(0) if idx is not None else 0, refs[1], refs[2], refs[3],
        out.data_ptr(), _lib.dtype_code(out.dtype), lse.data_ptr(), ws_ptr, ws_n,
    )
    _lib.check(rc, "sparse_decode")
    return out, lse


# -- a1 + a2 + a5 + a6: bound, top-K and decode of one layer in one call ----------------------------


def _select_desc(q: torch.Tensor, n_kv: int, block_size: int, scale: float, k: int, sink_block: int, cur_block: int, fill: int) -> _lib.DecodeDesc:
    n_q, d = q.reshape(-1, q.shape[-1]).shape
    return _lib.DecodeDesc(n_q, n_kv, d, block_size, float(scale), k, 1, sink_block, cur_block, fill, 0, 0)


class PreparedSelectDecode:
    """`lkv_select_decode` with its arguments converted once: the Quest bound of candidates
    cand_offset .. cand_offset + n_cand - 1 from metadata `[1, h, cap, d]`, the top k per head, and
    the block-sparse decode over sink + selected (from `sel`) + current. `desc.fill` /
    `desc.cur_block` and `n_cand` (`set_candidates`, up to the count the workspace was sized for) may
    change between calls."""

    def __init__(self, q: torch.Tensor, kmin: torch.Tensor, kmax: torch.Tensor, k: int, *, cand_offset: int, n_cand: int, block_size: int,
                 scale: float, sel: Source, sink: Source | None, sink_block: int, cur: Source | None, cur_block: int, fill: int,
                 out: torch.Tensor, lse: torch.Tensor, rank_mode: int = _lib.RANK_F32, out_idx: torch.Tensor | None = None,
                 ws: Workspace | None = None, max_cand: int | None = None) -> None:
        _lib.require_cuda(q, kmin, kmax, out, lse)
        n_kv, cap, d, hs = _meta_layout(kmin, kmax)
        qq = q.reshape(-1, d)
        if not qq.is_contiguous() or qq.shape[0] % n_kv:
            raise ValueError("query must be contiguous [n_q, d] with n_q a multiple of the KV heads")
        if cand_offset < 0 or n_cand <= 0 or cand_offset + n_cand > cap or not 0 < k <= n_cand:
            raise ValueError(f"candidates {cand_offset}..{cand_offset + n_cand} of {cap} metadata blocks, k={k}")
        if not out.is_contiguous() or out.numel() != qq.numel() or not lse.is_contiguous() or lse.numel() != qq.shape[0] or lse.dtype != torch.float32:
            raise ValueError("out must be contiguous [n_q, d] and lse contiguous float32 [n_q]")
        if out_idx is not None and (out_idx.dtype != torch.int32 or tuple(out_idx.shape) != (n_kv, k) or not out_idx.is_contiguous()):
            raise ValueError(f"out_idx must be contiguous int32 [{n_kv}, {k}]")
        self.desc = _select_desc(qq, n_kv, block_size, scale, k, sink_block, cur_block, fill)
        ws = ws or default_workspace(q.device)
        sizing = max(n_cand, max_cand or 0)
        ws_ptr, ws_n = ws.get(_lib.lib().lkv_select_decode_workspace_bytes(ctypes.byref(self.desc), sizing))
        self._c = [s.c() if s is not None else None for s in (sel, sink, cur)]
        refs = [ctypes.byref(c) if c is not None else None for c in self._c]
        self._keep = (q, kmin, kmax, out, lse, out_idx, ws.buf, sel, sink, cur)
        self._fn = _lib.lib().lkv_select_decode
        self._head = (ctypes.byref(self.desc), qq.data_ptr(), _lib.dtype_code(qq.dtype), address(kmin[0] if kmin.ndim == 4 else kmin),
                      address(kmax[0] if kmax.ndim == 4 else kmax), _lib.dtype_code(kmin.dtype), hs, cand_offset)
        self._tail = (rank_mode, refs[0], refs[1], refs[2], out.data_ptr(), _lib.dtype_code(out.dtype), lse.data_ptr(),
                      out_idx.data_ptr() if out_idx is not None else None, k, ws_ptr, ws_n)
        self.n_cand = n_cand
        self._sized = sizing
        self._cap = min(cap - cand_offset, sizing)
        self.device = q.device

    def set_candidates(self, n_cand: int) -> None:
        """A new candidate count, up to the one the workspace was sized for (the constructor's
        n_cand, or max_cand). The count decides where the top K is chosen and which kernel instance
        runs, so a HIP graph captured before the change must be captured again after it."""
        if not self.desc.k <= n_cand <= self._cap:
            raise ValueError(f"{n_cand} candidates for k={self.desc.k}: at most {self._cap} (the workspace was sized for {self._sized})")
        self.n_cand = n_cand

    def __call__(self) -> None:
        rc = self._fn(torch.cuda.current_stream(self.device).cuda_stream, *self._head, self.n_cand, *self._tail)
        if rc:
            _lib.check(rc, "select_decode")


def select_decode(q: torch.Tensor, kmin: torch.Tensor, kmax: torch.Tensor, k: int, *, cand_offset: int, n_cand: int, block_size: int, scale: float,
                  sel: Source, sink: Source | None = None, sink_block: int = -1, cur: Source | None = None, cur_block: int = -1, fill: int = 0,
                  rank_mode: int = _lib.RANK_F32, out: torch.Tensor | None = None, out_dtype: torch.dtype | None = None, lse: torch.Tensor | None = None,
                  out_idx: torch.Tensor | None = None, ws: Workspace | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Bound + top-k + block-sparse decode of one layer (lkv_select_decode). Returns (out [n_q, d], lse [n_q])."""
    qq = q.reshape(-1, q.shape[-1]).contiguous()
    n_q, d = qq.shape
    out_dtype = out_dtype or (out.dtype if out is not None else qq.dtype)
    out = out if out is not None else torch.empty((n_q, d), dtype=out_dtype, device=q.device)
    lse = lse if lse is not None else torch.empty((n_q,), dtype=torch.float32, device=q.device)
    PreparedSelectDecode(qq, kmin, kmax, k, cand_offset=cand_offset, n_cand=n_cand, block_size=block_size, scale=scale, sel=sel, sink=sink,
                         sink_block=sink_block, cur=cur, cur_block=cur_block, fill=fill, out=out, lse=lse, rank_mode=rank_mode, out_idx=out_idx, ws=ws)()
    return out, lse


# -- hybrid residency: hits from HBM slots, misses read in place and admitted -------------------------


@dataclass
class Residency:
    """HBM slots of one layer (`slots` [n_slots, h, 2, bs, d]) and the tables that say what they hold:
    block_slot [h, cap] (slot or -1), slot_block [h, n_slots] (block or -1), and `order` [h, n_slots]:
    each head's slots from least to most recently used, ties to the lower slot. All int32 on the GPU.
    With n_slots == k the order decides only which unhit slot a missed block lands in (every unhit
    slot is evicted), and the library accepts None there; `allocate` always keeps it, so the tables
    follow the reference's least-recently-used rule slot for slot."""

    slots: torch.Tensor
    block_slot: torch.Tensor
    slot_block: torch.Tensor
    order: torch.Tensor | None = None

    @classmethod
    def allocate(cls, k: int, h: int, cap_blocks: int, block_size: int, head_dim: int, dtype: torch.dtype, device: torch.device,
                 n_slots: int | None = None) -> Residency:
        n = k if n_slots is None else n_slots
        if n < k:
            raise ValueError(f"{n} slots cannot hold a selection of {k} blocks")
        order = torch.arange(n, dtype=torch.int32, device=device).repeat(h, 1)
        return cls(torch.zeros((n, h, 2, block_size, head_dim), dtype=dtype, device=device),
                   torch.full((h, cap_blocks), -1, dtype=torch.int32, device=device),
                   torch.full((h, n), -1, dtype=torch.int32, device=device), order)

    @property
    def n_slots(self) -> int:
        return self.slots.shape[0]

    def seed(self, first: int, n: int) -> None:
        """Record that slots 0..n-1 of every head hold blocks first..first+n-1 (the caller has written
        them), with the empty slots least recently used: the reference's seeded residency
        (lazykv/tiered.py:274-287). Device-side fills only."""
        dev = self.slot_block.device
        blocks = torch.arange(first, first + n, dtype=torch.int32, device=dev)
        self.slot_block[:, :n] = blocks
        self.block_slot[:, first : first + n] = torch.arange(n, dtype=torch.int32, device=dev)
        if self.order is not None:
            used = torch.cat([torch.arange(n, self.n_slots, device=dev), torch.arange(0, n, device=dev)]).to(torch.int32)
            self.order.copy_(used.expand_as(self.order))

    def tables(self) -> _lib.ResidencyTables:
        order = self.order
        return _lib.ResidencyTables(self.block_slot.data_ptr(), self.block_slot.stride(0), self.slot_block.data_ptr(), self.slot_block.stride(0),
                                    order.data_ptr() if order is not None else None, order.stride(0) if order is not None else 0)

    def check(self, n_kv: int, n_blocks: int, k: int) -> None:
        """Shapes the residency launch relies on: tables with contiguous rows covering the pool's
        blocks and the slots, and n_slots >= k."""
        n = self.n_slots
        for t, want in ((self.block_slot, n_blocks), (self.slot_block, n)) + (((self.order, n),) if self.order is not None else ()):
            if t.dtype != torch.int32 or t.ndim != 2 or t.shape[0] != n_kv or t.shape[1] < want or t.stride(1) != 1:
                raise ValueError(f"residency table must be int32 [{n_kv}, >= {want}] with contiguous rows, got {tuple(t.shape)} {t.dtype}")
        if n < k:
            raise ValueError(f"the slot pool holds {n} slots per head, fewer than k={k}")
        if n > k and self.order is None:
            raise ValueError(f"{n} slots for k={k} need the slots' use order")


def hybrid_decode(
    q: torch.Tensor,
    *,
    n_kv: int,
    block_size: int,
    scale: float,
    host: Source,
    res: Residency,
    idx: torch.Tensor,
    sink: Source | None = None,
    sink_block: int = -1,
    cur: Source | None = None,
    cur_block: int = -1,
    fill: int = 0,
    rem: Source | None = None,
    rem_range: tuple[int, int] = (0, 0),
    out: torch.Tensor | None = None,
    out_dtype: torch.dtype | None = None,
    lse: torch.Tensor | None = None,
    ws: Workspace | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """lkv_hybrid_decode: `sparse_decode` over `host` with the selected pairs in `res`'s slots read
    from HBM, the others read in place and admitted; with `rem`, also every block of `rem_range` the
    selection does not name (the exact tier's remainder). Updates `res`'s tables."""
    p = PreparedHybridDecode(q, n_kv=n_kv, block_size=block_size, scale=scale, host=host, res=res, idx=idx, sink=sink, sink_block=sink_block,
                             cur=cur, cur_block=cur_block, fill=fill, rem=rem, rem_range=rem_range, out=out, out_dtype=out_dtype, lse=lse, ws=ws)
    p()
    return p.out, p.lse


class PreparedHybridDecode:
    """`hybrid_decode` with its arguments converted once; `desc.fill` / `desc.cur_block` may change between calls."""

    def __init__(self, q: torch.Tensor, *, n_kv: int, block_size: int, scale: float, host: Source, res: Residency, idx: torch.Tensor, sink: Source | None,
                 sink_block: int, cur: Source | None, cur_block: int, fill: int, rem: Source | None = None, rem_range: tuple[int, int] = (0, 0),
                 out: torch.Tensor | None = None, out_dtype: torch.dtype | None = None, lse: torch.Tensor | None = None, ws: Workspace | None = None) -> None:
        _lib.require_cuda(q, idx, res.slots, res.block_slot, res.slot_block)
        qq = q.reshape(-1, q.shape[-1]).contiguous()
        n_q, d = qq.shape
        if idx.dtype != torch.int32 or idx.ndim != 2 or idx.shape[0] != n_kv or not idx.is_contiguous():
            raise ValueError(f"idx must be contiguous int32 [{n_kv}, k], got {tuple(idx.shape)} {idx.dtype}")
        k = idx.shape[1]
        res.check(n_kv, host.n_blocks, k)
        out_dtype = out_dtype or (out.dtype if out is not None else qq.dtype)
        self.out = out if out is not None else torch.empty((n_q, d), dtype=out_dtype, device=q.device)
        self.lse = lse if lse is not None else torch.empty((n_q,), dtype=torch.float32, device=q.device)
        r0, r1 = rem_range if rem is not None else (0, 0)
        self.desc = _lib.DecodeDesc(n_q, n_kv, d, block_size, float(scale), k, 1, sink_block, cur_block, fill, r0, r1)
        ws = ws or default_workspace(q.device)
        ws_ptr, ws_n = ws.get(_lib.lib().lkv_hybrid_decode_workspace_bytes(ctypes.byref(self.desc)))
        slot_src = pool_source(res.slots)
        self._c = [s.c() if s is not None else None for s in (host, slot_src, sink, cur, rem)]
        self._tables = res.tables()
        refs = [ctypes.byref(c) if c is not None else None for c in self._c]
        self._keep = (qq, idx, self.out, self.lse, ws.buf, host, res, sink, cur, rem)
        self._fn = _lib.lib().lkv_hybrid_decode
        self._args = (ctypes.byref(self.desc), qq.data_ptr(), _lib.dtype_code(qq.dtype), refs[0], refs[1], idx.data_ptr(), idx.stride(0),
                      ctypes.byref(self._tables), refs[2], refs[3], refs[4], self.out.data_ptr(), _lib.dtype_code(self.out.dtype),
                      self.lse.data_ptr(), ws_ptr, ws_n)
        self.device = q.device

    def __call__(self) -> None:
        rc = self._fn(torch.cuda.current_stream(self.device).cuda_stream, *self._args)
        if rc:
            _lib.check(rc, "hybrid_decode")


class PreparedSelectHybridDecode:
    """`lkv_select_hybrid_decode` with its arguments converted once: the Quest bound of candidates
    cand_offset .. cand_offset + n_cand - 1 from metadata `[1, h, cap, d]`, the top k per head chosen
    by the launch that updates `res`'s tables, and the hybrid decode over sink + selected (hits from
    `res`'s slots, misses from `host`) + current, plus, with `rem`, the exact tier's remainder.
    Equals `PreparedBoundTopk` followed by `PreparedHybridDecode`, bit for bit. `desc.fill` /
    `desc.cur_block` and `n_cand` (`set_candidates`, up to the count the workspace was sized for)
    may change between calls."""

    def __init__(self, q: torch.Tensor, kmin: torch.Tensor, kmax: torch.Tensor, k: int, *, cand_offset: int, n_cand: int, block_size: int,
                 scale: float, host: Source, res: Residency, sink: Source | None, sink_block: int, cur: Source | None, cur_block: int, fill: int,
                 out: torch.Tensor, lse: torch.Tensor, rem: Source | None = None, rem_range: tuple[int, int] = (0, 0), rank_mode: int = _lib.RANK_F32,
                 out_idx: torch.Tensor | None = None, ws: Workspace | None = None, max_cand: int | None = None) -> None:
        _lib.require_cuda(q, kmin, kmax, out, lse, res.slots, res.block_slot, res.slot_block)
        n_kv, cap, d, hs = _meta_layout(kmin, kmax)
        qq = q.reshape(-1, d)
        if not qq.is_contiguous() or qq.shape[0] % n_kv:
            raise ValueError("query must be contiguous [n_q, d] with n_q a multiple of the KV heads")
        if cand_offset < 0 or n_cand <= 0 or cand_offset + n_cand > cap or not 0 < k <= n_cand:
            raise ValueError(f"candidates {cand_offset}..{cand_offset + n_cand} of {cap} metadata blocks, k={k}")
        if not out.is_contiguous() or out.numel() != qq.numel() or not lse.is_contiguous() or lse.numel() != qq.shape[0] or lse.dtype != torch.float32:
            raise ValueError("out must be contiguous [n_q, d] and lse contiguous float32 [n_q]")
        if out_idx is not None and (out_idx.dtype != torch.int32 or tuple(out_idx.shape) != (n_kv, k) or not out_idx.is_contiguous()):
            raise ValueError(f"out_idx must be contiguous int32 [{n_kv}, {k}]")
        res.check(n_kv, host.n_blocks, k)
        self.desc = _select_desc(qq, n_kv, block_size, scale, k, sink_block, cur_block, fill)
        if rem is not None:
            self.desc.rem_first, self.desc.rem_last = rem_range
        ws = ws or default_workspace(q.device)
        sizing = max(n_cand, max_cand or 0)
        ws_ptr, ws_n = ws.get(_lib.lib().lkv_select_hybrid_decode_workspace_bytes(ctypes.byref(self.desc), sizing))
        self._c = [s.c() if s is not None else None for s in (host, pool_source(res.slots), sink, cur, rem)]
        self._tables = res.tables()
        refs = [ctypes.byref(c) if c is not None else None for c in self._c]
        self._keep = (q, kmin, kmax, out, lse, out_idx, ws.buf, host, res, sink, cur, rem)
        self._fn = _lib.lib().lkv_select_hybrid_decode
        self._head = (ctypes.byref(self.desc), qq.data_ptr(), _lib.dtype_code(qq.dtype), address(kmin[0] if kmin.ndim == 4 else kmin),
                      address(kmax[0] if kmax.ndim == 4 else kmax), _lib.dtype_code(kmin.dtype), hs, cand_offset)
        self._tail = (rank_mode, refs[0], refs[1], ctypes.byref(self._tables), refs[2], refs[3], refs[4], out.data_ptr(), _lib.dtype_code(out.dtype),
                      lse.data_ptr(), out_idx.data_ptr() if out_idx is not None else None, k, ws_ptr, ws_n)
        self.n_cand = n_cand
        self._sized = sizing
        self._cap = min(cap - cand_offset, sizing)
        self.device = q.device

    def set_candidates(self, n_cand: int) -> None:
        """A new candidate count, up to the one the workspace was sized for (the constructor's
        n_cand, or max_cand). A HIP graph captured before the change keeps the old count: capture
        again after it."""
        if not self.desc.k <= n_cand <= self._cap:
            raise ValueError(f"{n_cand} candidates for k={self.desc.k}: at most {self._cap} (the workspace was sized for {self._sized})")
        self.n_cand = n_cand

    def __call__(self) -> None:
        rc = self._fn(torch.cuda.current_stream(self.device).cuda_stream, *self._head, self.n_cand, *self._tail)
        if rc:
            _lib.check(rc, "select_hybrid_decode")


def select_hybrid_decode(q: torch.Tensor, kmin: torch.Tensor, kmax: torch.Tensor, k: int, *, cand_offset: int, n_cand: int, block_size: int,
                         scale: float, host: Source, res: Residency, sink: Source | None = None, sink_block: int = -1, cur: Source | None = None,
                         cur_block: int = -1, fill: int = 0, rem: Source | None = None, rem_range: tuple[int, int] = (0, 0),
                         rank_mode: int = _lib.RANK_F32, out: torch.Tensor | None = None, out_dtype: torch.dtype | None = None,
                         lse: torch.Tensor | None = None, out_idx: torch.Tensor | None = None, ws: Workspace | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Bound + top-k + hybrid decode of one layer (lkv_select_hybrid_decode), with the exact tier's
    remainder when `rem` is given. Returns (out [n_q, d], lse [n_q])."""
    qq = q.reshape(-1, q.shape[-1]).contiguous()
    n_q, d = qq.shape
    out_dtype = out_dtype or (out.dtype if out is not None else qq.dtype)
    out = out if out is not None else torch.empty((n_q, d), dtype=out_dtype, device=q.device)
    lse = lse if lse is not None else torch.empty((n_q,), dtype=torch.float32, device=q.device)
    PreparedSelectHybridDecode(qq, kmin, kmax, k, cand_offset=cand_offset, n_cand=n_cand, block_size=block_size, scale=scale, host=host, res=res,
                               sink=sink, sink_block=sink_block, cur=cur, cur_block=cur_block, fill=fill, out=out, lse=lse, rem=rem, rem_range=rem_range,
                               rank_mode=rank_mode, out_idx=out_idx, ws=ws)()
    return out, lse


# -- a8: merge --------------------------------------------------------------------------------------


def merge_lse(out_a: torch.Tensor, lse_a: torch.Tensor, out_b: torch.Tensor, lse_b: torch.Tensor, out_dtype: torch.dtype | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    _lib.require_cuda(out_a, lse_a, out_b, lse_b)
    if out_a.shape != out_b.shape or lse_a.shape != lse_b.shape or out_a.shape[:-1] != lse_a.shape:
        raise ValueError(f"partials must match: {tuple(out_a.shape)}/{tuple(lse_a.shape)} vs {tuple(out_b.shape)}/{tuple(lse_b.shape)}")
    dt = torch.promote_types(out_a.dtype, out_b.dtype)
    a = out_a.to(dt).contiguous()
    b = out_b.to(dt).contiguous()
    la = lse_a.float().contiguous()
    lb = lse_b.float().contiguous()
    d = a.shape[-1]
    rows = a.numel() // d if d else 0
    out = torch.empty(a.shape, dtype=out_dtype or dt, device=a.device)
    lse = torch.empty(la.shape, dtype=torch.float32, device=a.device)
    rc = _lib.lib().lkv_merge_lse(_lib.stream_of(a), a.data_ptr(), la.data_ptr(), b.data_ptr(), lb.data_ptr(), _lib.dtype_code(dt), rows, d, out.data_ptr(), _lib.dtype_code(out.dtype), lse.data_ptr())
    _lib.check(rc, "merge_lse")
    return out, lse


# -- a4, a10, a11: stores ---------------------------------------------------------------------------


def store_blocks(
    src: Source,
    *,
    n_kv: int,
    head_dim: int,
    block_size: int,
    first_block: int,
    n_blocks: int,
    dst: Source | None = None,
    kmin: torch.Tensor | None = None,
    kmax: torch.Tensor | None = None,
    stream: int | None = None,
) -> None:
    """Copy / int8-pack blocks and write their key min/max metadata (lkv_store_blocks).

    kmin/kmax are the full `[1, h, cap, d]` metadata tensors; block b of head h lands at [0, h, b].
    """
    mh, mdt, kmin_p, kmax_p = 0, _lib.F16, None, None
    if kmin is not None:
        _lib.require_cuda(kmin, kmax)
        n, cap, d, mh = _meta_layout(kmin, kmax)
        if n != n_kv or d != head_dim or first_block + n_blocks > cap:
            raise ValueError(f"metadata {tuple(kmin.shape)} cannot hold blocks {first_block}..{first_block + n_blocks} of {n_kv} heads")
        mdt = _lib.dtype_code(kmin.dtype)
        kmin_p, kmax_p = address(kmin), address(kmax)
    if first_block + n_blocks > src.n_blocks or (dst is not None and first_block + n_blocks > dst.n_blocks):
        raise ValueError("block range exceeds the source or destination")
    s = src.c()
    dd = dst.c() if dst is not None else None
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    rc = _lib.lib().lkv_store_blocks(stream, ctypes.byref(s), ctypes.byref(dd) if dd is not None else None, n_kv, head_dim, block_size, first_block, n_blocks, kmin_p, kmax_p, mdt, mh)
    _lib.check(rc, "store_blocks")


def packed_pair_bytes(block_size: int, head_dim: int) -> int:
    return int(_lib.lib().lkv_packed_pair_bytes(block_size, head_dim))


def pack_int8(pairs: torch.Tensor) -> torch.Tensor:
    """`[m, 2, bs, d]` model dtype -> `[m, P]` uint8 records (lkv_pack_int8)."""
    _lib.require_cuda(pairs)
    m, two, bs, d = pairs.shape
    x = pairs.contiguous()
    out = torch.empty((m, packed_pair_bytes(bs, d)), dtype=torch.uint8, device=pairs.device)
    _lib.check(_lib.lib().lkv_pack_int8(_lib.stream_of(x), x.data_ptr(), _lib.dtype_code(x.dtype), m, bs, d, out.data_ptr()), "pack_int8")
    return out


def unpack_int8(records: torch.Tensor, block_size: int, head_dim: int, dtype: torch.dtype) -> torch.Tensor:
    """`[m, P]` uint8 records -> `[m, 2, bs, d]` (lkv_unpack_int8)."""
    _lib.require_cuda(records)
    r = records.contiguous()
    out = torch.empty((r.shape[0], 2, block_size, head_dim), dtype=dtype, device=records.device)
    _lib.check(_lib.lib().lkv_unpack_int8(_lib.stream_of(r), r.data_ptr(), r.shape[0], block_size, head_dim, _lib.dtype_code(dtype), out.data_ptr()), "unpack_int8")
    return out


def stream_read(src_addr: int, nbytes: int, blocks: int, sink: torch.Tensor) -> None:
    """Launch the link probe over `nbytes` at a device-visible address; sink is uint32 [>= blocks] on the GPU."""
    _lib.check(_lib.lib().lkv_stream_read(_lib.stream_of(sink), src_addr, nbytes, blocks, sink.data_ptr()), "stream_read")


# -- prepared launches ------------------------------------------------------------------------------


class PreparedBoundTopk:
    """`bound_topk` with every argument converted once; calling it only launches.

    For loops that issue the same selection per step (a decode step over many layers), or for
    capture into a HIP graph: the stream is read at call time.
    """

    def __init__(self, q: torch.Tensor, kmin: torch.Tensor, kmax: torch.Tensor, k: int, *, cand_offset: int, n_cand: int, out_idx: torch.Tensor | None = None,
                 rank_mode: int = _lib.RANK_F32, ws: Workspace | None = None, out_bound: torch.Tensor | None = None) -> None:
        """k == 0 with `out_bound` [h, n_cand] float32: the bounds only."""
        _lib.require_cuda(q, kmin, kmax)
        n_kv, cap, d, hs = _meta_layout(kmin, kmax)
        if cand_offset < 1 or cand_offset + n_cand > cap or k > n_cand:
            raise ValueError("candidate range outside the metadata, or k > n_cand")
        if k > 0 and (out_idx is None or out_idx.dtype != torch.int32 or tuple(out_idx.shape) != (n_kv, k) or not out_idx.is_contiguous()):
            raise ValueError(f"out_idx must be contiguous int32 [{n_kv}, {k}]")
        if k == 0 and (out_bound is None or out_bound.dtype != torch.float32 or tuple(out_bound.shape) != (n_kv, n_cand) or not out_bound.is_contiguous()):
            raise ValueError(f"bounds only: out_bound must be contiguous float32 [{n_kv}, {n_cand}]")
        qq = q.reshape(-1, d)
        if not qq.is_contiguous() or qq.shape[0] % n_kv:
            raise ValueError("query must be contiguous [n_q, d] with n_q a multiple of the KV heads")
        ws = ws or default_workspace(q.device)
        ws_ptr, ws_n = ws.get(_lib.lib().lkv_bound_topk_workspace_bytes(n_kv, n_cand, k))
        self._keep = (q, kmin, kmax, out_idx, out_bound, ws.buf)
        self._fn = _lib.lib().lkv_bound_topk
        self._args = (qq.data_ptr(), _lib.dtype_code(qq.dtype), address(kmin[0] if kmin.ndim == 4 else kmin), address(kmax[0] if kmax.ndim == 4 else kmax),
                      _lib.dtype_code(kmin.dtype), hs, qq.shape[0], n_kv, d, cand_offset, n_cand, k, rank_mode, 0,
                      out_idx.data_ptr() if out_idx is not None else None, max(k, 1), out_bound.data_ptr() if out_bound is not None else None, ws_ptr, ws_n)
        self.device = q.device

    def __call__(self) -> None:
        rc = self._fn(torch.cuda.current_stream(self.device).cuda_stream, *self._args)
        if rc:
            _lib.check(rc, "bound_topk")


class PreparedDecode:
    """`sparse_decode` with every argument converted once; `desc` fields (fill, cur_block, rem
    range) may be updated between calls without re-preparing."""

    def __init__(self, q: torch.Tensor, *, n_kv: int, block_size: int, scale: float, sel: Source | None, idx: torch.Tensor | None, sink: Source | None, sink_block: int,
                 cur: Source | None, cur_block: int, fill: int, out: torch.Tensor, lse: torch.Tensor, rem: Source | None = None, rem_range: tuple[int, int] = (0, 0),
                 attend_selected: bool = True, ws: Workspace | None = None, max_rem_blocks: int = 0) -> None:
        qq = q.reshape(-1, q.shape[-1])
        n_q, d = qq.shape
        k = idx.shape[1] if idx is not None else 0
        self.desc = _lib.DecodeDesc(n_q, n_kv, d, block_size, float(scale), k, 1 if attend_selected else 0, sink_block, cur_block, fill, rem_range[0], rem_range[1])
        # Size the workspace for the largest remainder this call will be updated to.
        sizing = _lib.DecodeDesc(n_q, n_kv, d, block_size, float(scale), k, 1 if attend_selected else 0, sink_block, cur_block, fill, 0, max(rem_range[1] - rem_range[0], max_rem_blocks))
        ws = ws or default_workspace(q.device)
        ws_ptr, ws_n = ws.get(max(_lib.lib().lkv_sparse_decode_workspace_bytes(ctypes.byref(self.desc)), _lib.lib().lkv_sparse_decode_workspace_bytes(ctypes.byref(sizing))))
        self._c = [s.c() if s is not None else None for s in (sel, sink, cur, rem)]
        refs = [ctypes.byref(c) if c is not None else None for c in self._c]
        self._keep = (q, idx, out, lse, ws.buf, sel, sink, cur, rem)
        self._fn = _lib.lib().lkv_sparse_decode
        self._args = (ctypes.byref(self.desc), qq.data_ptr(), _lib.dtype_code(qq.dtype), refs[0], idx.data_ptr() if idx is not None else None, k,
                      refs[1], refs[2], refs[3], out.data_ptr(), _lib.dtype_code(out.dtype), lse.data_ptr(), ws_ptr, ws_n)
        self.device = q.device

    def __call__(self) -> None:
        rc = self._fn(torch.cuda.current_stream(self.device).cuda_stream, *self._args)
        if rc:
            _lib.check(rc, "sparse_decode")
