"""The allocation-free decode entry point (lkv_sparse_decode_static) against lkv_sparse_decode.

Both are called through the C ABI on the same inputs: the static entry point keeps its partials in
the library's per-device scratch array instead of a caller workspace, and must give the same output
and LSE bit for bit, on two calls in a row (the second smaller, so it reuses what the first left in
the array), with nothing allocated by torch's allocator during either call, and it must refuse a
shape whose partials exceed the array."""

from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _case(seed: int, n_kv: int, g: int, d: int, bs: int, n_blocks: int, k: int, fill: int, rem: bool):  # noqa: ANN202
    """A host-pool decode (selected pairs in mapped host memory), optionally with an exact remainder."""
    from lazykv_amd import kernels
    from lazykv_amd.pinned import pinned_empty

    gen = torch.Generator().manual_seed(seed)
    pool = (torch.randn((n_blocks, n_kv, 2, bs, d), generator=gen) * 1.3).to(torch.bfloat16)
    host = pinned_empty(tuple(pool.shape), pool.dtype)
    host.copy_(pool)
    hbm = pool.cuda()
    q = torch.randn((n_kv * g, d), generator=gen).to(torch.bfloat16).cuda()
    idx = torch.stack([torch.randperm(n_blocks - 2, generator=gen)[:k] + 1 for _ in range(n_kv)]).sort(dim=1).values.to(torch.int32).cuda()
    sel = kernels.pool_source(host)
    slots = kernels.pool_source(hbm)
    rem_src = kernels.pool_source(hbm) if rem else None
    desc = kernels._lib.DecodeDesc(n_kv * g, n_kv, d, bs, d**-0.5, k, 1, 0, n_blocks - 1, fill, 1 if rem else 0, n_blocks - 1 if rem else 0)
    return dict(q=q, idx=idx, sel=sel, sink=slots, cur=slots, rem=rem_src, desc=desc, keep=(host, hbm))


def _call(lib, case, static: bool, out: torch.Tensor, lse: torch.Tensor, ws: torch.Tensor | None = None) -> int:  # noqa: ANN001
    from lazykv_amd import _lib

    srcs = [case[n].c() if case[n] is not None else None for n in ("sel", "sink", "cur", "rem")]
    refs = [ctypes.byref(c) if c is not None else None for c in srcs]
    stream = torch.cuda.current_stream().cuda_stream
    common = (stream, ctypes.byref(case["desc"]), case["q"].data_ptr(), _lib.BF16, refs[0], case["idx"].data_ptr(), case["idx"].stride(0),
              refs[1], refs[2], refs[3], out.data_ptr(), _lib.F32, lse.data_ptr())
    if static:
        return lib.lkv_sparse_decode_static(*common)
    return lib.lkv_sparse_decode(*common, ws.data_ptr(), ws.numel())


def test_static_decode_equals_the_workspace_decode_on_consecutive_calls() -> None:
    from lazykv_amd import _lib

    lib = _lib.lib()
    torch.cuda.set_device(0)
    cases = [
        ("8 kv heads, d 128, exact remainder", _case(1, 8, 4, 128, 16, 700, 48, 9, rem=True)),
        ("2 kv heads, d 64, no remainder (smaller)", _case(2, 2, 4, 64, 16, 90, 8, 16, rem=False)),
    ]
    for name, case in cases:
        print(f"static decode case: {name}", flush=True)
        n_q, d = case["q"].shape
        need = lib.lkv_sparse_decode_workspace_bytes(ctypes.byref(case["desc"]))
        assert 0 < need <= _lib.STATIC_SCRATCH_BYTES
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        want_o = torch.empty((n_q, d), dtype=torch.float32, device="cuda")
        want_l = torch.empty((n_q,), dtype=torch.float32, device="cuda")
        got_o = torch.full((n_q, d), float("nan"), dtype=torch.float32, device="cuda")
        got_l = torch.full((n_q,), float("nan"), dtype=torch.float32, device="cuda")
        _lib.check(_call(lib, case, False, want_o, want_l, ws), "sparse_decode")
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated()
        _lib.check(_call(lib, case, True, got_o, got_l), "sparse_decode_static")
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated() == before
        assert torch.equal(got_o, want_o) and torch.equal(got_l, want_l), name
        assert torch.isfinite(got_o).all() and torch.isfinite(got_l).all()


def test_static_decode_refuses_partials_beyond_its_scratch() -> None:
    from lazykv_amd import _lib

    lib = _lib.lib()
    # 64 KV heads, groups of 8, d 128 and a long remainder: partials well past 16 MiB.
    desc = _lib.DecodeDesc(512, 64, 128, 16, 0.088, 0, 0, -1, -1, 0, 0, 1 << 20)
    assert lib.lkv_sparse_decode_workspace_bytes(ctypes.byref(desc)) > _lib.STATIC_SCRATCH_BYTES
    dummy = torch.zeros(16, device="cuda")
    src = _lib.KVSource(dummy.data_ptr(), dummy.data_ptr(), 0, 0, 1 << 20, _lib.BF16, _lib.BF16, 0)
    rc = lib.lkv_sparse_decode_static(torch.cuda.current_stream().cuda_stream, ctypes.byref(desc), dummy.data_ptr(), _lib.BF16, None, None, 0,
                                      None, None, ctypes.byref(src), dummy.data_ptr(), _lib.F32, dummy.data_ptr())
    assert rc == _lib.LKV_ERR_INVALID
    assert "allocation-free" in lib.lkv_last_error().decode()
