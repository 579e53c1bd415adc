"""The C ABI (CPU): the library loads, exports every function include/lazykv_hip.h declares, and
rejects bad arguments before touching a device."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "lazykv_hip.h"


def _declared() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lkv_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from lazykv_amd import _lib

    return _lib.lib()


def test_header_declares_the_hot_path_entry_points() -> None:
    names = _declared()
    for want in ("lkv_bound_topk", "lkv_sparse_decode", "lkv_merge_lse", "lkv_store_blocks", "lkv_pack_int8", "lkv_unpack_int8", "lkv_host_alloc", "lkv_last_error"):
        assert want in names


def test_library_exports_every_declared_symbol(lib) -> None:  # noqa: ANN001
    for name in _declared():
        assert hasattr(lib, name), name


def test_binding_covers_every_declared_symbol() -> None:
    from lazykv_amd import _lib

    assert sorted(_lib.SIGNATURES) == _declared()


def test_abi_version_and_record_width(lib) -> None:  # noqa: ANN001
    from oracle import reference as R

    assert lib.lkv_abi_version() == 4
    for bs, d in ((16, 64), (16, 128), (8, 64), (64, 64)):
        assert lib.lkv_packed_pair_bytes(bs, d) == R.packed_pair_bytes(bs, d)


def test_workspace_sizes_are_host_only(lib) -> None:  # noqa: ANN001
    from lazykv_amd import _lib

    assert lib.lkv_bound_topk_workspace_bytes(8, 8190, 512) >= 8 * 8190 * 4
    desc = _lib.DecodeDesc(32, 8, 128, 16, 0.088, 512, 1, 0, 8191, 16, 0, 0)
    assert lib.lkv_sparse_decode_workspace_bytes(ctypes.byref(desc)) > 8 * 4 * 128 * 4
    bad = _lib.DecodeDesc(30, 8, 128, 16, 0.088, 512, 1, 0, 8191, 16, 0, 0)
    assert lib.lkv_sparse_decode_workspace_bytes(ctypes.byref(bad)) == 0


def test_bad_arguments_are_rejected_before_any_launch(lib) -> None:  # noqa: ANN001
    from lazykv_amd import _lib

    dummy = ctypes.c_void_p(16)
    rc = lib.lkv_bound_topk(0, dummy, _lib.BF16, dummy, dummy, _lib.BF16, 0, 32, 8, 96, 1, 100, 10, 0, 0, dummy, 10, None, dummy, 1 << 20)
    assert rc == _lib.LKV_ERR_INVALID
    assert b"head_dim" in lib.lkv_last_error()
    rc = lib.lkv_bound_topk(0, dummy, _lib.BF16, dummy, dummy, _lib.BF16, 1 << 20, 32, 8, 128, 1, 100, 101, 0, 0, dummy, 101, None, dummy, 1 << 20)
    assert rc == _lib.LKV_ERR_INVALID and b"k=101" in lib.lkv_last_error()
    rc = lib.lkv_pack_int8(0, None, _lib.BF16, 4, 16, 128, None)
    assert rc == _lib.LKV_ERR_INVALID
    desc = _lib.DecodeDesc(32, 8, 128, 17, 0.088, 0, 1, 0, -1, 1, 0, 0)
    rc = lib.lkv_sparse_decode(0, ctypes.byref(desc), dummy, _lib.BF16, None, None, 0, None, None, None, dummy, _lib.BF16, dummy, dummy, 1 << 20)
    assert rc == _lib.LKV_ERR_INVALID and b"block_size" in lib.lkv_last_error()
    desc = _lib.DecodeDesc(32, 8, 128, 260, 0.088, 0, 1, 0, -1, 1, 0, 0)  # past the largest block size (256)
    rc = lib.lkv_sparse_decode(0, ctypes.byref(desc), dummy, _lib.BF16, None, None, 0, None, None, None, dummy, _lib.BF16, dummy, dummy, 1 << 20)
    assert rc == _lib.LKV_ERR_INVALID and b"block_size" in lib.lkv_last_error()
    # The one-call decode step: more candidates than any selection takes, k past them.
    desc = _lib.DecodeDesc(32, 8, 128, 16, 0.088, 512, 1, 0, 1, 16, 0, 0)
    rc = lib.lkv_select_decode(0, ctypes.byref(desc), dummy, _lib.BF16, dummy, dummy, _lib.BF16, 1 << 30, 1, 300000, 0, None, None, None,
                               dummy, _lib.BF16, dummy, None, 0, dummy, 1 << 30)
    assert rc == _lib.LKV_ERR_INVALID and b"300000 candidate blocks" in lib.lkv_last_error()
    rc = lib.lkv_select_decode(0, ctypes.byref(desc), dummy, _lib.BF16, dummy, dummy, _lib.BF16, 1 << 24, 1, 500, 0, None, None, None,
                               dummy, _lib.BF16, dummy, None, 0, dummy, 1 << 24)
    assert rc == _lib.LKV_ERR_INVALID and b"k=512" in lib.lkv_last_error()


def test_errors_map_to_the_reference_exception_types() -> None:
    from lazykv_amd import _lib

    _lib.lib().lkv_pack_int8(0, None, _lib.BF16, 4, 16, 128, None)
    with pytest.raises(ValueError, match="NULL"):
        _lib.check(_lib.LKV_ERR_INVALID, "pack")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.LKV_ERR_HIP, "x")


def test_product_modules_import_without_the_oracle() -> None:
    """The product path never imports the oracle: scan the package sources."""
    for path in (ROOT / "lazykv_amd").rglob("*.py"):
        src = path.read_text()
        assert "import oracle" not in src and "from oracle" not in src, path


def test_cpu_tensors_are_refused_not_computed() -> None:
    import torch

    from lazykv_amd import quant

    with pytest.raises(RuntimeError, match="GPU"):
        quant.pack(torch.zeros((1, 2, 16, 64), dtype=torch.bfloat16))
