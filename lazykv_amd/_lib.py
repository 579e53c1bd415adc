"""ctypes binding of liblazykv_hip.so (the C ABI declared in include/lazykv_hip.h).

The library is built in-tree by `python -c "import __graft_entry__; __graft_entry__.build()"`
(or `make -C lazykv_amd`). There is no fallback: if the library is missing, or a call returns an
error, this module raises. torch is imported first so the HIP runtime the library binds to is the
one torch already loaded (the loader shares it by soname).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

SO_PATH = Path(__file__).resolve().parent / "liblazykv_hip.so"

LKV_OK, LKV_ERR_INVALID, LKV_ERR_HIP, LKV_ERR_UNSUPPORTED = 0, -1, -2, -3
F16, BF16, F32, INT8_RECORD = 0, 1, 2, 3
SORTED = 1
RANK_F32, RANK_MODEL = 0, 1
HOST_COHERENT = 1
SRC_HOST = 1
SELECT_IN_DECODE_MAX_CAND = 8192  # lkv_select_decode chooses the top K inside the decode launch up to this many candidates


def selects_in_decode(n_cand: int, host: bool, group: int, int8: bool = False, head_dim: int = 128, model_query: bool = True) -> bool:
    """Whether lkv_select_decode chooses the top K inside its decode launch, as the library decides.
    The decode launch must take the instance the unfused decode takes, and hold at most 16 candidates
    per thread, never beyond SELECT_IN_DECODE_MAX_CAND. Pairs in HBM with a query group of at most 4
    take 512-thread workgroups: matrix-core ones for a model-dtype query (`model_query`: the pools'
    dtype, 16-byte aligned), int8-capable ones for int8 records (except head_dim 128 with a group of
    4, which takes 256); an HBM launch with any other query has no selecting instance of its own and
    selects in its own launch. Everything else takes 256 threads."""
    if not host and group <= 4:
        if int8:
            threads = 256 if (head_dim == 128 and group == 4) else 512
        elif model_query:
            threads = 512
        else:
            return False
    else:
        threads = 256
    return n_cand <= min(SELECT_IN_DECODE_MAX_CAND, 16 * threads)


STATIC_SCRATCH_BYTES = 16 * 1024 * 1024  # LKV_STATIC_SCRATCH_BYTES: the allocation-free decode's partials per device

_DTYPE_CODES = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32}


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}; expected float16, bfloat16 or float32") from None


class KVSource(ctypes.Structure):
    """lkv_kv_source: where one set of KV blocks lives (see include/lazykv_hip.h)."""

    _fields_ = [
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("block_stride", ctypes.c_int64),
        ("head_stride", ctypes.c_int64),
        ("n_blocks", ctypes.c_int64),
        ("dtype", ctypes.c_int32),
        ("deq_dtype", ctypes.c_int32),
        ("flags", ctypes.c_int32),
    ]


class DecodeDesc(ctypes.Structure):
    """lkv_decode_desc: shape and sequence state of one decode-attention call."""

    _fields_ = [
        ("n_q", ctypes.c_int32),
        ("n_kv", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("k", ctypes.c_int32),
        ("attend_selected", ctypes.c_int32),
        ("sink_block", ctypes.c_int32),
        ("cur_block", ctypes.c_int32),
        ("fill", ctypes.c_int32),
        ("rem_first", ctypes.c_int32),
        ("rem_last", ctypes.c_int32),
    ]


class ResidencyTables(ctypes.Structure):
    """lkv_residency: a hybrid tier's tables (which block each HBM slot holds, and their use order)."""

    _fields_ = [
        ("block_slot", ctypes.c_void_p),
        ("block_slot_stride", ctypes.c_int64),
        ("slot_block", ctypes.c_void_p),
        ("slot_block_stride", ctypes.c_int64),
        ("order", ctypes.c_void_p),
        ("order_stride", ctypes.c_int64),
    ]


_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_U = ctypes.c_uint64
_SZ = ctypes.c_size_t

# name -> (restype, argtypes). Every int-returning function is a status code.
SIGNATURES: dict[str, tuple] = {
    "lkv_last_error": (ctypes.c_char_p, []),
    "lkv_abi_version": (_I, []),
    "lkv_host_alloc": (_I, [_SZ, _I, ctypes.POINTER(ctypes.c_void_p)]),
    "lkv_host_free": (_I, [_P]),
    "lkv_host_device_pointer": (_I, [_P, ctypes.POINTER(ctypes.c_void_p)]),
    "lkv_bound_topk_workspace_bytes": (_SZ, [_I, _I, _I]),
    "lkv_bound_topk": (_I, [_U, _P, _I, _P, _P, _I, _I64, _I, _I, _I, _I, _I, _I, _I, _I, _P, _I64, _P, _P, _SZ]),
    "lkv_sparse_decode_workspace_bytes": (_SZ, [ctypes.POINTER(DecodeDesc)]),
    "lkv_sparse_decode": (
        _I,
        [_U, ctypes.POINTER(DecodeDesc), _P, _I, ctypes.POINTER(KVSource), _P, _I64, ctypes.POINTER(KVSource),
         ctypes.POINTER(KVSource), ctypes.POINTER(KVSource), _P, _I, _P, _P, _SZ],
    ),
    "lkv_sparse_decode_static": (
        _I,
        [_U, ctypes.POINTER(DecodeDesc), _P, _I, ctypes.POINTER(KVSource), _P, _I64, ctypes.POINTER(KVSource),
         ctypes.POINTER(KVSource), ctypes.POINTER(KVSource), _P, _I, _P],
    ),
    "lkv_select_decode_workspace_bytes": (_SZ, [ctypes.POINTER(DecodeDesc), _I]),
    "lkv_select_decode": (
        _I,
        [_U, ctypes.POINTER(DecodeDesc), _P, _I, _P, _P, _I, _I64, _I, _I, _I, ctypes.POINTER(KVSource), ctypes.POINTER(KVSource),
         ctypes.POINTER(KVSource), _P, _I, _P, _P, _I64, _P, _SZ],
    ),
    "lkv_hybrid_decode_workspace_bytes": (_SZ, [ctypes.POINTER(DecodeDesc)]),
    "lkv_hybrid_decode": (
        _I,
        [_U, ctypes.POINTER(DecodeDesc), _P, _I, ctypes.POINTER(KVSource), ctypes.POINTER(KVSource), _P, _I64,
         ctypes.POINTER(ResidencyTables), ctypes.POINTER(KVSource), ctypes.POINTER(KVSource), ctypes.POINTER(KVSource), _P, _I, _P, _P, _SZ],
    ),
    "lkv_select_hybrid_decode_workspace_bytes": (_SZ, [ctypes.POINTER(DecodeDesc), _I]),
    "lkv_select_hybrid_decode": (
        _I,
        [_U, ctypes.POINTER(DecodeDesc), _P, _I, _P, _P, _I, _I64, _I, _I, _I, ctypes.POINTER(KVSource), ctypes.POINTER(KVSource),
         ctypes.POINTER(ResidencyTables), ctypes.POINTER(KVSource), ctypes.POINTER(KVSource), ctypes.POINTER(KVSource), _P, _I, _P, _P,
         _I64, _P, _SZ],
    ),
    "lkv_merge_lse": (_I, [_U, _P, _P, _P, _P, _I, _I64, _I, _P, _I, _P]),
    "lkv_store_blocks": (_I, [_U, ctypes.POINTER(KVSource), ctypes.POINTER(KVSource), _I, _I, _I, _I, _I, _P, _P, _I, _I64]),
    "lkv_pack_int8": (_I, [_U, _P, _I, _I64, _I, _I, _P]),
    "lkv_unpack_int8": (_I, [_U, _P, _I64, _I, _I, _I, _P]),
    "lkv_packed_pair_bytes": (_I64, [_I, _I]),
    "lkv_stream_read": (_I, [_U, _P, _SZ, _I, _P]),
}

_LIB: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded library, with every exported signature declared. Raises if it is not built."""
    global _LIB  # noqa: PLW0603 -- a loaded library handle
    if _LIB is None:
        if not SO_PATH.exists():
            raise RuntimeError(f"{SO_PATH.name} is not built; run __graft_entry__.build() (or make -C lazykv_amd)")
        handle = ctypes.CDLL(str(SO_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def check(rc: int, what: str) -> None:
    """Raise on a non-zero status: ValueError for bad arguments (as the reference does), else RuntimeError."""
    if rc == LKV_OK:
        return
    msg = lib().lkv_last_error().decode(errors="replace")
    if rc == LKV_ERR_INVALID:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what} failed ({rc}): {msg}")


def stream_of(t: torch.Tensor) -> int:
    """The current HIP stream of the tensor's device, as the integer the C ABI takes."""
    return torch.cuda.current_stream(t.device).cuda_stream


def require_cuda(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if not t.is_cuda:
            raise RuntimeError("lazykv_amd runs on the GPU: got a CPU tensor (there is no CPU path)")
