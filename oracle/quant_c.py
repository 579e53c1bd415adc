"""ctypes wrapper of `oracle/quant_ref.c` (test infrastructure only; see `oracle/__init__.py`)."""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_SO = _HERE / "_build" / "liboracle_quant.so"
_LIB = None
_DT = {"f16": 0, "bf16": 1}


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _SO


def _lib() -> ctypes.CDLL:
    global _LIB  # noqa: PLW0603 -- a loaded library handle
    if _LIB is None:
        if not _SO.exists():
            build()
        lib = ctypes.CDLL(str(_SO))
        lib.oq_pack.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
        lib.oq_unpack.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
        lib.oq_packed_pair_bytes.restype = ctypes.c_int64
        lib.oq_packed_pair_bytes.argtypes = [ctypes.c_int, ctypes.c_int]
        _LIB = lib
    return _LIB


def pack(pairs: np.ndarray, dtype: str) -> np.ndarray:
    """`[m, 2, bs, d]` uint16 bits -> `[m, P]` uint8 records."""
    pairs = np.ascontiguousarray(pairs, dtype=np.uint16)
    m, _, bs, d = pairs.shape
    out = np.empty((m, _lib().oq_packed_pair_bytes(bs, d)), dtype=np.uint8)
    _lib().oq_pack(pairs.ctypes.data, _DT[dtype], m, bs, d, out.ctypes.data)
    return out


def unpack(rec: np.ndarray, bs: int, d: int, dtype: str) -> np.ndarray:
    """`[m, P]` uint8 records -> `[m, 2, bs, d]` uint16 bits."""
    rec = np.ascontiguousarray(rec, dtype=np.uint8)
    out = np.empty((rec.shape[0], 2, bs, d), dtype=np.uint16)
    _lib().oq_unpack(rec.ctypes.data, rec.shape[0], bs, d, _DT[dtype], out.ctypes.data)
    return out
