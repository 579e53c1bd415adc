"""Write the int8 warm/cold-tier golden vectors from the reference's own `pack` / `unpack`.

Run once, in the build container (the reference tree is not present on GPU machines):

    python tests/golden/make_quant_vectors.py

The reference's quantiser is `lazykv/quant.py` (pack :73-87, unpack :90-105, _affine :59-70). It
imports only torch, so it is loaded here by file path and run on the CPU. Its outputs are the
only thing that can pin the exact bytes torch produces (rounding of the float32 divide, the
half-to-even `round_`, the float16 casts of scale and zero). The inputs cover what those
bytes depend on:

* seeded N(0,1) data with per-channel scales in U[0.5, 2], as the decode workloads use;
* constant groups (zero range, where the scale clamps to float32 `tiny`);
* a key channel and a value token carrying a x500 outlier;
* groups whose quotient lands exactly on k + 0.5 (min 0, max 255, so the scale is 1.0),
  which pins the half-to-even rule;
* negative-only groups and mixed signs.

The fixture holds inputs and expected outputs only: for every case, the input pair bits, the
packed records and the unpacked pair bits in the input's dtype.
"""

from __future__ import annotations

import importlib.util
from pathlib import Path

import numpy as np
import torch

REF_QUANT = Path("/root/reference/lazykv/quant.py")
OUT = Path(__file__).resolve().parent / "quant_vectors.npz"


def _load_reference():
    spec = importlib.util.spec_from_file_location("reference_quant", REF_QUANT)
    mod = importlib.util.module_from_spec(spec)
    assert spec.loader is not None
    spec.loader.exec_module(mod)
    return mod


def _case(gen: torch.Generator, m: int, bs: int, d: int, dtype: torch.dtype) -> torch.Tensor:
    """[m, 2, bs, d] pairs: pair 0 random, pair 1 with edge groups, the rest random."""
    s_k = torch.rand((1, 1, d), generator=gen) * 1.5 + 0.5
    s_v = torch.rand((1, 1, d), generator=gen) * 1.5 + 0.5
    k = torch.randn((m, bs, d), generator=gen) * s_k
    v = torch.randn((m, bs, d), generator=gen) * s_v
    if m > 1:
        # Pair 1: edge groups.
        k[1, :, 0] = 3.5  # constant key channel
        v[1, 0, :] = -1.25  # constant value token
        k[1, :, 1] *= 500.0  # outlier key channel
        v[1, 1, :] *= 500.0  # outlier value token
        # A key channel and a value token spanning [0, 255] exactly, so scale == 1.0 and the
        # quotients are the values themselves: x.5 entries hit the half-to-even rule.
        halves = torch.arange(bs, dtype=torch.float32) + 0.5
        k[1, :, 2] = halves
        k[1, 0, 2], k[1, 1, 2] = 0.0, 255.0
        hv = (torch.arange(d, dtype=torch.float32) % 120) + 0.5
        v[1, 2, :] = hv
        v[1, 2, 0], v[1, 2, 1] = 0.0, 255.0
        k[1, :, 3] = -k[1, :, 3].abs() - 1.0  # negative-only key channel
    if m > 2:
        # Pair 2: entirely constant.
        k[2] = 0.75
        v[2] = -2.0
    return torch.stack([k, v], dim=1).to(dtype)


def main() -> None:
    ref = _load_reference()
    gen = torch.Generator().manual_seed(20261201)
    arrays: dict[str, np.ndarray] = {}
    geoms = [(16, 64), (16, 128), (8, 16), (64, 64)]
    for dtype, tag in ((torch.float16, "f16"), (torch.bfloat16, "bf16")):
        for bs, d in geoms:
            x = _case(gen, 3, bs, d, dtype)
            packed = ref.pack(x)
            back = ref.unpack(packed, bs, d, dtype)
            key = f"{tag}_bs{bs}_d{d}"
            arrays[f"{key}_in"] = x.view(torch.int16).numpy().view(np.uint16)
            arrays[f"{key}_packed"] = packed.numpy()
            arrays[f"{key}_unpacked"] = back.view(torch.int16).numpy().view(np.uint16)
            assert packed.shape == (3, ref.packed_pair_bytes(bs, d))
    arrays["packed_pair_bytes"] = np.array([[bs, d, ref.packed_pair_bytes(bs, d)] for bs, d in geoms], dtype=np.int64)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(arrays)} arrays)")


if __name__ == "__main__":
    main()
