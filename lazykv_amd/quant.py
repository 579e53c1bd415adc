"""int8 warm/cold-tier records on the GPU, bit-exact with lazykv/quant.py.

Same record format, names and errors as the reference (:42-105): per (block, head) pair, keys
quantised per channel and values per token, asymmetric min/max over 256 levels, float16 scale and
zero, one contiguous uint8 record `kq | vq | k scale | k zero | v scale | v zero`. The arithmetic
is the reference's float32 sequence (correctly rounded divide, half-to-even rounding, separately
rounded multiply and add on the way back), run by the `lkv_pack_int8` / `lkv_unpack_int8` kernels.
"""

from __future__ import annotations

import torch

from lazykv_amd import kernels

SCALE_DTYPE = torch.float16
_LEVELS = 255


def packed_pair_bytes(block_size: int, head_dim: int) -> int:
    """Bytes of one packed (block, head) pair: both int8 payloads plus the four scale arrays (:46-49)."""
    scale = SCALE_DTYPE.itemsize
    return 2 * block_size * head_dim + 2 * scale * head_dim + 2 * scale * block_size


def _offsets(block_size: int, head_dim: int) -> tuple[int, ...]:
    """Cut points of the record: k payload, v payload, k scale, k zero, v scale, v zero (:52-56)."""
    s = SCALE_DTYPE.itemsize
    n = block_size * head_dim
    return (n, 2 * n, 2 * n + s * head_dim, 2 * n + 2 * s * head_dim, 2 * n + 2 * s * head_dim + s * block_size)


def pack(blocks: torch.Tensor) -> torch.Tensor:
    """Pack KV pairs `[..., 2, block_size, head_dim]` into uint8 records `[..., packed_pair_bytes]` (:73-87)."""
    *lead, two, bs, d = blocks.shape
    if two != 2:
        raise ValueError(f"expected a [..., 2, block_size, head_dim] KV pair, got {tuple(blocks.shape)}")
    packed = kernels.pack_int8(blocks.reshape(-1, 2, bs, d))
    return packed.view(*lead, packed.shape[-1])


def unpack(packed: torch.Tensor, block_size: int, head_dim: int, dtype: torch.dtype) -> torch.Tensor:
    """Dequantise uint8 records `[m, packed_pair_bytes]` back to `[m, 2, block_size, head_dim]` (:90-105)."""
    if packed.ndim != 2 or packed.shape[1] != packed_pair_bytes(block_size, head_dim):
        raise ValueError(f"expected [m, {packed_pair_bytes(block_size, head_dim)}] uint8 records, got {tuple(packed.shape)}")
    return kernels.unpack_int8(packed, block_size, head_dim, dtype)
