"""The gfx950 code objects in the built library (CPU): every kernel runs from registers, with no
private (scratch) memory and no spilled registers. The hot decode kernel once slid into spills
when a new code path raised its register use; this reads each kernel's resource metadata, as the
compiler recorded it in the AMDGPU metadata note, so such a change fails here instead of showing
up only as a slower kernel."""

from __future__ import annotations

import re
import struct
from pathlib import Path

import msgpack
import pytest

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "lazykv_amd" / "liblazykv_hip.so"
EM_AMDGPU = 224
PT_NOTE = 4
NT_AMDGPU_METADATA = 32


def _notes(elf: bytes):  # noqa: ANN202
    """(name, type, desc) of every note in the PT_NOTE segments of a little-endian ELF64 image."""
    phoff = struct.unpack_from("<Q", elf, 32)[0]
    phentsize, phnum = struct.unpack_from("<HH", elf, 54)
    for i in range(phnum):
        p_type, _, p_offset, _, _, p_filesz = struct.unpack_from("<IIQQQQ", elf, phoff + i * phentsize)
        if p_type != PT_NOTE:
            continue
        pos, end = p_offset, p_offset + p_filesz
        while pos + 12 <= end:
            namesz, descsz, ntype = struct.unpack_from("<III", elf, pos)
            name_at = pos + 12
            desc_at = name_at + ((namesz + 3) & ~3)
            yield elf[name_at : name_at + namesz].rstrip(b"\0"), ntype, elf[desc_at : desc_at + descsz]
            pos = desc_at + ((descsz + 3) & ~3)


def _kernels() -> list[dict]:
    """Kernel metadata of every gfx950 code object embedded in the library."""
    data = LIB.read_bytes()
    found = []
    at = data.find(b"\x7fELF", 1)  # offset 0 is the host library itself
    while at >= 0:
        if struct.unpack_from("<H", data, at + 18)[0] == EM_AMDGPU:
            for name, ntype, desc in _notes(data[at:]):
                if name == b"AMDGPU" and ntype == NT_AMDGPU_METADATA:
                    meta = msgpack.unpackb(desc, raw=False, strict_map_key=False)
                    assert meta["amdhsa.target"].endswith("gfx950"), meta["amdhsa.target"]
                    found.extend(meta["amdhsa.kernels"])
        at = data.find(b"\x7fELF", at + 1)
    return found


@pytest.fixture(scope="module")
def kernels() -> list[dict]:
    if not LIB.exists():
        pytest.fail(f"{LIB} is not built: run __graft_entry__.build() first")
    return _kernels()


def test_every_kernel_of_the_path_is_in_the_library(kernels) -> None:  # noqa: ANN001
    names = " ".join(k[".name"] for k in kernels)
    for want in ("bound_kernel", "select_kernel", "select_stream_kernel", "sparse_decode_kernel", "decode_merge_kernel", "decode_merge_wave_kernel",
                 "residency_kernel", "store_blocks_kernel", "merge_lse_kernel", "stream_read_kernel"):
        assert want in names, want


def test_no_kernel_uses_private_memory(kernels) -> None:  # noqa: ANN001
    bad = [(k[".name"], k[".private_segment_fixed_size"]) for k in kernels if k[".private_segment_fixed_size"] != 0]
    assert not bad, f"{len(bad)} kernels use private memory: {bad[:5]}"


def _decode_group(name: str) -> int | None:
    """G of a sparse_decode_kernel<D, MT, G, NT, I8> instance, from its mangled name."""
    m = re.search(r"sparse_decode_kernelILi\d+ELi\d+ELi(\d+)E", name)
    return int(m.group(1)) if m else None


def test_no_kernel_spills_registers(kernels) -> None:  # noqa: ANN001
    """No spills, except the decode kernels for 8 query heads per KV head at d 128: their 64
    accumulators and 64 query values exceed 256 VGPRs, and the compiler parks the overflow in
    accumulation registers (private memory stays at zero, checked above)."""
    bad = [(k[".name"], k[".vgpr_spill_count"]) for k in kernels
           if k.get(".vgpr_spill_count", 0) != 0 and not (_decode_group(k[".name"]) == 8 and k[".agpr_count"] > 0)]
    assert not bad, f"{len(bad)} kernels spill VGPRs: {bad[:5]}"


def test_model_dtype_decode_kernels_fit_eight_wave_workgroups(kernels) -> None:  # noqa: ANN001
    """The 512-thread decode kernels (no int8 code) keep at most 256 VGPRs, so two waves fit on
    each SIMD and one workgroup per CU stays resident."""
    hbm = [k for k in kernels if "sparse_decode_kernel" in k[".name"] and k[".max_flat_workgroup_size"] == 512]
    assert hbm
    assert all(k[".vgpr_count"] <= 256 and k[".agpr_count"] == 0 for k in hbm), [(k[".name"], k[".vgpr_count"]) for k in hbm]
