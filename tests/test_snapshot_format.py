"""The snapshot file format on the CPU (lazykv/snapshot.py:16-20,116-123): the header framing,
alignment and the refusal of foreign files."""

from __future__ import annotations

import json

import pytest

from lazykv_amd import snapshot


def test_foreign_files_are_refused(tmp_path) -> None:  # noqa: ANN001
    p = tmp_path / "x.bin"
    p.write_bytes(b"\x07" * 64)
    with pytest.raises(ValueError, match="not a LazyKV snapshot"):
        snapshot.read_header(p)
    head = json.dumps({"magic": "something-else"}).encode()
    p.write_bytes(len(head).to_bytes(8, "little") + head)
    with pytest.raises(ValueError, match="not a LazyKV snapshot"):
        snapshot.read_header(p)


def test_header_framing_and_alignment(tmp_path) -> None:  # noqa: ANN001
    """8-byte little-endian length, JSON, zero padding to 4096; sections start on that boundary."""
    head = json.dumps({"magic": snapshot.MAGIC, "length": 3, "sections": {"logits": [0, 8]}}).encode()
    p = tmp_path / "s.lkv"
    p.write_bytes(len(head).to_bytes(8, "little") + head + b"\0" * (4096 - 8 - len(head)) + b"\0" * 4096)
    header, base = snapshot.read_header(p)
    assert header["length"] == 3 and base == 4096
    assert snapshot.ALIGN == 4096 and snapshot.MAGIC == "lazykv-snapshot-1"
    assert [snapshot._pad(n) for n in (0, 1, 4096, 4097)] == [0, 4096, 4096, 8192]
