"""Segment framing of compressed payloads: ``<u64 little-endian len><bytes>``
per segment (incremental.py:1721-1722, parsed at incremental.py:1782-1796)."""

from __future__ import annotations

import pytest

from altxs_amd.coder import frame, iter_framed_segments


def test_frame_layout_and_round_trip():
    segs = [b"", b"\x01", bytes(range(256)) * 3, b"xyz"]
    blob = frame(segs)
    # hand-built layout: the length is 8 bytes, least significant first
    assert blob[:8] == b"\0" * 8
    assert blob[8:16] == b"\x01" + b"\0" * 7 and blob[16:17] == b"\x01"
    assert blob[17:25] == (768).to_bytes(8, "little")
    assert len(blob) == 8 * 4 + sum(map(len, segs))
    assert list(iter_framed_segments(blob)) == segs
    assert list(iter_framed_segments(b"")) == []


def test_truncated_payloads_raise():
    blob = frame([b"abcdef", b"gh"])
    with pytest.raises(ValueError, match="truncated segment header"):
        list(iter_framed_segments(blob[:3]))
    with pytest.raises(ValueError, match="need 6, have 2"):
        list(iter_framed_segments(blob[:10]))
    with pytest.raises(ValueError, match="truncated segment at offset"):
        list(iter_framed_segments(blob[:-1]))
