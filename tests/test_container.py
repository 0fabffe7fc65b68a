"""The `.qvr` container on the CPU: files written here are byte-identical to the reference's
(src/internal/file_format.cc:150-188) for indexes that hold no vectors, and the loader rejects
the corruptions the reference rejects (src/internal/file_format.cc:200-287) with its messages.

Vector-holding files need the device and are covered in test_io_gpu.py.
"""

import os
import struct

import numpy as np
import pytest

import quiver_amd as quiver
from oracle import qvr


def _write_flat(tmp_path, reference, metric="l2"):
    path = tmp_path / f"ref_{metric}.qvr"
    reference.flat(24, metric).save(path)
    return path


@pytest.mark.parametrize("metric", ["l2", "ip", "cosine"])
def test_empty_flat_file_matches_reference_bytes(tmp_path, reference, metric):
    ours, theirs = tmp_path / "ours.qvr", tmp_path / "theirs.qvr"
    quiver.FlatIndex(24, metric).save(ours)
    reference.flat(24, metric).save(theirs)
    assert ours.read_bytes() == theirs.read_bytes()
    back = quiver.FlatIndex.load(theirs)
    assert (back.dim, back.metric, len(back)) == (24, metric, 0)
    assert len(reference.flat_load(ours)) == 0


@pytest.mark.parametrize("store", [False, True])
def test_untrained_ivfpq_file_matches_reference_bytes(tmp_path, reference, store):
    ours, theirs = tmp_path / "ours.qvr", tmp_path / "theirs.qvr"
    quiver.IvfPqIndex(32, "cosine", nlist=8, m=4, store_vectors=store, train_iterations=7).save(ours)
    reference.ivfpq(32, "cosine", nlist=8, m=4, train_iterations=7, store_vectors=store).save(theirs)
    assert ours.read_bytes() == theirs.read_bytes()
    back = quiver.IvfPqIndex.load(theirs)
    assert (back.dim, back.nlist, back.m, back.metric, back.is_trained, len(back)) == (32, 8, 4, "cosine",
                                                                                       False, 0)
    assert len(reference.ivfpq_load(ours)) == 0


def test_container_layout_is_the_documented_one(tmp_path):
    """Header fields, section table and 64-byte alignment, read back with the Python reader."""
    path = tmp_path / "f.qvr"
    quiver.FlatIndex(5, "ip").save(path)
    raw = path.read_bytes()
    assert raw[:8] == b"QUIVERDB"
    version, kind, endian, nsec, size = struct.unpack_from("<IIIIQ", raw, 8)
    assert (version, kind, endian, nsec, size) == (1, 1, 0x01020304, 3, len(raw))
    assert len(raw) % 64 == 0
    sections = qvr.read_sections(path)
    assert [s for s in sections if not s.startswith("__")] == ["META", "VECT", "LABL"]
    dim, count, metric, reserved = struct.unpack("<QQII", sections["META"])
    assert (dim, count, metric, reserved) == (5, 0, 1, 0)


def _flip(path, offset):
    raw = bytearray(path.read_bytes())
    raw[offset] ^= 0x01
    path.write_bytes(bytes(raw))


def _section_offset(path, tag):
    raw = path.read_bytes()
    n = struct.unpack_from("<I", raw, 20)[0]
    for i in range(n):
        t, _crc, off, size = struct.unpack_from("<4sIQQ", raw, 64 + 24 * i)
        if t == tag:
            return off, size
    raise KeyError(tag)


def test_section_checksum_is_verified_unless_disabled(tmp_path, reference):
    path = _write_flat(tmp_path, reference)
    off, size = _section_offset(path, b"META")
    assert size == 24
    _flip(path, off + 20)  # the reserved word of the META payload
    with pytest.raises(ValueError, match="checksum mismatch in section 'META'"):
        quiver.FlatIndex.load(path)
    assert len(quiver.FlatIndex.load(path, verify_checksums=False)) == 0
    with pytest.raises(ValueError, match="checksum mismatch"):
        reference.flat_load(path)


def test_header_and_table_corruption_is_rejected(tmp_path, reference):
    path = _write_flat(tmp_path, reference)
    _flip(path, 12)  # kind
    with pytest.raises(ValueError, match="header checksum mismatch"):
        quiver.FlatIndex.load(path)
    path = _write_flat(tmp_path, reference)
    _flip(path, 64 + 4)  # CRC field of the first table entry
    with pytest.raises(ValueError, match="section table checksum mismatch"):
        quiver.FlatIndex.load(path, verify_checksums=False)


def test_truncation_kind_and_magic(tmp_path, reference):
    path = _write_flat(tmp_path, reference)
    raw = path.read_bytes()
    path.write_bytes(raw[:-64])
    with pytest.raises(ValueError, match="truncated or padded"):
        quiver.FlatIndex.load(path)
    path.write_bytes(raw)
    with pytest.raises(ValueError, match="different index type"):
        quiver.IvfPqIndex.load(path)
    path.write_bytes(b"NOTQUIVR" + raw[8:])
    with pytest.raises(ValueError, match="bad magic"):
        quiver.FlatIndex.load(path)
    path.write_bytes(raw[:40])
    with pytest.raises(ValueError, match="too small"):
        quiver.FlatIndex.load(path)
    with pytest.raises(ValueError, match="cannot open"):
        quiver.FlatIndex.load(tmp_path / "missing.qvr")


def test_bad_meta_values_are_rejected(tmp_path, reference):
    """A META section with an impossible dimension fails with the reference's message."""
    path = tmp_path / "bad.qvr"
    quiver.FlatIndex(8).save(path)
    off, _ = _section_offset(path, b"META")
    raw = bytearray(path.read_bytes())
    struct.pack_into("<Q", raw, off, 0)
    path.write_bytes(bytes(raw))
    with pytest.raises(ValueError, match="bad dimension"):
        quiver.FlatIndex.load(path, verify_checksums=False)


def test_save_replaces_atomically(tmp_path):
    path = tmp_path / "idx.qvr"
    quiver.FlatIndex(4).save(path)
    quiver.FlatIndex(6).save(path)
    assert quiver.FlatIndex.load(path).dim == 6
    assert sorted(os.listdir(tmp_path)) == ["idx.qvr"]  # no temporary left behind
