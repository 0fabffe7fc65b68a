"""ORACLE — test infrastructure, NOT product code.

Read-only parser for the reference's ``.qvr`` container (src/internal/file_format.h:1-9,39-58):
a 64-byte header, a table of 24-byte section entries (tag, crc32c, offset, size), and raw
little-endian sections. Used to take the trained state (CENT / PQCB) and the CSR inverted lists
(LOFF / CODE / LABL / VECT, src/ivfpq_index.cc:465-503) out of an index the compiled reference
saved, so the oracle and the device path can be run on exactly the reference's trained state.
Checksums are not verified here (the file was just written by the reference in the same process
tree).
"""

from __future__ import annotations

import struct
from typing import Dict

import numpy as np


def _fourcc(s: str) -> int:
    b = s.encode()
    return b[0] | b[1] << 8 | b[2] << 16 | b[3] << 24


def read_sections(path: str) -> Dict[str, bytes]:
    with open(path, "rb") as f:
        raw = f.read()
    magic, version, kind, endian, nsec = struct.unpack_from("<8sIIII", raw, 0)
    out = {}
    for i in range(nsec):
        tag, _crc, off, size = struct.unpack_from("<IIQQ", raw, 64 + 24 * i)
        name = bytes([tag & 255, tag >> 8 & 255, tag >> 16 & 255, tag >> 24 & 255]).decode()
        out[name] = raw[off:off + size]
    out["__kind__"] = kind
    return out


def read_ivfpq(path: str) -> dict:
    """Dict with params and numpy arrays: centroids [nlist, dim], codebook [m, 256, dsub],
    offsets [nlist+1], codes [count, m], labels [count], vectors [count, dim] or None."""
    s = read_sections(path)
    dim, nlist, m, count, iters, seed, metric, store, trained, _ = struct.unpack_from(
        "<QQQQQQIIII", s["META"], 0)
    out = dict(dim=dim, nlist=nlist, m=m, count=count, train_iterations=iters, seed=seed,
               metric=["l2", "ip", "cosine"][metric], store_vectors=bool(store),
               trained=bool(trained))
    if trained:
        out["centroids"] = np.frombuffer(s["CENT"], dtype=np.float32).reshape(nlist, dim).copy()
        out["codebook"] = np.frombuffer(s["PQCB"], dtype=np.float32).reshape(m, 256, dim // m).copy()
    out["offsets"] = np.frombuffer(s["LOFF"], dtype=np.uint64).copy()
    out["codes"] = np.frombuffer(s["CODE"], dtype=np.uint8).reshape(count, m).copy()
    out["labels"] = np.frombuffer(s["LABL"], dtype=np.uint64).copy()
    out["vectors"] = (np.frombuffer(s["VECT"], dtype=np.float32).reshape(count, dim).copy()
                      if store else None)
    return out
