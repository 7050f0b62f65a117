"""Python mirror of the storage.build stages around the PQ build.

``residuals_and_norms`` is stage 2 of storage.build
(src/index/storage.zig:355-376), the per-token ``residualsAndNormsChunk``
(:255-278) run over every token at once on the GPU.  ``doc_payload_size``,
``write_doc_layouts`` and ``crc32`` produce the .tac sections that carry the
PQ codes (:674-686, :705-749) and the image's footer checksum (:612-617).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import errors
from ._native import c_u32, c_u64, lib


def _ptr(a: np.ndarray) -> ctypes.c_void_p:
    return ctypes.c_void_p(a.ctypes.data)


def residuals_and_norms(vectors: np.ndarray, dim: int, centroids: np.ndarray,
                        assignments: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(residuals [n][dim], norms [n]) for token vectors and their centroid ids.

    residual = (vector - centroid) * fl(1 / norm) when norm > 0, where norm is
    the square root of the in-order fp32 fold of squared differences.  An
    assignment outside the centroid table raises InvalidArgument.
    """
    v = np.ascontiguousarray(vectors, dtype=np.float32).reshape(-1)
    c = np.ascontiguousarray(centroids, dtype=np.float32).reshape(-1)
    a = np.ascontiguousarray(assignments, dtype=np.uint32).reshape(-1)
    if dim == 0 or v.size % dim != 0 or c.size % dim != 0 or v.size // dim != a.size:
        raise errors.DimMismatch("DimMismatch")
    n = a.size
    out = np.empty((n, dim), dtype=np.float32)
    norms = np.empty(n, dtype=np.float32)
    if n == 0:
        return out, norms
    errors.check(lib.tac_residuals(_ptr(v), n, dim, _ptr(c), c.size // dim, _ptr(a), _ptr(out),
                                   _ptr(norms)))
    return out, norms


def doc_payload_size(doc_offsets: np.ndarray, m: int, code_bytes: int = 1) -> int:
    """docPayloadSize (storage.zig:674-686): bytes of all per-doc layouts."""
    o = np.ascontiguousarray(doc_offsets, dtype=np.uint64)
    out = c_u64(0)
    errors.check(lib.tac_doc_payload_bytes(_ptr(o), max(o.size - 1, 0), m, code_bytes,
                                           ctypes.byref(out)))
    return int(out.value)


def write_doc_layouts(doc_offsets: np.ndarray, assignments: np.ndarray, codes: np.ndarray,
                      m: int) -> tuple[np.ndarray, np.ndarray]:
    """writeDocLayouts (storage.zig:705-749): (doc_index [n_docs+1] u64, payload bytes).

    ``codes`` is token-major [n_tokens][m], uint8 or uint16 (little-endian
    in the payload).
    """
    o = np.ascontiguousarray(doc_offsets, dtype=np.uint64)
    a = np.ascontiguousarray(assignments, dtype=np.uint32).reshape(-1)
    c = np.ascontiguousarray(codes)
    if c.dtype not in (np.uint8, np.uint16):
        raise errors.InvalidArgument("codes must be uint8 or uint16")
    cb = c.dtype.itemsize
    if c.size != a.size * m:
        raise errors.DimMismatch("DimMismatch")
    n_docs = o.size - 1
    total = doc_payload_size(o, m, cb)
    idx = np.empty(n_docs + 1, np.uint64)
    pay = np.empty(max(total, 8), np.uint8)
    errors.check(lib.tac_write_doc_layouts(_ptr(o), n_docs, a.size, _ptr(a), _ptr(c), m, cb,
                                           _ptr(idx), _ptr(pay), total))
    return idx, pay[:total]


def crc32(data) -> int:
    """std.hash.Crc32 of a byte buffer (the .tac footer checksum)."""
    b = np.frombuffer(data, dtype=np.uint8) if isinstance(data, (bytes, bytearray, memoryview)) \
        else np.ascontiguousarray(data).reshape(-1).view(np.uint8)
    out = c_u32(0)
    errors.check(lib.tac_crc32(_ptr(b) if b.size else None, b.size, ctypes.byref(out)))
    return int(out.value)
