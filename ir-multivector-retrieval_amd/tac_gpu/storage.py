"""Python mirror of the storage.build stages around the PQ build.

``residuals_and_norms`` is stage 2 of storage.build
(src/index/storage.zig:355-376), the per-token ``residualsAndNormsChunk``
(:255-278) run over every token at once on the GPU.  ``doc_payload_size``,
``write_doc_layouts`` and ``crc32`` produce the .tac sections that carry the
PQ codes (:674-686, :705-749) and the image's footer checksum (:612-617).
"""
from __future__ import annotations

import ctypes
import zlib

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


# ---- .tac header with the PQ shape carried at run time ----------------------
# The reference's Header (src/index/storage.zig:52-71) stores pq_M, pq_bits and
# sub_dim, but parse rejects any pq_M other than constants.PQ_M and any
# pq_bits other than 8 (:776-778), and parsePq sizes the codebook section from
# the constants (:935-952).  The rules below carry the trained shape instead:
# pq_M = m, pq_bits = log2(ksub), codes of 1 byte when pq_bits <= 8, else 2
# (little-endian), and a codebook section of m * 2^pq_bits * sub_dim f32.

INDEX_MAGIC = b"TAC_IDX1"          # src/constants.zig:43
INDEX_VERSION = 2                  # src/constants.zig:45
HEADER_REGION_SIZE = 128           # src/index/storage.zig:76
_HEADER_DTYPE = np.dtype([
    ("magic", "S8"), ("version", "<u4"), ("dim", "<u4"), ("kappa", "<u4"), ("pq_M", "<u4"),
    ("pq_bits", "u1"), ("_pad0", "V3"), ("sub_dim", "<u4"), ("n_docs", "<u8"),
    ("n_tokens", "<u8"), ("centroids_off", "<u8"), ("hnsw_off", "<u8"), ("pq_off", "<u8"),
    ("ilist_off", "<u8"), ("doc_off", "<u8"), ("doc_tok_off", "<u8"), ("norms_off", "<u8"),
    ("footer_off", "<u8")])
SECTION_FIELDS = ("centroids_off", "hnsw_off", "pq_off", "ilist_off", "doc_off", "doc_tok_off",
                  "norms_off", "footer_off")


def pq_bits_of(ksub: int) -> int:
    """pq_bits for a codebook of ksub codewords: ksub must be a power of two
    between 2 and 65536 (the code fits 1 or 2 bytes)."""
    if ksub < 2 or ksub > 65536 or ksub & (ksub - 1):
        raise errors.InvalidArgument("ksub must be a power of two in [2, 65536]")
    return ksub.bit_length() - 1


def code_bytes_of(pq_bits: int) -> int:
    return 1 if pq_bits <= 8 else 2


def pq_section_bytes(m: int, pq_bits: int, sub_dim: int) -> int:
    """Bytes of the codebook section: [m][2^pq_bits][sub_dim] f32 (parsePq, :935-952)."""
    return m * (1 << pq_bits) * sub_dim * 4


def pack_header(*, dim: int, kappa: int, m: int, ksub: int, n_docs: int, n_tokens: int,
                offsets: dict) -> bytes:
    """The 128-byte header region (serialise, :630-650) for a PQ of m x ksub."""
    if dim == 0 or m == 0 or dim % m:
        raise errors.DimNotDivisibleByM("DimNotDivisibleByM")
    h = np.zeros(1, _HEADER_DTYPE)
    h["magic"], h["version"], h["dim"], h["kappa"] = INDEX_MAGIC, INDEX_VERSION, dim, kappa
    h["pq_M"], h["pq_bits"], h["sub_dim"] = m, pq_bits_of(ksub), dim // m
    h["n_docs"], h["n_tokens"] = n_docs, n_tokens
    for f in SECTION_FIELDS:
        h[f] = offsets[f]
    out = bytearray(HEADER_REGION_SIZE)
    out[:_HEADER_DTYPE.itemsize] = h.tobytes()
    return bytes(out)


def parse_header(image) -> dict:
    """parse's header checks (:764-797) with the PQ shape read from the header:
    magic, version, 1 <= pq_bits <= 16, sub_dim * pq_M == dim, dim and kappa
    non-zero, section offsets monotonic from 128 and inside the image, the
    footer CRC-32, then the centroid and codebook sections large enough.  Raises
    InvalidIndex / UnsupportedVersion / IndexCorrupt as the reference does."""
    b = np.frombuffer(bytes(image), np.uint8)
    if b.size < HEADER_REGION_SIZE + 8:
        raise errors.InvalidIndex("image shorter than the header region")
    h = np.frombuffer(b[:_HEADER_DTYPE.itemsize].tobytes(), _HEADER_DTYPE)[0]
    if bytes(h["magic"]) != INDEX_MAGIC:
        raise errors.InvalidIndex("magic")
    if int(h["version"]) != INDEX_VERSION:
        raise errors.UnsupportedVersion("version")
    m, bits, sub, dim = int(h["pq_M"]), int(h["pq_bits"]), int(h["sub_dim"]), int(h["dim"])
    if m == 0 or not 1 <= bits <= 16:
        raise errors.InvalidIndex("pq_M / pq_bits")
    if sub * m != dim or dim == 0 or int(h["kappa"]) == 0:
        raise errors.InvalidIndex("dim / sub_dim / kappa")
    offs = [int(h[f]) for f in SECTION_FIELDS]
    if offs[0] != HEADER_REGION_SIZE:
        raise errors.InvalidIndex("centroids_off")
    for a, c in zip(offs, offs[1:]):
        if c < a or c > b.size:
            raise errors.InvalidIndex("section offsets")
    footer = offs[-1]
    if footer + 8 > b.size:
        raise errors.InvalidIndex("footer")
    stored = int(np.frombuffer(b[footer:footer + 4].tobytes(), "<u4")[0])
    if zlib.crc32(b[:footer].tobytes()) != stored:  # host CRC-32, std.hash.Crc32's
        raise errors.IndexCorrupt("footer CRC-32")
    # Section sizes after the CRC, in parse's order: centroids (:799-802),
    # then (past the HNSW section, not read here) parsePq's codebooks (:942).
    if int(h["hnsw_off"]) - int(h["centroids_off"]) < int(h["kappa"]) * dim * 4:
        raise errors.InvalidIndex("centroid section")
    if int(h["ilist_off"]) - int(h["pq_off"]) < pq_section_bytes(m, bits, sub):
        raise errors.InvalidIndex("codebook section")
    out = {f: int(h[f]) for f in _HEADER_DTYPE.names if f not in ("magic", "_pad0")}
    out["code_bytes"] = code_bytes_of(bits)
    out["ksub"] = 1 << bits
    return out


def read_doc_layouts(doc_index: np.ndarray, payload: np.ndarray, m: int, code_bytes: int):
    """The per-document layouts (:705-749) read back: a list of
    (centroid ids u32 [n_d], codes [n_d][m] u8 or u16) per document.  Raises
    InvalidIndex when a layout runs past its slot or its padding is not zero."""
    idx = np.ascontiguousarray(doc_index, dtype=np.uint64)
    pay = np.ascontiguousarray(payload, dtype=np.uint8)
    ct = np.uint8 if code_bytes == 1 else np.dtype("<u2")
    docs = []
    for d in range(idx.size - 1):
        lo, hi = int(idx[d]), int(idx[d + 1])
        if hi < lo or hi > pay.size or hi - lo < 4:
            raise errors.InvalidIndex("doc_index")
        n_d = int(np.frombuffer(pay[lo:lo + 4].tobytes(), "<u4")[0])
        need = 4 + 4 * n_d + n_d * m * code_bytes
        if (need + 7) // 8 * 8 != hi - lo:
            raise errors.InvalidIndex("layout size")
        ids = np.frombuffer(pay[lo + 4:lo + 4 + 4 * n_d].tobytes(), "<u4")
        codes = np.frombuffer(pay[lo + 4 + 4 * n_d:lo + need].tobytes(), ct).reshape(n_d, m)
        if pay[lo + need:hi].any():
            raise errors.InvalidIndex("padding")
        docs.append((ids.astype(np.uint32), codes))
    return docs
