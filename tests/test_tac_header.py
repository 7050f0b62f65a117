"""The .tac header and per-document layouts with the PQ shape carried at run
time (src/index/storage.zig:52-71 Header, :764-797 parse, :705-749 layouts).

CPU tests: header round trips and rejections, and layouts written by the
oracle read back.  The GPU test writes layouts through the C ABI at m16 with
u16 codes (ksub 1024) and parses the whole image back.
"""
import zlib

import numpy as np
import pytest

from tac_gpu import errors, storage
from oracle import binding as orc


def _image(*, dim, kappa, m, ksub, doc_off, assignments, codes, write):
    """A .tac-shaped image: header, centroids, empty hnsw, codebooks, empty
    inverted lists, doc index + layouts, empty doc_tok / norms, CRC footer."""
    rng = np.random.default_rng(dim + m + ksub)
    sub = dim // m
    cents = rng.standard_normal((kappa, dim)).astype(np.float32).tobytes()
    cb = rng.standard_normal((m, ksub, sub)).astype(np.float32).tobytes()
    idx, pay = write(doc_off, assignments, codes, m)
    doc = idx.astype("<u8").tobytes() + pay.tobytes()
    offs, cur = {}, storage.HEADER_REGION_SIZE
    for name, blob in (("centroids_off", cents), ("hnsw_off", b""), ("pq_off", cb),
                       ("ilist_off", b""), ("doc_off", doc), ("doc_tok_off", b""),
                       ("norms_off", b"")):
        offs[name] = cur
        cur += (len(blob) + 7) // 8 * 8
    offs["footer_off"] = cur
    body = bytearray(cur + 8)
    hdr = storage.pack_header(dim=dim, kappa=kappa, m=m, ksub=ksub, n_docs=doc_off.size - 1,
                              n_tokens=int(doc_off[-1]), offsets=offs)
    body[:len(hdr)] = hdr
    for name, blob in (("centroids_off", cents), ("pq_off", cb), ("doc_off", doc)):
        body[offs[name]:offs[name] + len(blob)] = blob
    body[cur:cur + 4] = np.uint32(zlib.crc32(bytes(body[:cur]))).astype("<u4").tobytes()
    return bytes(body), offs, idx, pay


def _oracle_write(off, a, codes, m):
    st, idx, pay = orc.write_doc_layouts(off, a, codes, m, codes.dtype.itemsize)
    assert st == 0
    return idx, pay


def _docs(seed, n_docs, m, code_dtype, ksub):
    rng = np.random.default_rng(seed)
    lens = rng.integers(0, 30, n_docs)
    lens[::7] = 0
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint64)
    n = int(off[-1])
    a = rng.integers(0, 1000, n).astype(np.uint32)
    codes = rng.integers(0, ksub, (n, m)).astype(code_dtype)
    return off, a, codes


@pytest.mark.parametrize("dim,m,ksub", [(64, 16, 256), (64, 32, 256), (64, 8, 256),
                                        (64, 16, 1024), (128, 32, 65536), (64, 64, 2)])
def test_header_round_trip_and_layouts(dim, m, ksub):
    code_dtype = np.uint8 if ksub <= 256 else np.uint16
    off, a, codes = _docs(dim + m + ksub, 200, m, code_dtype, ksub)
    img, offs, idx, pay = _image(dim=dim, kappa=1000, m=m, ksub=ksub, doc_off=off,
                                 assignments=a, codes=codes, write=_oracle_write)
    h = storage.parse_header(img)
    assert (h["pq_M"], h["ksub"], h["sub_dim"], h["dim"]) == (m, ksub, dim // m, dim)
    assert h["code_bytes"] == (1 if ksub <= 256 else 2)
    assert h["pq_bits"] == int(np.log2(ksub))
    assert h["n_docs"] == off.size - 1 and h["n_tokens"] == int(off[-1])
    # the codebook section holds m x ksub x sub_dim floats
    assert h["ilist_off"] - h["pq_off"] == storage.pq_section_bytes(m, h["pq_bits"], dim // m)
    docs = storage.read_doc_layouts(idx, pay, m, h["code_bytes"])
    for d, (ids, cd) in enumerate(docs):
        lo, hi = int(off[d]), int(off[d + 1])
        assert np.array_equal(ids, a[lo:hi]) and np.array_equal(cd, codes[lo:hi])


def test_header_rejections():
    off, a, codes = _docs(3, 20, 16, np.uint16, 1024)
    img, offs, idx, pay = _image(dim=64, kappa=10, m=16, ksub=1024, doc_off=off, assignments=a,
                                 codes=codes, write=_oracle_write)
    storage.parse_header(img)

    def patched(pos, raw):
        b = bytearray(img)
        b[pos:pos + len(raw)] = raw
        return bytes(b)

    with pytest.raises(errors.InvalidIndex):        # magic
        storage.parse_header(patched(0, b"TAC_IDX0"))
    with pytest.raises(errors.UnsupportedVersion):  # version
        storage.parse_header(patched(8, np.uint32(1).tobytes()))
    with pytest.raises(errors.InvalidIndex):        # sub_dim * pq_M != dim
        storage.parse_header(patched(20, np.uint32(8).tobytes()))
    with pytest.raises(errors.InvalidIndex):        # pq_bits out of range
        storage.parse_header(patched(24, bytes([17])))
    def recrc(image):
        b = bytearray(image)
        f = offs["footer_off"]
        b[f:f + 4] = np.uint32(zlib.crc32(bytes(b[:f]))).astype("<u4").tobytes()
        return bytes(b)

    # The section sizes are checked after the footer CRC, as parse does
    # (storage.zig:793-797, then :799-802 and parsePq :942): a short codebook
    # section under a stale CRC is IndexCorrupt, under a valid one InvalidIndex.
    with pytest.raises(errors.IndexCorrupt):
        storage.parse_header(patched(24, bytes([11])))
    with pytest.raises(errors.InvalidIndex, match="codebook section"):
        storage.parse_header(recrc(patched(24, bytes([11]))))
    with pytest.raises(errors.InvalidIndex, match="centroid section"):  # kappa 10 -> 11
        storage.parse_header(recrc(patched(16, np.uint32(11).tobytes())))
    with pytest.raises(errors.IndexCorrupt):        # one payload byte flipped
        pos = offs["doc_off"] + 8 * (off.size) + 5
        storage.parse_header(patched(pos, bytes([img[pos] ^ 1])))
    with pytest.raises(errors.InvalidIndex):        # non-monotonic offsets
        storage.parse_header(patched(48 + 8, np.uint64(offs["pq_off"] + 8).tobytes()))
    with pytest.raises(errors.InvalidArgument):
        storage.pq_bits_of(1000)
    with pytest.raises(errors.InvalidIndex):        # layout padding not zero
        bad = pay.copy()
        n0 = int(np.frombuffer(bad[:4].tobytes(), "<u4")[0])
        end = 4 + 4 * n0 + n0 * 16 * 2
        if end % 8 == 0:
            pytest.skip("first layout has no padding")
        bad[end] = 1
        storage.read_doc_layouts(idx, bad, 16, 2)


@pytest.mark.gpu
@pytest.mark.parametrize("m,ksub", [(16, 1024), (16, 256), (32, 65536)])
def test_image_through_the_c_abi(gpu, m, ksub):
    """Layouts written by tac_write_doc_layouts at a runtime shape (m16 with
    u16 codes among them) parse back to the inputs, and the image's CRC-32
    from tac_crc32 is the footer parse checks."""
    dim = 64 if m <= 16 else 128
    code_dtype = np.uint8 if ksub <= 256 else np.uint16
    off, a, codes = _docs(m + ksub, 3000, m, code_dtype, ksub)
    img, offs, idx, pay = _image(dim=dim, kappa=1000, m=m, ksub=ksub, doc_off=off,
                                 assignments=a, codes=codes, write=storage.write_doc_layouts)
    ridx, rpay = _oracle_write(off, a, codes, m)
    assert np.array_equal(idx, ridx) and np.array_equal(pay, rpay)
    h = storage.parse_header(img)
    assert storage.crc32(np.frombuffer(img[:h["footer_off"]], np.uint8)) == \
        int(np.frombuffer(img[h["footer_off"]:h["footer_off"] + 4], "<u4")[0])
    docs = storage.read_doc_layouts(idx, pay, h["pq_M"], h["code_bytes"])
    for d, (ids, cd) in enumerate(docs):
        lo, hi = int(off[d]), int(off[d + 1])
        assert np.array_equal(ids, a[lo:hi]) and np.array_equal(cd, codes[lo:hi])
