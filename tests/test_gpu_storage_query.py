"""GPU .tac layouts, CRC-32, distance table and refine against the oracle and
zlib, bit for bit, through the C ABI."""
import ctypes
import zlib

import numpy as np
import pytest

from oracle import binding as orc
from tac_gpu import device, errors, lib, pq, retrieval, storage
from test_storage_query_oracle import synthetic_index

pytestmark = pytest.mark.gpu


def _crc_device(data: bytes, misalign: int) -> int:
    buf = device.DeviceArray((len(data) + 32,), np.uint8)
    p = ctypes.c_void_p(buf.ptr.value + misalign)
    if data:
        errors.check(lib.tac_gpu_memcpy_htod(p, ctypes.c_char_p(data), len(data)))
    out = ctypes.c_uint32(0)
    errors.check(lib.tac_crc32_device(p, len(data), ctypes.byref(out), None))
    return out.value


@pytest.mark.parametrize("n", [0, 1, 15, 16, 17, 1023, 1024, 1025, 262_144 + 5, 3_000_017])
def test_crc_matches_zlib(gpu, n):
    data = np.random.default_rng(n).integers(0, 256, n, dtype=np.uint8).tobytes()
    want = zlib.crc32(data)
    assert storage.crc32(data) == want
    for mis in (0, 1, 7, 15):
        assert _crc_device(data, mis) == want


def test_crc_after_workspace_release(gpu):
    data = np.random.default_rng(4).integers(0, 256, 100_003, dtype=np.uint8).tobytes()
    assert storage.crc32(data) == zlib.crc32(data)
    errors.check(lib.tac_gpu_release_workspace())
    assert storage.crc32(data) == zlib.crc32(data)


def test_crc_large_image(gpu):
    data = np.random.default_rng(1).integers(0, 256, 300 * 2**20 + 333, dtype=np.uint8)
    assert storage.crc32(data) == zlib.crc32(data.tobytes())


@pytest.mark.parametrize("m,cb", [(32, 1), (16, 1), (3, 1), (16, 2), (5, 2)])
def test_doc_layouts_match_oracle(gpu, m, cb):
    rng = np.random.default_rng(m + 7 * cb)
    lens = rng.integers(0, 40, 3000)
    lens[::17] = 0
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint64)
    n = int(off[-1])
    a = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    codes = rng.integers(0, 256 if cb == 1 else 65536, (n, m)).astype(
        np.uint8 if cb == 1 else np.uint16)
    idx, pay = storage.write_doc_layouts(off, a, codes, m)
    st, ridx, rpay = orc.write_doc_layouts(off, a, codes, m, cb)
    assert st == 0
    assert np.array_equal(idx, ridx) and np.array_equal(pay, rpay)


def test_doc_layouts_full_corpus_scale(gpu):
    """1,521,797 tokens in documents of 1-100 tokens, m16 u8 codes."""
    rng = np.random.default_rng(5)
    lens = rng.integers(1, 101, 40_000)
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint64)
    off = off[off <= 1_521_797]
    off = np.append(off, np.uint64(1_521_797)) if off[-1] != 1_521_797 else off
    n = int(off[-1])
    a = rng.integers(0, 32768, n).astype(np.uint32)
    codes = rng.integers(0, 256, (n, 16)).astype(np.uint8)
    idx, pay = storage.write_doc_layouts(off, a, codes, 16)
    st, ridx, rpay = orc.write_doc_layouts(off, a, codes, 16, 1)
    assert st == 0 and np.array_equal(idx, ridx) and np.array_equal(pay, rpay)
    assert storage.crc32(pay) == zlib.crc32(rpay.tobytes())


def test_doc_layouts_errors(gpu):
    a = np.zeros(4, np.uint32)
    codes = np.zeros((4, 2), np.uint8)
    with pytest.raises(errors.InvalidArgument):  # decreasing offsets
        storage.write_doc_layouts(np.array([0, 3, 2, 4], np.uint64), a, codes, 2)
    # device entry: offsets past n_tokens are caught on the device
    d_off = device.DeviceArray.from_host(np.array([0, 2, 9], np.uint64))
    d_a = device.DeviceArray.from_host(a)
    d_c = device.DeviceArray.from_host(codes)
    d_i = device.DeviceArray((3,), np.uint64)
    d_p = device.DeviceArray((256,), np.uint8)
    st = lib.tac_write_doc_layouts_device(d_off.ptr, 2, 4, d_a.ptr, d_c.ptr, 2, 1, d_i.ptr,
                                          d_p.ptr, 256, None)
    assert st == errors.InvalidArgument.status
    d_off2 = device.DeviceArray.from_host(np.array([0, 2, 4], np.uint64))
    st = lib.tac_write_doc_layouts_device(d_off2.ptr, 2, 4, d_a.ptr, d_c.ptr, 2, 1, d_i.ptr,
                                          d_p.ptr, 8, None)
    assert st == errors.BufferTooSmall.status


@pytest.mark.parametrize("dim,m,ksub,n_q", [(64, 16, 256, 32), (64, 32, 256, 1),
                                            (64, 8, 1024, 7), (128, 32, 256, 100),
                                            (96, 32, 256, 3), (30, 10, 5, 2)])
def test_distance_table_matches_oracle(gpu, dim, m, ksub, n_q):
    rng = np.random.default_rng(dim + m + n_q)
    cb = rng.standard_normal((m, ksub, dim // m)).astype(np.float32)
    q = rng.standard_normal((n_q, dim)).astype(np.float32)
    p = pq.PQ(dim=dim, sub_dim=dim // m, codebooks=cb.reshape(-1), m=m, ksub=ksub)
    got = p.build_distance_table(q, n_q)
    st, ref = orc.pq_distance_table(q, n_q, dim, m, ksub, cb)
    assert st == 0
    assert np.array_equal(got.reshape(-1).view(np.uint32), ref.view(np.uint32))


def test_distance_table_errors(gpu):
    p = pq.PQ(dim=8, sub_dim=2, codebooks=np.zeros(4 * 256 * 2, np.float32), m=4)
    with pytest.raises(errors.NQMismatch):
        p.build_distance_table(np.zeros(8, np.float32), 0)
    with pytest.raises(errors.NQMismatch):
        p.build_distance_table(np.zeros(9, np.float32), 1)


def _index_and_query(seed, dim, m, ksub, n_q, n_docs=300):
    cents, cb, off, idx, pay, norms, codes, assign = synthetic_index(
        seed, n_docs=n_docs, dim=dim, m=m, ksub=ksub, kappa=40)
    rng = np.random.default_rng(seed + 1)
    q = rng.standard_normal((n_q, dim)).astype(np.float32)
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    _, table = orc.pq_distance_table(q, n_q, dim, m, ksub, cb)
    ix = retrieval.DocIndex(dim, m, ksub, cents, idx, pay, off, norms)
    return ix, table, q


@pytest.mark.parametrize("dim,m,ksub,n_q", [(32, 32, 256, 2), (64, 16, 256, 32),
                                            (128, 32, 256, 65), (96, 32, 256, 100),
                                            (64, 32, 1024, 5), (20, 10, 256, 1)])
def test_refine_matches_oracle(gpu, dim, m, ksub, n_q):
    ix, table, q = _index_and_query(dim * 3 + n_q, dim, m, ksub, n_q)
    cand = np.concatenate([np.arange(ix.n_docs), [5, 5, 0, ix.n_docs - 1]]).astype(np.uint32)
    np.random.default_rng(0).shuffle(cand)
    got = retrieval.refine(ix, table, q, n_q, cand)
    for j, d in enumerate(cand):
        st, want = orc.refine(q, n_q, dim, ix.centroids, table, m, ksub, ix.doc_index,
                              ix.doc_payload, ix.doc_token_offsets, ix.residual_norms, int(d))
        assert st == 0
        assert got[j].tobytes() == want.tobytes(), (j, d, got[j], want)


def test_refine_errors_first_failing_candidate(gpu):
    ix, table, q = _index_and_query(11, 32, 32, 256, 2, n_docs=60)
    with pytest.raises(errors.DocOutOfRange):
        retrieval.refine(ix, table, q, 2, [0, 1, 9999, 3])
    with pytest.raises(errors.TableSizeMismatch):
        retrieval.refine(ix, table[:-1], q, 2, [0])
    with pytest.raises(errors.QueryShapeMismatch):
        retrieval.refine(ix, table, q[:1], 2, [0])
    bad = ix.doc_payload.copy()
    d = next(i for i in range(ix.n_docs) if ix.doc_token_offsets[i + 1] > ix.doc_token_offsets[i])
    bad[int(ix.doc_index[d]) + 4: int(ix.doc_index[d]) + 8] = 255  # centroid id 0xFFFFFFFF
    ix_bad = retrieval.DocIndex(ix.dim, ix.m, ix.ksub, ix.centroids, ix.doc_index, bad,
                                ix.doc_token_offsets, ix.residual_norms)
    with pytest.raises(errors.DocLayoutCorrupt):
        retrieval.refine(ix_bad, table, q, 2, [d])
    # the candidate before the corrupt one decides when both fail
    with pytest.raises(errors.DocOutOfRange):
        retrieval.refine(ix_bad, table, q, 2, [9999, d])
    # a clean call after the errors
    assert retrieval.refine(ix, table, q, 2, [0]).shape == (1,)
