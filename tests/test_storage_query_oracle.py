"""Pins the oracle's .tac layout writer, CRC-32 and refine, and checks on the
CPU the CRC decomposition the GPU kernels use.  No GPU needed.

Pins:
- CRC-32: the CRC catalogue's check value for "123456789" and Python's zlib
  (an independent implementation) over lengths around every boundary.
- Document layouts: a byte image built independently with struct.pack from
  the field list of src/index/storage.zig:705-749, and the size formula of
  :674-686.
- refine: a hand-worked score, and the reference's own refine tests
  (src/retrieval/refine.zig:196-272 brute-force MaxSim within 1e-3,
  :274-305 determinism, :307-336 DocOutOfRange, :338-end shape errors).
"""
import struct
import zlib

import numpy as np
import pytest

from oracle import binding as orc

ST_OK, ST_QSHAPE, ST_TABLE, ST_DOC_RANGE, ST_CORRUPT, ST_SMALL = 0, 16, 17, 18, 19, 20


# ---- CRC-32 ----------------------------------------------------------------

def test_crc_check_value():
    assert orc.crc32(b"123456789") == 0xCBF43926
    assert orc.crc32(b"") == 0


@pytest.mark.parametrize("n", [1, 15, 16, 17, 1023, 1024, 1025, 4096 + 7, 300_001])
def test_crc_matches_zlib(n):
    data = np.random.default_rng(n).integers(0, 256, n, dtype=np.uint8).tobytes()
    assert orc.crc32(data) == zlib.crc32(data)


POLY = 0xEDB88320


def mulmod(a, b):
    """Product of two polynomials mod P, reflected (bit 31 = x^0)."""
    p = 0
    for i in range(32):
        if (a >> (31 - i)) & 1:
            p ^= b
        b = (b >> 1) ^ POLY if b & 1 else b >> 1
    return p


def raw_crc(data, reg=0):
    """CRC register after `data` from register `reg`, no pre/post complement."""
    return (~zlib.crc32(data, ~reg & 0xFFFFFFFF)) & 0xFFFFFFFF


def x8_powers():
    t = 0x40000000  # x^1
    for _ in range(3):
        t = mulmod(t, t)
    out = []
    for _ in range(64):
        out.append(t)
        t = mulmod(t, t)
    return out


def shift(r, count, sh, pw):
    j = 0
    while count:
        if count & 1:
            r = mulmod(pw[j + sh], r)
        count >>= 1
        j += 1
    return r


@pytest.mark.parametrize("n,mis", [(0, 0), (5, 3), (5000, 0), (5000, 9), (70_000, 1)])
def test_crc_decomposition_used_by_the_kernels(n, mis):
    """head (to 16-byte alignment) + whole 256-byte leaves + tail, from the
    all-ones preset, equals zlib's CRC.  Each leaf is four 64-byte chains
    joined by x^(8*64) shifts, and leaves combine pairwise by x^(8 len)."""
    data = np.random.default_rng(n + mis).integers(0, 256, n, dtype=np.uint8).tobytes()
    pw = x8_powers()
    L, LOG2, SUB, SUB_LOG2 = 256, 8, 64, 6
    head = min((16 - mis) % 16, n)
    leaves = (n - head) // L
    tail = n - head - leaves * L

    def leaf_crc(j):
        base = head + j * L
        ways = [raw_crc(data[base + w * SUB: base + (w + 1) * SUB]) for w in range(4)]
        r = ways[0]
        for w in range(1, 4):
            r = mulmod(pw[SUB_LOG2], r) ^ ways[w]
        return r

    nodes = [(leaf_crc(j), 1) for j in range(leaves)]
    while len(nodes) > 1:  # pairwise tree, as the block reduction does
        nxt = []
        for k in range(0, len(nodes), 2):
            if k + 1 < len(nodes):
                (a, na), (b, nb) = nodes[k], nodes[k + 1]
                nxt.append((shift(a, nb, LOG2, pw) ^ b, na + nb))
            else:
                nxt.append(nodes[k])
        nodes = nxt
    body = nodes[0][0] if nodes else 0
    r = raw_crc(data[:head], 0xFFFFFFFF)
    r = shift(r, leaves, LOG2, pw) ^ body
    r = raw_crc(data[n - tail:], r) if tail else r
    assert r ^ 0xFFFFFFFF == zlib.crc32(data)


def test_slicing_by_8_step():
    """Eight bytes at once through tables T_k (byte then k zero bytes) equal
    eight byte steps."""
    T0 = []
    for i in range(256):
        r = i
        for _ in range(8):
            r = (r >> 1) ^ POLY if r & 1 else r >> 1
        T0.append(r)
    T = [T0]
    for k in range(1, 8):
        T.append([(v >> 8) ^ T0[v & 0xFF] for v in T[k - 1]])
    rng = np.random.default_rng(3)
    for _ in range(200):
        reg = int(rng.integers(0, 2**32))
        b = rng.integers(0, 256, 8, dtype=np.uint8).tobytes()
        lo, hi = struct.unpack("<II", b)
        x = reg ^ lo
        got = (T[7][x & 0xFF] ^ T[6][(x >> 8) & 0xFF] ^ T[5][(x >> 16) & 0xFF] ^ T[4][x >> 24]
               ^ T[3][hi & 0xFF] ^ T[2][(hi >> 8) & 0xFF] ^ T[1][(hi >> 16) & 0xFF]
               ^ T[0][hi >> 24])
        assert got == raw_crc(b, reg)


def test_shift_table_rows_multiply():
    """The kernels multiply by x^(8 * 2^j) as the XOR of table row j's
    entries x^(8 * 2^j) * x^i over the coefficients i of the register."""
    pw = x8_powers()
    rng = np.random.default_rng(9)
    for j in (0, 6, 8, 17, 40):
        row, v = [], pw[j]
        for _ in range(32):
            row.append(v)
            v = (v >> 1) ^ POLY if v & 1 else v >> 1
        for reg in rng.integers(0, 2**32, 20):
            reg = int(reg)
            got = 0
            for i in range(32):
                if (reg >> (31 - i)) & 1:
                    got ^= row[i]
            assert got == mulmod(reg, pw[j])


def test_shift_is_zero_bytes():
    pw = x8_powers()
    for reg in (0x12345678, 0xFFFFFFFF, 1):
        assert shift(reg, 3, 0, pw) == raw_crc(b"\0\0\0", reg)


# ---- document layouts --------------------------------------------------------

def layout_by_hand(doc_offsets, assign, codes, m, cb):
    idx, pay = [], b""
    for d in range(len(doc_offsets) - 1):
        idx.append(len(pay))
        lo, hi = doc_offsets[d], doc_offsets[d + 1]
        n_d = hi - lo
        rec = struct.pack("<I", n_d) + struct.pack(f"<{n_d}I", *assign[lo:hi])
        flat = codes[lo:hi].reshape(-1)
        rec += struct.pack(f"<{flat.size}{'B' if cb == 1 else 'H'}", *flat.tolist())
        rec += b"\0" * (-len(rec) % 8)
        pay += rec
    idx.append(len(pay))
    return np.array(idx, np.uint64), np.frombuffer(pay, np.uint8)


@pytest.mark.parametrize("m,cb", [(32, 1), (3, 1), (16, 2), (5, 2)])
def test_doc_layouts_match_hand_built_bytes(m, cb):
    rng = np.random.default_rng(m * 10 + cb)
    lens = [3, 0, 1, 8, 0, 0, 13, 2]
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint64)
    n = int(off[-1])
    a = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    codes = rng.integers(0, 256 if cb == 1 else 1024, (n, m)).astype(
        np.uint8 if cb == 1 else np.uint16)
    st, idx, pay = orc.write_doc_layouts(off, a, codes, m, cb)
    assert st == ST_OK
    hidx, hpay = layout_by_hand(off.tolist(), a.tolist(), codes, m, cb)
    assert np.array_equal(idx, hidx) and np.array_equal(pay, hpay)
    assert orc.doc_payload_bytes(off, m, cb) == hpay.size
    assert orc.write_doc_layouts(off, a, codes, m, cb, payload_len=hpay.size - 1)[0] == ST_SMALL


def test_reference_fixture_sizes():
    # PQ_M = 32, u8 codes: a doc of n_d tokens takes align8(4 + 36 n_d) bytes
    off = np.array([0, 1, 3, 3], np.uint64)
    assert orc.doc_payload_bytes(off, 32, 1) == 40 + 80 + 8


# ---- refine ------------------------------------------------------------------

def tiny_index():
    # dim 2, m 1 (dsub 2), ksub 2; doc 0 has two tokens, doc 1 none
    cents = np.array([[1, 0], [0, 1]], np.float32)
    cb = np.array([[[0.5, 0.0], [0.0, 0.5]]], np.float32)
    off = np.array([0, 2, 2], np.uint64)
    assign = np.array([0, 1], np.uint32)
    codes = np.array([[1], [0]], np.uint8)
    norms = np.array([2.0, 1.0], np.float32)
    _, idx, pay = orc.write_doc_layouts(off, assign, codes, 1, 1)
    return cents, cb, off, idx, pay, norms


def test_refine_hand_worked():
    cents, cb, off, idx, pay, norms = tiny_index()
    q = np.array([[1, 2]], np.float32)
    st, table = orc.pq_distance_table(q, 1, 2, 1, 2, cb)
    assert st == ST_OK and table.tolist() == [0.5, 1.0]
    # token 0: <q, c0> + 2 * table[code 1] = 1 + 2 = 3; token 1: 2 + 1 * 0.5 = 2.5
    assert orc.refine(q, 1, 2, cents, table, 1, 2, idx, pay, off, norms, 0) == (ST_OK, 3.0)
    assert orc.refine(q, 1, 2, cents, table, 1, 2, idx, pay, off, norms, 1) == (ST_OK, 0.0)


def test_refine_errors():
    cents, cb, off, idx, pay, norms = tiny_index()
    q = np.array([[1, 2]], np.float32)
    _, table = orc.pq_distance_table(q, 1, 2, 1, 2, cb)
    assert orc.refine(q, 1, 2, cents, table, 1, 2, idx, pay, off, norms, 9999)[0] == ST_DOC_RANGE
    assert orc.refine(q, 1, 2, cents, table[:1], 1, 2, idx, pay, off, norms, 0)[0] == ST_TABLE
    assert orc.refine(q, 0, 2, cents, table, 1, 2, idx, pay, off, norms, 0)[0] == ST_QSHAPE
    bad = pay.copy()
    bad[4] = 7  # centroid id 7 of a 2-centroid table
    assert orc.refine(q, 1, 2, cents, table, 1, 2, idx, bad, off, norms, 0)[0] == ST_CORRUPT
    short_off = np.array([0, 1, 2], np.uint64)  # token range disagrees with n_d
    assert orc.refine(q, 1, 2, cents, table, 1, 2, idx, pay, short_off, norms, 0)[0] == ST_CORRUPT


def synthetic_index(seed, n_docs=50, dim=32, m=32, ksub=256, kappa=16):
    """Docs of unit tokens around kappa centroids, residuals PQ-coded with
    codebooks trained by the oracle (the reference's refine fixture shape:
    dim 32, 50 docs, kappa 16)."""
    rng = np.random.default_rng(seed)
    cents = rng.standard_normal((kappa, dim)).astype(np.float32)
    cents /= np.linalg.norm(cents, axis=1, keepdims=True)
    lens = rng.integers(0, 16, n_docs)
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint64)
    n = int(off[-1])
    assign = rng.integers(0, kappa, n).astype(np.uint32)
    tok = cents[assign] + 0.3 * rng.standard_normal((n, dim)).astype(np.float32)
    tok /= np.linalg.norm(tok, axis=1, keepdims=True)
    st, res, norms = orc.residuals(tok.astype(np.float32), dim, cents, assign)
    assert st == ST_OK
    assert n >= ksub, "the fixture needs at least ksub tokens for its initial codebooks"
    init = res[rng.permutation(n)[:ksub]].reshape(ksub, m, dim // m).transpose(1, 0, 2)
    tr = orc.pq_train(res, dim, m, ksub, init=np.ascontiguousarray(init), max_iters=5)
    codes = orc.pq_encode(res, dim, m, ksub, tr.codebooks)
    _, idx, pay = orc.write_doc_layouts(off, assign, codes, m, 1 if ksub <= 256 else 2)
    return cents, tr.codebooks.reshape(m, ksub, dim // m), off, idx, pay, norms, codes, assign


def test_refine_matches_brute_force_maxsim():  # refine.zig:196-272
    cents, cb, off, idx, pay, norms, codes, assign = synthetic_index(2002)
    dim, m = 32, 32
    q = np.stack([cents[0], cents[2]]).astype(np.float32)
    _, table = orc.pq_distance_table(q, 2, dim, m, 256, cb)
    for d in range(50):
        st, got = orc.refine(q, 2, dim, cents, table, m, 256, idx, pay, off, norms, d)
        assert st == ST_OK
        lo, hi = int(off[d]), int(off[d + 1])
        if hi == lo:
            assert got == 0.0
            continue
        recon = cents[assign[lo:hi]] + norms[lo:hi, None] * np.concatenate(
            [cb[mm][codes[lo:hi, mm]] for mm in range(m)], axis=1)
        bf = np.sum(np.max(q.astype(np.float64) @ recon.T.astype(np.float64), axis=1))
        assert abs(got - bf) < 1e-3


def test_refine_deterministic():  # refine.zig:274-305
    cents, cb, off, idx, pay, norms, _, _ = synthetic_index(3003)
    q = np.stack([cents[0], cents[1]]).astype(np.float32)
    _, table = orc.pq_distance_table(q, 2, 32, 32, 256, cb)
    a = orc.refine(q, 2, 32, cents, table, 32, 256, idx, pay, off, norms, 7)
    b = orc.refine(q, 2, 32, cents, table, 32, 256, idx, pay, off, norms, 7)
    assert a[0] == ST_OK and a[1].tobytes() == b[1].tobytes()
