"""ctypes binding of the CPU oracle (oracle/_build/libpq_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the timed CPU
baseline, never as part of the product path.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "_build" / "libpq_oracle.so"

_vp, _u64, _u32, _f32 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_float


class FitExtras(ctypes.Structure):
    _fields_ = [("trace", _vp), ("empties", _vp), ("wcss_trace", _vp)]


class TrainExtras(ctypes.Structure):
    _fields_ = [("trace", _vp), ("iters_run", _vp), ("wcss", _vp), ("empties", _vp)]


class TacParams(ctypes.Structure):
    _fields_ = [("kappa_total", _u32), ("mu", _u32), ("tau", _u32), ("epsilon", _u32),
                ("theta", _u32), ("max_iters", _u32), ("tol", _f32), ("seed", _u64),
                ("n_threads", _u32)]


class Xoshiro(ctypes.Structure):
    _fields_ = [("s", _u64 * 4)]


def _load():
    if not LIB_PATH.exists():
        raise ImportError(f"{LIB_PATH} is not built (make -C oracle)")
    L = ctypes.CDLL(os.fspath(LIB_PATH))
    L.orc_l2sq.restype = _f32
    L.orc_l2sq.argtypes = [_vp, _vp, _u32]
    L.orc_dot.restype = _f32
    L.orc_dot.argtypes = [_vp, _vp, _u32]
    L.orc_argmin.restype = _u64
    L.orc_argmin.argtypes = [_vp, _u64]
    L.orc_argmax.restype = _u64
    L.orc_argmax.argtypes = [_vp, _u64]
    L.orc_zig_prng_init.argtypes = [ctypes.POINTER(Xoshiro), _u64]
    L.orc_zig_next.restype = _u64
    L.orc_zig_next.argtypes = [ctypes.POINTER(Xoshiro)]
    L.orc_zig_uint_less_than.restype = _u64
    L.orc_zig_uint_less_than.argtypes = [ctypes.POINTER(Xoshiro), _u64]
    L.orc_zig_float_f64.restype = ctypes.c_double
    L.orc_zig_float_f64.argtypes = [ctypes.POINTER(Xoshiro)]
    L.orc_weighted_sample.restype = ctypes.c_int
    L.orc_weighted_sample.argtypes = [ctypes.POINTER(Xoshiro), _vp, _u64,
                                      ctypes.POINTER(_u64)]
    L.orc_kmeans_fit.restype = ctypes.c_int
    L.orc_kmeans_fit.argtypes = [_vp, _u64, _u32, _u32, _u32, _f32, _u64, _u32, _vp, _vp, _vp,
                                 ctypes.POINTER(_f32), ctypes.POINTER(_u32),
                                 ctypes.POINTER(FitExtras)]
    L.orc_pq_train.restype = ctypes.c_int
    L.orc_pq_train.argtypes = [_vp, _u64, _u32, _u32, _u32, _vp, _u64, _u32, _f32, _u32, _vp,
                               ctypes.POINTER(TrainExtras)]
    L.orc_set_scalar.restype = None
    L.orc_set_scalar.argtypes = [ctypes.c_int]
    L.orc_set_lane_count.restype = ctypes.c_int
    L.orc_set_lane_count.argtypes = [_u32]
    L.orc_lane_count.restype = _u32
    L.orc_lane_count.argtypes = []
    L.orc_pq_encode.restype = ctypes.c_int
    L.orc_pq_encode.argtypes = [_vp, _u64, _u32, _u32, _u32, _vp, _vp, _u32]
    L.orc_pq_near_ties.restype = ctypes.c_int
    L.orc_pq_near_ties.argtypes = [_vp, _u64, _u32, _u32, _u32, _vp, _f32,
                                   ctypes.POINTER(_u64), _u32]
    L.orc_pq_decode.restype = ctypes.c_int
    L.orc_pq_decode.argtypes = [_vp, _u64, _u32, _u32, _u32, _vp, _vp]
    L.orc_pq_distance_table.restype = ctypes.c_int
    L.orc_pq_distance_table.argtypes = [_vp, _u32, _u32, _u32, _u32, _vp, _vp, _u64]
    L.orc_residuals.restype = ctypes.c_int
    L.orc_residuals.argtypes = [_vp, _u64, _u32, _vp, _u32, _vp, _vp, _vp]
    L.orc_doc_payload_bytes.restype = _u64
    L.orc_doc_payload_bytes.argtypes = [_vp, _u64, _u32, _u32]
    L.orc_write_doc_layouts.restype = ctypes.c_int
    L.orc_write_doc_layouts.argtypes = [_vp, _u64, _vp, _vp, _u32, _u32, _vp, _vp, _u64]
    L.orc_crc32.restype = _u32
    L.orc_crc32.argtypes = [_vp, _u64]
    L.orc_refine.restype = ctypes.c_int
    L.orc_refine.argtypes = [_vp, _u32, _u32, _vp, _u32, _vp, _u64, _u32, _u32, _vp, _vp, _u64,
                             _vp, _vp, _u64, _u64, _u64, ctypes.POINTER(_f32)]
    L.orc_tac_allocate_tail.restype = ctypes.c_int
    L.orc_tac_allocate_tail.argtypes = [_vp, _u64, _vp, _u32, _u32, _u32, ctypes.POINTER(_u32)]
    L.orc_tac_damped_phase2.restype = ctypes.c_int
    L.orc_tac_damped_phase2.argtypes = [_vp, _vp, _u64, _vp, _vp, _u32, _u32, _u32]
    L.orc_tac_bound_phase3.restype = ctypes.c_int
    L.orc_tac_bound_phase3.argtypes = [_vp, _u64, _vp, _u32, _u32, _u32, _u32]
    L.orc_tac_reconcile_phase4.restype = ctypes.c_int
    L.orc_tac_reconcile_phase4.argtypes = [_vp, _u64, _vp, _vp, _u32, _u32, _u32, _u32, _u32]
    L.orc_tac_allocate_budgets.restype = ctypes.c_int
    L.orc_tac_allocate_budgets.argtypes = [_vp, _vp, _u64, _vp, _vp, ctypes.POINTER(TacParams)]
    L.orc_tac_spreads.restype = None
    L.orc_tac_spreads.argtypes = [_vp, _u32, _vp, _vp, _u64, _vp]
    L.orc_tac_cluster_flat.restype = ctypes.c_int
    L.orc_tac_cluster_flat.argtypes = [_vp, _u64, _vp, _u64, _u32, ctypes.POINTER(TacParams),
                                       _vp, _vp, _vp, ctypes.POINTER(_f32), ctypes.POINTER(_u64)]
    return L


lib = _load()


def _p(a):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def l2sq(a, b) -> np.float32:
    a, b = _f32(a).reshape(-1), _f32(b).reshape(-1)
    assert a.size == b.size
    return np.float32(lib.orc_l2sq(_p(a), _p(b), a.size))


def dot(a, b) -> np.float32:
    a, b = _f32(a).reshape(-1), _f32(b).reshape(-1)
    return np.float32(lib.orc_dot(_p(a), _p(b), a.size))


def argmin(v) -> int:
    v = _f32(v).reshape(-1)
    return int(lib.orc_argmin(_p(v), v.size))


def argmax(v) -> int:
    v = _f32(v).reshape(-1)
    return int(lib.orc_argmax(_p(v), v.size))


class ZigPrng:
    """Restated Zig std.Random.DefaultPrng (parity unpinned)."""

    def __init__(self, seed: int):
        self.state = Xoshiro()
        lib.orc_zig_prng_init(ctypes.byref(self.state), seed & (2**64 - 1))

    def next(self) -> int:
        return int(lib.orc_zig_next(ctypes.byref(self.state)))

    def uint_less_than(self, n: int) -> int:
        return int(lib.orc_zig_uint_less_than(ctypes.byref(self.state), n))

    def float_f64(self) -> float:
        return float(lib.orc_zig_float_f64(ctypes.byref(self.state)))

    def weighted_sample(self, w) -> tuple[int, int]:
        w = _f32(w).reshape(-1)
        out = _u64(0)
        st = lib.orc_weighted_sample(ctypes.byref(self.state), _p(w), w.size, ctypes.byref(out))
        return st, int(out.value)


@dataclass
class FitResult:
    status: int
    centroids: np.ndarray
    assignments: np.ndarray
    wcss: float
    iters_run: int
    trace: np.ndarray | None
    empties: np.ndarray | None
    wcss_trace: np.ndarray | None


def kmeans_fit(vectors, dim: int, k: int, *, max_iters: int = 25, tol: float = 1e-4,
               seed: int = 0, n_threads: int = 1, init=None, trace: bool = False) -> FitResult:
    v = _f32(vectors).reshape(-1)
    n = v.size // dim if dim else 0
    cent = np.zeros(max(k, 1) * max(dim, 1), dtype=np.float32)
    assign = np.zeros(max(n, 1), dtype=np.uint32)
    init_a = None if init is None else _f32(init).reshape(-1)
    tr = np.zeros((max_iters, k * dim), np.float32) if trace and max_iters else None
    emp = np.zeros(max_iters, np.uint32) if trace and max_iters else None
    wtr = np.zeros(max_iters, np.float32) if trace and max_iters else None
    ex = FitExtras(_p(tr), _p(emp), _p(wtr))
    wcss, iters = _f32_c(), _u32(0)
    st = lib.orc_kmeans_fit(_p(v), n, dim, k, max_iters, tol, seed & (2**64 - 1), n_threads,
                            _p(init_a), _p(cent), _p(assign), ctypes.byref(wcss),
                            ctypes.byref(iters), ctypes.byref(ex))
    return FitResult(st, cent[:k * dim], assign[:n], float(wcss.value), int(iters.value), tr, emp,
                     wtr)


def _f32_c():
    return ctypes.c_float(0.0)


@dataclass
class TrainResult:
    status: int
    codebooks: np.ndarray
    iters_run: np.ndarray
    wcss: np.ndarray
    empties: np.ndarray
    trace: np.ndarray | None


def pq_train(residuals, dim: int, m: int, ksub: int, *, init=None, seed: int = 0,
             max_iters: int = 25, tol: float = 1e-4, n_threads: int = 1,
             trace: bool = False) -> TrainResult:
    r = _f32(residuals).reshape(-1)
    n = r.size // dim if dim else 0
    dsub = dim // m if m else 0
    cb = np.zeros(max(m * ksub * dsub, 1), dtype=np.float32)
    init_a = None if init is None else _f32(init).reshape(-1)
    it = np.zeros(max(m, 1), np.uint32)
    wc = np.zeros(max(m, 1), np.float32)
    em = np.zeros(max(m, 1), np.uint32)
    tr = np.zeros((max_iters, m * ksub * dsub), np.float32) if trace and max_iters else None
    ex = TrainExtras(_p(tr), _p(it), _p(wc), _p(em))
    st = lib.orc_pq_train(_p(r), n, dim, m, ksub, _p(init_a), seed & (2**64 - 1), max_iters, tol,
                          n_threads, _p(cb), ctypes.byref(ex))
    return TrainResult(st, cb[:m * ksub * dsub], it[:m], wc[:m], em[:m], tr)


def pq_encode(residuals, dim: int, m: int, ksub: int, codebooks, n_threads: int = 1):
    r = _f32(residuals).reshape(-1)
    n = r.size // dim
    out = np.zeros((n, m), dtype=np.uint8 if ksub <= 256 else np.uint16)
    cb = _f32(codebooks).reshape(-1)
    st = lib.orc_pq_encode(_p(r), n, dim, m, ksub, _p(cb), _p(out), n_threads)
    assert st == 0, st
    return out


def pq_near_ties(residuals, dim: int, m: int, ksub: int, codebooks, rel_tol: float = 1e-5,
                 n_threads: int = 1) -> int:
    r = _f32(residuals).reshape(-1)
    cb = _f32(codebooks).reshape(-1)
    out = _u64(0)
    st = lib.orc_pq_near_ties(_p(r), r.size // dim, dim, m, ksub, _p(cb), rel_tol,
                              ctypes.byref(out), n_threads)
    assert st == 0, st
    return int(out.value)


def pq_decode(codes, dim: int, m: int, ksub: int, codebooks):
    c = np.ascontiguousarray(codes, dtype=np.uint8 if ksub <= 256 else np.uint16)
    n = c.size // m
    out = np.zeros((n, dim), np.float32)
    cb = _f32(codebooks).reshape(-1)
    st = lib.orc_pq_decode(_p(c), n, dim, m, ksub, _p(cb), _p(out))
    assert st == 0, st
    return out


def pq_distance_table(queries, n_q: int, dim: int, m: int, ksub: int, codebooks,
                      table_len: int | None = None):
    q = _f32(queries).reshape(-1)
    cb = _f32(codebooks).reshape(-1)
    tl = m * ksub * n_q if table_len is None else table_len
    out = np.zeros(max(tl, 1), np.float32)
    st = lib.orc_pq_distance_table(_p(q), n_q, dim, m, ksub, _p(cb), _p(out), tl)
    return st, out[:tl]


def residuals(vectors, dim: int, centroids, assignments):
    """(status, residuals [n][dim], norms [n]) of storage.zig:255-278."""
    v = _f32(vectors).reshape(-1)
    c = _f32(centroids).reshape(-1)
    a = np.ascontiguousarray(assignments, dtype=np.uint32).reshape(-1)
    n = a.size
    r = np.zeros((n, dim), np.float32)
    nr = np.zeros(n, np.float32)
    st = lib.orc_residuals(_p(v), n, dim, _p(c), c.size // dim if dim else 0, _p(a), _p(r),
                           _p(nr))
    return st, r, nr


def doc_payload_bytes(doc_offsets, m: int, code_bytes: int) -> int:
    o = np.ascontiguousarray(doc_offsets, dtype=np.uint64)
    return int(lib.orc_doc_payload_bytes(_p(o), o.size - 1, m, code_bytes))


def write_doc_layouts(doc_offsets, assignments, codes, m: int, code_bytes: int,
                      payload_len: int | None = None):
    """(status, doc_index [n_docs+1] u64, payload bytes) of storage.zig:705-749."""
    o = np.ascontiguousarray(doc_offsets, dtype=np.uint64)
    a = np.ascontiguousarray(assignments, dtype=np.uint32)
    c = np.ascontiguousarray(codes, dtype=np.uint8 if code_bytes == 1 else np.uint16)
    n_docs = o.size - 1
    need = doc_payload_bytes(o, m, code_bytes)
    plen = need if payload_len is None else payload_len
    idx = np.zeros(n_docs + 1, np.uint64)
    pay = np.zeros(max(plen, 1), np.uint8)
    st = lib.orc_write_doc_layouts(_p(o), n_docs, _p(a), _p(c), m, code_bytes, _p(idx), _p(pay),
                                   plen)
    return st, idx, pay[:plen]


def crc32(data) -> int:
    b = np.frombuffer(bytes(data), dtype=np.uint8) if not isinstance(data, np.ndarray) \
        else np.ascontiguousarray(data).view(np.uint8).reshape(-1)
    return int(lib.orc_crc32(_p(b) if b.size else None, b.size))


def refine(query, n_q: int, dim: int, centroids, table, m: int, ksub: int, doc_index, payload,
           doc_token_offsets, norms, doc_id: int):
    """(status, score) of refine.zig:83-145 for one candidate document."""
    q = _f32(query).reshape(-1)
    c = _f32(centroids).reshape(-1)
    t = _f32(table).reshape(-1)
    di = np.ascontiguousarray(doc_index, dtype=np.uint64)
    pay = np.ascontiguousarray(payload, dtype=np.uint8)
    dto = np.ascontiguousarray(doc_token_offsets, dtype=np.uint64)
    nr = _f32(norms).reshape(-1)
    out = _f32_c()
    st = lib.orc_refine(_p(q), n_q, dim, _p(c), c.size // dim, _p(t), t.size, m, ksub, _p(di),
                        _p(pay), pay.size, _p(dto), _p(nr), nr.size, di.size - 1, doc_id,
                        ctypes.byref(out))
    return st, np.float32(out.value)


# ---- TAC (src/tac/tac.zig) ---------------------------------------------------

# Paper defaults (src/constants.zig TAC_MU / TAC_TAU / TAC_EPSILON / TAC_THETA).
TAC_DEFAULTS = dict(mu=128, tau=256, epsilon=4, theta=39, max_iters=25, tol=1e-4)


def tac_params(kappa_total: int, seed: int, **kw) -> TacParams:
    d = dict(TAC_DEFAULTS, n_threads=1)
    d.update(kw)
    return TacParams(kappa_total, d["mu"], d["tau"], d["epsilon"], d["theta"], d["max_iters"],
                     d["tol"], seed & (2**64 - 1), d["n_threads"])


def _u32a(a):
    return np.ascontiguousarray(a, dtype=np.uint32)


def tac_allocate_tail(freqs, mu, tau, kappa_total):
    f = _u32a(freqs)
    kappa = np.zeros(max(f.size, 1), np.uint32)
    b = _u32(0)
    st = lib.orc_tac_allocate_tail(_p(f), f.size, _p(kappa), mu, tau, kappa_total,
                                   ctypes.byref(b))
    return st, kappa[:f.size], int(b.value)


def tac_damped_phase2(freqs, spreads, kappa, budget_active, mu, tau):
    f, sp = _u32a(freqs), _f32(spreads)
    k = _u32a(kappa).copy()
    frac = np.zeros(max(f.size, 1), np.float32)
    st = lib.orc_tac_damped_phase2(_p(f), _p(sp), f.size, _p(k), _p(frac), budget_active, mu, tau)
    return st, k, frac[:f.size]


def tac_bound_phase3(freqs, kappa, mu, tau, epsilon, theta):
    f = _u32a(freqs)
    k = _u32a(kappa).copy()
    st = lib.orc_tac_bound_phase3(_p(f), f.size, _p(k), mu, tau, epsilon, theta)
    return st, k


def tac_reconcile_phase4(freqs, kappa, frac, kappa_total, mu, tau, epsilon, theta):
    f, fr = _u32a(freqs), _f32(frac)
    k = _u32a(kappa).copy()
    st = lib.orc_tac_reconcile_phase4(_p(f), f.size, _p(k), _p(fr), kappa_total, mu, tau,
                                      epsilon, theta)
    return st, k


def tac_allocate_budgets(freqs, spreads, params: TacParams):
    f, sp = _u32a(freqs), _f32(spreads)
    k = np.zeros(max(f.size, 1), np.uint32)
    frac = np.zeros(max(f.size, 1), np.float32)
    st = lib.orc_tac_allocate_budgets(_p(f), _p(sp), f.size, _p(k), _p(frac), ctypes.byref(params))
    return st, k[:f.size], frac[:f.size]


def tac_spreads(vectors, dim, group_offsets, group_indices):
    v = _f32(vectors).reshape(-1)
    go, gi = _u32a(group_offsets), _u32a(group_indices)
    nd = go.size - 1
    out = np.zeros(max(nd, 1), np.float32)
    lib.orc_tac_spreads(_p(v), dim, _p(go), _p(gi), nd, _p(out))
    return out[:nd]


@dataclass
class TacResult:
    status: int
    centroids: np.ndarray
    assignments: np.ndarray
    kappa_per_token: np.ndarray
    wcss_total: float


def tac_cluster_flat(token_ids, vectors, dim: int, params: TacParams) -> TacResult:
    ids = _u32a(token_ids).reshape(-1)
    v = _f32(vectors).reshape(-1)
    nd = int(ids.max()) + 1 if ids.size else 1
    cent = np.zeros(max(params.kappa_total * max(dim, 1), 1), np.float32)
    asg = np.zeros(max(ids.size, 1), np.uint32)
    kpt = np.zeros(nd, np.uint32)
    w, ndo = _f32_c(), _u64(0)
    st = lib.orc_tac_cluster_flat(_p(ids), ids.size, _p(v), v.size, dim, ctypes.byref(params),
                                  _p(cent), _p(asg), _p(kpt), ctypes.byref(w), ctypes.byref(ndo))
    return TacResult(st, cent[:params.kappa_total * dim], asg[:ids.size], kpt,
                     float(np.float32(w.value)))


class scalar_distances:
    """Within the block, every oracle distance goes through orc_l2sq pair by
    pair (the per-pair form the vectorized d <= 8 path is checked against)."""

    def __enter__(self):
        lib.orc_set_scalar(1)
        return self

    def __exit__(self, *exc):
        lib.orc_set_scalar(0)
        return False


class lane_count:
    """Within the block the oracle's generic vec path (src/util/vec.zig:16,
    :90-103, :159-175) runs with `lanes` vector lanes (4, 8 or 16), the
    value of std.simd.suggestVectorLength(f32) on the host being matched."""

    def __init__(self, lanes: int):
        self.lanes = lanes

    def __enter__(self):
        self.prev = int(lib.orc_lane_count())
        st = lib.orc_set_lane_count(self.lanes)
        assert st == 0, f"lane count {self.lanes} rejected"
        return self

    def __exit__(self, *exc):
        lib.orc_set_lane_count(self.prev)
        return False
