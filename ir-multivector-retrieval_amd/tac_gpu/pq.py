"""Python mirror of the reference's ``tac.index.pq`` module over the C ABI.

Names, argument meaning and error behaviour follow src/index/pq.zig:
``train`` (pq.zig:158-291), ``PQ.encode`` (:59-76), ``PQ.decode`` (:79-88),
``PQ.codebookEntry`` (:52-56).  The subspace count ``m`` and codebook size
``ksub`` are compile-time constants in the reference (src/constants.zig:16-18)
and keyword arguments here, defaulting to the reference's values.
All computation runs on the GPU through ``libtac_gpu.so``.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import errors
from ._native import TrainExtras, lib

PQ_M = 32          # src/constants.zig:16
PQ_BITS = 8        # src/constants.zig:17
PQ_CENTROIDS = 256  # src/constants.zig:18

# Reference defaults of the per-subspace k-means (src/index/pq.zig:319-325).
DEFAULT_MAX_ITERS = 25
DEFAULT_TOL = 1e-4
# A tolerance that never triggers the early break: exactly max_iters run.
TOL_NEVER = float("-inf")


def _ptr(a: np.ndarray | None) -> ctypes.c_void_p | None:
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def code_dtype(ksub: int) -> np.dtype:
    return np.dtype(np.uint8) if ksub <= 256 else np.dtype(np.uint16)


def _validate(flat_len: int, dim: int, m: int) -> None:
    # Order of src/index/pq.zig:165-168.
    if dim == 0:
        raise errors.DimMismatch("DimMismatch")
    if dim % m != 0:
        raise errors.DimNotDivisibleByM("DimNotDivisibleByM")
    if flat_len == 0:
        raise errors.EmptyCorpus("EmptyCorpus")
    if flat_len % dim != 0:
        raise errors.DimMismatch("DimMismatch")


@dataclass
class TrainStats:
    """Per-subspace results the reference keeps in KMeansResult."""

    iters_run: np.ndarray
    wcss: np.ndarray
    empties: np.ndarray
    trace: np.ndarray | None = None


@dataclass
class PQ:
    """Trained codebooks; layout codebook[m][c][k] (src/index/pq.zig:14-15)."""

    dim: int
    sub_dim: int
    codebooks: np.ndarray  # float32 [m * ksub * sub_dim]
    m: int = PQ_M
    ksub: int = PQ_CENTROIDS
    stats: TrainStats | None = field(default=None, repr=False)

    def codebook_entry(self, mm: int, c: int) -> np.ndarray:
        base = (mm * self.ksub + c) * self.sub_dim
        return self.codebooks[base:base + self.sub_dim]

    def encode(self, residual: np.ndarray) -> np.ndarray:
        """Encode one residual into m codes (PQ.encode, pq.zig:59-76)."""
        r = np.ascontiguousarray(residual, dtype=np.float32).reshape(-1)
        if r.size != self.dim:
            raise errors.DimMismatch("DimMismatch")
        return self.encode_many(r.reshape(1, self.dim))[0]

    def encode_many(self, residuals: np.ndarray) -> np.ndarray:
        """Encode n residuals at once; codes are token-major [n][m]."""
        r = np.ascontiguousarray(residuals, dtype=np.float32)
        if r.size % self.dim != 0:
            raise errors.DimMismatch("DimMismatch")
        n = r.size // self.dim
        out = np.empty((n, self.m), dtype=code_dtype(self.ksub))
        if n == 0:
            return out
        cb = np.ascontiguousarray(self.codebooks, dtype=np.float32)
        errors.check(lib.tac_pq_encode(_ptr(r), n, self.dim, self.m, self.ksub, _ptr(cb),
                                       _ptr(out)))
        return out

    def decode(self, codes: np.ndarray) -> np.ndarray:
        """Decode m codes back into a dim-length residual (pq.zig:79-88)."""
        c = np.ascontiguousarray(codes, dtype=code_dtype(self.ksub)).reshape(-1)
        if c.size != self.m:
            raise errors.DimMismatch("DimMismatch")
        return self.decode_many(c.reshape(1, self.m))[0]

    def build_distance_table(self, query_tokens: np.ndarray, n_q: int) -> np.ndarray:
        """PQ.buildDistanceTable (pq.zig:92-123): float32 [m][ksub][n_q] of
        dot(query_i[m-th sub-vector], codeword)."""
        if n_q == 0:
            raise errors.NQMismatch("NQMismatch")
        q = np.ascontiguousarray(query_tokens, dtype=np.float32).reshape(-1)
        if q.size != n_q * self.dim:
            raise errors.NQMismatch("NQMismatch")
        out = np.empty((self.m, self.ksub, n_q), dtype=np.float32)
        cb = np.ascontiguousarray(self.codebooks, dtype=np.float32)
        errors.check(lib.tac_pq_distance_table(_ptr(q), n_q, self.dim, self.m, self.ksub,
                                               _ptr(cb), _ptr(out), out.size))
        return out

    def decode_many(self, codes: np.ndarray) -> np.ndarray:
        c = np.ascontiguousarray(codes, dtype=code_dtype(self.ksub))
        if c.size % self.m != 0:
            raise errors.DimMismatch("DimMismatch")
        n = c.size // self.m
        out = np.empty((n, self.dim), dtype=np.float32)
        if n == 0:
            return out
        cb = np.ascontiguousarray(self.codebooks, dtype=np.float32)
        errors.check(lib.tac_pq_decode(_ptr(c), n, self.dim, self.m, self.ksub, _ptr(cb),
                                       _ptr(out)))
        return out


def train(residuals: np.ndarray, dim: int, seed: int, n_threads: int = 1, *, m: int = PQ_M,
          ksub: int = PQ_CENTROIDS, max_iters: int = DEFAULT_MAX_ITERS,
          tol: float = DEFAULT_TOL, init_codebooks: np.ndarray | None = None,
          trace: bool = False) -> PQ:
    """pq.train (src/index/pq.zig:158-291).

    ``n_threads`` is accepted for signature parity and ignored: the GPU path
    runs every subspace at once.  ``init_codebooks`` ([m][ksub][dsub]) seeds
    the Lloyd loop of each subspace; without it the reference uses k-means++.
    """
    del n_threads
    r = np.ascontiguousarray(residuals, dtype=np.float32).reshape(-1)
    _validate(r.size, dim, m)
    n = r.size // dim
    sub_dim = dim // m
    cb = np.empty(m * ksub * sub_dim, dtype=np.float32)
    init = None
    if init_codebooks is not None:
        init = np.ascontiguousarray(init_codebooks, dtype=np.float32).reshape(-1)
        if init.size != cb.size:
            raise errors.OutBufferWrongSize("OutBufferWrongSize")
    iters = np.zeros(m, dtype=np.uint32)
    wcss = np.zeros(m, dtype=np.float32)
    empties = np.zeros(m, dtype=np.uint32)
    tr = np.empty((max_iters, m * ksub * sub_dim), dtype=np.float32) if trace else None
    ex = TrainExtras(
        iters.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
        wcss.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
        empties.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
        tr.ctypes.data_as(ctypes.POINTER(ctypes.c_float)) if tr is not None else None,
    )
    errors.check(lib.tac_pq_train(_ptr(r), n, dim, m, ksub, _ptr(init), seed & (2**64 - 1),
                                  max_iters, tol, _ptr(cb), ctypes.byref(ex)))
    return PQ(dim=dim, sub_dim=sub_dim, codebooks=cb, m=m, ksub=ksub,
              stats=TrainStats(iters, wcss, empties, tr))
