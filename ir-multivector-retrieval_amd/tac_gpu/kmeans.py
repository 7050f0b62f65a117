"""Python mirror of the reference's ``tac.tac.kmeans`` (src/tac/kmeans.zig).

``fit`` keeps the reference's parameters (KMeansParams, kmeans.zig:28-41) and
result (KMeansResult, :43-54); the Lloyd loop runs on the GPU through
``tac_kmeans_fit``.  ``init_centroids`` replaces k-means++ seeding.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import errors
from ._native import lib


@dataclass
class KMeansResult:
    centroids: np.ndarray    # float32 [k * dim]
    assignments: np.ndarray  # uint32 [n]
    wcss: float
    iters_run: int


def fit(vectors: np.ndarray, dim: int, k: int, *, seed: int = 0, max_iters: int = 25,
        tol: float = 1e-4, n_threads: int = 1,
        init_centroids: np.ndarray | None = None) -> KMeansResult:
    del n_threads  # the GPU assigns every vector at once
    v = np.ascontiguousarray(vectors, dtype=np.float32).reshape(-1)
    # src/tac/kmeans.zig:73-76
    if k == 0:
        raise errors.KmeansBudgetTooSmall("KmeansBudgetTooSmall")
    if dim == 0:
        raise errors.DimMismatch("DimMismatch")
    if v.size == 0:
        raise errors.EmptyVectorSet("EmptyVectorSet")
    if v.size % dim != 0:
        raise errors.DimMismatch("DimMismatch")
    n = v.size // dim
    cent = np.empty(k * dim, dtype=np.float32)
    assign = np.empty(n, dtype=np.uint32)
    init = None
    if init_centroids is not None:
        init = np.ascontiguousarray(init_centroids, dtype=np.float32).reshape(-1)
        if init.size != cent.size:
            raise errors.DimMismatch("DimMismatch")
    wcss = ctypes.c_float(0.0)
    iters = ctypes.c_uint32(0)
    errors.check(lib.tac_kmeans_fit(
        ctypes.c_void_p(v.ctypes.data), n, dim, k, max_iters, tol, seed & (2**64 - 1),
        None if init is None else ctypes.c_void_p(init.ctypes.data),
        ctypes.c_void_p(cent.ctypes.data), ctypes.c_void_p(assign.ctypes.data),
        ctypes.byref(wcss), ctypes.byref(iters)))
    return KMeansResult(cent, assign, float(wcss.value), int(iters.value))
