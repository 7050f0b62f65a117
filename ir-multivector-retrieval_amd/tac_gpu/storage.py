"""Python mirror of the storage.build stages around the PQ build.

``residuals_and_norms`` is stage 2 of storage.build
(src/index/storage.zig:355-376), the per-token ``residualsAndNormsChunk``
(:255-278) run over every token at once on the GPU.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import errors
from ._native import lib


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
