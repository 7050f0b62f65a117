"""Python mirror of the query side that consumes PQ codes.

``DocIndex`` holds the sections of a parsed .tac Index that refine reads
(src/index/storage.zig:86-124): centroids, the per-document layouts written
by writeDocLayouts, the doc token offsets and the residual norms.
``refine`` is src/retrieval/refine.zig:83-145 for a batch of candidate
documents of one query, run on the GPU; its errors are RefineError's.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import errors
from ._native import DocIndex as _DocIndexC
from ._native import lib


def _ptr(a: np.ndarray) -> ctypes.c_void_p:
    return ctypes.c_void_p(a.ctypes.data)


@dataclass
class DocIndex:
    dim: int
    m: int
    ksub: int
    centroids: np.ndarray          # float32 [kappa][dim]
    doc_index: np.ndarray          # uint64 [n_docs + 1]
    doc_payload: np.ndarray        # uint8 per-doc layouts
    doc_token_offsets: np.ndarray  # uint64 [n_docs + 1]
    residual_norms: np.ndarray     # float32 [n_tokens]

    def __post_init__(self):
        self.centroids = np.ascontiguousarray(self.centroids, dtype=np.float32)
        self.doc_index = np.ascontiguousarray(self.doc_index, dtype=np.uint64)
        self.doc_payload = np.ascontiguousarray(self.doc_payload, dtype=np.uint8)
        self.doc_token_offsets = np.ascontiguousarray(self.doc_token_offsets, dtype=np.uint64)
        self.residual_norms = np.ascontiguousarray(self.residual_norms, dtype=np.float32)

    @property
    def n_docs(self) -> int:
        return self.doc_index.size - 1

    def c_view(self) -> _DocIndexC:
        return _DocIndexC(self.dim, self.centroids.size // self.dim, self.m, self.ksub,
                          self.n_docs, self.residual_norms.size, self.doc_payload.size,
                          _ptr(self.centroids), _ptr(self.doc_index),
                          _ptr(self.doc_payload) if self.doc_payload.size else None,
                          _ptr(self.doc_token_offsets), _ptr(self.residual_norms))


def refine(index: DocIndex, distance_table: np.ndarray, query_tokens: np.ndarray, n_q: int,
           doc_ids) -> np.ndarray:
    """Exact MaxSim scores (float32) of candidate documents `doc_ids`."""
    t = np.ascontiguousarray(distance_table, dtype=np.float32).reshape(-1)
    q = np.ascontiguousarray(query_tokens, dtype=np.float32).reshape(-1)
    if n_q == 0 or q.size != n_q * index.dim:
        raise errors.QueryShapeMismatch("QueryShapeMismatch")
    ids = np.ascontiguousarray(doc_ids, dtype=np.uint32).reshape(-1)
    out = np.empty(ids.size, dtype=np.float32)
    view = index.c_view()
    errors.check(lib.tac_refine(ctypes.byref(view), _ptr(t), t.size, _ptr(q), n_q,
                                _ptr(ids) if ids.size else None, ids.size,
                                _ptr(out) if ids.size else None))
    return out
