"""Token-aware clustering on the device: the mirror of the reference's
``tac.tac`` (src/tac/tac.zig) — ``ClusteringParams`` (:35-58),
``ClusteringResult`` (:408-427) and ``clusterFlat`` (:563-830) — over
``tac_cluster_flat`` of include/tac_gpu.h.  Errors raise the
ClusteringError / KMeansError classes of ``tac_gpu.errors``."""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import errors
from ._native import ClusterParams, lib

# src/constants.zig: TAC_MU, TAC_TAU, TAC_EPSILON, TAC_THETA
TAC_MU, TAC_TAU, TAC_EPSILON, TAC_THETA = 128, 256, 4, 39


@dataclass
class ClusteringParams:
    kappa_total: int
    seed: int
    mu: int = TAC_MU
    tau: int = TAC_TAU
    epsilon: int = TAC_EPSILON
    theta: int = TAC_THETA
    max_iters: int = 25
    tol: float = 1e-4
    n_threads: int = 1  # groups wcss_total only (tac.zig:688-820)

    def native(self) -> ClusterParams:
        return ClusterParams(self.kappa_total, self.mu, self.tau, self.epsilon, self.theta,
                             self.max_iters, self.tol, self.seed & (2**64 - 1),
                             max(int(self.n_threads), 1))


@dataclass
class ClusteringResult:
    centroids: np.ndarray        # kappa_total x dim, token-id order
    assignments: np.ndarray      # n_tokens global centroid ids
    kappa_per_token: np.ndarray  # n_distinct = max(token id) + 1
    wcss_total: float


def cluster_flat(token_ids, vectors, dim: int, p: ClusteringParams) -> ClusteringResult:
    """clusterFlat: per-token budgets, then kmeans.fit per token, on the GPU.
    `vectors` may also be a device.DeviceArray of n_tokens * dim floats
    (tac_cluster_flat_device: no upload)."""
    ids = np.ascontiguousarray(token_ids, dtype=np.uint32).reshape(-1)
    on_device = hasattr(vectors, "ptr") and hasattr(vectors, "nbytes")
    if on_device:
        # the device entry point reads f32 values (its length check, in the
        # reference's error order, sees nbytes / 4 of them); an array of
        # another dtype is refused before any call, since an f64 or integer
        # array would otherwise be read as f32 bits
        if np.dtype(getattr(vectors, "dtype", np.float32)) != np.float32:
            raise errors.InvalidArgument("device vectors must be float32")
        vptr, vlen = vectors.ptr, vectors.nbytes // 4
    else:
        v = np.ascontiguousarray(vectors, dtype=np.float32).reshape(-1)
        vptr, vlen = v.ctypes.data_as(ctypes.c_void_p), v.size
    nd = int(ids.max()) + 1 if ids.size else 1
    cent = np.zeros(max(p.kappa_total * max(dim, 1), 1), np.float32)
    asg = np.zeros(max(ids.size, 1), np.uint32)
    kpt = np.zeros(nd, np.uint32)
    wcss = ctypes.c_float(0.0)
    nd_out = ctypes.c_uint64(0)
    prm = p.native()
    fn = lib.tac_cluster_flat_device if on_device else lib.tac_cluster_flat
    errors.check(fn(
        ids.ctypes.data_as(ctypes.c_void_p), ids.size, vptr, vlen,
        dim, ctypes.byref(prm), cent.ctypes.data_as(ctypes.c_void_p),
        asg.ctypes.data_as(ctypes.c_void_p), kpt.ctypes.data_as(ctypes.c_void_p), nd,
        ctypes.byref(wcss), ctypes.byref(nd_out)))
    return ClusteringResult(cent[:p.kappa_total * dim].reshape(p.kappa_total, dim),
                            asg[:ids.size], kpt, float(np.float32(wcss.value)))
