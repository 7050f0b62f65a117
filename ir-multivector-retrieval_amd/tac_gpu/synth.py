"""Synthetic PQ build workloads (host generator ``libtac_synth.so``).

Residual corpora follow one recipe: unit-sphere centres in R^dim, vectors
``normalize(centre_j + N(0, sigma^2 I))`` with j uniform or Zipf(s), residual
``vector - centre_j``.  Initial codebooks are the first ksub points of a
seeded shuffle, per subspace.
"""
from __future__ import annotations

import ctypes
import functools
import os
from dataclasses import dataclass

import numpy as np

from ._native import SYNTH_PATH


@dataclass(frozen=True)
class Workload:
    name: str
    n: int
    dim: int
    n_centers: int
    zipf: float        # 0: uniform centre popularity
    sigma: float
    m: int
    ksub: int
    iters: int
    seed: int = 0

    @property
    def dsub(self) -> int:
        return self.dim // self.m


# Small chunk (117,645 x 64, uniform over 10,240 centres) and the full corpus
# shape (1,521,797 x 64, Zipf 1.1 over 32,768 centres); both m=16, ksub=256,
# 20 Lloyd iterations.
WORKLOADS = {
    "chunk-117k": Workload("chunk-117k", 117_645, 64, 10_240, 0.0, 0.15, 16, 256, 20),
    "corpus-1.52m": Workload("corpus-1.52m", 1_521_797, 64, 32_768, 1.1, 0.15, 16, 256, 20),
    "corpus-1.52m-m32d2": Workload("corpus-1.52m-m32d2", 1_521_797, 64, 32_768, 1.1, 0.15, 32,
                                   256, 20),
    "corpus-1.52m-m8d8": Workload("corpus-1.52m-m8d8", 1_521_797, 64, 32_768, 1.1, 0.15, 8, 256,
                                  20),
    "corpus-1.52m-k1024": Workload("corpus-1.52m-k1024", 1_521_797, 64, 32_768, 1.1, 0.15, 16,
                                   1024, 20),
    # Paper-scale training sample: 60M residuals, Zipf 1.05 over 262,144
    # centres, sigma 0.12, 25 Lloyd iterations.
    "paper-60m": Workload("paper-60m", 60_000_000, 64, 262_144, 1.05, 0.12, 16, 256, 25),
    # Encode-only stream: 200M residuals generated as the paper-scale corpus,
    # encoded in 10M-vector chunks against fixed N(0, 0.05^2) codebooks.
    "stream-200m": Workload("stream-200m", 200_000_000, 64, 262_144, 1.05, 0.12, 16, 256, 0),
}


def _lib() -> ctypes.CDLL:
    if not SYNTH_PATH.exists():
        raise ImportError(f"{SYNTH_PATH} is not built")
    lib = ctypes.CDLL(os.fspath(SYNTH_PATH))
    vp, u64, u32 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32
    lib.tac_synth_centers.argtypes = [u64, u32, u32, vp]
    lib.tac_synth_residuals.argtypes = [u64, u64, u32, u32, vp, ctypes.c_double, ctypes.c_float,
                                        u64, vp, vp, u32]
    lib.tac_synth_shuffle_init.argtypes = [vp, u64, u32, u32, u32, u64, vp]
    lib.tac_synth_gauss_codebooks.argtypes = [u64, u32, u32, u32, ctypes.c_float, vp]
    lib.tac_synth_shuffle_prefix.argtypes = [u64, u64, u32, vp]
    for f in (lib.tac_synth_centers, lib.tac_synth_residuals, lib.tac_synth_shuffle_init,
              lib.tac_synth_gauss_codebooks, lib.tac_synth_shuffle_prefix):
        f.restype = ctypes.c_int
    return lib


_L = None


def lib() -> ctypes.CDLL:
    global _L
    if _L is None:
        _L = _lib()
    return _L


def _p(a: np.ndarray) -> ctypes.c_void_p:
    return ctypes.c_void_p(a.ctypes.data)


@functools.lru_cache(maxsize=4)
def _centers(seed: int, n_centers: int, dim: int) -> np.ndarray:
    out = np.empty((n_centers, dim), dtype=np.float32)
    assert lib().tac_synth_centers(seed, n_centers, dim, _p(out)) == 0
    out.setflags(write=False)
    return out


def centers(seed: int, n_centers: int, dim: int) -> np.ndarray:
    """Unit-sphere centres (cached: chunked generation reuses them)."""
    return _centers(seed, n_centers, dim).copy()


def residuals(w: Workload, n: int | None = None, first: int = 0, threads: int | None = None,
              with_ids: bool = False):
    """Residual rows first .. first+n-1 of workload w (default: all of it)."""
    n = w.n if n is None else n
    c = _centers(w.seed, w.n_centers, w.dim)
    out = np.empty((n, w.dim), dtype=np.float32)
    ids = np.empty(n, dtype=np.uint32) if with_ids else None
    t = threads or min(16, os.cpu_count() or 1)
    assert lib().tac_synth_residuals(w.seed, n, w.dim, w.n_centers, _p(c), w.zipf, w.sigma, first,
                                     _p(out), _p(ids) if ids is not None else None, t) == 0
    return (out, ids) if with_ids else out


def shuffle_init(x: np.ndarray, m: int, ksub: int, seed: int) -> np.ndarray:
    """[m][ksub][dsub] codebooks from the first ksub points of a seeded shuffle."""
    n, dim = x.shape
    out = np.empty((m, ksub, dim // m), dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert lib().tac_synth_shuffle_init(_p(x), n, dim, m, ksub, seed, _p(out)) == 0
    return out


def _gpu_lib() -> ctypes.CDLL:
    path = SYNTH_PATH.with_name("libtac_synth_gpu.so")
    if not path.exists():
        raise ImportError(f"{path} is not built")
    lib = ctypes.CDLL(os.fspath(path))
    vp, u64, u32 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32
    lib.tac_synth_residuals_device.argtypes = [u64, u64, u32, u32, vp, vp, ctypes.c_float, u64,
                                               vp, vp]
    lib.tac_synth_residuals_device.restype = ctypes.c_int
    return lib


_GL = None


def zipf_cdf(n_centers: int, s: float) -> np.ndarray:
    """Normalised Zipf(s) CDF over centres, accumulated in index order as
    synth.c does."""
    acc = np.cumsum(np.power(np.arange(1, n_centers + 1, dtype=np.float64), -s))
    cdf = acc / acc[-1]
    cdf[-1] = 1.0
    return cdf


class DeviceCorpus:
    """Residual rows of a workload generated on the device (the kernel form of
    the same generator), for inputs too large to generate on the host."""

    def __init__(self, w: Workload):
        global _GL
        from . import device
        if _GL is None:
            _GL = _gpu_lib()
        self.w = w
        self.centers = device.DeviceArray.from_host(
            np.ascontiguousarray(_centers(w.seed, w.n_centers, w.dim)))
        self.cdf = (device.DeviceArray.from_host(zipf_cdf(w.n_centers, w.zipf))
                    if w.zipf > 0 else None)

    def fill(self, out, n: int, first: int = 0) -> None:
        """Rows first .. first+n-1 into the device array `out` ([>= n][dim] f32)."""
        from . import device
        assert out.nbytes >= n * self.w.dim * 4
        st = _GL.tac_synth_residuals_device(
            self.w.seed, n, self.w.dim, self.w.n_centers, self.centers.ptr,
            self.cdf.ptr if self.cdf is not None else None, self.w.sigma, first, out.ptr, None)
        assert st == 0, st
        device.synchronize()

    def shuffle_init(self, x, n: int, m: int, ksub: int, seed: int) -> np.ndarray:
        """shuffle_init's codebooks, read from the device rows x[0 .. n)."""
        dim = self.w.dim
        dsub = dim // m
        out = np.empty((m, ksub, dsub), np.float32)
        pre = np.empty(ksub, np.uint64)
        row = np.empty(dim, np.float32)
        for mm in range(m):
            assert lib().tac_synth_shuffle_prefix(seed + mm, n, ksub, _p(pre)) == 0
            for c in range(ksub):
                x.read_row(int(pre[c]), row)
                out[mm, c] = row[mm * dsub:(mm + 1) * dsub]
        return out

    def free(self) -> None:
        self.centers.free()
        if self.cdf is not None:
            self.cdf.free()


def gauss_codebooks(seed: int, m: int, ksub: int, dsub: int, sigma: float) -> np.ndarray:
    out = np.empty((m, ksub, dsub), dtype=np.float32)
    assert lib().tac_synth_gauss_codebooks(seed, m, ksub, dsub, sigma, _p(out)) == 0
    return out


def workload(name: str, n: int | None = None):
    """(residuals, init codebooks) of a named workload, optionally truncated to n rows."""
    w = WORKLOADS[name]
    x = residuals(w, n)
    return w, x, shuffle_init(x, w.m, w.ksub, w.seed)


# Token-aware clustering input: token id = a Zipf draw over `vocab` themes
# (unit-sphere centres), vector = theme + residual noise scaled per token by
# 0.5 + (id mod 7) / 4, so that token spreads differ.
TAC_WORKLOADS = {
    # 1.52M token vectors of dim 64 over a BERT-sized vocabulary (30,522 ids),
    # Zipf 1.05, kappa_total 40,960: ~29k micro tokens, ~500 active tokens
    # with up to ~1,000 centroids, 1.1e8 (row, centroid) pairs per iteration.
    "tac-1.52m": dict(n=1_521_797, dim=64, vocab=30_522, zipf=1.05, sigma=0.15, seed=0,
                      kappa_total=40_960),
}


def tac_vectors(n: int, dim: int, vocab: int, zipf: float, sigma: float, seed: int):
    """(token_ids u32 [n], vectors f32 [n][dim]) of a synthetic token dump."""
    w = Workload("tac", n, dim, vocab, zipf, sigma, 16, 256, 1, seed)
    r, ids = residuals(w, n, with_ids=True)
    c = _centers(seed, vocab, dim)
    scale = (0.5 + (ids % 7).astype(np.float32) / 4.0).astype(np.float32)
    v = (c[ids] + r * scale[:, None]).astype(np.float32)
    return ids, v


def tac_workload(name: str, n: int | None = None):
    d = TAC_WORKLOADS[name]
    ids, v = tac_vectors(n or d["n"], d["dim"], d["vocab"], d["zipf"], d["sigma"], d["seed"])
    return d, ids, v
