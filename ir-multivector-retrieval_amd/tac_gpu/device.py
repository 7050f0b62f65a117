"""Device memory, device-resident entry points and kernel timing.

Used by callers that keep residuals resident in HBM across train and encode
(the way storage.build chains them, src/index/storage.zig:378-401) and by
the benchmark.  Memory comes from the library's own HIP runtime, so no other
GPU framework has to be loaded in the process.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import errors
from ._native import DeviceInfo, Profile, TrainExtras, lib
from .pq import code_dtype


def device_count() -> int:
    c = ctypes.c_int(0)
    lib.tac_gpu_device_count(ctypes.byref(c))
    return int(c.value)


def device_info(device: int = 0) -> dict:
    info = DeviceInfo()
    errors.check(lib.tac_gpu_get_device_info(device, ctypes.byref(info)))
    return {
        "name": info.name.decode(errors="replace"),
        "arch": info.arch.decode(errors="replace"),
        "compute_units": info.compute_units,
        "clock_khz": info.clock_khz,
        "global_mem_bytes": int(info.global_mem_bytes),
    }


def set_lane_count(lanes: int) -> None:
    """vec.lane_count of the host whose reference build is being matched
    (src/util/vec.zig:16): 16 (AVX-512, the default), 8 (AVX2) or 4 (NEON)."""
    errors.check(lib.tac_gpu_set_lane_count(lanes))


def lane_count() -> int:
    v = ctypes.c_uint32(0)
    errors.check(lib.tac_gpu_get_lane_count(ctypes.byref(v)))
    return int(v.value)


class lanes:
    """Within the block the library's generic vec path uses `n` lanes."""

    def __init__(self, n: int):
        self.n = n

    def __enter__(self):
        self.prev = lane_count()
        set_lane_count(self.n)
        return self

    def __exit__(self, *exc):
        set_lane_count(self.prev)
        return False


def synchronize() -> None:
    errors.check(lib.tac_gpu_synchronize())


class DeviceArray:
    """A flat device allocation with a numpy dtype and shape."""

    def __init__(self, shape, dtype):
        self.shape = tuple(int(s) for s in np.atleast_1d(shape)) if not isinstance(shape, tuple) \
            else tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = ctypes.c_void_p()
        errors.check(lib.tac_gpu_malloc(ctypes.byref(p), self.nbytes))
        self.ptr = p

    @classmethod
    def from_host(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        errors.check(lib.tac_gpu_memcpy_htod(d.ptr, ctypes.c_void_p(a.ctypes.data), a.nbytes))
        return d

    def copy_from_host(self, a: np.ndarray) -> None:
        """Overwrite the leading a.nbytes bytes with host data."""
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise errors.OutBufferWrongSize(f"{a.nbytes} bytes into a {self.nbytes}-byte buffer")
        errors.check(lib.tac_gpu_memcpy_htod(self.ptr, ctypes.c_void_p(a.ctypes.data), a.nbytes))

    def read_row(self, i: int, out: np.ndarray) -> None:
        """Copy row i of a 2-D array into the host array `out`."""
        nb = out.nbytes
        errors.check(lib.tac_gpu_memcpy_dtoh(ctypes.c_void_p(out.ctypes.data),
                                             ctypes.c_void_p(self.ptr.value + i * nb), nb))

    def to_host(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        errors.check(lib.tac_gpu_memcpy_dtoh(ctypes.c_void_p(out.ctypes.data), self.ptr,
                                             self.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            lib.tac_gpu_free(self.ptr)
            self.ptr = ctypes.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def train_device(x: DeviceArray, n: int, dim: int, m: int, ksub: int, init: DeviceArray | None,
                 out: DeviceArray, max_iters: int, tol: float, stats: bool = False,
                 seed: int = 0, trace: bool = False):
    """tac_pq_train_device on resident buffers; optional per-subspace stats
    (iters_run, wcss, empties) and, with trace, the codebooks after every
    iteration as a fourth array [max_iters][m][ksub][dsub].
    init None seeds every subspace with k-means++ (seed +% subspace)."""
    ex = None
    arrays = None
    if stats or trace:
        arrays = (np.zeros(m, np.uint32), np.zeros(m, np.float32), np.zeros(m, np.uint32))
        tr = None
        if trace:
            tr = np.zeros((max_iters, m, ksub, dim // m), np.float32)
            arrays = arrays + (tr,)
        ex = TrainExtras(arrays[0].ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                         arrays[1].ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                         arrays[2].ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                         None if tr is None else tr.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    errors.check(lib.tac_pq_train_device(x.ptr, n, dim, m, ksub,
                                         init.ptr if init is not None else None,
                                         seed & (2**64 - 1), max_iters, tol, out.ptr,
                                         ctypes.byref(ex) if ex else None, None))
    return arrays


def train_encode_device(x: DeviceArray, n: int, dim: int, m: int, ksub: int,
                        init: DeviceArray | None, out: DeviceArray, codes: DeviceArray,
                        max_iters: int, tol: float, seed: int = 0, trace: bool = False):
    """tac_pq_train_encode_device: train (as train_device) and encode the same
    resident residuals into `codes` [n][m], as storage.build chains them.
    Returns the per-subspace stats (and trace) as train_device does."""
    assert codes.dtype == code_dtype(ksub)
    arrays = (np.zeros(m, np.uint32), np.zeros(m, np.float32), np.zeros(m, np.uint32))
    tr = None
    if trace:
        tr = np.zeros((max_iters, m, ksub, dim // m), np.float32)
        arrays = arrays + (tr,)
    ex = TrainExtras(arrays[0].ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                     arrays[1].ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                     arrays[2].ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                     None if tr is None else tr.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    errors.check(lib.tac_pq_train_encode_device(x.ptr, n, dim, m, ksub,
                                                init.ptr if init is not None else None,
                                                seed & (2**64 - 1), max_iters, tol, out.ptr,
                                                codes.ptr, ctypes.byref(ex), None))
    return arrays


def encode_device(x: DeviceArray, n: int, dim: int, m: int, ksub: int, cb: DeviceArray,
                  codes: DeviceArray) -> None:
    assert codes.dtype == code_dtype(ksub)
    errors.check(lib.tac_pq_encode_device(x.ptr, n, dim, m, ksub, cb.ptr, codes.ptr, None))


def residuals_device(v: DeviceArray, n: int, dim: int, cent: DeviceArray, n_cent: int,
                     assign: DeviceArray, out: DeviceArray, norms: DeviceArray) -> None:
    """tac_residuals_device on resident buffers (out may be v itself)."""
    errors.check(lib.tac_residuals_device(v.ptr, n, dim, cent.ptr, n_cent, assign.ptr, out.ptr,
                                          norms.ptr, None))


@dataclass
class KernelTimes:
    transpose_ms: float
    transpose_launches: int
    assign_ms: float
    assign_launches: int
    update_ms: float
    update_iters: int
    encode_ms: float
    encode_launches: int
    exact_rescans: int
    residual_ms: float = 0.0
    residual_launches: int = 0
    crc_ms: float = 0.0
    crc_launches: int = 0
    refine_ms: float = 0.0
    refine_launches: int = 0
    cluster_kpp_ms: float = 0.0
    cluster_lloyd_ms: float = 0.0
    cluster_calls: int = 0
    cluster_prep_ms: float = 0.0
    cluster_call_ms: float = 0.0
    cand_vectors: int = 0
    cand_deferred: int = 0
    cand_assign_ms: float = 0.0
    cand_assign_iters: int = 0
    train_streams: int = 1
    cell_subspaces: int = 0
    screen_vectors: int = 0
    screen_deferred: int = 0


def profile_enable(on: bool = True) -> None:
    lib.tac_gpu_profile_enable(1 if on else 0)


def profile_read(reset: bool = True) -> KernelTimes:
    p = Profile()
    errors.check(lib.tac_gpu_profile_read(ctypes.byref(p), 1 if reset else 0))
    return KernelTimes(p.transpose_ms, p.transpose_launches, p.assign_ms, p.assign_launches,
                       p.update_ms, p.update_iters, p.encode_ms, p.encode_launches,
                       p.exact_rescans, p.residual_ms, p.residual_launches, p.crc_ms,
                       p.crc_launches, p.refine_ms, p.refine_launches, p.cluster_kpp_ms,
                       p.cluster_lloyd_ms, p.cluster_calls, p.cluster_prep_ms,
                       p.cluster_call_ms, p.cand_vectors, p.cand_deferred, p.cand_assign_ms,
                       p.cand_assign_iters, p.train_streams, p.cell_subspaces,
                       p.screen_vectors, p.screen_deferred)


def profile_kernels(reset: bool = True) -> dict:
    """Per-kernel HIP-event times recorded while profiling was enabled:
    {kernel name: (total ms, launches)}."""
    from ._native import KernelTime
    count = ctypes.c_uint32(0)
    errors.check(lib.tac_gpu_profile_kernels(None, 0, ctypes.byref(count), 0))
    arr = (KernelTime * max(count.value, 1))()
    errors.check(lib.tac_gpu_profile_kernels(arr, count.value, ctypes.byref(count),
                                             1 if reset else 0))
    return {k.name.decode(): (float(k.ms), int(k.launches)) for k in arr[:count.value]}
