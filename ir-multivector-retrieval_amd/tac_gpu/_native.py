"""ctypes binding of ``libtac_gpu.so`` (the gfx950 PQ build library).

The library is built in-tree into ``lib/`` next to this package.  There is no
fallback: if the shared object is missing, importing this module raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent.parent
LIB_DIR = PKG_ROOT / "lib"
LIB_PATH = LIB_DIR / "libtac_gpu.so"
SYNTH_PATH = LIB_DIR / "libtac_synth.so"

c_f32_p = ctypes.POINTER(ctypes.c_float)
c_u32_p = ctypes.POINTER(ctypes.c_uint32)
c_void_p = ctypes.c_void_p
c_u64 = ctypes.c_uint64
c_u32 = ctypes.c_uint32
c_int = ctypes.c_int


class TrainExtras(ctypes.Structure):
    _fields_ = [
        ("iters_run", c_u32_p),
        ("wcss", c_f32_p),
        ("empties", c_u32_p),
        ("trace", c_f32_p),
    ]


class KernelTime(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 96), ("ms", ctypes.c_double), ("launches", c_u64)]


class DeviceInfo(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 256),
        ("arch", ctypes.c_char * 64),
        ("compute_units", c_int),
        ("clock_khz", c_int),
        ("global_mem_bytes", c_u64),
        ("lds_bytes_per_block", c_u64),
    ]


class Profile(ctypes.Structure):
    _fields_ = [
        ("transpose_ms", ctypes.c_double),
        ("transpose_launches", c_u64),
        ("assign_ms", ctypes.c_double),
        ("assign_launches", c_u64),
        ("update_ms", ctypes.c_double),
        ("update_iters", c_u64),
        ("encode_ms", ctypes.c_double),
        ("encode_launches", c_u64),
        ("exact_rescans", c_u64),
        ("residual_ms", ctypes.c_double),
        ("residual_launches", c_u64),
        ("crc_ms", ctypes.c_double),
        ("crc_launches", c_u64),
        ("refine_ms", ctypes.c_double),
        ("refine_launches", c_u64),
        ("cluster_kpp_ms", ctypes.c_double),
        ("cluster_lloyd_ms", ctypes.c_double),
        ("cluster_calls", c_u64),
        ("cluster_prep_ms", ctypes.c_double),
        ("cluster_call_ms", ctypes.c_double),
        ("cand_vectors", c_u64),
        ("cand_deferred", c_u64),
        ("cand_assign_ms", ctypes.c_double),
        ("cand_assign_iters", c_u64),
        ("train_streams", c_u64),
        ("cell_subspaces", c_u64),
        ("screen_vectors", c_u64),
        ("screen_deferred", c_u64),
    ]


class ClusterParams(ctypes.Structure):
    """tac_cluster_params (ClusteringParams, src/tac/tac.zig:35-58)."""

    _fields_ = [
        ("kappa_total", c_u32), ("mu", c_u32), ("tau", c_u32), ("epsilon", c_u32),
        ("theta", c_u32), ("max_iters", c_u32), ("tol", ctypes.c_float), ("seed", c_u64),
        ("n_threads", c_u32),
    ]


class DocIndex(ctypes.Structure):
    """tac_doc_index: the parts of a parsed .tac Index that refine reads."""

    _fields_ = [
        ("dim", c_u32), ("kappa", c_u32), ("m", c_u32), ("ksub", c_u32),
        ("n_docs", c_u64), ("n_tokens", c_u64), ("payload_len", c_u64),
        ("centroids", c_void_p), ("doc_index", c_void_p), ("doc_payload", c_void_p),
        ("doc_token_offsets", c_void_p), ("residual_norms", c_void_p),
    ]


# Every exported symbol with (restype, argtypes).  include/tac_gpu.h is the
# source of truth; tests check that this table and the header agree.
SIGNATURES = {
    "tac_gpu_strerror": (ctypes.c_char_p, [c_int]),
    "tac_gpu_last_error": (ctypes.c_char_p, []),
    "tac_gpu_device_count": (c_int, [ctypes.POINTER(c_int)]),
    "tac_gpu_get_device_info": (c_int, [c_int, ctypes.POINTER(DeviceInfo)]),
    "tac_gpu_set_device": (c_int, [c_int]),
    "tac_gpu_set_lane_count": (c_int, [c_u32]),
    "tac_gpu_get_lane_count": (c_int, [ctypes.POINTER(c_u32)]),
    "tac_gpu_malloc": (c_int, [ctypes.POINTER(c_void_p), c_u64]),
    "tac_gpu_free": (c_int, [c_void_p]),
    "tac_gpu_memcpy_htod": (c_int, [c_void_p, c_void_p, c_u64]),
    "tac_gpu_memcpy_dtoh": (c_int, [c_void_p, c_void_p, c_u64]),
    "tac_gpu_memcpy_dtod": (c_int, [c_void_p, c_void_p, c_u64]),
    "tac_gpu_synchronize": (c_int, []),
    "tac_gpu_release_workspace": (c_int, []),
    "tac_pq_train": (
        c_int,
        [c_void_p, c_u64, c_u32, c_u32, c_u32, c_void_p, c_u64, c_u32, ctypes.c_float,
         c_void_p, ctypes.POINTER(TrainExtras)],
    ),
    "tac_pq_train_device": (
        c_int,
        [c_void_p, c_u64, c_u32, c_u32, c_u32, c_void_p, c_u64, c_u32, ctypes.c_float,
         c_void_p, ctypes.POINTER(TrainExtras), c_void_p],
    ),
    "tac_pq_train_encode_device": (
        c_int,
        [c_void_p, c_u64, c_u32, c_u32, c_u32, c_void_p, c_u64, c_u32, ctypes.c_float,
         c_void_p, c_void_p, ctypes.POINTER(TrainExtras), c_void_p],
    ),
    "tac_pq_encode": (c_int, [c_void_p, c_u64, c_u32, c_u32, c_u32, c_void_p, c_void_p]),
    "tac_pq_encode_device": (
        c_int, [c_void_p, c_u64, c_u32, c_u32, c_u32, c_void_p, c_void_p, c_void_p]),
    "tac_pq_encode_device_noalloc": (
        c_int, [c_void_p, c_u64, c_u32, c_u32, c_u32, c_void_p, c_void_p, c_void_p]),
    "tac_pq_decode": (c_int, [c_void_p, c_u64, c_u32, c_u32, c_u32, c_void_p, c_void_p]),
    "tac_kmeans_fit": (
        c_int,
        [c_void_p, c_u64, c_u32, c_u32, c_u32, ctypes.c_float, c_u64, c_void_p, c_void_p,
         c_void_p, c_f32_p, c_u32_p],
    ),
    "tac_residuals": (
        c_int, [c_void_p, c_u64, c_u32, c_void_p, c_u32, c_void_p, c_void_p, c_void_p]),
    "tac_residuals_device": (
        c_int, [c_void_p, c_u64, c_u32, c_void_p, c_u32, c_void_p, c_void_p, c_void_p, c_void_p]),
    "tac_doc_payload_bytes": (c_int, [c_void_p, c_u64, c_u32, c_u32, ctypes.POINTER(c_u64)]),
    "tac_write_doc_layouts": (
        c_int, [c_void_p, c_u64, c_u64, c_void_p, c_void_p, c_u32, c_u32, c_void_p, c_void_p,
                c_u64]),
    "tac_write_doc_layouts_device": (
        c_int, [c_void_p, c_u64, c_u64, c_void_p, c_void_p, c_u32, c_u32, c_void_p, c_void_p,
                c_u64, c_void_p]),
    "tac_crc32": (c_int, [c_void_p, c_u64, c_u32_p]),
    "tac_crc32_device": (c_int, [c_void_p, c_u64, c_u32_p, c_void_p]),
    "tac_pq_distance_table": (
        c_int, [c_void_p, c_u32, c_u32, c_u32, c_u32, c_void_p, c_void_p, c_u64]),
    "tac_pq_distance_table_device": (
        c_int, [c_void_p, c_u32, c_u32, c_u32, c_u32, c_void_p, c_void_p, c_u64, c_void_p]),
    "tac_refine": (
        c_int, [ctypes.POINTER(DocIndex), c_void_p, c_u64, c_void_p, c_u32, c_void_p, c_u32,
                c_void_p]),
    "tac_refine_device": (
        c_int, [ctypes.POINTER(DocIndex), c_void_p, c_u64, c_void_p, c_u32, c_void_p, c_u32,
                c_void_p, c_void_p]),
    "tac_cluster_flat": (
        c_int, [c_void_p, c_u64, c_void_p, c_u64, c_u32, ctypes.POINTER(ClusterParams), c_void_p,
                c_void_p, c_void_p, c_u64, c_f32_p, ctypes.POINTER(c_u64)]),
    "tac_cluster_flat_device": (
        c_int, [c_void_p, c_u64, c_void_p, c_u64, c_u32, ctypes.POINTER(ClusterParams), c_void_p,
                c_void_p, c_void_p, c_u64, c_f32_p, ctypes.POINTER(c_u64)]),
    "tac_gpu_profile_enable": (c_int, [c_int]),
    "tac_gpu_profile_read": (c_int, [ctypes.POINTER(Profile), c_int]),
    "tac_gpu_profile_kernels": (
        c_int, [ctypes.POINTER(KernelTime), c_u32, ctypes.POINTER(c_u32), c_int]),
}

STATUS_NAMES = [
    "Ok", "DimNotDivisibleByM", "DimMismatch", "EmptyCorpus", "OutBufferWrongSize",
    "NQMismatch", "KmeansBudgetTooSmall", "EmptyVectorSet", "EmptyDistribution", "NonFinite",
    "AllZero", "OutOfMemory", "NoDevice", "HipError", "InvalidArgument", "Unsupported",
    "QueryShapeMismatch", "TableSizeMismatch", "DocOutOfRange", "DocLayoutCorrupt",
    "BufferTooSmall", "BudgetTooSmall", "BudgetTooLarge", "InvalidThresholds", "EmptyTokenDump",
]


def _load() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
            "(or `make -C ir-multivector-retrieval_amd`) first")
    lib = ctypes.CDLL(os.fspath(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()
