"""tac_gpu — MI355X (gfx950) product-quantization build path.

Drop-in for the reference's ``tac.index.pq`` (``train``, ``PQ.encode``,
``PQ.decode``, ``PQ.buildDistanceTable``), ``tac.tac.kmeans.fit``, the
residual stage and PQ-carrying .tac sections of ``storage.build``, the
refine phase of retrieval, and ``tac.tac.clusterFlat`` (token-aware
clustering); every call runs hand-written HIP kernels through the C ABI
declared in include/tac_gpu.h.
"""
from . import errors, kmeans, pq, retrieval, storage, tac  # noqa: F401
from ._native import LIB_PATH, lib  # noqa: F401
from .pq import PQ, PQ_BITS, PQ_CENTROIDS, PQ_M, TOL_NEVER, train  # noqa: F401
