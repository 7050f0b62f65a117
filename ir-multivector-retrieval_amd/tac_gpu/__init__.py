"""tac_gpu — MI355X (gfx950) product-quantization build path.

Drop-in for the reference's ``tac.index.pq`` (``train``, ``PQ.encode``,
``PQ.decode``), ``tac.tac.kmeans.fit`` and the residual stage of
``storage.build``; every call runs hand-written HIP kernels through the C ABI
declared in include/tac_gpu.h.
"""
from . import errors, kmeans, pq, storage  # noqa: F401
from ._native import LIB_PATH, lib  # noqa: F401
from .pq import PQ, PQ_BITS, PQ_CENTROIDS, PQ_M, TOL_NEVER, train  # noqa: F401
