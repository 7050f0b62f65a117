"""Error types named after the reference's Zig error sets.

``PqError`` (src/index/pq.zig:32-38), ``KMeansError`` (src/tac/kmeans.zig:56-60)
and ``RngError`` (src/util/rng.zig:14-18) become one exception hierarchy; a
C-ABI status maps to exactly one class.
"""
from __future__ import annotations

from ._native import STATUS_NAMES, lib


class TacError(Exception):
    """Base class of every status the library reports."""

    status = -1


class DimNotDivisibleByM(TacError):
    status = 1


class DimMismatch(TacError):
    status = 2


class EmptyCorpus(TacError):
    status = 3


class OutBufferWrongSize(TacError):
    status = 4


class NQMismatch(TacError):
    status = 5


class KmeansBudgetTooSmall(TacError):
    status = 6


class EmptyVectorSet(TacError):
    status = 7


class EmptyDistribution(TacError):
    status = 8


class NonFinite(TacError):
    status = 9


class AllZero(TacError):
    status = 10


class OutOfMemory(TacError):
    status = 11


class NoDevice(TacError):
    status = 12


class HipError(TacError):
    status = 13


class InvalidArgument(TacError):
    status = 14


class Unsupported(TacError):
    status = 15


class QueryShapeMismatch(TacError):
    status = 16


class TableSizeMismatch(TacError):
    status = 17


class DocOutOfRange(TacError):
    status = 18


class DocLayoutCorrupt(TacError):
    status = 19


class BufferTooSmall(TacError):
    status = 20


class BudgetTooSmall(TacError):
    status = 21


class BudgetTooLarge(TacError):
    status = 22


class InvalidThresholds(TacError):
    status = 23


class EmptyTokenDump(TacError):
    status = 24


# StorageError (src/index/storage.zig:40-47) raised by the host-side .tac
# header and layout parser; no C-ABI status carries them.
class InvalidIndex(TacError):
    status = None


class UnsupportedVersion(TacError):
    status = None


class IndexCorrupt(TacError):
    status = None


_BY_STATUS = {cls.status: cls for cls in TacError.__subclasses__() if cls.status is not None}


def check(status: int) -> None:
    """Raise the exception class of a non-zero C-ABI status."""
    if status == 0:
        return
    cls = _BY_STATUS.get(status, TacError)
    name = STATUS_NAMES[status] if 0 <= status < len(STATUS_NAMES) else f"status {status}"
    detail = ""
    if status in (HipError.status, OutOfMemory.status, NoDevice.status):
        msg = lib.tac_gpu_last_error()
        if msg:
            detail = ": " + msg.decode(errors="replace")
    raise cls(name + detail)
