"""The recall worker's exact maximum-inner-product archive (``ArchiveIndex`` of
src/lazy_recall/recall/cpu_worker.py:94-134, over ``HeadArchive`` :17-92) on the host, without
faiss: liblazyrecall_archive.so (csrc/archive.cpp), loaded with ctypes. Same constructor,
methods, properties, argument shapes, results and error messages as the reference class; the
CPU worker process (cpu_worker.py:136-182) can construct it in place of its own.

Equal inner products rank in the order the rows were indexed (the scan order of a faiss flat
index); faiss itself leaves the order of exact ties unspecified.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

LIBRARY_PATH = Path(__file__).resolve().parent / "liblazyrecall_archive.so"

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
SIGNATURES = {
    "lra_last_error": ([], ctypes.c_char_p),
    "lra_create": ([_I64, _I64, _I64, _I64, ctypes.c_int], _P),
    "lra_destroy": ([_P], None),
    "lra_add": ([_P, _P, _P, _I64], ctypes.c_int),
    "lra_remove": ([_P, _P, _I64], ctypes.c_int),
    "lra_search": ([_P, _P, _I64, _P, _P, _P], ctypes.c_int),
    "lra_size": ([_P], _I64),
    "lra_dropped": ([_P], _I64),
}
_library = None


def load() -> ctypes.CDLL:
    global _library
    if _library is None:
        if not LIBRARY_PATH.exists():
            raise RuntimeError(f"{LIBRARY_PATH.name} is not built; run "
                               "`python -m code_for_iclr27_amd.build`")
        library = ctypes.CDLL(os.fspath(LIBRARY_PATH))
        for name, (argtypes, restype) in SIGNATURES.items():
            function = getattr(library, name)
            function.argtypes, function.restype = argtypes, restype
        _library = library
    return _library


def _raise(status: int) -> None:
    if status:
        raise ValueError(load().lra_last_error().decode())


class ArchiveIndex:
    """cpu_worker.py:94-134: one bounded exact-MIPS archive per (layer, KV head)."""

    def __init__(self, layers, heads, dimension, threads, capacity):
        self.layers, self.heads, self.dimension = int(layers), int(heads), int(dimension)
        self._handle = load().lra_create(self.layers, self.heads, self.dimension, int(capacity),
                                         int(threads))
        if not self._handle:
            raise ValueError(load().lra_last_error().decode())

    def __del__(self):
        handle, self._handle = getattr(self, "_handle", None), None
        if handle and _library is not None:
            _library.lra_destroy(handle)

    @property
    def size(self):
        return int(load().lra_size(self._handle))

    @property
    def dropped(self):
        return int(load().lra_dropped(self._handle))

    def add(self, metadata, payload):
        metadata = np.ascontiguousarray(metadata, dtype=np.int64)
        payload = np.ascontiguousarray(payload, dtype=np.uint16)
        if metadata.shape != (len(payload), 3) or payload.shape[1:] != (2, self.dimension):
            raise ValueError("Archive payload shape mismatch")
        _raise(load().lra_add(self._handle, metadata.ctypes.data, payload.ctypes.data,
                              len(metadata)))

    def remove(self, metadata):
        metadata = np.ascontiguousarray(np.asarray(metadata, dtype=np.int64).reshape(-1, 3))
        _raise(load().lra_remove(self._handle, metadata.ctypes.data, len(metadata)))

    def search(self, queries, topk):
        segments = self.layers * self.heads
        queries = np.ascontiguousarray(np.asarray(queries, dtype=np.float32).reshape(-1, self.dimension))
        if len(queries) < segments:
            raise ValueError("One query per (layer, head) is required")
        topk = int(topk)
        metadata = np.empty((segments * topk, 3), dtype=np.int64)
        payload = np.empty((segments * topk, 2, self.dimension), dtype=np.uint16)
        count = ctypes.c_int64(0)
        _raise(load().lra_search(self._handle, queries.ctypes.data, topk, metadata.ctypes.data,
                                 payload.ctypes.data, ctypes.byref(count)))
        return metadata[:count.value].copy(), payload[:count.value].copy()
