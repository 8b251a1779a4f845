"""ctypes wrapper over tile_oracle.c.  TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py."""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "libtile_oracle.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _SO


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        lib = ctypes.CDLL(_SO)
        lib.oracle_tile_counts.restype = ctypes.c_int
        lib.oracle_tile_counts.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64] * 3 + [ctypes.c_void_p]
        _lib = lib
    return _lib


def tile_counts(doc_ids, q_bits=None, kv_bits=None, block: int = 128) -> np.ndarray:
    """Brute-force int64[nt, nt] allowed-pair counts per tile (tile_oracle.c)."""
    lib = _load()
    doc = np.ascontiguousarray(doc_ids, dtype=np.int32)
    T = doc.shape[0]
    if q_bits is None:
        words = 0
        qb = np.zeros(1, dtype=np.uint64)
        kb = np.zeros(1, dtype=np.uint64)
    else:
        qb = np.ascontiguousarray(q_bits, dtype=np.uint64)
        kb = np.ascontiguousarray(kv_bits, dtype=np.uint64)
        words = qb.shape[0]
    nt = (T + block - 1) // block
    counts = np.zeros((nt, nt), dtype=np.int64)
    rc = lib.oracle_tile_counts(doc.ctypes.data, qb.ctypes.data, kb.ctypes.data,
                                T, words, block, counts.ctypes.data)
    if rc != 0:
        raise ValueError("oracle_tile_counts rejected its arguments")
    return counts
