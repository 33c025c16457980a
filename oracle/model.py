"""Model-level pieces of the oracle — TEST INFRASTRUCTURE ONLY.

quantize_q8 restates the reference's offline quantizer (scripts/quantize.py:7-23)
in numpy; q8_matmul / q8_matmul_bulk bind the C restatements of the
reference's Q8 products (oracle/model_oracle.c, src/model_q8.cpp:92-125 and
:382-420).  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg use this module.
"""
from __future__ import annotations

import ctypes

import numpy as np

from .attn import lib as _attn_lib
from .attn import max_threads

Q8_BLOCK = 32
Q8_BLOCK_BYTES = 36

_f32p = ctypes.POINTER(ctypes.c_float)
_bound = False


def _lib():
    global _bound
    L = _attn_lib()
    if not _bound:
        c_int = ctypes.c_int
        L.oracle_q8_matmul.argtypes = [_f32p, _f32p, ctypes.c_void_p, c_int, c_int, c_int]
        L.oracle_q8_matmul.restype = None
        L.oracle_q8_matmul_bulk.argtypes = [_f32p, _f32p, ctypes.c_void_p, c_int, c_int, c_int, c_int]
        L.oracle_q8_matmul_bulk.restype = None
        _bound = True
    return L


def quantize_q8(weights: np.ndarray):
    """scripts/quantize.py:7-23 over a [d][n] fp32 matrix, row-major in blocks
    of 32: scale = max|w|/127 (1e-9 for an all-zero block), q = round-half-even
    (w/scale) clipped to int8.  Returns (scales [d][n/32] f32, q [d][n] int8)."""
    w = np.ascontiguousarray(weights, dtype=np.float32)
    d, n = w.shape
    assert n % Q8_BLOCK == 0
    blocks = w.reshape(d, n // Q8_BLOCK, Q8_BLOCK)
    absmax = np.max(np.abs(blocks), axis=2)
    scale = (absmax / np.float32(127.0)).astype(np.float32)
    scale = np.where(absmax != 0, scale, np.float32(1e-9)).astype(np.float32)
    q = np.round(blocks / scale[:, :, None]).astype(np.float32)
    q = np.clip(q, -128, 127).astype(np.int8)
    return scale, q.reshape(d, n)


def pack_q8(scale: np.ndarray, q: np.ndarray) -> np.ndarray:
    """BlockQ8 rows (src/model_q8.cpp:28-32) as bytes: [d][n/32][4 + 32]."""
    d, n = q.shape
    nb = n // Q8_BLOCK
    out = np.empty((d, nb, Q8_BLOCK_BYTES), np.uint8)
    out[:, :, :4] = np.ascontiguousarray(scale, dtype=np.float32).reshape(d, nb, 1).view(np.uint8)
    out[:, :, 4:] = q.reshape(d, nb, Q8_BLOCK).view(np.uint8)
    return out.reshape(-1)


def unpack_q8(w: np.ndarray, n: int, d: int):
    """Inverse of pack_q8: (scales [d][n/32] f32, q [d][n] int8)."""
    b = np.ascontiguousarray(w, dtype=np.uint8).reshape(d, n // Q8_BLOCK, Q8_BLOCK_BYTES)
    scale = np.ascontiguousarray(b[:, :, :4]).view(np.float32).reshape(d, n // Q8_BLOCK)
    q = np.ascontiguousarray(b[:, :, 4:]).view(np.int8).reshape(d, n)
    return scale, q


def q8_matmul(w: np.ndarray, x: np.ndarray, n: int, d: int, n_threads: int = 0) -> np.ndarray:
    """oracle_q8_matmul row by row: x [batch][n] (or [n]) -> [batch][d]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    one = x.ndim == 1
    x2 = x.reshape(-1, n)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    out = np.zeros((x2.shape[0], d), np.float32)
    t = n_threads or max_threads()
    for b in range(x2.shape[0]):
        _lib().oracle_q8_matmul(out[b].ctypes.data_as(_f32p), x2[b].ctypes.data_as(_f32p),
                                w.ctypes.data_as(ctypes.c_void_p), n, d, t)
    return out[0] if one else out


def q8_matmul_bulk(w: np.ndarray, x: np.ndarray, n: int, d: int, n_threads: int = 0) -> np.ndarray:
    """oracle_q8_matmul_bulk: x [batch][n] -> [batch][d], last block of each row only."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, n)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    out = np.zeros((x.shape[0], d), np.float32)
    _lib().oracle_q8_matmul_bulk(out.ctypes.data_as(_f32p), x.ctypes.data_as(_f32p),
                                 w.ctypes.data_as(ctypes.c_void_p), x.shape[0], n, d,
                                 n_threads or max_threads())
    return out
