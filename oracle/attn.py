"""ctypes bindings of the C oracle (oracle/attn_oracle.c) — TEST INFRASTRUCTURE ONLY.

Each wrapper takes numpy arrays and calls the C restatement of one reference
attention loop (src/model_q8.cpp).  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg use these.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_attn.so")
_V4_PATH = os.path.join(_HERE, "liboracle_attn_v4.so")
_lib = None

# Flags /proc/cpuinfo lists on a host that runs x86-64-v4 code.
_V4_FLAGS = {"avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"}
_BUILD_FLAGS = "-O3 -ffast-math -fopenmp -march={}"


def host_has_avx512() -> bool:
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("flags"):
                    return _V4_FLAGS <= set(ln.split(":", 1)[1].split())
    except OSError:
        pass
    return False


def use_timing_build() -> str:
    """For the benchmark's CPU baseline only: load the x86-64-v4 build (what
    -march=native selects on an AVX-512 host, the reference's build line) when
    this host runs it, else the x86-64-v3 one.  Must precede the first call.
    Returns the flags of the build in use."""
    global _LIB_PATH
    if _lib is None and host_has_avx512() and os.path.exists(_V4_PATH):
        _LIB_PATH = _V4_PATH
    return _BUILD_FLAGS.format("x86-64-v4" if _LIB_PATH == _V4_PATH else "x86-64-v3")

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run `make -C oracle`)")
        L = ctypes.CDLL(_LIB_PATH)
        c_int = ctypes.c_int
        L.oracle_softmax.argtypes = [_f32p, c_int]
        L.oracle_softmax.restype = None
        L.oracle_kv_append_decode.argtypes = [_f32p, _f32p, c_int, c_int, c_int, _f32p, _f32p,
                                              _i32p, c_int, _i32p, c_int]
        L.oracle_kv_append_decode.restype = None
        L.oracle_kv_scatter_prefill.argtypes = [_f32p, _f32p, c_int, c_int, c_int, _f32p, _f32p,
                                                _i32p, c_int, c_int]
        L.oracle_kv_scatter_prefill.restype = None
        L.oracle_decode_batch.argtypes = [_f32p, _f32p, c_int, c_int, c_int, _f32p, _f32p, _i32p,
                                          c_int, _i32p, c_int, c_int, c_int, c_int, c_int]
        L.oracle_decode_single_avx2.argtypes = [_f32p, _f32p, c_int, c_int, c_int, _f32p, _f32p,
                                                _i32p, c_int, c_int, c_int, c_int, c_int]
        L.oracle_prefill_chunk.argtypes = [_f32p, _f32p, c_int, c_int, c_int, _f32p, _f32p, _i32p,
                                           c_int, c_int, c_int, c_int, c_int, c_int]
        L.oracle_contiguous_attention.argtypes = [_f32p, _f32p, c_int, c_int, c_int, _f32p, _f32p,
                                                  c_int, c_int, c_int, c_int, c_int]
        L.oracle_rope.argtypes = [_f32p, _f32p, c_int, _i32p, _f32p, _f32p, c_int, c_int, c_int]
        L.oracle_rope.restype = None
        for name in ("oracle_decode_batch", "oracle_decode_single_avx2", "oracle_prefill_chunk",
                     "oracle_contiguous_attention", "oracle_max_threads"):
            getattr(L, name).restype = c_int
        _lib = L
    return _lib


def _f(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous, (a.dtype, a.flags)
    return a.ctypes.data_as(_f32p)


def _i(a: np.ndarray):
    assert a.dtype == np.int32 and a.flags.c_contiguous, (a.dtype, a.flags)
    return a.ctypes.data_as(_i32p)


def _pool_dims(k_pool: np.ndarray):
    # k_pool: [pages][layers][16][kv_dim]
    assert k_pool.ndim == 4 and k_pool.shape[2] == 16, k_pool.shape
    return k_pool.shape[1], k_pool.shape[3]


def softmax(x: np.ndarray) -> np.ndarray:
    y = np.ascontiguousarray(x, dtype=np.float32).copy()
    lib().oracle_softmax(_f(y), y.size)
    return y


def kv_append_decode(k_pool, v_pool, layer, k, v, tables, positions):
    L, kv_dim = _pool_dims(k_pool)
    tables = np.ascontiguousarray(tables, dtype=np.int32)
    positions = np.ascontiguousarray(positions, dtype=np.int32)
    lib().oracle_kv_append_decode(_f(k_pool), _f(v_pool), L, kv_dim, layer, _f(k), _f(v),
                                  _i(tables), tables.shape[1], _i(positions), positions.size)


def kv_scatter_prefill(k_pool, v_pool, layer, k, v, table, start_pos):
    L, kv_dim = _pool_dims(k_pool)
    table = np.ascontiguousarray(table, dtype=np.int32)
    lib().oracle_kv_scatter_prefill(_f(k_pool), _f(v_pool), L, kv_dim, layer, _f(k), _f(v),
                                    _i(table), int(start_pos), k.shape[0])


def decode_batch(k_pool, v_pool, layer, q, tables, positions, n_heads, n_kv_heads, head_dim,
                 n_threads=0):
    """Batched decode attention (src/model_q8.cpp:625-662). q: [B][H*hd] -> out [B][H*hd]."""
    L, kv_dim = _pool_dims(k_pool)
    tables = np.ascontiguousarray(tables, dtype=np.int32)
    positions = np.ascontiguousarray(positions, dtype=np.int32)
    q = np.ascontiguousarray(q, dtype=np.float32)
    out = np.zeros_like(q)
    rc = lib().oracle_decode_batch(_f(k_pool), _f(v_pool), L, kv_dim, layer, _f(q), _f(out),
                                   _i(tables), tables.shape[1], _i(positions), positions.size,
                                   n_heads, n_kv_heads, head_dim, n_threads)
    if rc != 0:
        raise RuntimeError(f"oracle_decode_batch failed: {rc}")
    return out


def decode_single_avx2(k_pool, v_pool, layer, q, table, pos, n_heads, n_kv_heads, head_dim,
                       n_threads=0):
    """Single-sequence AVX2 decode (src/model_q8.cpp:290-347). q: [H*hd]."""
    L, kv_dim = _pool_dims(k_pool)
    table = np.ascontiguousarray(table, dtype=np.int32)
    q = np.ascontiguousarray(q, dtype=np.float32)
    out = np.zeros_like(q)
    rc = lib().oracle_decode_single_avx2(_f(k_pool), _f(v_pool), L, kv_dim, layer, _f(q), _f(out),
                                         _i(table), int(pos), n_heads, n_kv_heads, head_dim,
                                         n_threads)
    if rc != 0:
        raise RuntimeError(f"oracle_decode_single_avx2 failed: {rc}")
    return out


def prefill_chunk(k_pool, v_pool, layer, q, table, start_pos, n_heads, n_kv_heads, head_dim,
                  n_threads=0):
    """Causal prefill for one sequence (src/model_q8.cpp:485-523). q: [T][H*hd]."""
    L, kv_dim = _pool_dims(k_pool)
    table = np.ascontiguousarray(table, dtype=np.int32)
    q = np.ascontiguousarray(q, dtype=np.float32)
    out = np.zeros_like(q)
    rc = lib().oracle_prefill_chunk(_f(k_pool), _f(v_pool), L, kv_dim, layer, _f(q), _f(out),
                                    _i(table), int(start_pos), q.shape[0], n_heads, n_kv_heads,
                                    head_dim, n_threads)
    if rc != 0:
        raise RuntimeError(f"oracle_prefill_chunk failed: {rc}")
    return out


def contiguous_attention(key_cache, value_cache, layer, q, pos, n_heads, n_kv_heads, head_dim,
                         n_threads=0):
    """Non-paged attention (src/model_q8.cpp:189-222). caches: [layers][seq_len][kv_dim]."""
    _, seq_len, kv_dim = key_cache.shape
    q = np.ascontiguousarray(q, dtype=np.float32)
    out = np.zeros_like(q)
    rc = lib().oracle_contiguous_attention(_f(key_cache), _f(value_cache), seq_len, kv_dim, layer,
                                           _f(q), _f(out), int(pos), n_heads, n_kv_heads,
                                           head_dim, n_threads)
    if rc != 0:
        raise RuntimeError(f"oracle_contiguous_attention failed: {rc}")
    return out


def rope(q, k, positions, freq_real, freq_imag, head_dim):
    """RoPE of the paged paths (src/model_q8.cpp:601-615); returns rotated copies.
    q: [rows][dim], k: [rows][kv_dim], positions: [rows], freq_*: [seq_len][hd/2]."""
    q = np.ascontiguousarray(q, dtype=np.float32).copy()
    k = np.ascontiguousarray(k, dtype=np.float32).copy()
    positions = np.ascontiguousarray(positions, dtype=np.int32)
    fr = np.ascontiguousarray(freq_real, dtype=np.float32)
    fi = np.ascontiguousarray(freq_imag, dtype=np.float32)
    assert positions.max() < fr.shape[0]
    lib().oracle_rope(_f(q), _f(k), q.shape[0], _i(positions), _f(fr), _f(fi), q.shape[1],
                      k.shape[1], head_dim)
    return q, k


def max_threads() -> int:
    return int(lib().oracle_max_threads())
