"""ctypes driver of the reference's own compiled code — TEST INFRASTRUCTURE ONLY.

oracle/_ref/libnitro_ref.so is built by `make -C oracle ref` from the
reference's src/model_q8.cpp (+ src/pagedMemory.hpp) and oracle/ref_harness.cpp.
It exists only where the reference checkout is present; callers must check
available() first.  Used by tests/golden/make_golden.py to record golden
vectors and by CPU tests to cross-check the oracle live.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from . import paged_memory as pm

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_ref", "libnitro_ref.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)


def available() -> bool:
    return os.path.exists(LIB_PATH)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        L = ctypes.CDLL(LIB_PATH)
        ci, vp, u64 = ctypes.c_int, ctypes.c_void_p, ctypes.c_uint64
        L.ref_hash_block_state.argtypes = [u64, _i32p, ci]
        L.ref_hash_block_state.restype = u64
        L.ref_set_threads.argtypes = [ci]
        L.ref_model_create.argtypes = [ci, ci, ci, ci, ci, ci, ci, ci, ci, ci, u64, ctypes.c_float]
        L.ref_model_create.restype = vp
        L.ref_model_serialize.argtypes = [vp, ctypes.POINTER(ctypes.c_uint8), u64]
        L.ref_model_serialize.restype = u64
        L.ref_read_logits.argtypes = [vp, ci, _f32p]
        L.ref_q8_matmul.argtypes = [_f32p, _f32p, vp, ci, ci]
        L.ref_q8_matmul.restype = None
        L.ref_q8_matmul_bulk.argtypes = [_f32p, _f32p, vp, ci, ci, ci]
        L.ref_q8_matmul_bulk.restype = None
        L.ref_world_create.argtypes = [ci, ci, ci, ci, ci, ci, ci, ci, ci, u64]
        L.ref_world_create.restype = vp
        L.ref_world_destroy.argtypes = [vp]
        L.ref_world_dims.argtypes = [vp, _i32p]
        L.ref_world_set_rope.argtypes = [vp, _f32p, _f32p]
        L.ref_op.argtypes = [vp, ci, ci, ci, u64, _i32p, ci, ctypes.POINTER(ctypes.c_int64)]
        L.ref_snapshot.argtypes = [vp, _i32p, ci]
        L.ref_decode_batch.argtypes = [vp, _i32p, _i32p, ci, _i32p]
        L.ref_forward_paged.argtypes = [vp, ci, ci, _i32p]
        L.ref_prefill_chunk.argtypes = [vp, ci, _i32p, ci, _i32p]
        L.ref_forward_contiguous.argtypes = [vp, ci, ci]
        L.ref_read_rows.argtypes = [vp, ci, _f32p, _f32p, _f32p, _f32p]
        L.ref_read_pool.argtypes = [vp, _f32p, _f32p]
        L.ref_write_pool.argtypes = [vp, _f32p, _f32p]
        L.ref_read_contiguous_cache.argtypes = [vp, _f32p, _f32p]
        L.ref_write_contiguous_cache.argtypes = [vp, _f32p, _f32p]
        L.ref_block_table.argtypes = [vp, ci, _i32p, ci]
        L.ref_rpc_send_ints.argtypes = [ci, _i32p, ci]
        L.ref_rpc_recv_ints.argtypes = [ci, _i32p, ci]
        L.ref_rpc_recv_structured_query.argtypes = [ci, ci, ctypes.POINTER(ctypes.c_uint64), _f32p, _f32p, _f32p]
        L.ref_sched_create.argtypes = [vp, ci]
        L.ref_sched_add.argtypes = [vp, ci, _i32p, ci]
        L.ref_sched_active.argtypes = [vp]
        L.ref_sched_step.argtypes = [vp]
        L.ref_sched_state.argtypes = [vp, _i32p, ci]
        _lib = L
    return _lib


def q8_matmul(w: np.ndarray, x: np.ndarray, n: int, d: int) -> np.ndarray:
    """The reference's matmul (BlockQ8) on one activation row x[n] -> [d]."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(d, np.float32)
    lib().ref_q8_matmul(out.ctypes.data_as(_f32p), x.ctypes.data_as(_f32p),
                        w.ctypes.data_as(ctypes.c_void_p), n, d)
    return out


def q8_matmul_bulk(w: np.ndarray, x: np.ndarray, n: int, d: int) -> np.ndarray:
    """The reference's matmul_bulk (BlockQ8) on x[batch][n] -> [batch][d]."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    batch = x.shape[0]
    out = np.zeros((batch, d), np.float32)
    lib().ref_q8_matmul_bulk(out.ctypes.data_as(_f32p), x.ctypes.data_as(_f32p),
                             w.ctypes.data_as(ctypes.c_void_p), batch, n, d)
    return out


def hash_block_state(parent: int, tokens) -> int:
    t = np.ascontiguousarray(tokens, dtype=np.int32)
    return int(lib().ref_hash_block_state(parent, t.ctypes.data_as(_i32p), t.size))


class RefWorld:
    """One reference KVBlock_Manager + PrefixCacheManager + request slots around
    a tiny model whose wo is the identity (so xb2 exposes the attention output)."""

    def __init__(self, n_heads=2, n_kv_heads=2, head_dim=16, n_layers=1, vocab=512,
                 seq_len=512, total_blocks=32, max_rows=256, max_seqs=8, seed=1, threads=1):
        L = lib()
        L.ref_set_threads(threads)
        self.h = L.ref_world_create(n_heads, n_kv_heads, head_dim, n_layers, vocab, seq_len,
                                    total_blocks, max_rows, max_seqs, seed)
        self.n_heads, self.n_kv_heads, self.head_dim = n_heads, n_kv_heads, head_dim
        self.n_layers, self.total_blocks, self.max_seqs = n_layers, total_blocks, max_seqs
        self.seq_len, self.max_rows = seq_len, max_rows
        self.dim = n_heads * head_dim
        self.kv_dim = n_kv_heads * head_dim

    @classmethod
    def random_model(cls, n_heads, n_kv_heads, head_dim, n_layers, vocab, seq_len, hidden_dim,
                     total_blocks, max_rows=64, max_seqs=8, seed=1, threads=1, out_scale=1.0):
        """A world whose model has every weight random (ref_model_create): for
        logits-level golden vectors of the forward passes.  out_scale > 1
        strengthens wo and w2 so the layers, not the token's own embedding,
        decide the argmax."""
        self = cls.__new__(cls)
        L = lib()
        L.ref_set_threads(threads)
        self.h = L.ref_model_create(n_heads, n_kv_heads, head_dim, n_layers, vocab, seq_len,
                                    hidden_dim, total_blocks, max_rows, max_seqs, seed, out_scale)
        self.n_heads, self.n_kv_heads, self.head_dim = n_heads, n_kv_heads, head_dim
        self.n_layers, self.total_blocks, self.max_seqs = n_layers, total_blocks, max_seqs
        self.seq_len, self.max_rows, self.vocab = seq_len, max_rows, vocab
        self.dim = n_heads * head_dim
        self.kv_dim = n_kv_heads * head_dim
        return self

    def serialize(self) -> np.ndarray:
        """The model in the reference's file layout (src/Server_Inference.cpp:45-69)."""
        n = lib().ref_model_serialize(self.h, None, 0)
        out = np.zeros(n, dtype=np.uint8)
        assert lib().ref_model_serialize(self.h, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), n) == n
        return out

    def logits(self, rows) -> np.ndarray:
        out = np.zeros((rows, self.vocab), dtype=np.float32)
        assert lib().ref_read_logits(self.h, rows, out.ctypes.data_as(_f32p)) == 0
        return out

    def close(self):
        if self.h:
            lib().ref_world_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_rope(self, real, imag):
        """RoPE tables [seq_len][head_dim/2] (the world starts with the identity rotation)."""
        real = np.ascontiguousarray(real, dtype=np.float32)
        imag = np.ascontiguousarray(imag, dtype=np.float32)
        assert real.shape == imag.shape == (self.seq_len, self.head_dim // 2)
        lib().ref_world_set_rope(self.h, real.ctypes.data_as(_f32p), imag.ctypes.data_as(_f32p))

    def op(self, op, a=0, b=0, h=0, toks=()):
        t = np.ascontiguousarray(toks, dtype=np.int32)
        res = ctypes.c_int64(0)
        st = lib().ref_op(self.h, op, a, b, h, t.ctypes.data_as(_i32p), t.size,
                          ctypes.byref(res))
        return int(st), int(res.value)

    def snapshot(self) -> dict:
        cap = 1 << 20
        buf = np.zeros(cap, dtype=np.int32)
        n = lib().ref_snapshot(self.h, buf.ctypes.data_as(_i32p), cap)
        assert n >= 0
        return pm.decode_snapshot(buf[:n], self.total_blocks, self.max_seqs)

    # ---- Continuous_Scheduler (src/pagedMemory.hpp:287-399) ---------------
    def sched_create(self, max_tokens_per_batch=256):
        assert lib().ref_sched_create(self.h, max_tokens_per_batch) == 0

    def sched_add(self, req_id, prompt):
        t = np.ascontiguousarray(prompt, dtype=np.int32)
        assert lib().ref_sched_add(self.h, req_id, t.ctypes.data_as(_i32p), t.size) == 0

    def sched_active(self) -> bool:
        return lib().ref_sched_active(self.h) != 0

    def sched_step(self) -> int:
        """0, or 1 when the reference called exit() (pool exhausted)."""
        return int(lib().ref_sched_step(self.h))

    def sched_state(self) -> np.ndarray:
        cap = 1 << 16
        buf = np.zeros(cap, dtype=np.int32)
        n = lib().ref_sched_state(self.h, buf.ctypes.data_as(_i32p), cap)
        assert n >= 0
        return buf[:n].copy()

    def block_table(self, slot) -> np.ndarray:
        buf = np.zeros(4096, dtype=np.int32)
        n = lib().ref_block_table(self.h, slot, buf.ctypes.data_as(_i32p), buf.size)
        assert n >= 0
        return buf[:n].copy()

    def pool(self):
        shape = (self.total_blocks, self.n_layers, 16, self.kv_dim)
        k = np.zeros(shape, dtype=np.float32)
        v = np.zeros(shape, dtype=np.float32)
        lib().ref_read_pool(self.h, k.ctypes.data_as(_f32p), v.ctypes.data_as(_f32p))
        return k, v

    def write_pool(self, k, v):
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        lib().ref_write_pool(self.h, k.ctypes.data_as(_f32p), v.ctypes.data_as(_f32p))

    def contiguous_cache(self):
        shape = (self.n_layers, self.seq_len, self.kv_dim)
        k = np.zeros(shape, dtype=np.float32)
        v = np.zeros(shape, dtype=np.float32)
        lib().ref_read_contiguous_cache(self.h, k.ctypes.data_as(_f32p), v.ctypes.data_as(_f32p))
        return k, v

    def write_contiguous_cache(self, k, v):
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        lib().ref_write_contiguous_cache(self.h, k.ctypes.data_as(_f32p),
                                         v.ctypes.data_as(_f32p))

    def rows(self, n):
        q = np.zeros((n, self.dim), dtype=np.float32)
        k = np.zeros((n, self.kv_dim), dtype=np.float32)
        v = np.zeros((n, self.kv_dim), dtype=np.float32)
        xb2 = np.zeros((n, self.dim), dtype=np.float32)
        assert lib().ref_read_rows(self.h, n, q.ctypes.data_as(_f32p), k.ctypes.data_as(_f32p),
                                   v.ctypes.data_as(_f32p), xb2.ctypes.data_as(_f32p)) == 0
        return q, k, v, xb2

    def decode_batch(self, slots, tokens):
        s = np.ascontiguousarray(slots, dtype=np.int32)
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        pos = np.zeros(s.size, dtype=np.int32)
        st = lib().ref_decode_batch(self.h, s.ctypes.data_as(_i32p), t.ctypes.data_as(_i32p),
                                    s.size, pos.ctypes.data_as(_i32p))
        assert st == 0
        return pos

    def forward_paged(self, slot, token) -> int:
        pos = np.zeros(1, dtype=np.int32)
        assert lib().ref_forward_paged(self.h, slot, token, pos.ctypes.data_as(_i32p)) == 0
        return int(pos[0])

    def prefill_chunk(self, slot, tokens) -> int:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        sp = np.zeros(1, dtype=np.int32)
        assert lib().ref_prefill_chunk(self.h, slot, t.ctypes.data_as(_i32p), t.size,
                                       sp.ctypes.data_as(_i32p)) == 0
        return int(sp[0])

    def forward_contiguous(self, token, pos):
        lib().ref_forward_contiguous(self.h, token, pos)
