"""Model-level pieces of the oracle — TEST INFRASTRUCTURE ONLY.

quantize_q8 restates the reference's offline quantizer (scripts/quantize.py:7-23)
in numpy; q8_matmul / q8_matmul_bulk bind the C restatements of the
reference's Q8 products (oracle/model_oracle.c, src/model_q8.cpp:92-125 and
:382-420).  OracleModel composes the C restatements into the reference's
forward passes (forward_paged, forward_prefill_chunk, forward_decode_batch).
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module.
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
        L.oracle_rms_norm.argtypes = [_f32p, _f32p, _f32p, c_int]
        L.oracle_rms_norm.restype = None
        L.oracle_swiglu.argtypes = [_f32p, _f32p, c_int]
        L.oracle_swiglu.restype = None
        L.oracle_f32_matmul.argtypes = [_f32p, _f32p, _f32p, c_int, c_int, c_int]
        L.oracle_f32_matmul.restype = None
        L.oracle_f32_matmul_bulk.argtypes = [_f32p, _f32p, _f32p, c_int, c_int, c_int, c_int]
        L.oracle_f32_matmul_bulk.restype = None
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


def scale_residual_outputs(blob: np.ndarray, factor: float) -> np.ndarray:
    """A copy of a model file (src/Server_Inference.cpp:45-69) with the block
    scales of wo and w2 multiplied by `factor` — what the reference driver's
    random model with out_scale=factor holds (exact for powers of two)."""
    b = np.array(blob, dtype=np.uint8, copy=True)
    D, Hd, L, H, Hkv, V, S = (int(v) for v in b[:28].view(np.int32))
    KV = D // H * Hkv
    q8b = lambda rows, cols: rows * (cols // Q8_BLOCK) * Q8_BLOCK_BYTES
    o_wo = 28 + V * D * 4 + L * D * 4 + L * (q8b(D, D) + 2 * q8b(KV, D))
    o_w2 = o_wo + L * q8b(D, D) + L * D * 4 + L * q8b(Hd, D)
    for off, nbytes in ((o_wo, L * q8b(D, D)), (o_w2, L * q8b(D, Hd))):
        blocks = b[off:off + nbytes].reshape(-1, Q8_BLOCK_BYTES)
        sc = blocks[:, :4].copy().view(np.float32) * np.float32(factor)
        blocks[:, :4] = sc.view(np.uint8).reshape(-1, 4)
        b[off:off + nbytes] = blocks.reshape(-1)
    return b


def _p(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_f32p)


def rms_norm(x: np.ndarray, weight: np.ndarray) -> np.ndarray:
    """src/model_q8.cpp:128-140 on every row of x."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(weight, dtype=np.float32)
    out = np.empty_like(x)
    for r in range(x.shape[0]):
        _lib().oracle_rms_norm(_p(out[r]), _p(x[r]), _p(w), x.shape[1])
    return out


def swiglu(hb: np.ndarray, hb2: np.ndarray) -> np.ndarray:
    hb = np.ascontiguousarray(hb, dtype=np.float32).copy()
    hb2 = np.ascontiguousarray(hb2, dtype=np.float32)
    _lib().oracle_swiglu(_p(hb), _p(hb2), hb.size)
    return hb


def f32_matmul(w: np.ndarray, x: np.ndarray, bulk: bool, n_threads: int = 0) -> np.ndarray:
    """x [rows][n] . w[d][n]^T with the reference's float matmul (one row at a
    time, :80-90) or matmul_bulk (:370-380)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    d, n = w.shape
    out = np.zeros((x.shape[0], d), np.float32)
    t = n_threads or max_threads()
    if bulk:
        _lib().oracle_f32_matmul_bulk(_p(out), _p(x), _p(w), x.shape[0], n, d, t)
    else:
        for r in range(x.shape[0]):
            _lib().oracle_f32_matmul(_p(out[r]), _p(x[r]), _p(w), n, d, t)
    return out


class OracleModel:
    """A model file (src/Server_Inference.cpp:45-69) on the host and the
    reference's forward passes over a paged KV pool [pages][L][16][kv_dim],
    composed from the C restatements."""

    def __init__(self, blob: np.ndarray):
        from . import attn

        self._attn = attn
        b = np.ascontiguousarray(blob, dtype=np.uint8)
        h = b[:28].view(np.int32)
        (self.dim, self.hidden, self.n_layers, self.n_heads, self.n_kv_heads, self.vocab,
         self.seq_len) = (int(v) for v in h)
        self.head_size = self.dim // self.n_heads
        self.kv_dim = self.n_kv_heads * self.head_size
        D, Hd, L, KV, V = self.dim, self.hidden, self.n_layers, self.kv_dim, self.vocab
        o = 28

        def take(nbytes):
            nonlocal o
            a = b[o:o + nbytes]
            o += nbytes
            return a

        f32 = lambda shape: take(4 * int(np.prod(shape))).view(np.float32).reshape(shape)
        q8 = lambda rows, cols: take(L * rows * (cols // Q8_BLOCK) * Q8_BLOCK_BYTES).reshape(L, -1)
        self.emb = f32((V, D))
        self.rms_att = f32((L, D))
        self.wq, self.wk, self.wv, self.wo = q8(D, D), q8(KV, D), q8(KV, D), q8(D, D)
        self.rms_ffn = f32((L, D))
        self.w1, self.w2, self.w3 = q8(Hd, D), q8(D, Hd), q8(Hd, D)
        self.rms_final = f32((D,))
        self.freq_real = f32((self.seq_len, self.head_size // 2))
        self.freq_imag = f32((self.seq_len, self.head_size // 2))

    def _q8(self, w, x, n, d, bulk):
        return q8_matmul_bulk(w, x, n, d) if bulk else q8_matmul(w, x, n, d)

    def _layers(self, x, k_pool, v_pool, bulk, attend):
        D, Hd, KV = self.dim, self.hidden, self.kv_dim
        for l in range(self.n_layers):
            xb = rms_norm(x, self.rms_att[l])
            q = self._q8(self.wq[l], xb, D, D, bulk)
            k = self._q8(self.wk[l], xb, D, KV, bulk)
            v = self._q8(self.wv[l], xb, D, KV, bulk)
            xb = attend(l, q, k, v)
            x = x + self._q8(self.wo[l], xb, D, D, bulk)
            xb = rms_norm(x, self.rms_ffn[l])
            hb = self._q8(self.w1[l], xb, D, Hd, bulk)
            hb2 = self._q8(self.w3[l], xb, D, Hd, bulk)
            x = x + self._q8(self.w2[l], swiglu(hb, hb2), Hd, D, bulk)
        return x

    def forward_decode_batch(self, k_pool, v_pool, tables, positions, tokens, bulk=True):
        """forward_decode_batch (src/model_q8.cpp:571-694) after the caller's
        allocate_next_token; bulk=False with one sequence is forward_paged
        (:244-368, full-row matmul and the single-sequence AVX2 attention).
        Appends this step's K/V into the pools; returns logits [B][vocab]."""
        A = self._attn
        positions = np.asarray(positions, np.int32)
        x = self.emb[np.asarray(tokens, np.int64)].copy()

        def attend(l, q, k, v):
            q, k = A.rope(q, k, positions, self.freq_real, self.freq_imag, self.head_size)
            A.kv_append_decode(k_pool, v_pool, l, k, v, tables, positions)
            if not bulk and len(positions) == 1:
                return A.decode_single_avx2(k_pool, v_pool, l, q[0], np.asarray(tables)[0],
                                            int(positions[0]), self.n_heads, self.n_kv_heads,
                                            self.head_size)[None, :]
            return A.decode_batch(k_pool, v_pool, l, q, tables, positions, self.n_heads,
                                  self.n_kv_heads, self.head_size)

        x = self._layers(x, k_pool, v_pool, bulk, attend)
        x = rms_norm(x, self.rms_final)
        return f32_matmul(self.emb, x, bulk=bulk)

    def forward_prefill_chunk(self, k_pool, v_pool, table, start_pos, tokens, bulk=True):
        """forward_prefill_chunk (src/model_q8.cpp:424-557) after the caller's
        allocate_next_token for the chunk: logits [vocab] of its last token.
        The reference's products there are matmul_bulk; bulk=False composes the
        same step from full-row products (matmul, :92-125)."""
        A = self._attn
        tokens = np.asarray(tokens, np.int64)
        positions = (start_pos + np.arange(tokens.size)).astype(np.int32)
        x = self.emb[tokens].copy()

        def attend(l, q, k, v):
            q, k = A.rope(q, k, positions, self.freq_real, self.freq_imag, self.head_size)
            A.kv_scatter_prefill(k_pool, v_pool, l, k, v, table, start_pos)
            return A.prefill_chunk(k_pool, v_pool, l, q, table, start_pos, self.n_heads,
                                   self.n_kv_heads, self.head_size)

        x = self._layers(x, k_pool, v_pool, bulk, attend)
        last = rms_norm(x[-1:], self.rms_final)
        return f32_matmul(self.emb, last, bulk=bulk)[0]
