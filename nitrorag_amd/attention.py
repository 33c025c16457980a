"""Device KV pool and paged-attention launches over the C ABI.

KVPool mirrors the storage side of the reference's KVBlock_Manager
(src/pagedMemory.hpp:86-111: pools [page][layer][16][kv_dim], fp32) on the
GPU.  Its methods launch the HIP kernels that replace the reference's
attention regions:
  kv_append / decode          forward_decode_batch  src/model_q8.cpp:616-662
                              (and forward_paged    src/model_q8.cpp:279-347, batch 1)
  kv_append_prefill / prefill forward_prefill_chunk src/model_q8.cpp:473-523
Device buffers are torch tensors (fp32, contiguous, on the GPU); calls run
on torch's current stream unless a stream is given.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _native as N


def _stream_ptr(stream):
    import torch

    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _dev(t, name: str):
    import torch

    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise TypeError(f"{name} must be a GPU tensor")
    if t.dtype != torch.float32 or not t.is_contiguous():
        raise TypeError(f"{name} must be contiguous float32")
    return ctypes.c_void_p(t.data_ptr())


def _host_i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int64).astype(np.int32))


class KVPool:
    """Device K/V pools with the reference layout, plus the uploaded batches."""

    def __init__(self, num_pages: int, num_layers: int, kv_dim: int, k=None, v=None,
                 contiguous: bool = False):
        h = ctypes.c_void_p()
        if k is None:
            N.call("nitro_kvpool_create", num_pages, num_layers, kv_dim, ctypes.byref(h))
            self._keep = None
        else:
            need = num_pages * num_layers * 16 * kv_dim
            if k.numel() != need or v.numel() != need:
                raise ValueError(f"pool tensors need {need} elements")
            if contiguous:
                N.call("nitro_kvpool_wrap_contiguous", _dev(k, "k"), _dev(v, "v"), num_pages * 16,
                       num_layers, kv_dim, ctypes.byref(h))
            else:
                N.call("nitro_kvpool_wrap", _dev(k, "k"), _dev(v, "v"), num_pages, num_layers,
                       kv_dim, ctypes.byref(h))
            self._keep = (k, v)
        self._h = h
        self.num_pages, self.num_layers, self.kv_dim = num_pages, num_layers, kv_dim
        self.decode_batch = 0      # sequences in the uploaded decode batch
        self.prefill_rows = 0      # packed rows in the uploaded prefill batch

    @staticmethod
    def _need(t, n: int, name: str):
        # n == 0: no batch uploaded yet; the C entry point reports NITRO_ERR_NO_BATCH
        if n and t.numel() != n:
            raise ValueError(f"{name} has {t.numel()} elements, expected {n}")

    @classmethod
    def wrap(cls, k, v):
        """Borrow torch tensors shaped [pages][layers][16][kv_dim]."""
        pages, layers, rows, kv_dim = k.shape
        assert rows == 16 and v.shape == k.shape
        return cls(pages, layers, kv_dim, k, v)

    @classmethod
    def wrap_contiguous(cls, key_cache, value_cache):
        """Borrow forward's non-paged caches shaped [layers][seq_len][kv_dim]
        (src/model_q8.cpp:189-222) as seq_len/16 pages per layer; the identity
        block table [0, 1, .., pos/16] then addresses rows 0..pos of a layer."""
        layers, seq_len, kv_dim = key_cache.shape
        assert value_cache.shape == key_cache.shape
        if seq_len % 16:
            raise ValueError("seq_len must be a multiple of 16")
        return cls(seq_len // 16, layers, kv_dim, key_cache, value_cache, contiguous=True)

    @property
    def handle(self):
        return self._h

    def close(self):
        if getattr(self, "_h", None):
            N.lib().nitro_kvpool_destroy(self._h)
            self._h = None
            self._keep = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def data_ptrs(self) -> tuple[int, int]:
        k, v = ctypes.c_void_p(), ctypes.c_void_p()
        N.call("nitro_kvpool_data", self._h, ctypes.byref(k), ctypes.byref(v))
        return k.value, v.value

    # ---------------------------------------------------------------- decode
    def upload_decode_batch(self, tables, positions, stream=None) -> None:
        t = _host_i32(tables)
        p = _host_i32(positions)
        if t.ndim != 2 or p.ndim != 1 or t.shape[0] != p.shape[0]:
            raise ValueError("tables must be [B][max_pages] and positions [B]")
        N.call("nitro_decode_batch_upload", self._h, t.ctypes.data_as(N._i32p),
               p.ctypes.data_as(N._i32p), p.size, t.shape[1], _stream_ptr(stream))
        self.decode_batch = p.size

    def kv_append(self, layer: int, k, v, stream=None) -> None:
        self._need(k, self.decode_batch * self.kv_dim, "k")
        self._need(v, self.decode_batch * self.kv_dim, "v")
        N.call("nitro_kv_append", self._h, layer, _dev(k, "k"), _dev(v, "v"), _stream_ptr(stream))

    def decode(self, layer: int, q, out, n_heads: int, n_kv_heads: int, head_dim: int,
               stream=None) -> None:
        self._need(q, self.decode_batch * n_heads * head_dim, "q")
        self._need(out, self.decode_batch * n_heads * head_dim, "out")
        N.call("nitro_paged_attn_decode", self._h, layer, _dev(q, "q"), _dev(out, "out"), n_heads,
               n_kv_heads, head_dim, _stream_ptr(stream))

    def decode_append(self, layer: int, q, k, v, out, n_heads: int, n_kv_heads: int, head_dim: int,
                      stream=None) -> None:
        """kv_append + decode in one call (one launch where no other sequence
        reads the page a sequence appends to)."""
        self._need(q, self.decode_batch * n_heads * head_dim, "q")
        self._need(out, self.decode_batch * n_heads * head_dim, "out")
        self._need(k, self.decode_batch * self.kv_dim, "k")
        self._need(v, self.decode_batch * self.kv_dim, "v")
        N.call("nitro_paged_attn_decode_append", self._h, layer, _dev(q, "q"), _dev(k, "k"), _dev(v, "v"),
               _dev(out, "out"), n_heads, n_kv_heads, head_dim, _stream_ptr(stream))

    # --------------------------------------------------------------- prefill
    def upload_prefill_batch(self, tables, start_pos, num_tokens, stream=None) -> None:
        t = _host_i32(tables)
        s = _host_i32(start_pos)
        n = _host_i32(num_tokens)
        if t.ndim != 2 or not (t.shape[0] == s.size == n.size):
            raise ValueError("tables must be [B][max_pages], start_pos and num_tokens [B]")
        N.call("nitro_prefill_batch_upload", self._h, t.ctypes.data_as(N._i32p),
               s.ctypes.data_as(N._i32p), n.ctypes.data_as(N._i32p), s.size, t.shape[1],
               _stream_ptr(stream))
        self.prefill_rows = int(n.sum())
        self.prefill_chunks = int(n.size)

    def kv_append_prefill(self, layer: int, k, v, stream=None) -> None:
        self._need(k, self.prefill_rows * self.kv_dim, "k")
        self._need(v, self.prefill_rows * self.kv_dim, "v")
        N.call("nitro_kv_append_prefill", self._h, layer, _dev(k, "k"), _dev(v, "v"),
               _stream_ptr(stream))

    def prefill(self, layer: int, q, out, n_heads: int, n_kv_heads: int, head_dim: int,
                stream=None) -> None:
        self._need(q, self.prefill_rows * n_heads * head_dim, "q")
        self._need(out, self.prefill_rows * n_heads * head_dim, "out")
        N.call("nitro_paged_attn_prefill", self._h, layer, _dev(q, "q"), _dev(out, "out"), n_heads,
               n_kv_heads, head_dim, _stream_ptr(stream))

    def prefill_append(self, layer: int, q, k, v, out, n_heads: int, n_kv_heads: int,
                       head_dim: int, stream=None) -> None:
        """kv_append_prefill then prefill (src/model_q8.cpp:473-523), in one
        launch where the batch allows it."""
        self._need(q, self.prefill_rows * n_heads * head_dim, "q")
        self._need(k, self.prefill_rows * self.kv_dim, "k")
        self._need(v, self.prefill_rows * self.kv_dim, "v")
        self._need(out, self.prefill_rows * n_heads * head_dim, "out")
        N.call("nitro_paged_attn_prefill_append", self._h, layer, _dev(q, "q"), _dev(k, "k"),
               _dev(v, "v"), _dev(out, "out"), n_heads, n_kv_heads, head_dim, _stream_ptr(stream))

    def prefill_counts(self) -> tuple:
        """(prefill_append calls so far, how many ran as one launch)."""
        n, one = ctypes.c_int64(), ctypes.c_int64()
        N.call("nitro_kvpool_prefill_counts", self._h, ctypes.byref(n), ctypes.byref(one))
        return n.value, one.value

    # ------------------------------------------------------------------ RoPE
    def rope_kv_append(self, layer: int, q, k, v, freq_real, freq_imag, n_heads: int,
                       n_kv_heads: int, head_dim: int, stream=None) -> None:
        """Rotates q and k in place (src/model_q8.cpp:601-615), appends k and v (:616-623)."""
        self._need(q, self.decode_batch * n_heads * head_dim, "q")
        self._need(k, self.decode_batch * self.kv_dim, "k")
        self._need(v, self.decode_batch * self.kv_dim, "v")
        self._rope("nitro_rope_kv_append", layer, q, k, v, freq_real, freq_imag, n_heads,
                   n_kv_heads, head_dim, stream)

    def rope_kv_append_prefill(self, layer: int, q, k, v, freq_real, freq_imag, n_heads: int,
                               n_kv_heads: int, head_dim: int, stream=None) -> None:
        """The same for the prefill batch rows (src/model_q8.cpp:451-484)."""
        self._need(q, self.prefill_rows * n_heads * head_dim, "q")
        self._need(k, self.prefill_rows * self.kv_dim, "k")
        self._need(v, self.prefill_rows * self.kv_dim, "v")
        self._rope("nitro_rope_kv_append_prefill", layer, q, k, v, freq_real, freq_imag, n_heads,
                   n_kv_heads, head_dim, stream)

    def _rope(self, fn, layer, q, k, v, freq_real, freq_imag, n_heads, n_kv_heads, head_dim,
              stream):
        if freq_real.shape != freq_imag.shape or freq_real.shape[-1] != head_dim // 2:
            raise ValueError("RoPE tables must both be [seq_len][head_dim/2]")
        N.call(fn, self._h, layer, _dev(q, "q"), _dev(k, "k"), _dev(v, "v"),
               _dev(freq_real, "freq_real"), _dev(freq_imag, "freq_imag"), freq_real.shape[0],
               n_heads, n_kv_heads, head_dim, _stream_ptr(stream))

    def take_device_errors(self) -> int:
        out = ctypes.c_int32()
        N.call("nitro_kvpool_take_device_errors", self._h, ctypes.byref(out))
        return out.value

    def decode_counts(self) -> tuple:
        """(decode launches so far, how many took the shared-prefix form)."""
        n, shared = ctypes.c_int64(), ctypes.c_int64()
        N.call("nitro_kvpool_decode_counts", self._h, ctypes.byref(n), ctypes.byref(shared))
        return n.value, shared.value
