"""The transformer step around the attention path (binding of nitro_model_*
and nitro_forward_*): weights in the reference's model file layout
(src/Server_Inference.cpp:45-69), forward passes of src/model_q8.cpp on the
device."""
from __future__ import annotations

import ctypes

import numpy as np

from . import _native as N
from .attention import _dev, _stream_ptr
from .q8 import FULL_ROWS, LAST_BLOCK  # noqa: F401  (re-exported semantics)

HEADER_FIELDS = ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "vocab_size", "seq_len")


class Model:
    """Device copy of a model file; forward passes over a KVPool's uploaded batch."""

    def __init__(self, blob):
        b = np.ascontiguousarray(np.frombuffer(bytes(blob), dtype=np.uint8)
                                 if not isinstance(blob, np.ndarray) else blob, dtype=np.uint8)
        h = ctypes.c_void_p()
        N.call("nitro_model_create", b.ctypes.data_as(ctypes.c_void_p), b.size, ctypes.byref(h))
        self._h = h
        cfg = np.zeros(7, np.int32)
        N.call("nitro_model_config", self._h, cfg.ctypes.data_as(N._i32p))
        self.config = dict(zip(HEADER_FIELDS, (int(v) for v in cfg)))
        self.dim, self.vocab = self.config["dim"], self.config["vocab_size"]
        self.n_layers = self.config["n_layers"]
        self.kv_dim = self.config["n_kv_heads"] * self.dim // self.config["n_heads"]

    @classmethod
    def from_file(cls, path: str) -> "Model":
        return cls(np.fromfile(path, dtype=np.uint8))

    @property
    def handle(self):
        return self._h

    def close(self):
        if getattr(self, "_h", None):
            N.call("nitro_model_destroy", self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _logits(self, rows, logits):
        import torch

        if logits is None:
            logits = torch.empty((rows, self.vocab), device="cuda")
        if tuple(logits.shape) != (rows, self.vocab):
            raise N.NitroError(N.INVALID_ARGUMENT, "model", f"logits must be [{rows}][{self.vocab}]")
        return logits

    def forward_decode_batch(self, pool, tokens, logits=None, semantics: int = LAST_BLOCK,
                             stream=None):
        """forward_decode_batch (src/model_q8.cpp:571-694; forward_paged with one
        token and FULL_ROWS): one token per sequence of the pool's uploaded
        decode batch.  Returns logits [batch][vocab] on the GPU."""
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int64).astype(np.int32))
        logits = self._logits(t.size, logits)
        N.call("nitro_forward_decode_batch", self._h, pool.handle, t.ctypes.data_as(N._i32p), t.size,
               _dev(logits, "logits"), semantics, _stream_ptr(stream))
        return logits

    def forward_prefill(self, pool, tokens, logits=None, semantics: int = LAST_BLOCK, stream=None):
        """forward_prefill_chunk (src/model_q8.cpp:424-557) for every chunk of the
        pool's uploaded prefill batch (tokens packed in batch order).  Returns
        the logits of each chunk's last token, [chunks][vocab] on the GPU."""
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int64).astype(np.int32))
        logits = self._logits(pool.prefill_chunks, logits)
        N.call("nitro_forward_prefill", self._h, pool.handle, t.ctypes.data_as(N._i32p), t.size,
               _dev(logits, "logits"), semantics, _stream_ptr(stream))
        return logits


def synthetic_model_file(dim: int, hidden_dim: int, n_layers: int, n_heads: int, n_kv_heads: int,
                         vocab_size: int, seq_len: int, seed: int = 0) -> np.ndarray:
    """A model file in the reference's layout (src/Server_Inference.cpp:45-69)
    with synthetic weights: embedding U[-1,1), rms weights U[0.5,1.5), Q8
    matrices of random int8 in [-127, 127] with per-block scales ~
    1/(127*sqrt(cols)) (unit scale activations), and RoPE tables
    cos/sin(pos * 10000^(-2i/head_size)).  For benchmarks and tests where no
    trained checkpoint is available; written straight into one buffer so a
    7B-shaped file (7.3 GB) takes seconds."""
    rng = np.random.default_rng(seed)
    head = dim // n_heads
    kv_dim = n_kv_heads * head
    q8n = lambda rows, cols: n_layers * rows * (cols // 32) * 36
    total = (28 + 4 * (vocab_size * dim + 2 * n_layers * dim + dim + seq_len * head)
             + 2 * q8n(dim, dim) + 2 * q8n(kv_dim, dim) + 2 * q8n(hidden_dim, dim) + q8n(dim, hidden_dim))
    out = np.empty(total, np.uint8)
    off = 0

    def put(b):
        nonlocal off
        out[off:off + b.size] = b
        off += b.size

    def f32(a):
        put(np.ascontiguousarray(a, dtype=np.float32).view(np.uint8).reshape(-1))

    def q8(rows, cols):
        nonlocal off
        nb = cols // 32
        blocks = out[off:off + q8n(rows, cols)].reshape(n_layers * rows, nb, 36)
        scale = (1.0 / (127.0 * np.sqrt(cols))) * (1.0 + 0.5 * rng.uniform(-1, 1, (n_layers * rows, nb, 1)))
        blocks[:, :, :4] = scale.astype(np.float32).view(np.uint8)
        q = rng.bit_generator.random_raw(n_layers * rows * nb * 4).view(np.int8).reshape(n_layers * rows, nb, 32)
        blocks[:, :, 4:] = np.maximum(q, -127).view(np.uint8)
        off += blocks.size

    put(np.array([dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len], np.int32).view(np.uint8))
    f32(rng.random((vocab_size, dim), dtype=np.float32) * 2.0 - 1.0)
    f32(rng.uniform(0.5, 1.5, (n_layers, dim)))
    q8(dim, dim)
    q8(kv_dim, dim)
    q8(kv_dim, dim)
    q8(dim, dim)
    f32(rng.uniform(0.5, 1.5, (n_layers, dim)))
    q8(hidden_dim, dim)
    q8(dim, hidden_dim)
    q8(hidden_dim, dim)
    f32(rng.uniform(0.5, 1.5, dim))
    ang = np.arange(seq_len)[:, None] * 10000.0 ** (-2.0 * np.arange(head // 2) / head)[None, :]
    f32(np.cos(ang))
    f32(np.sin(ang))
    assert off == total
    return out
