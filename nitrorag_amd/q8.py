"""Q8_0 matrix product on the GPU (binding of nitro_q8_matmul).

Weights are the reference's BlockQ8 rows (src/model_q8.cpp:28-32): a [d][n]
matrix is d rows of n/32 blocks of {float scale; int8 q[32]} (36 bytes), kept
on the device as a uint8 tensor.  Activations are fp32 [batch][n]; the
product out[b][i] = sum_k float(q[i][k]) * scale[i][k/32] * x[b][k] is fp32.
"""
from __future__ import annotations

from . import _native as N
from .attention import _dev, _stream_ptr

FULL_ROWS = 0    # matmul (src/model_q8.cpp:92-125)
LAST_BLOCK = 1   # matmul_bulk (src/model_q8.cpp:382-420): only the last 32 columns count
BLOCK = 32
BLOCK_BYTES = 36


def q8_matmul(w, x, out, semantics: int = FULL_ROWS, stream=None) -> None:
    """out[batch][d] = x[batch][n] . W[d][n]^T on the GPU, W packed BlockQ8 (uint8 tensor)."""
    import torch

    if x.dim() != 2 or out.dim() != 2:
        raise N.NitroError(N.INVALID_ARGUMENT, "q8_matmul", "x and out must be 2-D")
    batch, n = x.shape
    d = out.shape[1]
    if out.shape[0] != batch:
        raise N.NitroError(N.INVALID_ARGUMENT, "q8_matmul", "x and out batch sizes differ")
    if n % BLOCK:
        raise N.NitroError(N.INVALID_ARGUMENT, "q8_matmul", "n must be a multiple of 32")
    if w.dtype != torch.uint8 or w.numel() != d * (n // BLOCK) * BLOCK_BYTES:
        raise N.NitroError(N.INVALID_ARGUMENT, "q8_matmul",
                           f"w must hold {d} x {n // BLOCK} BlockQ8 ({d * (n // BLOCK) * BLOCK_BYTES} bytes)")
    if not w.is_contiguous():
        raise N.NitroError(N.INVALID_ARGUMENT, "q8_matmul", "w must be contiguous")
    if w.device.type != "cuda":
        raise TypeError("w must be a GPU tensor")
    N.call("nitro_q8_matmul", w.data_ptr(), _dev(x, "x"), _dev(out, "out"), batch, n, d,
           semantics, _stream_ptr(stream))
