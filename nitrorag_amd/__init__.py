"""MI355X (gfx950) paged-attention path for NitroRAG's inference engine.

The compute lives in libnitro_paged_attn.so (HIP kernels + C ABI, see
include/nitro_paged_attn.h); this package only binds it:
  paged_memory  BlockManager / Sequence / hash_block_state (src/pagedMemory.hpp semantics)
  attention     KVPool: device pools, batch uploads, KV append, decode, prefill
  q8            Q8_0 matrix product (BlockQ8 weights, fp32 activations)
  model         Model: the forward passes around attention (reference model file layout)
  build         compiles the library in-tree with hipcc for gfx950
"""
from ._native import NitroError, lib  # noqa: F401
from .attention import KVPool  # noqa: F401
from .model import Model  # noqa: F401
from .q8 import q8_matmul  # noqa: F401
from .scheduler import ContinuousScheduler  # noqa: F401
from .paged_memory import (BLOCK_SIZE, FNV_OFFSET_BASIS, BlockManager, Sequence,  # noqa: F401
                           hash_block_state, pack_block_tables)
