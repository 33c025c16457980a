"""Python handles over the C++ page bookkeeping (src/pagedMemory.hpp semantics).

BlockManager wraps one KVBlock_Manager + PrefixCacheManager pair
(src/pagedMemory.hpp:86-229); Sequence wraps Sequence (:233-285).  Method
names follow the reference.  Where the reference calls exit(1) these raise
NitroError with status OUT_OF_PAGES.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _native as N

BLOCK_SIZE = 16
FNV_OFFSET_BASIS = 14695981039346656037


def _i32_array(values) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(values, dtype=np.int64).astype(np.int32))


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(N._i32p)


def hash_block_state(parent_hash: int, tokens) -> int:
    """src/pagedMemory.hpp:14-24."""
    t = _i32_array(tokens)
    return int(N.lib().nitro_hash_block_state(parent_hash, _ptr(t), t.size))


class BlockManager:
    def __init__(self, total_blocks: int):
        h = ctypes.c_void_p()
        N.call("nitro_bm_create", total_blocks, ctypes.byref(h))
        self._h = h
        self.total_blocks = total_blocks

    @property
    def handle(self):
        return self._h

    def close(self):
        if getattr(self, "_h", None):
            N.lib().nitro_bm_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def allocate_block(self) -> int:
        out = ctypes.c_int32()
        N.call("nitro_bm_allocate_block", self._h, ctypes.byref(out))
        return out.value

    def inc_ref_count(self, i: int) -> None:
        N.call("nitro_bm_inc_ref_count", self._h, i)

    def free_block(self, i: int) -> None:
        N.call("nitro_bm_free_block", self._h, i)

    def force_free_block(self, i: int) -> None:
        N.call("nitro_bm_force_free_block", self._h, i)

    def get_free_count(self) -> int:
        out = ctypes.c_int32()
        N.call("nitro_bm_get_free_count", self._h, ctypes.byref(out))
        return out.value

    def get_block(self, i: int) -> dict:
        info = N.nitro_block_info()
        N.call("nitro_bm_get_block", self._h, i, ctypes.byref(info))
        return {"num_tokens": info.num_tokens, "ref_count": info.ref_count,
                "parent_id": info.parent_id, "child_count": info.child_count}

    def is_cached(self, i: int) -> bool:
        out = ctypes.c_int32()
        N.call("nitro_bm_is_cached", self._h, i, ctypes.byref(out))
        return bool(out.value)

    def check_cache(self, block_hash: int) -> int:
        out = ctypes.c_int32()
        N.call("nitro_bm_check_cache", self._h, block_hash, ctypes.byref(out))
        return out.value

    def insert_cache(self, block_hash: int, i: int, parent: int) -> None:
        N.call("nitro_bm_insert_cache", self._h, block_hash, i, parent)

    def evict_lru_block(self) -> None:
        N.call("nitro_bm_evict_lru_block", self._h)

    def _ids(self, fn: str) -> list[int]:
        n = ctypes.c_int32()
        N.call(fn, self._h, None, 0, ctypes.byref(n))
        buf = np.zeros(max(n.value, 1), dtype=np.int32)
        N.call(fn, self._h, _ptr(buf), buf.size, ctypes.byref(n))
        return buf[:n.value].tolist()

    def free_list(self) -> list[int]:
        return self._ids("nitro_bm_free_list")

    def evictable_leaves(self) -> list[int]:
        """Front (most recently made evictable) to back (next to evict)."""
        return self._ids("nitro_bm_evictable_leaves")

    def cache_entries(self) -> list[tuple[int, int]]:
        n = ctypes.c_int32()
        N.call("nitro_bm_cache_entries", self._h, None, None, 0, ctypes.byref(n))
        k = max(n.value, 1)
        hs = np.zeros(k, dtype=np.uint64)
        ids = np.zeros(k, dtype=np.int32)
        N.call("nitro_bm_cache_entries", self._h, hs.ctypes.data_as(N._u64p), _ptr(ids), k,
               ctypes.byref(n))
        return [(int(hs[i]), int(ids[i])) for i in range(n.value)]

    def reverse_entries(self) -> list[tuple[int, int]]:
        n = ctypes.c_int32()
        N.call("nitro_bm_reverse_entries", self._h, None, None, 0, ctypes.byref(n))
        k = max(n.value, 1)
        hs = np.zeros(k, dtype=np.uint64)
        ids = np.zeros(k, dtype=np.int32)
        N.call("nitro_bm_reverse_entries", self._h, _ptr(ids), hs.ctypes.data_as(N._u64p), k,
               ctypes.byref(n))
        return [(int(ids[i]), int(hs[i])) for i in range(n.value)]


class Sequence:
    def __init__(self, seq_id: int):
        h = ctypes.c_void_p()
        N.call("nitro_seq_create", seq_id, ctypes.byref(h))
        self._h = h
        self.seq_id = seq_id

    @property
    def handle(self):
        return self._h

    def close(self):
        if getattr(self, "_h", None):
            N.lib().nitro_seq_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def allocate_next_token(self, token: int, bm: BlockManager) -> None:
        N.call("nitro_seq_allocate_next_token", self._h, bm.handle, int(token))

    def flush_cache(self, bm: BlockManager) -> None:
        N.call("nitro_seq_flush_cache", self._h, bm.handle)

    def release(self, bm: BlockManager) -> None:
        N.call("nitro_seq_release", self._h, bm.handle)

    def prefix_walk(self, prompt, bm: BlockManager, start: int = 0,
                    require_empty_buffer: bool = False) -> int:
        t = _i32_array(prompt)
        out = ctypes.c_int32()
        N.call("nitro_seq_prefix_walk", self._h, bm.handle, _ptr(t), t.size, start,
               int(require_empty_buffer), ctypes.byref(out))
        return out.value

    def ingest_prompt(self, prompt, bm: BlockManager, enable_prefix_caching: bool) -> int:
        t = _i32_array(prompt)
        out = ctypes.c_int32()
        N.call("nitro_seq_ingest_prompt", self._h, bm.handle, _ptr(t), t.size,
               int(enable_prefix_caching), ctypes.byref(out))
        return out.value

    def _state(self):
        c, b, n = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
        h = ctypes.c_uint64()
        N.call("nitro_seq_state", self._h, ctypes.byref(c), ctypes.byref(h), ctypes.byref(b),
               ctypes.byref(n))
        return c.value, h.value, b.value, n.value

    @property
    def logical_token_count(self) -> int:
        return self._state()[0]

    @property
    def current_hash(self) -> int:
        return self._state()[1]

    def _list(self, fn: str) -> list[int]:
        n = ctypes.c_int32()
        N.call(fn, self._h, None, 0, ctypes.byref(n))
        buf = np.zeros(max(n.value, 1), dtype=np.int32)
        N.call(fn, self._h, _ptr(buf), buf.size, ctypes.byref(n))
        return buf[:n.value].tolist()

    @property
    def block_table(self) -> list[int]:
        return self._list("nitro_seq_block_table")

    @property
    def token_buffer(self) -> list[int]:
        return self._list("nitro_seq_token_buffer")


def pack_block_tables(seqs, max_pages: int | None = None) -> np.ndarray:
    """Dense int32 [len(seqs)][max_pages] block tables (unused entries 0)."""
    if max_pages is None:
        max_pages = max(1, max(len(s.block_table) for s in seqs))
    arr = (ctypes.c_void_p * len(seqs))(*[s.handle.value for s in seqs])
    out = np.zeros((len(seqs), max_pages), dtype=np.int32)
    N.call("nitro_pack_block_tables", arr, len(seqs), max_pages, _ptr(out))
    return out
