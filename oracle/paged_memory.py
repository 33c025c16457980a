"""Pure-Python restatement of the reference's page bookkeeping — TEST INFRASTRUCTURE ONLY.

Follows src/pagedMemory.hpp:9-285 (KVBlock_Manager, PrefixCacheManager,
Sequence, hash_block_state) and the prefix-hit walk of ingest_prompt
(src/model_q8.cpp:695-724) statement by statement, for small cases.  Where the
reference calls exit(1) this raises OutOfPages instead.  Pinned by the golden
traces that tests/golden/make_golden.py records from the reference's own
compiled code, and by the FNV-1a-64 specification vectors.
"""
from __future__ import annotations

import numpy as np

BLOCK_SIZE = 16
FNV_OFFSET_BASIS = 14695981039346656037
FNV_PRIME = 1099511628211
_MASK = (1 << 64) - 1


class OutOfPages(Exception):
    """The reference would have called exit(1) (src/pagedMemory.hpp:96,117,212)."""


def fnv1a64_bytes(data: bytes, state: int = FNV_OFFSET_BASIS) -> int:
    """FNV-1a 64 over a byte string (xor the byte, then multiply by the prime)."""
    h = state
    for byte in data:
        h ^= byte
        h = (h * FNV_PRIME) & _MASK
    return h


def hash_block_state(parent_hash: int, tokens) -> int:
    """src/pagedMemory.hpp:14-24 — FNV-1a continued from parent_hash over each
    int32 token's 4 little-endian bytes."""
    return fnv1a64_bytes(np.asarray(tokens, dtype="<i4").tobytes(), parent_hash)


class KVBlock:
    __slots__ = ("physical_id", "num_tokens", "ref_count", "parent_id", "child_count")

    def __init__(self, i: int):
        self.physical_id = i
        self.num_tokens = 0
        self.ref_count = 0
        self.parent_id = -1
        self.child_count = 0


class KVBlockManager:
    """src/pagedMemory.hpp:86-160 (bookkeeping only; K/V storage lives elsewhere)."""

    def __init__(self, total_blocks: int):
        self.blocks = [KVBlock(i) for i in range(total_blocks)]
        self.free_list = list(range(total_blocks))

    def allocate_block(self, cache: "PrefixCacheManager") -> int:  # :113-128
        if not self.free_list:
            cache.evict_lru_block()
            if not self.free_list:
                raise OutOfPages("Out of Memory. Eviction Failed")
        i = self.free_list.pop()
        b = self.blocks[i]
        b.ref_count = 1
        b.num_tokens = 0
        b.parent_id = -1
        b.child_count = 0
        return i

    def inc_ref_count(self, i: int, cache: "PrefixCacheManager") -> None:  # :129-132
        self.blocks[i].ref_count += 1
        cache.evaluate_evictability(i)

    def get_free_count(self) -> int:  # :134-136
        return len(self.free_list)

    def free_block(self, i: int, cache: "PrefixCacheManager") -> None:  # :137-144
        self.blocks[i].ref_count -= 1
        cache.evaluate_evictability(i)
        if self.blocks[i].ref_count == 0 and not cache.is_cached(i):
            self.blocks[i].num_tokens = 0
            self.free_list.append(i)

    def force_free_block(self, i: int) -> None:  # :145-151
        b = self.blocks[i]
        b.num_tokens = 0
        b.ref_count = 0
        b.parent_id = -1
        b.child_count = 0
        self.free_list.append(i)

    def get_block(self, i: int) -> KVBlock:  # :154-156
        return self.blocks[i]


class PrefixCacheManager:
    """src/pagedMemory.hpp:163-229.  evictable_leaves is kept front->back as a
    Python list (index 0 = front = most recently made evictable)."""

    def __init__(self, mem: KVBlockManager, total_blocks: int):
        self.mem = mem
        self.cache_map: dict[int, int] = {}
        self.reverse_map: dict[int, int] = {}
        self.evictable_leaves: list[int] = []
        self.min_free_blocks = max(1, int(total_blocks * 0.05))
        self.target_free_blocks = max(2, int(total_blocks * 0.2))

    def is_cached(self, i: int) -> bool:  # :168-170
        return i in self.reverse_map

    def evaluate_evictability(self, i: int) -> None:  # :171-186
        if not self.is_cached(i):
            return
        b = self.mem.get_block(i)
        evictable = b.ref_count == 0 and b.child_count == 0
        in_lru = i in self.evictable_leaves
        if evictable and not in_lru:
            self.evictable_leaves.insert(0, i)
        elif not evictable and in_lru:
            self.evictable_leaves.remove(i)

    def check_cache(self, h: int) -> int:  # :187-192
        return self.cache_map.get(h, -1)

    def insert_cache(self, h: int, i: int, parent: int) -> None:  # :193-205
        self.cache_map[h] = i
        self.reverse_map[i] = h
        b = self.mem.get_block(i)
        b.parent_id = parent
        b.child_count = 0
        if parent != -1:
            self.mem.get_block(parent).child_count += 1
            self.evaluate_evictability(parent)
        self.evaluate_evictability(i)

    def evict_lru_block(self) -> None:  # :206-229
        if self.mem.get_free_count() >= self.min_free_blocks:
            return
        while self.mem.get_free_count() < self.target_free_blocks:
            if not self.evictable_leaves:
                if self.mem.get_free_count() > 0:
                    break
                raise OutOfPages("High Traffic.No evictable leaves left!")
            evict_id = self.evictable_leaves.pop()
            # reverse_map[evict_id] default-constructs 0 when absent (std::unordered_map::operator[])
            h = self.reverse_map.get(evict_id, 0)
            self.cache_map.pop(h, None)
            self.reverse_map.pop(evict_id, None)
            parent = self.mem.get_block(evict_id).parent_id
            if parent != -1:
                self.mem.get_block(parent).child_count -= 1
                self.evaluate_evictability(parent)
            self.mem.force_free_block(evict_id)


class Sequence:
    """src/pagedMemory.hpp:233-285."""

    def __init__(self, seq_id: int):
        self.seq_id = seq_id
        self.block_table: list[int] = []
        self.logical_token_count = 0
        self.current_hash = FNV_OFFSET_BASIS
        self.token_buffer: list[int] = []

    def allocate_next_token(self, token: int, mem: KVBlockManager,
                            cache: PrefixCacheManager) -> None:  # :245-264
        if len(self.token_buffer) == BLOCK_SIZE:
            self.current_hash = hash_block_state(self.current_hash, self.token_buffer)
            finished = self.block_table[-1]
            parent = self.block_table[-2] if len(self.block_table) > 1 else -1
            cache.insert_cache(self.current_hash, finished, parent)
            self.token_buffer.clear()
        if self.logical_token_count % BLOCK_SIZE == 0:
            self.block_table.append(mem.allocate_block(cache))
        self.token_buffer.append(token)
        mem.get_block(self.block_table[-1]).num_tokens += 1
        self.logical_token_count += 1

    def flush_cache(self, cache: PrefixCacheManager) -> None:  # :265-273
        if len(self.token_buffer) == BLOCK_SIZE:
            self.current_hash = hash_block_state(self.current_hash, self.token_buffer)
            parent = self.block_table[-2] if len(self.block_table) > 1 else -1
            cache.insert_cache(self.current_hash, self.block_table[-1], parent)

    def release(self, mem: KVBlockManager, cache: PrefixCacheManager) -> None:  # :274-283
        for i in self.block_table:
            mem.free_block(i, cache)
        self.block_table.clear()
        self.token_buffer.clear()
        self.logical_token_count = 0
        self.current_hash = FNV_OFFSET_BASIS


def ingest_prompt(prompt, seq: Sequence, mem: KVBlockManager, cache: PrefixCacheManager,
                  enable_prefix_caching: bool) -> int:
    """Bookkeeping of src/model_q8.cpp:695-724: the prefix-hit walk over full
    16-token chunks, then allocate_next_token for every remaining token (what
    forward_prefill_chunk does first, :428-430).  Returns logical_token_count."""
    p = 0
    prompt = list(prompt)
    if enable_prefix_caching:
        while p + BLOCK_SIZE <= len(prompt):
            chunk = prompt[p:p + BLOCK_SIZE]
            h = hash_block_state(seq.current_hash, chunk)
            hit = cache.check_cache(h)
            if hit != -1:
                mem.inc_ref_count(hit, cache)
                seq.block_table.append(hit)
                seq.logical_token_count += BLOCK_SIZE
                seq.current_hash = h
                p += BLOCK_SIZE
            else:
                break
    for tok in prompt[p:]:
        seq.allocate_next_token(tok, mem, cache)
    return seq.logical_token_count


# ---- trace replay (shared op codes with the reference driver) --------------
OP_ALLOC, OP_INC, OP_FREE, OP_FORCE_FREE, OP_CHECK, OP_INSERT, OP_EVICT = 1, 2, 3, 4, 5, 6, 7
OP_SEQ_NEW, OP_SEQ_APPEND, OP_SEQ_FLUSH, OP_SEQ_RELEASE, OP_INGEST = 8, 9, 10, 11, 12
OP_FREE_COUNT, OP_IS_CACHED = 13, 14


class World:
    """A block manager, its prefix cache and sequence slots, driven by op tuples
    (op, a, b, hash, tokens) — the same ops the reference driver accepts."""

    def __init__(self, total_blocks: int, max_seqs: int):
        self.mem = KVBlockManager(total_blocks)
        self.cache = PrefixCacheManager(self.mem, total_blocks)
        self.seqs: list[Sequence | None] = [None] * max_seqs

    def op(self, op: int, a: int = 0, b: int = 0, h: int = 0, toks=()) -> tuple[int, int]:
        """Returns (status, result): status 1 = the reference would have exited."""
        try:
            if op == OP_ALLOC:
                return 0, self.mem.allocate_block(self.cache)
            if op == OP_INC:
                self.mem.inc_ref_count(a, self.cache)
            elif op == OP_FREE:
                self.mem.free_block(a, self.cache)
            elif op == OP_FORCE_FREE:
                self.mem.force_free_block(a)
            elif op == OP_CHECK:
                return 0, self.cache.check_cache(h)
            elif op == OP_INSERT:
                self.cache.insert_cache(h, a, b)
            elif op == OP_EVICT:
                self.cache.evict_lru_block()
            elif op == OP_FREE_COUNT:
                return 0, self.mem.get_free_count()
            elif op == OP_IS_CACHED:
                return 0, int(self.cache.is_cached(a))
            elif op == OP_SEQ_NEW:
                self.seqs[a] = Sequence(a)
            elif op == OP_SEQ_APPEND:
                self.seqs[a].allocate_next_token(b, self.mem, self.cache)
            elif op == OP_SEQ_FLUSH:
                self.seqs[a].flush_cache(self.cache)
            elif op == OP_SEQ_RELEASE:
                self.seqs[a].release(self.mem, self.cache)
            elif op == OP_INGEST:
                return 0, ingest_prompt(toks, self.seqs[a], self.mem, self.cache, b != 0)
            else:
                return 2, 0
        except OutOfPages:
            return 1, 0
        return 0, 0

    def snapshot(self) -> dict:
        return {
            "free_list": list(self.mem.free_list),
            "blocks": [[b.ref_count, b.num_tokens, b.parent_id, b.child_count]
                       for b in self.mem.blocks],
            "lru": list(self.cache.evictable_leaves),
            "cache_map": sorted([h, i] for h, i in self.cache.cache_map.items()),
            "reverse_map": sorted([i, h] for i, h in self.cache.reverse_map.items()),
            "seqs": [None if s is None else {
                "count": s.logical_token_count, "hash": s.current_hash,
                "buffer": list(s.token_buffer), "table": list(s.block_table)}
                for s in self.seqs],
        }


def decode_snapshot(words, total_blocks: int, max_seqs: int) -> dict:
    """Parses the int32 stream written by the reference driver's ref_snapshot."""
    w = [int(x) for x in words]
    i = 0

    def take(n):
        nonlocal i
        out = w[i:i + n]
        i += n
        return out

    def u64(lo, hi):
        return (lo & 0xffffffff) | ((hi & 0xffffffff) << 32)

    n = take(1)[0]
    free_list = take(n)
    blocks = [take(4) for _ in range(total_blocks)]
    n = take(1)[0]
    lru = take(n)
    n = take(1)[0]
    cache_map = []
    for _ in range(n):
        lo, hi, bid = take(3)
        cache_map.append([u64(lo, hi), bid])
    n = take(1)[0]
    reverse_map = []
    for _ in range(n):
        bid, lo, hi = take(3)
        reverse_map.append([bid, u64(lo, hi)])
    seqs = []
    for _ in range(max_seqs):
        if take(1)[0] == 0:
            seqs.append(None)
            continue
        count, lo, hi = take(3)
        nb = take(1)[0]
        buf = take(nb)
        nt = take(1)[0]
        table = take(nt)
        seqs.append({"count": count, "hash": u64(lo, hi), "buffer": buf, "table": table})
    assert i == len(w), (i, len(w))
    return {"free_list": free_list, "blocks": blocks, "lru": lru, "cache_map": cache_map,
            "reverse_map": reverse_map, "seqs": seqs}
