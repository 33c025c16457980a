"""The shipped C++ page bookkeeping (through the C ABI) replays the reference's
own traces bit-exactly: per-op results and full-state digests (free-list
order, per-page counts/parents, LRU order, prefix-cache maps, block tables)."""
import ctypes
import os
import re

import numpy as np
import pytest

import nitrorag_amd as na
from nitrorag_amd import _native as N
from make_golden import state_digest
from oracle import paged_memory as pm

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


class ProductWorld:
    """The reference driver's op set, executed by the shipped library."""

    def __init__(self, total_blocks, max_seqs):
        self.bm = na.BlockManager(total_blocks)
        self.total_blocks = total_blocks
        self.seqs = [None] * max_seqs

    def op(self, op, a=0, b=0, h=0, toks=()):
        bm = self.bm
        try:
            if op == pm.OP_ALLOC:
                return 0, bm.allocate_block()
            if op == pm.OP_INC:
                bm.inc_ref_count(a)
            elif op == pm.OP_FREE:
                bm.free_block(a)
            elif op == pm.OP_FORCE_FREE:
                bm.force_free_block(a)
            elif op == pm.OP_CHECK:
                return 0, bm.check_cache(h)
            elif op == pm.OP_INSERT:
                bm.insert_cache(h, a, b)
            elif op == pm.OP_EVICT:
                bm.evict_lru_block()
            elif op == pm.OP_FREE_COUNT:
                return 0, bm.get_free_count()
            elif op == pm.OP_IS_CACHED:
                return 0, int(bm.is_cached(a))
            elif op == pm.OP_SEQ_NEW:
                if self.seqs[a] is not None:
                    self.seqs[a].close()
                self.seqs[a] = na.Sequence(a)
            elif op == pm.OP_SEQ_APPEND:
                self.seqs[a].allocate_next_token(b, bm)
            elif op == pm.OP_SEQ_FLUSH:
                self.seqs[a].flush_cache(bm)
            elif op == pm.OP_SEQ_RELEASE:
                self.seqs[a].release(bm)
            elif op == pm.OP_INGEST:
                return 0, self.seqs[a].ingest_prompt(toks, bm, b != 0)
            else:
                return 2, 0
        except na.NitroError as e:
            if e.status == N.OUT_OF_PAGES:
                return 1, 0
            raise
        return 0, 0

    def snapshot(self):
        bm = self.bm
        blocks = []
        for i in range(self.total_blocks):
            b = bm.get_block(i)
            blocks.append([b["ref_count"], b["num_tokens"], b["parent_id"], b["child_count"]])
        seqs = []
        for s in self.seqs:
            if s is None:
                seqs.append(None)
                continue
            seqs.append({"count": s.logical_token_count, "hash": s.current_hash,
                         "buffer": s.token_buffer, "table": s.block_table})
        return {"free_list": bm.free_list(), "blocks": blocks, "lru": bm.evictable_leaves(),
                "cache_map": [[h, i] for h, i in bm.cache_entries()],
                "reverse_map": [[i, h] for i, h in bm.reverse_entries()], "seqs": seqs}


def replay(world, trace):
    for i, (op, want) in enumerate(zip(trace["ops"], trace["steps"])):
        st, res = world.op(op["op"], op.get("a", 0), op.get("b", 0), op.get("h", 0),
                           op.get("toks", ()))
        got = [st, res, state_digest(world.snapshot())]
        assert got == want, (trace["name"], i, op, got, want)
    assert world.snapshot() == trace["final"]


def test_product_bookkeeping_replays_reference_traces(golden_traces):
    for trace in golden_traces:
        replay(ProductWorld(trace["total_blocks"], trace["max_seqs"]), trace)


def test_product_hash_matches_reference_golden(golden_fnv):
    for c in golden_fnv["cases"]:
        assert na.hash_block_state(c["parent"], c["tokens"]) == c["hash"]
    assert na.hash_block_state(na.FNV_OFFSET_BASIS, []) == na.FNV_OFFSET_BASIS


def test_product_bookkeeping_random_vs_oracle():
    """Longer random workloads than the fixtures: product and Python restatement agree."""
    from make_golden import low_level_workload, seq_workload
    for seed, blocks in ((201, 17), (202, 40), (203, 150)):
        for ops in (seq_workload(seed, blocks, 6, 300), low_level_workload(seed, blocks, 300)):
            a, b = ProductWorld(blocks, 6), pm.World(blocks, 6)
            for op in ops:
                args = (op["op"], op.get("a", 0), op.get("b", 0), op.get("h", 0),
                        op.get("toks", ()))
                assert a.op(*args) == b.op(*args)
            assert a.snapshot() == b.snapshot()


def test_scheduler_prefix_walk_variant():
    """The scheduler's walk stops when the token buffer is non-empty
    (src/pagedMemory.hpp:346); ingest_prompt's does not (src/model_q8.cpp:699)."""
    bm = na.BlockManager(16)
    a = na.Sequence(0)
    prompt = list(range(50, 98))
    a.ingest_prompt(prompt, bm, False)
    a.flush_cache(bm)  # 48 tokens: pages 0,1 inserted on the way, page 2 by the flush
    b = na.Sequence(1)
    b.allocate_next_token(7, bm)  # buffer non-empty, current_hash still the FNV basis
    assert b.prefix_walk(prompt, bm, 0, require_empty_buffer=True) == 0
    # ingest's walk hits anyway and appends the shared pages after b's own page
    assert b.prefix_walk(prompt, bm, 0, require_empty_buffer=False) == 48
    assert b.block_table[1:] == a.block_table and b.logical_token_count == 49
    c = na.Sequence(2)
    assert c.prefix_walk(prompt, bm, 0, require_empty_buffer=True) == 48
    assert c.block_table == a.block_table
    assert all(bm.get_block(i)["ref_count"] == 3 for i in a.block_table)


def test_errors_are_status_codes():
    bm = na.BlockManager(2)
    with pytest.raises(na.NitroError) as e:
        bm.get_block(2)
    assert e.value.status == N.INVALID_ARGUMENT
    s = na.Sequence(0)
    for t in range(32):
        s.allocate_next_token(t, bm)
    with pytest.raises(na.NitroError) as e:  # third page: pool of 2, nothing evictable
        s.allocate_next_token(99, bm)
    assert e.value.status == N.OUT_OF_PAGES
    with pytest.raises(na.NitroError):
        na.BlockManager(0)


def test_pack_block_tables():
    bm = na.BlockManager(32)
    seqs = [na.Sequence(i) for i in range(3)]
    for i, s in enumerate(seqs):
        s.ingest_prompt(list(range(1 + 20 * i)), bm, False)
    t = na.pack_block_tables(seqs, 4)
    for i, s in enumerate(seqs):
        bt = s.block_table
        assert t[i, :len(bt)].tolist() == bt and np.all(t[i, len(bt):] == 0)
    with pytest.raises(na.NitroError) as e:
        na.pack_block_tables(seqs, 1)
    assert e.value.status == N.BAD_BLOCK_TABLE


def header_functions():
    with open(os.path.join(ROOT, "include", "nitro_paged_attn.h")) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nitro_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    names = header_functions()
    assert len(names) >= 40
    lib = N.lib()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the binding declares a prototype for each of them
    assert sorted(N.SIGNATURES) == names


def test_device_entry_points_reject_bad_arguments_without_gpu():
    """Argument checks run before any device work (safe on a CPU-only host)."""
    lib = N.lib()
    assert lib.nitro_kvpool_create(0, 1, 64, ctypes.byref(ctypes.c_void_p())) == N.INVALID_ARGUMENT
    assert lib.nitro_kvpool_create(4, 1, 66, ctypes.byref(ctypes.c_void_p())) == N.UNSUPPORTED
    assert lib.nitro_paged_attn_decode(None, 0, None, None, 1, 1, 64, None) == N.INVALID_ARGUMENT
    assert lib.nitro_kv_append(None, 0, None, None, None) == N.INVALID_ARGUMENT
    assert lib.nitro_status_string(4) == b"out of pages"
