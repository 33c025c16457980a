"""Pins the Python restatement of the reference's page bookkeeping and FNV-1a
prefix hash against the reference's own traces and the FNV specification."""
import numpy as np
import pytest

from make_golden import state_digest
from oracle import paged_memory as pm
from oracle import ref


def test_fnv1a64_specification_vectors():
    # Published FNV-1a 64-bit test vectors.
    assert pm.fnv1a64_bytes(b"") == 0xCBF29CE484222325
    assert pm.fnv1a64_bytes(b"a") == 0xAF63DC4C8601EC8C
    assert pm.fnv1a64_bytes(b"foobar") == 0x85944171F73967E8


def test_hash_block_state_closed_form():
    rng = np.random.default_rng(3)
    toks = rng.integers(-2**31, 2**31, size=48, dtype=np.int64).astype(np.int32)
    # block k's hash == FNV-1a-64 over the LE bytes of tokens[0..16k)
    h = pm.FNV_OFFSET_BASIS
    for k in range(3):
        h = pm.hash_block_state(h, toks[16 * k:16 * (k + 1)])
        assert h == pm.fnv1a64_bytes(toks[:16 * (k + 1)].astype("<i4").tobytes())
    # byte order: token 0x64636261 hashes like the string "abcd"
    assert pm.hash_block_state(pm.FNV_OFFSET_BASIS, [0x64636261]) == pm.fnv1a64_bytes(b"abcd")


def test_fnv_matches_reference_golden(golden_fnv):
    for c in golden_fnv["cases"]:
        assert pm.hash_block_state(c["parent"], c["tokens"]) == c["hash"]
    h = pm.FNV_OFFSET_BASIS
    for want in golden_fnv["shared_263_chain"]:
        h = pm.hash_block_state(h, [263] * 16)
        assert h == want


def replay(world, trace):
    for i, (op, want) in enumerate(zip(trace["ops"], trace["steps"])):
        st, res = world.op(op["op"], op.get("a", 0), op.get("b", 0), op.get("h", 0),
                           op.get("toks", ()))
        got = [st, res, state_digest(world.snapshot())]
        assert got == want, (trace["name"], i, op, got, want)
    assert world.snapshot() == trace["final"]


def test_python_bookkeeping_replays_reference_traces(golden_traces):
    assert len(golden_traces) >= 6
    for trace in golden_traces:
        replay(pm.World(trace["total_blocks"], trace["max_seqs"]), trace)


def test_traces_cover_evictions_and_exhaustion(golden_traces):
    statuses = [s[0] for t in golden_traces for s in t["steps"]]
    assert 1 in statuses  # the reference exited (pool exhausted, nothing evictable)
    ops = {op["op"] for t in golden_traces for op in t["ops"]}
    assert {pm.OP_ALLOC, pm.OP_INC, pm.OP_FREE, pm.OP_FORCE_FREE, pm.OP_CHECK, pm.OP_INSERT,
            pm.OP_EVICT, pm.OP_SEQ_NEW, pm.OP_SEQ_APPEND, pm.OP_SEQ_FLUSH, pm.OP_SEQ_RELEASE,
            pm.OP_INGEST} <= ops


def test_lifo_fresh_pool_and_exp4_sharing(golden_traces):
    exp4 = next(t for t in golden_traces if t["name"] == "exp4_shared_prompt")
    fin = exp4["final"]
    # both users released: the 16 shared pages stay cached (not freed), LIFO order kept
    assert len(fin["cache_map"]) == 16
    w = pm.World(100, 2)
    w.op(pm.OP_SEQ_NEW, 0)
    w.op(pm.OP_INGEST, 0, 1, toks=[263] * 256)
    assert w.seqs[0].block_table == list(range(99, 83, -1))  # fresh pool hands out N-1, N-2, ...
    w.op(pm.OP_SEQ_FLUSH, 0)
    w.op(pm.OP_SEQ_NEW, 1)
    w.op(pm.OP_INGEST, 1, 1, toks=[263] * 256)
    assert w.seqs[1].block_table == w.seqs[0].block_table
    assert all(w.mem.blocks[i].ref_count == 2 for i in w.seqs[0].block_table)


@pytest.mark.skipif(not ref.available(), reason="reference build (oracle/_ref) not present")
def test_python_bookkeeping_live_random_vs_reference():
    import random

    from make_golden import run_trace, seq_workload
    for seed in range(3):
        rng = random.Random(seed)
        blocks = rng.choice([10, 20, 33])
        trace = run_trace("live", blocks, 5, seq_workload(100 + seed, blocks, 5, 120))
        replay(pm.World(blocks, 5), trace)
