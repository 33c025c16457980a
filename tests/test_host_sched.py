"""The shipped continuous scheduler's host half (nitro_sched_create / add_request
/ plan / commit, C ABI) against the reference's Continuous_Scheduler
(src/pagedMemory.hpp:287-399) recorded in tests/golden/sched_traces.*: fed the
reference's tokens, every step leaves the same scheduler state words and the
same block-manager state, and plans the same forward work as the oracle.
Host code only (no device calls)."""
import numpy as np
import pytest

import nitrorag_amd as na
from nitrorag_amd import _native as N
from oracle import paged_memory as pm
from oracle import scheduler as sc


def _native_bm(bm, total):
    blocks = []
    for i in range(total):
        b = bm.get_block(i)
        blocks.append([b["ref_count"], b["num_tokens"], b["parent_id"], b["child_count"]])
    return {"free_list": bm.free_list(), "blocks": blocks, "lru": bm.evictable_leaves(),
            "cache_map": [[h, i] for h, i in bm.cache_entries()],
            "reverse_map": [[i, h] for i, h in bm.reverse_entries()]}


def _golden_bm(tr, t):
    d = pm.decode_snapshot(tr.bm(t), tr.total_blocks, 0)
    d.pop("seqs")
    return d


def test_native_scheduler_replays_reference_steps(golden_sched):
    _, traces = golden_sched
    for tr in traces:
        bm = na.BlockManager(tr.total_blocks)
        S = na.ContinuousScheduler(bm, tr.budget, 20)
        mem = pm.KVBlockManager(tr.total_blocks)
        cache = pm.PrefixCacheManager(mem, tr.total_blocks)
        O = sc.ContinuousScheduler(mem, cache, tr.budget)
        last = max(tr.arrivals)
        t = 0
        while True:
            for rid, prompt in tr.arrivals.get(t, []):
                S.add_request(rid, prompt)
                O.add_request(sc.Request(rid, prompt))
            if not S.has_active_requests() and t >= last:
                assert not O.has_active_requests()
                break
            p = S.plan()
            q = O.plan()
            # the planned forward work equals the oracle's
            assert p.decode_ids == [r.req_id for r in q.decode_reqs], (tr.name, t)
            assert p.decode_tokens == q.decode_tokens and p.decode_positions == q.decode_positions
            if q.prefill_req is None:
                assert p.prefill_id == -1 and p.prefill_length == 0
            else:
                assert (p.prefill_id, p.prefill_start, p.prefill_length, p.prefill_finishes) == (
                    q.prefill_req.req_id, q.prefill_start, len(q.prefill_tokens),
                    q.prefill_req.is_prefill_done)
                assert S.prompts[p.prefill_id][p.prefill_start:p.prefill_start + p.prefill_length] == \
                    q.prefill_tokens
            after = {r["req_id"]: r for r in sc.decode_state(tr.state(t))["requests"]}
            pt = after[p.prefill_id]["next"] if p.prefill_id >= 0 else 0
            dt = [after[i]["next"] for i in p.decode_ids]
            S.commit(pt, dt)
            O.commit(q, pt, dt)
            assert S.state_words() == tr.state(t), (tr.name, t)
            assert _native_bm(bm, tr.total_blocks) == _golden_bm(tr, t), (tr.name, t)
            t += 1
        assert t == tr.steps
        # observers agree with the state words
        for r in sc.decode_state(tr.state(t - 1))["requests"]:
            st = S.request_status(r["req_id"])
            assert S.generated(r["req_id"]) == r["generated"]
            assert (st["prefill_idx"], st["is_prefill_done"], st["is_finished"],
                    st["next_token_to_process"], st["logical_token_count"]) == (
                r["prefill_idx"], r["done"], r["finished"], r["next"], r["count"])
            S.drop_request(r["req_id"])  # finished and released by the last step
        assert S.state_words() == [0, 0, 0]
        S.close()


def _status(fn):
    with pytest.raises(na.NitroError) as e:
        fn()
    return e.value.status


def test_scheduler_argument_and_order_errors():
    bm = na.BlockManager(8)
    S = na.ContinuousScheduler(bm, 4, 2)
    assert _status(lambda: S.add_request(0, [])) == N.INVALID_ARGUMENT
    S.add_request(0, [1, 2, 3])
    assert _status(lambda: S.add_request(0, [4])) == N.INVALID_ARGUMENT       # duplicate id
    assert _status(lambda: S.commit(0, [])) == N.INVALID_ARGUMENT            # nothing planned
    p = S.plan()
    assert (p.prefill_id, p.prefill_length, p.prefill_finishes) == (0, 3, True)
    assert _status(lambda: S.plan()) == N.INVALID_ARGUMENT                   # not committed
    assert _status(lambda: S.add_request(1, [5])) == N.INVALID_ARGUMENT
    assert _status(lambda: S.commit(7, [1])) == N.INVALID_ARGUMENT           # no decode rows
    S.commit(7, [])
    assert _status(lambda: S.drop_request(0)) == N.INVALID_ARGUMENT          # still running
    assert _status(lambda: S.drop_request(9)) == N.INVALID_ARGUMENT
    p = S.plan()
    assert p.decode_ids == [0] and p.decode_tokens == [7] and p.decode_positions == [3]
    S.commit(0, [8])
    assert S.request_status(0)["is_finished"] == 1 and S.generated(0) == [7, 8]
    assert _status(lambda: S.drop_request(0)) == N.INVALID_ARGUMENT          # not yet released
    p = S.plan()                                                             # releases it
    assert p.decode_ids == [] and p.prefill_id == -1
    S.commit(0, [])
    assert not S.has_active_requests()
    S.drop_request(0)
    lib = N.lib()
    assert lib.nitro_sched_create(None, 4, 2, None) == N.INVALID_ARGUMENT
    assert lib.nitro_sched_step(None, None, None, 0, None) == N.INVALID_ARGUMENT


def test_scheduler_out_of_pages_is_a_status():
    """Where the reference calls exit(1) (src/pagedMemory.hpp:117) the
    scheduler returns NITRO_ERR_OUT_OF_PAGES."""
    bm = na.BlockManager(2)
    S = na.ContinuousScheduler(bm, 256, 20)
    S.add_request(0, list(range(40)))  # needs 3 pages
    assert _status(lambda: S.plan()) == N.OUT_OF_PAGES
