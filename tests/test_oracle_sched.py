"""The oracle's continuous scheduler (oracle/scheduler.py) against the
reference's own Continuous_Scheduler (src/pagedMemory.hpp:287-399), recorded
step by step on a tiny random model in tests/golden/sched_traces.*.

- teacher-forced: the oracle's bookkeeping, fed the reference's tokens, gives
  the same scheduler state and block-manager snapshot after every step;
- free-running: the oracle scheduler on the oracle model reproduces every
  token the reference chose and the logits the reference left behind;
- the reference's argmax (src/model_q8.cpp:559-569) on its recorded logits
  gives its recorded tokens, and its quirks hold on hand-made rows."""
import numpy as np
import pytest

from oracle import paged_memory as pm
from oracle import scheduler as sc
from oracle.model import OracleModel, scale_residual_outputs


def _bm_dict(mem, cache):
    return {"free_list": list(mem.free_list),
            "blocks": [[b.ref_count, b.num_tokens, b.parent_id, b.child_count] for b in mem.blocks],
            "lru": list(cache.evictable_leaves),
            "cache_map": sorted([h, i] for h, i in cache.cache_map.items()),
            "reverse_map": sorted([i, h] for i, h in cache.reverse_map.items())}


def _golden_bm(tr, t):
    d = pm.decode_snapshot(tr.bm(t), tr.total_blocks, 0)
    d.pop("seqs")
    return d


def _forced_forward(tr, t):
    """Tokens the reference chose at step t, read from its state after t."""
    after = {r["req_id"]: r for r in sc.decode_state(tr.state(t))["requests"]}

    def forward(p):
        pt = after[p.prefill_req.req_id]["next"] if p.prefill_req is not None else None
        return pt, [after[r.req_id]["next"] for r in p.decode_reqs]
    return forward


def _replay(tr, forward_for_step, budget=None):
    mem = pm.KVBlockManager(tr.total_blocks)
    cache = pm.PrefixCacheManager(mem, tr.total_blocks)
    S = sc.ContinuousScheduler(mem, cache, tr.budget if budget is None else budget)
    last = max(tr.arrivals)
    t = 0
    while True:
        for rid, prompt in tr.arrivals.get(t, []):
            S.add_request(sc.Request(rid, prompt))
        if not S.has_active_requests() and t >= last:
            break
        yield t, S, S.step(forward_for_step(t)), mem, cache
        t += 1
    assert t == tr.steps


def test_teacher_forced_bookkeeping_matches_reference(golden_sched):
    _, traces = golden_sched
    for tr in traces:
        for t, S, p, mem, cache in _replay(tr, lambda t, tr=tr: _forced_forward(tr, t)):
            assert S.state_words() == tr.state(t), (tr.name, t)
            assert _bm_dict(mem, cache) == _golden_bm(tr, t), (tr.name, t)


def test_scenarios_cover_the_schedulers_branches(golden_sched):
    """Chunked prefill, an exhausted budget, prefix hits (including a prompt
    that is entirely cached), eviction and the insert_cache overwrite."""
    _, traces = golden_sched
    seen = set()
    for tr in traces:
        prev_cache = set()
        for t in range(tr.steps):
            st = sc.decode_state(tr.state(t))
            bm = _golden_bm(tr, t)
            for r in st["requests"]:
                if r["done"] and not r["generated"] and r["count"] % 16 == 0 and r["count"] > 0:
                    seen.add("fully_cached_prompt")
                if 0 < r["prefill_idx"] and not r["done"]:
                    seen.add("chunked")
            if st["waiting"] and tr.budget <= len(st["running"]):
                seen.add("budget_exhausted")
            cached = {i for i, _ in bm["reverse_map"]}
            if prev_cache - cached:
                seen.add("evicted")
            if len(bm["reverse_map"]) > len(bm["cache_map"]):
                seen.add("stale_reverse_entry")
            if any(b[0] > 1 for b in bm["blocks"]):
                seen.add("shared_page")
            prev_cache = cached
    assert seen == {"fully_cached_prompt", "chunked", "budget_exhausted", "evicted",
                    "stale_reverse_entry", "shared_page"}, seen


@pytest.fixture(scope="module")
def sched_model(golden_sched, golden_model):
    meta, _ = golden_sched
    blob, _, _ = golden_model
    return OracleModel(scale_residual_outputs(blob, meta["out_scale"]))


def test_oracle_model_reproduces_reference_steps(golden_sched, sched_model):
    _, traces = golden_sched
    for tr in traces:
        fwd = sc.OracleForward(sched_model, tr.total_blocks)
        for t, S, p, mem, cache in _replay(tr, lambda t: fwd):
            assert S.state_words() == tr.state(t), (tr.name, t)
            idx, val = tr.top(t)
            if tr.kind(t) == 1:
                got = np.take_along_axis(fwd.decode_logits, idx, axis=1)
            elif tr.kind(t) == 2:
                got = fwd.prefill_logits[idx]
            else:
                assert fwd.decode_logits is None and fwd.prefill_logits is None
                continue
            np.testing.assert_allclose(got, val, atol=1e-3, rtol=1e-4, err_msg=f"{tr.name} step {t}")


def test_reference_argmax_on_recorded_rows(golden_sched):
    """The recorded rows' top entry is the token the step chose (decode rows in
    running order; a lone prefill row when its request finished prefill)."""
    _, traces = golden_sched
    for tr in traces:
        for t in range(tr.steps):
            if tr.kind(t) == 0:
                continue
            idx, val = tr.top(t)
            before = sc.decode_state(tr.state(t - 1)) if t else None
            after = {r["req_id"]: r for r in sc.decode_state(tr.state(t))["requests"]}
            if tr.kind(t) == 1:
                running = [rid for rid in before["running"] if not before["requests"][
                    [r["req_id"] for r in before["requests"]].index(rid)]["finished"]]
                assert len(running) == len(idx), (tr.name, t)
                for rid, row_i, row_v in zip(running, idx, val):
                    assert row_v[0] > 0 and row_v[0] > row_v[1]
                    assert after[rid]["next"] == row_i[0], (tr.name, t, rid)


def test_argmax_quirks():
    assert sc.argmax([-1.0, -0.5, -2.0]) == 0           # nothing above 0.0 -> index 0
    assert sc.argmax([0.0, 0.0]) == 0
    assert sc.argmax([0.5, 2.0, 2.0, 1.0]) == 1         # first of equal maxima
    assert sc.argmax([np.nan, 1.0, np.nan, 3.0]) == 3   # NaN never wins
    assert sc.argmax([-0.0, 1e-30]) == 1
