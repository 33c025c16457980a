"""GPU parity of the continuous scheduler's device step (nitro_sched_step: host
plan, one forward over the prefill chunk's rows and the decode rows together
over device-resident block tables, argmax on the device, commit) against the
reference's own Continuous_Scheduler (src/pagedMemory.hpp:287-399) stepping
the same tiny model, recorded in tests/golden/sched_traces.*.

Every step must leave the reference's scheduler state word for word — which
includes every token the device argmax chose (the fixture's decisions win by
at least 0.16, far above fp32 rounding) — and the logits the reference left
behind must match within |gpu - ref| <= 2e-3 + 1e-3*|ref| on the recorded
top entries of each row."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LOGIT_ATOL, LOGIT_RTOL = 2e-3, 1e-3


@pytest.fixture(scope="module", autouse=True)
def gpu():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    import nitrorag_amd  # noqa: F401
    yield
    torch.cuda.synchronize()


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def test_scheduler_steps_match_reference(golden_sched, golden_model):
    import nitrorag_amd as na
    from nitrorag_amd.q8 import LAST_BLOCK
    from oracle import scheduler as sc
    from oracle.model import scale_residual_outputs

    meta, traces = golden_sched
    blob, _, _ = golden_model
    model = na.Model(scale_residual_outputs(blob, meta["out_scale"]))
    for tr in traces:
        say(f"scheduler scenario {tr.name}: {tr.steps} steps, {tr.total_blocks} pages, "
            f"budget {tr.budget}")
        pool = na.KVPool(tr.total_blocks, model.n_layers, model.kv_dim)
        bm = na.BlockManager(tr.total_blocks)
        S = na.ContinuousScheduler(bm, tr.budget, meta["max_generated"])
        last = max(tr.arrivals)
        t = 0
        while True:
            for rid, prompt in tr.arrivals.get(t, []):
                S.add_request(rid, prompt)
            if not S.has_active_requests() and t >= last:
                break
            before = sc.decode_state(S.state_words())
            S.step(model, pool, LAST_BLOCK)
            got = S.state_words()
            assert got == tr.state(t), (tr.name, t, sc.decode_state(got), sc.decode_state(tr.state(t)))
            lg = S.last_logits()
            idx, val = tr.top(t)
            after = sc.decode_state(got)
            finished_prefill = any(r["done"] and not b["done"] and r["generated"]
                                   for r, b in zip(after["requests"], before["requests"]))
            if tr.kind(t) == 1:
                rows = lg[1:] if finished_prefill else lg
            elif tr.kind(t) == 2 and finished_prefill:
                rows = lg
            else:
                rows = None
            if rows is not None:
                assert rows.shape[0] == idx.shape[0], (tr.name, t)
                g = np.take_along_axis(rows, idx, axis=1)
                bound = LOGIT_ATOL + LOGIT_RTOL * np.abs(val)
                assert np.all(np.abs(g - val) <= bound), (tr.name, t, np.abs(g - val).max())
            t += 1
        assert t == tr.steps
        assert pool.take_device_errors() == 0
        S.close()
        pool.close()


def test_scheduler_finishes_requests_the_model_cannot_run(golden_model):
    """A request the model cannot run no longer fails the step (and with it every
    later step): the device step binds the model's limits, finishes a queued
    prompt that cannot fit seq_len unserved, and finishes a running request
    that would decode at seq_len with the tokens it has; add_request then
    refuses such prompts up front."""
    import nitrorag_amd as na
    from nitrorag_amd.q8 import LAST_BLOCK

    blob, meta, _ = golden_model
    model = na.Model(blob)
    seq_len = model.config["seq_len"]
    pool = na.KVPool(16, model.n_layers, model.kv_dim)
    bm = na.BlockManager(16)
    S = na.ContinuousScheduler(bm, 256, 1000)
    S.add_request(0, [1] * (seq_len + 1))  # no limits bound yet: queued
    S.step(model, pool, LAST_BLOCK)
    st = S.request_status(0)
    assert st["is_finished"] == 1 and st["generated"] == 0 and st["logical_token_count"] == 0
    assert not S.has_active_requests()
    with pytest.raises(na.NitroError):
        S.add_request(1, [1] * (seq_len + 1))
    S.drop_request(0)
    assert bm.get_free_count() == 16
    S2 = na.ContinuousScheduler(bm, 256, 1000)
    S2.add_request(1, [2] * (seq_len - 1))
    S2.plan()
    S2.commit(5, [])                      # host path: the prompt's one chunk
    S2.plan()
    S2.commit(0, [6])                     # decode at position seq_len - 1
    S2.step(model, pool, LAST_BLOCK)      # would decode at seq_len: finished instead
    st = S2.request_status(1)
    assert st["is_finished"] == 1 and S2.generated(1) == [5, 6]
    assert not S2.has_active_requests()
    assert pool.take_device_errors() == 0


def test_device_argmax_quirks():
    """nitro_argmax on hand-made rows against the oracle's restatement of the
    reference's argmax (src/model_q8.cpp:559-569): all values <= 0 -> 0,
    first of equal maxima, NaN never wins; rows of odd length take the
    scalar path."""
    import torch

    from nitrorag_amd.scheduler import argmax
    from oracle import scheduler as sc

    rng = np.random.default_rng(5)
    for vocab in (32000, 160, 1001, 7):
        rows = rng.standard_normal((9, vocab)).astype(np.float32)
        rows[1] = -np.abs(rows[1])                       # nothing above 0
        rows[2] = 0.0
        rows[3, :] = -1.0
        rows[3, [vocab // 3, vocab - 1]] = 5.0           # equal maxima
        rows[4, vocab - 1] = 100.0                        # maximum in the last entry
        rows[5, ::2] = np.nan
        rows[5, 1 % vocab] = 50.0
        rows[6] = np.abs(rows[6]) * 1e-30                 # tiny positives
        rows[7, :] = 2.0                                  # all equal -> 0
        got = argmax(torch.from_numpy(rows).cuda()).cpu().numpy()
        want = [sc.argmax(r) for r in rows]
        assert got.tolist() == want, (vocab, got.tolist(), want)


def test_scheduler_reads_shared_prompts_once(monkeypatch):
    """Requests whose prompts are prefix-cache hits begin with the same pages,
    and the scheduler step hands its host tables to the decode batch, so its
    attention takes the shared-prefix form (those rows read once per member
    set).  An MHA model (the form's case) serves 8 requests of one 128-token
    prompt (8 shared pages) and 2 others, with the form forced on (these
    batches are far below the size where the library takes it by itself) and
    off: every step must leave the same scheduler state (hence the same
    tokens) and logits within 1e-4 + 1e-3|x|, and the form must have run."""
    import nitrorag_amd as na
    from nitrorag_amd.model import LAST_BLOCK, synthetic_model_file

    dim, hid, L, H, V, S = 128, 256, 2, 4, 200, 256
    blob = synthetic_model_file(dim, hid, L, H, H, V, S, seed=23)
    rng = np.random.default_rng(23)
    shared = rng.integers(0, V, 128).astype(np.int32)
    prompts = [shared] * 8 + [rng.integers(0, V, 70).astype(np.int32), rng.integers(0, V, 130).astype(np.int32)]
    runs = {}
    for form in ("2", "0"):
        monkeypatch.setenv("NITRO_DECODE_PREFIX", form)
        say(f"scheduler over shared prompts, shared-prefix form {form}")
        model = na.Model(blob)
        pool = na.KVPool(300, L, model.kv_dim)
        sched = na.ContinuousScheduler(na.BlockManager(300), 256, 12)
        for rid, pr in enumerate(prompts):
            sched.add_request(rid, pr)
        steps = []
        while sched.has_active_requests():
            sched.step(model, pool, LAST_BLOCK)
            steps.append((sched.state_words(), sched.last_logits().copy()))
            assert len(steps) < 200
        runs[form] = (steps, pool.decode_counts())
        assert pool.take_device_errors() == 0
        sched.close()
        pool.close()
    (on, (n_on, shared_on)), (off, (n_off, shared_off)) = runs["2"], runs["0"]
    assert shared_on > 0 and shared_off == 0 and n_on == n_off, (n_on, shared_on, n_off, shared_off)
    assert len(on) == len(off)
    for t, ((w1, l1), (w0, l0)) in enumerate(zip(on, off)):
        assert w1 == w0, t
        assert l1.shape == l0.shape and np.all(np.abs(l1 - l0) <= 1e-4 + 1e-3 * np.abs(l0)), t
