"""Pure-Python restatement of the reference's continuous scheduler — TEST INFRASTRUCTURE ONLY.

Follows Request and Continuous_Scheduler (src/pagedMemory.hpp:287-399)
statement by statement over the bookkeeping restatement in paged_memory.py,
with the forward passes split out: `plan()` is everything step() decides and
allocates before its two forward calls (including the allocate_next_token
loops at the top of forward_prefill_chunk, src/model_q8.cpp:428-430, and of
forward_decode_batch, :578-582, taken in batch order as one OpenMP thread
runs them), and `commit()` is what it does with the argmax tokens afterwards.
`step(forward)` runs both around a caller-supplied forward.

Pinned by tests/golden/sched_traces.* (the reference's own scheduler, compiled
from its sources, stepping a tiny random model): per-step scheduler state and
block-manager snapshots must match word for word.
"""
from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field

import numpy as np

from . import paged_memory as pm


class Request:
    """src/pagedMemory.hpp:287-300."""

    def __init__(self, req_id: int, prompt):
        self.req_id = int(req_id)
        self.prompt_tokens = [int(t) for t in prompt]
        self.generated_tokens: list[int] = []
        self.prefill_idx = 0
        self.is_prefill_done = False
        self.is_finished = False
        self.next_token_to_process = -1
        self.seq = pm.Sequence(self.req_id)


@dataclass
class StepPlan:
    """The two forward calls one step makes: at most one prefill chunk
    (request, tokens, start position) and the decode rows in running order."""
    prefill_req: Request | None = None
    prefill_tokens: list = field(default_factory=list)
    prefill_start: int = 0
    decode_reqs: list = field(default_factory=list)
    decode_tokens: list = field(default_factory=list)
    decode_positions: list = field(default_factory=list)


def argmax(row) -> int:
    """src/model_q8.cpp:559-569: first index of the largest value above 0.0,
    index 0 when no value exceeds 0.0 (NaN never wins)."""
    best, best_i = 0.0, 0
    for i, v in enumerate(np.asarray(row, dtype=np.float32).tolist()):
        if v > best:
            best, best_i = v, i
    return best_i


class ContinuousScheduler:
    """src/pagedMemory.hpp:303-399.  max_tokens_per_batch is the reference's
    member (256); max_generated is its hard-coded finish length (20, :393)."""

    def __init__(self, mem: pm.KVBlockManager, cache: pm.PrefixCacheManager,
                 max_tokens_per_batch: int = 256, max_generated: int = 20):
        self.mem, self.cache = mem, cache
        self.waiting_queue: deque[Request] = deque()
        self.running_batch: list[Request] = []
        self.max_tokens_per_batch = max_tokens_per_batch
        self.max_generated = max_generated
        self.requests: list[Request] = []  # every request, in the order added

    def add_request(self, req: Request) -> None:  # :309-312
        req.next_token_to_process = req.prompt_tokens[0]
        self.waiting_queue.append(req)
        self.requests.append(req)

    def has_active_requests(self) -> bool:  # :313-315
        return bool(self.waiting_queue) or bool(self.running_batch)

    def plan(self) -> StepPlan:
        mem, cache = self.mem, self.cache
        # :317-326 release the requests that finished last step
        kept = []
        for r in self.running_batch:
            if r.is_finished:
                r.seq.release(mem, cache)
            else:
                kept.append(r)
        self.running_batch = kept
        budget = self.max_tokens_per_batch
        p = StepPlan()
        # :332-340 one decode row per running request (all have finished prefill)
        for r in self.running_batch:
            if r.is_prefill_done:
                p.decode_tokens.append(r.next_token_to_process)
                p.decode_positions.append(r.seq.logical_token_count)
                p.decode_reqs.append(r)
                budget -= 1
        # :343-377 at most one prefill chunk, from the head of the queue
        if self.waiting_queue and budget > 0:
            r = self.waiting_queue[0]
            while (r.prefill_idx + pm.BLOCK_SIZE <= len(r.prompt_tokens)
                   and not r.seq.token_buffer):
                chunk = r.prompt_tokens[r.prefill_idx:r.prefill_idx + pm.BLOCK_SIZE]
                h = pm.hash_block_state(r.seq.current_hash, chunk)
                hit = cache.check_cache(h)
                if hit == -1:
                    break
                mem.inc_ref_count(hit, cache)
                r.seq.block_table.append(hit)
                r.seq.logical_token_count += pm.BLOCK_SIZE
                r.seq.current_hash = h
                r.prefill_idx += pm.BLOCK_SIZE
            remaining = len(r.prompt_tokens) - r.prefill_idx
            n = min(remaining, budget)
            if n > 0:
                p.prefill_tokens = r.prompt_tokens[r.prefill_idx:r.prefill_idx + n]
                p.prefill_req = r
            if r.prefill_idx + n == len(r.prompt_tokens):
                r.is_prefill_done = True
                self.running_batch.append(r)
                self.waiting_queue.popleft()
            else:
                r.prefill_idx += n
        # forward_prefill_chunk's allocations (src/model_q8.cpp:428-430), then
        # forward_decode_batch's (:578-582), in that order
        if p.prefill_req is not None:
            seq = p.prefill_req.seq
            p.prefill_start = seq.logical_token_count
            for t in p.prefill_tokens:
                seq.allocate_next_token(t, mem, cache)
        for r, t in zip(p.decode_reqs, p.decode_tokens):
            r.seq.allocate_next_token(t, mem, cache)
        return p

    def commit(self, p: StepPlan, prefill_token: int | None, decode_tokens) -> None:
        """:380-397 with the argmax tokens of the two forwards."""
        if p.prefill_req is not None and p.prefill_req.is_prefill_done:
            p.prefill_req.next_token_to_process = int(prefill_token)
            p.prefill_req.generated_tokens.append(int(prefill_token))
        for r, t in zip(p.decode_reqs, decode_tokens):
            r.next_token_to_process = int(t)
            r.generated_tokens.append(int(t))
            if len(r.generated_tokens) >= self.max_generated:
                r.is_finished = True

    def step(self, forward) -> StepPlan:
        """forward(plan) -> (prefill_token or None, [decode tokens])."""
        p = self.plan()
        pt, dt = forward(p)
        self.commit(p, pt, dt)
        return p

    # ---- observation (the word stream the reference driver writes) --------
    def state_words(self) -> list[int]:
        """Same layout as ref_sched_state: running ids, waiting ids, then per
        request (in the order added) its fields, generated tokens and sequence."""
        o = [len(self.running_batch), *[r.req_id for r in self.running_batch]]
        o += [len(self.waiting_queue), *[r.req_id for r in self.waiting_queue]]
        o.append(len(self.requests))
        for r in self.requests:
            o += [r.req_id, r.prefill_idx, int(r.is_prefill_done), int(r.is_finished),
                  r.next_token_to_process, len(r.generated_tokens), *r.generated_tokens]
            s = r.seq
            h = s.current_hash
            o += [s.logical_token_count, _i32(h & 0xffffffff), _i32(h >> 32)]
            o += [len(s.token_buffer), *s.token_buffer, len(s.block_table), *s.block_table]
        return o


def _i32(u: int) -> int:
    return u - (1 << 32) if u >= (1 << 31) else u


def decode_state(words) -> dict:
    """Parses a scheduler word stream into a dict (for readable diffs)."""
    w = [int(x) for x in words]
    i = 0

    def take(n):
        nonlocal i
        out = w[i:i + n]
        i += n
        return out

    running = take(take(1)[0])
    waiting = take(take(1)[0])
    reqs = []
    for _ in range(take(1)[0]):
        rid, pidx, done, fin, nxt = take(5)
        gen = take(take(1)[0])
        count, lo, hi = take(3)
        buf = take(take(1)[0])
        table = take(take(1)[0])
        reqs.append(dict(req_id=rid, prefill_idx=pidx, done=done, finished=fin, next=nxt,
                         generated=gen, count=count,
                         hash=(lo & 0xffffffff) | ((hi & 0xffffffff) << 32),
                         buffer=buf, table=table))
    assert i == len(w), "trailing words in scheduler state"
    return dict(running=running, waiting=waiting, requests=reqs)


class OracleForward:
    """The reference's two forward calls of one step on the oracle model
    (oracle.model.OracleModel) over host K/V pools [pages][L][16][kv_dim];
    returns the argmax tokens and keeps the logits rows of the step."""

    def __init__(self, model, total_blocks: int):
        shape = (total_blocks, model.n_layers, pm.BLOCK_SIZE, model.kv_dim)
        self.model = model
        self.k = np.zeros(shape, np.float32)
        self.v = np.zeros(shape, np.float32)
        self.prefill_logits = None
        self.decode_logits = None

    def __call__(self, p: StepPlan):
        self.prefill_logits = self.decode_logits = None
        pt = None
        if p.prefill_req is not None:
            table = np.asarray(p.prefill_req.seq.block_table, np.int32)[None, :]
            lg = self.model.forward_prefill_chunk(self.k, self.v, table, p.prefill_start,
                                                  p.prefill_tokens)
            self.prefill_logits = np.asarray(lg, np.float32).reshape(-1)
            pt = argmax(self.prefill_logits)
        dt = []
        if p.decode_reqs:
            tables = pm_pack([r.seq.block_table for r in p.decode_reqs])
            lg = self.model.forward_decode_batch(self.k, self.v, tables, p.decode_positions,
                                                 p.decode_tokens, bulk=True)
            self.decode_logits = np.asarray(lg, np.float32)
            dt = [argmax(row) for row in self.decode_logits]
        return pt, dt


def pm_pack(tables) -> np.ndarray:
    width = max(1, max(len(t) for t in tables))
    out = np.zeros((len(tables), width), np.int32)
    for i, t in enumerate(tables):
        out[i, :len(t)] = t
    return out
