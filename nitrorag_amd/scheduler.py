"""The continuous scheduler (binding of nitro_sched_*): Request and
Continuous_Scheduler of src/pagedMemory.hpp:287-399 over a BlockManager, with
each step either run whole on the device (`step`: one forward over the
prefill chunk's rows and the decode rows together, argmax on the device) or
split around a caller-supplied forward (`plan` / `commit`)."""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import _native as N
from .attention import _stream_ptr
from .q8 import LAST_BLOCK


def argmax(logits, out=None, stream=None):
    """argmax (src/model_q8.cpp:559-569) of each row of a [rows][vocab] fp32
    GPU tensor: the first index of the largest value above 0.0, 0 when none
    exceeds 0.0.  Returns an int32 GPU tensor [rows]."""
    import torch

    from .attention import _dev

    rows, vocab = logits.shape
    if out is None:
        out = torch.empty(rows, dtype=torch.int32, device=logits.device)
    if out.dtype != torch.int32 or out.device.type != "cuda" or not out.is_contiguous() or out.numel() < rows:
        raise TypeError("out must be a contiguous int32 GPU tensor with one entry per row")
    N.call("nitro_argmax", _dev(logits, "logits"), rows, vocab, ctypes.c_void_p(out.data_ptr()),
           _stream_ptr(stream))
    return out


@dataclass
class StepPlan:
    """The two forward calls of one step: the prefill chunk (request id,
    prompt[start:start + length], whether it completes the prompt) and the
    decode rows in running order."""
    prefill_id: int = -1
    prefill_start: int = 0
    prefill_length: int = 0
    prefill_finishes: bool = False
    decode_ids: list = field(default_factory=list)
    decode_tokens: list = field(default_factory=list)
    decode_positions: list = field(default_factory=list)


class ContinuousScheduler:
    """Continuous_Scheduler (src/pagedMemory.hpp:303-399).  The block manager
    must outlive the scheduler.  max_tokens_per_batch is the reference's
    per-step token budget (256); max_generated its finish length (20)."""

    def __init__(self, block_manager, max_tokens_per_batch: int = 256, max_generated: int = 20):
        h = ctypes.c_void_p()
        N.call("nitro_sched_create", block_manager.handle, max_tokens_per_batch, max_generated,
               ctypes.byref(h))
        self._h = h
        self._bm = block_manager  # kept alive with the scheduler
        self.prompts: dict[int, list] = {}
        self._vocab = 0

    @property
    def handle(self):
        return self._h

    def close(self):
        if getattr(self, "_h", None):
            N.call("nitro_sched_destroy", self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def add_request(self, req_id: int, prompt) -> None:
        """new Request(req_id, prompt) + add_request (:309-312)."""
        t = np.ascontiguousarray(np.asarray(prompt, dtype=np.int64).astype(np.int32))
        N.call("nitro_sched_add_request", self._h, int(req_id), t.ctypes.data_as(N._i32p), t.size)
        self.prompts[int(req_id)] = t.tolist()

    def set_limits(self, seq_len: int, vocab: int) -> None:
        """Admission limits (0 = none): add_request then refuses a prompt with a
        token outside [0, vocab) or with len + max_generated - 1 > seq_len.  A
        device step sets them from its model."""
        N.call("nitro_sched_set_limits", self._h, int(seq_len), int(vocab))

    def has_active_requests(self) -> bool:
        v = ctypes.c_int32()
        N.call("nitro_sched_has_active_requests", self._h, ctypes.byref(v))
        return bool(v.value)

    def step(self, model, pool, semantics: int = LAST_BLOCK, stream=None) -> None:
        """One whole step on the device (synchronises the stream)."""
        N.call("nitro_sched_step", self._h, model.handle, pool.handle, semantics, _stream_ptr(stream))
        self._vocab = model.vocab

    def plan(self) -> StepPlan:
        """step() up to its forward calls (all bookkeeping included)."""
        cap = max(1, len(self.prompts))
        pre = np.zeros(4, np.int32)
        ids, toks, pos = (np.zeros(cap, np.int32) for _ in range(3))
        n = ctypes.c_int32()
        N.call("nitro_sched_plan", self._h, pre.ctypes.data_as(N._i32p), ids.ctypes.data_as(N._i32p),
               toks.ctypes.data_as(N._i32p), pos.ctypes.data_as(N._i32p), cap, ctypes.byref(n))
        B = n.value
        return StepPlan(int(pre[0]), int(pre[2]), int(pre[1]), bool(pre[3]), ids[:B].tolist(),
                        toks[:B].tolist(), pos[:B].tolist())

    def commit(self, prefill_token, decode_tokens) -> None:
        t = np.ascontiguousarray(np.asarray(decode_tokens, dtype=np.int64).astype(np.int32))
        N.call("nitro_sched_commit", self._h, int(prefill_token or 0), t.ctypes.data_as(N._i32p), t.size)

    def last_logits(self) -> np.ndarray:
        """Logits rows of the last device step: the prefill chunk's last row
        first when it completed its prompt, then the decode rows."""
        rows = ctypes.c_int32()
        N.call("nitro_sched_last_logits", self._h, None, 0, ctypes.byref(rows))
        out = np.zeros((rows.value, self._vocab), np.float32)
        if rows.value:
            N.call("nitro_sched_last_logits", self._h,
                   out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), rows.value, ctypes.byref(rows))
        return out

    def state_words(self) -> list:
        n = ctypes.c_int32()
        N.call("nitro_sched_state", self._h, None, 0, ctypes.byref(n))
        buf = np.zeros(max(1, n.value), np.int32)
        N.call("nitro_sched_state", self._h, buf.ctypes.data_as(N._i32p), buf.size, ctypes.byref(n))
        return buf[:n.value].tolist()

    def generated(self, req_id: int) -> list:
        n = ctypes.c_int32()
        N.call("nitro_sched_generated", self._h, int(req_id), None, 0, ctypes.byref(n))
        buf = np.zeros(max(1, n.value), np.int32)
        N.call("nitro_sched_generated", self._h, int(req_id), buf.ctypes.data_as(N._i32p), buf.size,
               ctypes.byref(n))
        return buf[:n.value].tolist()

    def request_status(self, req_id: int) -> dict:
        st = np.zeros(6, np.int32)
        N.call("nitro_sched_request_status", self._h, int(req_id), st.ctypes.data_as(N._i32p))
        keys = ("prefill_idx", "is_prefill_done", "is_finished", "next_token_to_process",
                "generated", "logical_token_count")
        return dict(zip(keys, (int(v) for v in st)))

    def drop_request(self, req_id: int) -> None:
        N.call("nitro_sched_drop_request", self._h, int(req_id))
        self.prompts.pop(int(req_id), None)
