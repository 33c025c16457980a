"""Records golden vectors from the reference's own compiled code.

Run in a container that has the reference checkout (needs oracle/_ref, built
by `make -C oracle ref`):

    python tests/golden/make_golden.py

Writes, next to this script:
  fnv.json                   hash_block_state outputs (src/pagedMemory.hpp:14-24)
  block_manager_traces.json  op scripts over KVBlock_Manager / PrefixCacheManager /
                             Sequence / ingest_prompt with, per op, the status, the
                             result and a digest of the full bookkeeping state, plus
                             the final state (src/pagedMemory.hpp:86-285,
                             src/model_q8.cpp:695-724)
  attention.json + attention.npz
                             inputs and outputs of forward_decode_batch, forward_paged,
                             forward_prefill_chunk (fresh, continued, after a prefix
                             hit) and forward, observed through xb2 (see
                             oracle/ref_harness.cpp).  Pools are regenerated in the
                             tests from counter_pool(seed); the npz holds q, the K/V
                             rows written by the call, the block tables and the
                             observed outputs.  Pool digests are over the observed
                             layer only.
  q8_matmul.json + q8_matmul.npz
                             the reference's matmul and matmul_bulk (BlockQ8) on
                             packed Q8 matrices and fp32 activations
  model_tiny.bin + model_forward.json + model_forward.npz
                             a tiny random model in the reference's file layout and
                             the logits of forward_prefill_chunk / forward_paged /
                             forward_decode_batch over a scripted session
  rpc.json                   the reference's NitroRPC send_ints bytes and recv_ints /
                             recv_structured_query decodes over socket pairs
  sched_traces.json + sched_traces.npz
                             steps of the reference's Continuous_Scheduler over the tiny
                             model with wo/w2 scaled by 64: scheduler state and
                             block-manager snapshot words per step, and the top logits
                             of the rows each step left behind
"""
from __future__ import annotations

import hashlib
import json
import os
import random
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, HERE)

from oracle import paged_memory as pm  # noqa: E402
from oracle import ref  # noqa: E402
from synth import counter_pool, counter_uniform, rope_tables  # noqa: E402


def state_digest(snap: dict) -> str:
    return hashlib.sha256(json.dumps(snap, sort_keys=True, separators=(",", ":"))
                          .encode()).hexdigest()[:16]


def array_digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()[:16]


# ---------------------------------------------------------------- FNV -------
def make_fnv():
    rng = random.Random(0xF17)
    cases = []
    for n in [0, 1, 2, 15, 16, 16, 16, 17, 33, 64]:
        toks = [rng.randrange(-2**31, 2**31) if rng.random() < 0.3 else rng.randrange(0, 32000)
                for _ in range(n)]
        parent = pm.FNV_OFFSET_BASIS if rng.random() < 0.5 else rng.getrandbits(64)
        cases.append({"parent": parent, "tokens": toks,
                      "hash": ref.hash_block_state(parent, toks)})
    shared = [263] * 16  # the reference benchmark's shared prompt token (src/model_q8.cpp:788)
    h = pm.FNV_OFFSET_BASIS
    chain = []
    for _ in range(16):
        h = ref.hash_block_state(h, shared)
        chain.append(h)
    return {"cases": cases, "shared_263_chain": chain}


# ---------------------------------------------------- block manager traces --
def run_trace(name, total_blocks, max_seqs, ops):
    W = ref.RefWorld(n_heads=2, n_kv_heads=2, head_dim=16, n_layers=1, vocab=512, seq_len=512,
                     total_blocks=total_blocks, max_rows=512, max_seqs=max_seqs, seed=3)
    steps = []
    for op in ops:
        st, res = W.op(op["op"], op.get("a", 0), op.get("b", 0), op.get("h", 0),
                       op.get("toks", ()))
        steps.append([st, res, state_digest(W.snapshot())])
    final = W.snapshot()
    W.close()
    return {"name": name, "total_blocks": total_blocks, "max_seqs": max_seqs, "ops": ops,
            "steps": steps, "final": final}


def seq_workload(seed, total_blocks, max_seqs, n_ops, families=3, max_tokens=380):
    """Sequences ingesting prompts from a few shared-prefix families, appending,
    flushing and releasing, under pool pressure (evictions, exhaustion)."""
    rng = random.Random(seed)
    fams = [[rng.randrange(1, 500) for _ in range(rng.choice([16, 32, 48, 64]))]
            for _ in range(families)]
    live = {}
    ops = []
    for _ in range(n_ops):
        r = rng.random()
        free_slots = [s for s in range(max_seqs) if s not in live]
        if free_slots and (r < 0.25 or not live):
            s = rng.choice(free_slots)
            ops.append({"op": pm.OP_SEQ_NEW, "a": s})
            fam = rng.choice(fams)
            tail = [rng.randrange(1, 500) for _ in range(rng.randrange(0, 40))]
            prompt = fam[: rng.choice([len(fam), len(fam) - 16 if len(fam) > 16 else len(fam)])] + tail
            if rng.random() < 0.2:
                prompt = [rng.randrange(1, 500) for _ in range(rng.randrange(1, 50))]
            ops.append({"op": pm.OP_INGEST, "a": s, "b": int(rng.random() < 0.8), "toks": prompt})
            live[s] = len(prompt)
        elif r < 0.55:
            s = rng.choice(list(live))
            for _ in range(rng.randrange(1, 20)):
                if live[s] >= max_tokens:
                    break
                ops.append({"op": pm.OP_SEQ_APPEND, "a": s, "b": rng.randrange(1, 500)})
                live[s] += 1
        elif r < 0.65:
            s = rng.choice(list(live))
            ops.append({"op": pm.OP_SEQ_FLUSH, "a": s})
        elif r < 0.85:
            s = rng.choice(list(live))
            ops.append({"op": pm.OP_SEQ_RELEASE, "a": s})
            del live[s]
        elif r < 0.9:
            ops.append({"op": pm.OP_FREE_COUNT})
        else:
            ops.append({"op": pm.OP_IS_CACHED, "a": rng.randrange(total_blocks)})
    return ops


def low_level_workload(seed, total_blocks, n_ops):
    rng = random.Random(seed)
    hashes = [rng.getrandbits(64) for _ in range(12)]
    ops = []
    allocated = []
    for _ in range(n_ops):
        r = rng.random()
        if r < 0.3:
            ops.append({"op": pm.OP_ALLOC})
            allocated.append(None)
        elif r < 0.4:
            ops.append({"op": pm.OP_INC, "a": rng.randrange(total_blocks)})
        elif r < 0.6:
            ops.append({"op": pm.OP_FREE, "a": rng.randrange(total_blocks)})
        elif r < 0.62:
            ops.append({"op": pm.OP_FORCE_FREE, "a": rng.randrange(total_blocks)})
        elif r < 0.8:
            parent = -1 if rng.random() < 0.4 else rng.randrange(total_blocks)
            ops.append({"op": pm.OP_INSERT, "a": rng.randrange(total_blocks), "b": parent,
                        "h": rng.choice(hashes)})
        elif r < 0.9:
            ops.append({"op": pm.OP_CHECK, "h": rng.choice(hashes)})
        elif r < 0.95:
            ops.append({"op": pm.OP_EVICT})
        else:
            ops.append({"op": pm.OP_FREE_COUNT})
    return ops


def exp4_workload():
    """The reference benchmark's prefix-cache experiment shape (src/model_q8.cpp:917-939):
    user A ingests 256 x token 263 and flushes; user B hits every page."""
    p = [263] * 256
    return [{"op": pm.OP_SEQ_NEW, "a": 0}, {"op": pm.OP_INGEST, "a": 0, "b": 1, "toks": p},
            {"op": pm.OP_SEQ_FLUSH, "a": 0}, {"op": pm.OP_SEQ_NEW, "a": 1},
            {"op": pm.OP_INGEST, "a": 1, "b": 1, "toks": p}, {"op": pm.OP_SEQ_FLUSH, "a": 1},
            {"op": pm.OP_SEQ_APPEND, "a": 1, "b": 7}, {"op": pm.OP_SEQ_RELEASE, "a": 0},
            {"op": pm.OP_SEQ_RELEASE, "a": 1}, {"op": pm.OP_FREE_COUNT}]


def make_traces():
    return [
        run_trace("seq_pressure_24", 24, 6, seq_workload(11, 24, 6, 160)),
        run_trace("seq_roomy_96", 96, 8, seq_workload(12, 96, 8, 220, families=4)),
        run_trace("seq_tight_12", 12, 4, seq_workload(13, 12, 4, 120, families=2, max_tokens=120)),
        run_trace("low_level_16", 16, 1, low_level_workload(14, 16, 300)),
        run_trace("low_level_40", 40, 1, low_level_workload(15, 40, 400)),
        run_trace("exp4_shared_prompt", 1000 // 10, 2, exp4_workload()),
    ]


# ------------------------------------------------------------- attention ---
class Recorder:
    def __init__(self):
        self.meta = []
        self.arrays = {}

    def add(self, name, meta, **arrays):
        meta = dict(meta, name=name)
        self.meta.append(meta)
        for k, v in arrays.items():
            self.arrays[f"{name}/{k}"] = v


def tables_of(W, slots, max_pages):
    t = np.zeros((len(slots), max_pages), dtype=np.int32)
    for i, s in enumerate(slots):
        bt = W.block_table(s)
        t[i, : len(bt)] = bt
    return t


def case_decode(rec, name, H, Hkv, hd, L, blocks, lens, seed):
    W = ref.RefWorld(n_heads=H, n_kv_heads=Hkv, head_dim=hd, n_layers=L, total_blocks=blocks,
                     seed=seed, max_seqs=len(lens))
    for s, n in enumerate(lens):
        W.op(pm.OP_SEQ_NEW, s)
        for t in range(n):
            W.op(pm.OP_SEQ_APPEND, s, 1 + (t * 7 + s) % 400)
    pool_seed = 1000 + seed
    W.write_pool(counter_pool(pool_seed, blocks, L, W.kv_dim),
                 counter_pool(pool_seed + 1, blocks, L, W.kv_dim))
    toks = [5 + 3 * s for s in range(len(lens))]
    pos = W.decode_batch(list(range(len(lens))), toks)
    q, k, v, xb2 = W.rows(len(lens))
    max_pages = max(p // 16 + 1 for p in pos) + 1
    tables = tables_of(W, range(len(lens)), max_pages)
    kp, vp = W.pool()
    rec.add(name, {"kind": "decode_batch", "H": H, "Hkv": Hkv, "hd": hd, "layers": L,
                   "pages": blocks, "layer": L - 1, "pool_seed": pool_seed, "observed": 32,
                   "k_pool_digest": array_digest(kp[:, L - 1]),
                   "v_pool_digest": array_digest(vp[:, L - 1])},
            q=q, k=k, v=v, xb2_obs=xb2[:, -32:], tables=tables, positions=pos)
    W.close()


def case_single(rec, name, H, Hkv, hd, L, blocks, n_past, seed):
    W = ref.RefWorld(n_heads=H, n_kv_heads=Hkv, head_dim=hd, n_layers=L, total_blocks=blocks,
                     seed=seed, max_seqs=1)
    W.op(pm.OP_SEQ_NEW, 0)
    for t in range(n_past):
        W.op(pm.OP_SEQ_APPEND, 0, 1 + (t * 5) % 300)
    pool_seed = 2000 + seed
    W.write_pool(counter_pool(pool_seed, blocks, L, W.kv_dim),
                 counter_pool(pool_seed + 1, blocks, L, W.kv_dim))
    pos = W.forward_paged(0, 42)
    q, k, v, xb2 = W.rows(1)
    table = W.block_table(0)
    kp, vp = W.pool()
    rec.add(name, {"kind": "decode_single", "H": H, "Hkv": Hkv, "hd": hd, "layers": L,
                   "pages": blocks, "layer": L - 1, "pool_seed": pool_seed, "pos": int(pos),
                   "observed": H * hd, "k_pool_digest": array_digest(kp[:, L - 1]),
                   "v_pool_digest": array_digest(vp[:, L - 1])},
            q=q, k=k, v=v, xb2_obs=xb2, table=table)
    W.close()


def case_prefill(rec, name, H, Hkv, hd, L, blocks, chunks, seed):
    """One sequence, prefill chunks of the given sizes; records the last chunk."""
    W = ref.RefWorld(n_heads=H, n_kv_heads=Hkv, head_dim=hd, n_layers=L, total_blocks=blocks,
                     seed=seed, max_seqs=1)
    W.op(pm.OP_SEQ_NEW, 0)
    pool_seed = 3000 + seed
    W.write_pool(counter_pool(pool_seed, blocks, L, W.kv_dim),
                 counter_pool(pool_seed + 1, blocks, L, W.kv_dim))
    earlier_k, earlier_v, starts = [], [], []
    tok = 1
    for ci, n in enumerate(chunks):
        toks = list(range(tok, tok + n))
        tok += n
        sp = W.prefill_chunk(0, toks)
        starts.append(sp)
        q, k, v, xb2 = W.rows(n)
        if ci < len(chunks) - 1:
            earlier_k.append(k)
            earlier_v.append(v)
    table = W.block_table(0)
    kp, vp = W.pool()
    arrays = dict(q=q, k=k, v=v, xb2_obs=xb2[:, -32:], table=table,
                  chunk_starts=np.array(starts, dtype=np.int32))
    if earlier_k:
        arrays["earlier_k"] = np.concatenate(earlier_k)
        arrays["earlier_v"] = np.concatenate(earlier_v)
    rec.add(name, {"kind": "prefill", "H": H, "Hkv": Hkv, "hd": hd, "layers": L,
                   "pages": blocks, "layer": L - 1, "pool_seed": pool_seed,
                   "start_pos": int(starts[-1]), "observed": 32,
                   "k_pool_digest": array_digest(kp[:, L - 1]),
                   "v_pool_digest": array_digest(vp[:, L - 1])}, **arrays)
    W.close()


def case_prefix_hit(rec, name, H, Hkv, hd, L, blocks, shared, tail_a, tail_b, seed):
    """Seq A ingests shared+tail_a with the prefix cache on and flushes; seq B
    ingests shared+tail_b, hits the shared pages and prefills only its tail."""
    W = ref.RefWorld(n_heads=H, n_kv_heads=Hkv, head_dim=hd, n_layers=L, total_blocks=blocks,
                     seed=seed, max_seqs=2)
    pool_seed = 4000 + seed
    W.write_pool(counter_pool(pool_seed, blocks, L, W.kv_dim),
                 counter_pool(pool_seed + 1, blocks, L, W.kv_dim))
    base = list(range(100, 100 + shared))
    pa = base + list(range(300, 300 + tail_a))
    pb = base + list(range(400, 400 + tail_b))
    W.op(pm.OP_SEQ_NEW, 0)
    W.op(pm.OP_INGEST, 0, 1, toks=pa)
    qa, ka, va, _ = W.rows(len(pa))
    W.op(pm.OP_SEQ_FLUSH, 0)
    W.op(pm.OP_SEQ_NEW, 1)
    st, count = W.op(pm.OP_INGEST, 1, 1, toks=pb)
    hits = shared // 16
    n_b = len(pb) - 16 * hits
    qb, kb, vb, xb2 = W.rows(n_b)
    ta, tb = W.block_table(0), W.block_table(1)
    kp, vp = W.pool()
    rec.add(name, {"kind": "prefix_hit", "H": H, "Hkv": Hkv, "hd": hd, "layers": L,
                   "pages": blocks, "layer": L - 1, "pool_seed": pool_seed,
                   "start_pos": 16 * hits, "hits": hits, "observed": 32,
                   "k_pool_digest": array_digest(kp[:, L - 1]),
                   "v_pool_digest": array_digest(vp[:, L - 1])},
            q=qb, k=kb, v=vb, xb2_obs=xb2[:, -32:], table=tb, table_a=ta, k_a=ka, v_a=va)
    W.close()


def case_contiguous(rec, name, H, Hkv, hd, n_pos, seed):
    W = ref.RefWorld(n_heads=H, n_kv_heads=Hkv, head_dim=hd, n_layers=1, total_blocks=4,
                     seed=seed, max_seqs=1, seq_len=256)
    for pos in range(n_pos):
        W.forward_contiguous(1 + (pos * 11) % 400, pos)
    q, k, v, xb2 = W.rows(1)
    kc, vc = W.contiguous_cache()
    rec.add(name, {"kind": "contiguous", "H": H, "Hkv": Hkv, "hd": hd, "pos": n_pos - 1,
                   "observed": H * hd},
            q=q, xb2_obs=xb2, key_rows=kc[0, :n_pos], value_rows=vc[0, :n_pos])
    W.close()


def rope_pair(H, Hkv, hd, blocks, seed, max_seqs, seq_len=128):
    """Two one-layer worlds with equal weights: A keeps the identity rotation, so
    its q/k are the pre-RoPE values of B, which uses Llama-style tables."""
    A = ref.RefWorld(n_heads=H, n_kv_heads=Hkv, head_dim=hd, n_layers=1, total_blocks=blocks,
                     seed=seed, max_seqs=max_seqs, seq_len=seq_len)
    B = ref.RefWorld(n_heads=H, n_kv_heads=Hkv, head_dim=hd, n_layers=1, total_blocks=blocks,
                     seed=seed, max_seqs=max_seqs, seq_len=seq_len)
    fr, fi = rope_tables(seq_len, hd)
    B.set_rope(fr, fi)
    return A, B


def case_rope_decode(rec, name, H, Hkv, hd, blocks, lens, seed):
    A, B = rope_pair(H, Hkv, hd, blocks, seed, len(lens))
    pool_seed = 5000 + seed
    for W in (A, B):
        for s, n in enumerate(lens):
            W.op(pm.OP_SEQ_NEW, s)
            for t in range(n):
                W.op(pm.OP_SEQ_APPEND, s, 1 + (t * 7 + s) % 400)
        W.write_pool(counter_pool(pool_seed, blocks, 1, W.kv_dim),
                     counter_pool(pool_seed + 1, blocks, 1, W.kv_dim))
    toks = [5 + 3 * s for s in range(len(lens))]
    pa = A.decode_batch(list(range(len(lens))), toks)
    pb = B.decode_batch(list(range(len(lens))), toks)
    assert np.array_equal(pa, pb)
    qa, ka, va, _ = A.rows(len(lens))
    qb, kb, vb, xb2 = B.rows(len(lens))
    assert np.array_equal(va, vb)
    max_pages = max(p // 16 + 1 for p in pb) + 1
    tables = tables_of(B, range(len(lens)), max_pages)
    kp, vp = B.pool()
    rec.add(name, {"kind": "rope_decode", "H": H, "Hkv": Hkv, "hd": hd, "layers": 1,
                   "pages": blocks, "layer": 0, "pool_seed": pool_seed, "observed": 32,
                   "seq_len": B.seq_len, "rope_base": 10000.0,
                   "k_pool_digest": array_digest(kp[:, 0]), "v_pool_digest": array_digest(vp[:, 0])},
            q_pre=qa, k_pre=ka, v=vb, q=qb, k=kb, xb2_obs=xb2[:, -32:], tables=tables,
            positions=pb)
    A.close()
    B.close()


def case_rope_single(rec, name, H, Hkv, hd, blocks, n_past, seed):
    A, B = rope_pair(H, Hkv, hd, blocks, seed, 1)
    pool_seed = 6000 + seed
    for W in (A, B):
        W.op(pm.OP_SEQ_NEW, 0)
        for t in range(n_past):
            W.op(pm.OP_SEQ_APPEND, 0, 1 + (t * 5) % 300)
        W.write_pool(counter_pool(pool_seed, blocks, 1, W.kv_dim),
                     counter_pool(pool_seed + 1, blocks, 1, W.kv_dim))
    pos = A.forward_paged(0, 42)
    assert B.forward_paged(0, 42) == pos
    qa, ka, va, _ = A.rows(1)
    qb, kb, vb, xb2 = B.rows(1)
    kp, vp = B.pool()
    rec.add(name, {"kind": "rope_single", "H": H, "Hkv": Hkv, "hd": hd, "layers": 1,
                   "pages": blocks, "layer": 0, "pool_seed": pool_seed, "pos": int(pos),
                   "observed": H * hd, "seq_len": B.seq_len, "rope_base": 10000.0,
                   "k_pool_digest": array_digest(kp[:, 0]), "v_pool_digest": array_digest(vp[:, 0])},
            q_pre=qa, k_pre=ka, v=vb, q=qb, k=kb, xb2_obs=xb2, table=B.block_table(0))
    A.close()
    B.close()


def case_rope_prefill(rec, name, H, Hkv, hd, blocks, chunks, seed):
    """One sequence, prefill chunks of the given sizes with RoPE; records every chunk's
    pre/post q and k and the last chunk's observed output."""
    A, B = rope_pair(H, Hkv, hd, blocks, seed, 1)
    pool_seed = 7000 + seed
    for W in (A, B):
        W.op(pm.OP_SEQ_NEW, 0)
        W.write_pool(counter_pool(pool_seed, blocks, 1, W.kv_dim),
                     counter_pool(pool_seed + 1, blocks, 1, W.kv_dim))
    arrays = {}
    tok = 1
    starts = []
    for ci, n in enumerate(chunks):
        toks = list(range(tok, tok + n))
        tok += n
        sa = A.prefill_chunk(0, toks)
        sb = B.prefill_chunk(0, toks)
        assert sa == sb
        starts.append(sb)
        qa, ka, va, _ = A.rows(n)
        qb, kb, vb, xb2 = B.rows(n)
        arrays.update({f"q_pre{ci}": qa, f"k_pre{ci}": ka, f"v{ci}": vb, f"q{ci}": qb,
                       f"k{ci}": kb})
    kp, vp = B.pool()
    rec.add(name, {"kind": "rope_prefill", "H": H, "Hkv": Hkv, "hd": hd, "layers": 1,
                   "pages": blocks, "layer": 0, "pool_seed": pool_seed, "chunks": len(chunks),
                   "observed": 32, "seq_len": B.seq_len, "rope_base": 10000.0,
                   "k_pool_digest": array_digest(kp[:, 0]), "v_pool_digest": array_digest(vp[:, 0])},
            xb2_obs=xb2[:, -32:], table=B.block_table(0), chunk_starts=np.array(starts, np.int32),
            **arrays)
    A.close()
    B.close()


def make_attention():
    rec = Recorder()
    case_decode(rec, "decode_mha_hd16_l2", 4, 4, 16, 2, 24, [0, 15, 16, 37], 21)
    case_decode(rec, "decode_gqa_h8kv2_hd16", 8, 2, 16, 1, 32, [3, 31, 32, 50, 64], 22)
    case_decode(rec, "decode_hd64", 2, 2, 64, 1, 32, [1, 47, 80], 23)
    case_decode(rec, "decode_hd128", 1, 1, 128, 1, 16, [0, 20, 33], 24)
    case_single(rec, "single_hd32_l2", 4, 4, 32, 2, 16, 45, 31)
    case_single(rec, "single_gqa_hd64", 4, 2, 64, 1, 16, 70, 32)
    case_single(rec, "single_pos0", 2, 2, 64, 1, 8, 0, 33)
    case_prefill(rec, "prefill_fresh_hd16_l2", 4, 4, 16, 2, 16, [37], 41)
    case_prefill(rec, "prefill_continued_gqa", 4, 2, 16, 1, 16, [20, 25], 42)
    case_prefill(rec, "prefill_hd64", 2, 2, 64, 1, 16, [33], 43)
    case_prefix_hit(rec, "prefix_hit_gqa_l2", 4, 2, 16, 2, 24, 32, 8, 20, 51)
    case_decode(rec, "decode_gqa_h4kv2_hd32", 4, 2, 32, 2, 32, [0, 16, 31, 77], 25)
    case_prefill(rec, "prefill_gqa_hd32_l2", 4, 2, 32, 2, 16, [19, 30], 44)
    case_prefix_hit(rec, "prefix_hit_hd32", 2, 2, 32, 1, 24, 48, 5, 21, 52)
    case_rope_decode(rec, "rope_decode_gqa_hd32", 4, 2, 32, 32, [0, 17, 40, 63], 71)
    case_rope_decode(rec, "rope_decode_hd64", 2, 2, 64, 24, [5, 33], 72)
    case_rope_single(rec, "rope_single_hd32", 4, 4, 32, 16, 50, 73)
    case_rope_prefill(rec, "rope_prefill_hd32", 4, 4, 32, 16, [21, 30], 74)
    case_contiguous(rec, "contiguous_hd16", 4, 4, 16, 30, 61)
    case_contiguous(rec, "contiguous_gqa_hd32", 4, 2, 32, 19, 62)
    return rec


Q8_CASES = [
    # name, n, d, batch, seed
    ("q8_n64_d48_b3", 64, 48, 3, 91),
    ("q8_n96_d40_b2", 96, 40, 2, 92),      # odd number of blocks per row
    ("q8_n32_d16_b4", 32, 16, 4, 93),      # one block per row
    ("q8_n256_d96_b5", 256, 96, 5, 94),
    ("q8_n128_d33_b1", 128, 33, 1, 95),    # rows not a multiple of 16
]


def make_q8():
    """Q8 products (src/model_q8.cpp:92-125 matmul, :382-420 matmul_bulk) of the
    reference build on matrices quantised with oracle.model.quantize_q8 (a
    restatement of scripts/quantize.py).  Row 0 holds an all-zero block (scale
    1e-9) and a block with one large outlier."""
    from oracle import model as om

    arrays, meta = {}, {}
    for name, n, d, batch, seed in Q8_CASES:
        W = counter_uniform(seed, d * n).reshape(d, n) * np.float32(0.05)
        W[0, :32] = 0.0
        if n >= 64:
            W[0, 32:64] *= np.float32(0.01)
            W[0, 40] = np.float32(3.0)
        scale, q = om.quantize_q8(W)
        w = om.pack_q8(scale, q)
        x = counter_uniform(seed + 1000, batch * n).reshape(batch, n)
        full = np.stack([ref.q8_matmul(w, x[b], n, d) for b in range(batch)])
        bulk = ref.q8_matmul_bulk(w, x, n, d)
        arrays[f"{name}/w"] = w
        arrays[f"{name}/x"] = x
        arrays[f"{name}/full"] = full
        arrays[f"{name}/bulk"] = bulk
        meta[name] = dict(n=n, d=d, batch=batch)
    return meta, arrays


MODEL = dict(n_heads=4, n_kv_heads=2, head_dim=32, n_layers=2, vocab=160, seq_len=128,
             hidden_dim=96, total_blocks=48)


def make_model():
    """Logits of the reference's forward passes on a tiny random model
    (ref_model_create), over a script that mixes forward_prefill_chunk (fresh
    and continued chunks), forward_paged and forward_decode_batch, one
    reference thread (forward_decode_batch allocates inside an OpenMP loop).
    Returns (model file bytes, meta, arrays)."""
    W = ref.RefWorld.random_model(**MODEL, max_rows=64, max_seqs=4, seed=4242, threads=1)
    blob = W.serialize()
    rng = np.random.default_rng(4343)
    V = MODEL["vocab"]
    toks = lambda n: rng.integers(0, V, size=n).astype(np.int32)
    for slot in range(3):
        W.op(pm.OP_SEQ_NEW, slot)
    script = [("prefill", [0], toks(37)), ("prefill", [1], toks(20)), ("prefill", [1], toks(13))]
    script += [("paged", [2], toks(1)) for _ in range(5)]
    script += [("decode", [0, 1], toks(2)) for _ in range(3)]
    script += [("decode", [0, 1, 2], toks(3)) for _ in range(2)]
    script += [("prefill", [2], toks(11)), ("decode", [2, 0], toks(2))]
    meta, arrays = [], {}
    for i, (kind, slots, t) in enumerate(script):
        if kind == "prefill":
            start = W.prefill_chunk(slots[0], t)
            lg = W.logits(1)
            meta.append(dict(kind=kind, slots=slots, start=start))
        elif kind == "paged":
            pos = W.forward_paged(slots[0], int(t[0]))
            lg = W.logits(1)
            meta.append(dict(kind=kind, slots=slots, pos=pos))
        else:
            pos = W.decode_batch(slots, t)
            lg = W.logits(len(slots))
            meta.append(dict(kind=kind, slots=slots, pos=[int(p) for p in pos]))
        arrays[f"{i}/tokens"] = t
        arrays[f"{i}/logits"] = lg
    tables = {str(slot): W.block_table(slot).tolist() for slot in range(3)}
    W.close()
    return blob, dict(model=MODEL, script=meta, final_tables=tables), arrays


# Scheduler scenarios over the tiny model with wo/w2 scaled by SCHED_OUT_SCALE
# (so the layers, not the token's own embedding, decide the argmax).  Each is
# (name, total_blocks, max_tokens_per_batch, {step: [(req_id, prompt_len or
# prompt source)]}); prompts are drawn from SCHED_PROMPT_SEED.
SCHED_OUT_SCALE = 64.0
SCHED_PROMPT_SEED = 9
SCHED_TOP = 16


def sched_scenarios():
    rng = np.random.default_rng(SCHED_PROMPT_SEED)
    V = MODEL["vocab"]
    tok = lambda n: [int(t) for t in rng.integers(0, V, n)]
    shared = tok(40)
    s = [("shared_prompt", 48, 256, {0: [(i, shared) for i in range(5)]})]
    s.append(("chunked", 48, 24, {0: [(0, tok(70)), (1, tok(33))], 3: [(2, tok(50))],
                                  6: [(3, tok(5))]}))
    s.append(("budget_exhausted", 48, 3, {0: [(0, tok(20)), (1, tok(9)), (2, tok(5)),
                                              (3, tok(7))]}))
    p = tok(32)
    s.append(("full_hit", 48, 256, {0: [(0, p)], 2: [(1, p), (2, p + tok(5))], 4: [(3, p[:16])]}))
    s.append(("eviction", 16, 256, {0: [(0, tok(40)), (1, tok(40))], 10: [(2, tok(40))],
                                    22: [(3, tok(40))], 25: [(4, tok(40))], 30: [(5, tok(24))]}))
    return s


def make_sched():
    """Steps of the reference's Continuous_Scheduler (src/pagedMemory.hpp:287-399)
    over the tiny model, one reference thread.  Per step: the scheduler state
    words (ref_sched_state), the block-manager snapshot words (ref_snapshot),
    and the largest SCHED_TOP logits (value, index) of every row the step left
    in s->logits: the decode rows when a decode batch ran, else the prefill
    chunk's last row.  The same steps replayed by the oracle scheduler on the
    oracle model must agree, and every argmax decision must win by a margin
    well above fp32 rounding (checked here, so the fixture is robust)."""
    from oracle import scheduler as sc
    from oracle.model import OracleModel, scale_residual_outputs

    meta, arrays = [], {}
    min_gap = np.inf
    for name, total, budget, arrivals in sched_scenarios():
        W = ref.RefWorld.random_model(**dict(MODEL, total_blocks=total), max_rows=256, max_seqs=0,
                                      seed=4242, threads=1, out_scale=SCHED_OUT_SCALE)
        blob = W.serialize()
        base = np.fromfile(os.path.join(HERE, "model_tiny.bin"), dtype=np.uint8)
        assert np.array_equal(blob, scale_residual_outputs(base, SCHED_OUT_SCALE))
        W.sched_create(budget)
        mem = pm.KVBlockManager(total)
        cache = pm.PrefixCacheManager(mem, total)
        S = sc.ContinuousScheduler(mem, cache, budget)
        fwd = sc.OracleForward(OracleModel(blob), total)
        states, bms, tops_v, tops_i, rows, kinds = [], [], [], [], [], []
        t, last = 0, max(arrivals)
        evicted = False
        while True:
            for rid, prompt in arrivals.get(t, []):
                W.sched_add(rid, prompt)
                S.add_request(sc.Request(rid, prompt))
            if not W.sched_active() and t >= last:
                assert not S.has_active_requests()
                break
            cached_before = set(cache.reverse_map)
            assert W.sched_step() == 0, (name, t)
            p = S.step(fwd)
            evicted |= bool(cached_before - set(cache.reverse_map))
            st = W.sched_state()
            assert st.tolist() == S.state_words(), (name, t)
            snap = W.snapshot()
            bm_words = _snapshot_words(W)
            states.append(st)
            bms.append(bm_words)
            if p.decode_reqs:
                lg = W.logits(len(p.decode_reqs))
                np.testing.assert_allclose(lg, fwd.decode_logits, atol=1e-3, rtol=1e-4)
                kinds.append(1)
            elif p.prefill_req is not None:
                lg = W.logits(1)
                np.testing.assert_allclose(lg[0], fwd.prefill_logits, atol=1e-3, rtol=1e-4)
                kinds.append(2)
            else:
                lg = np.zeros((0, MODEL["vocab"]), np.float32)
                kinds.append(0)
            decided = list(fwd.decode_logits) if fwd.decode_logits is not None else []
            if p.prefill_req is not None and p.prefill_req.is_prefill_done:
                decided.append(fwd.prefill_logits)
            for row in decided:
                srt = np.sort(row)[::-1]
                min_gap = min(min_gap, srt[0] - srt[1], srt[0])
            idx = np.argsort(-lg, axis=1, kind="stable")[:, :SCHED_TOP].astype(np.int32)
            tops_i.append(idx)
            tops_v.append(np.take_along_axis(lg, idx, axis=1))
            rows.append(len(lg))
            assert snap["free_list"] == list(mem.free_list), (name, t)
            t += 1
        if name == "eviction":
            assert evicted, "eviction scenario never evicted"
        W.close()
        off = lambda parts: np.cumsum([0] + [len(x) for x in parts]).astype(np.int64)
        arrays[f"{name}/state"] = np.concatenate(states).astype(np.int32)
        arrays[f"{name}/state_off"] = off(states)
        arrays[f"{name}/bm"] = np.concatenate(bms).astype(np.int32)
        arrays[f"{name}/bm_off"] = off(bms)
        arrays[f"{name}/top_val"] = np.concatenate(tops_v).astype(np.float32)
        arrays[f"{name}/top_idx"] = np.concatenate(tops_i).astype(np.int32)
        arrays[f"{name}/rows"] = np.asarray(rows, np.int32)
        arrays[f"{name}/kind"] = np.asarray(kinds, np.int32)
        meta.append(dict(name=name, total_blocks=total, max_tokens_per_batch=budget, steps=t,
                         arrivals={str(k): [[rid, list(pr)] for rid, pr in v]
                                   for k, v in arrivals.items()}))
    assert min_gap > 0.05, f"an argmax decision wins by only {min_gap}"
    return dict(model=MODEL, seed=4242, out_scale=SCHED_OUT_SCALE, max_generated=20,
                top=SCHED_TOP, min_gap=float(min_gap), scenarios=meta), arrays


def _snapshot_words(W) -> np.ndarray:
    cap = 1 << 20
    buf = np.zeros(cap, dtype=np.int32)
    n = ref.lib().ref_snapshot(W.h, buf.ctypes.data_as(ref._i32p), cap)
    assert n >= 0
    return buf[:n].copy()


def make_rpc():
    """The reference's NitroRPC (src/NitroRPC.hpp) over UNIX socket pairs: the
    bytes send_ints puts on the wire for a set of int vectors, and what
    recv_ints / recv_structured_query decode from hand-made messages
    (including a message cut short, which the reference reports as failure)."""
    import ctypes
    import socket

    L = ref.lib()
    rng = np.random.default_rng(99)
    out = []

    def drain(sock):
        sock.setblocking(False)
        data = b""
        while True:
            try:
                chunk = sock.recv(1 << 16)
            except BlockingIOError:
                break
            if not chunk:
                break
            data += chunk
        return data

    vectors = [[], [7], [1, 2, 3], [-1, 2**31 - 1, -2**31, 0],
               [int(v) for v in rng.integers(-2**31, 2**31, 300)]]
    for vals in vectors:
        a, b = socket.socketpair()
        arr = np.asarray(vals, np.int32)
        assert L.ref_rpc_send_ints(a.fileno(), arr.ctypes.data_as(ref._i32p), arr.size) == 0
        wire = drain(b)
        a.close(), b.close()
        out.append(dict(kind="send_ints", values=vals, wire=wire.hex()))
    for vals in vectors[1:]:
        a, b = socket.socketpair()
        msg = np.asarray([len(vals)] + vals, np.int32).tobytes()
        b.sendall(msg)
        buf = np.zeros(max(1, len(vals)), np.int32)
        n = L.ref_rpc_recv_ints(a.fileno(), buf.ctypes.data_as(ref._i32p), buf.size)
        a.close(), b.close()
        out.append(dict(kind="recv_ints", wire=msg.hex(), count=int(n), values=buf[:max(n, 0)].tolist()))
    # a message cut short: count 5, two values, then the peer closes
    a, b = socket.socketpair()
    msg = np.asarray([5, 10, 20], np.int32).tobytes()
    b.sendall(msg)
    b.close()
    buf = np.zeros(8, np.int32)
    n = L.ref_rpc_recv_ints(a.fileno(), buf.ctypes.data_as(ref._i32p), buf.size)
    a.close()
    out.append(dict(kind="recv_ints_truncated", wire=msg.hex(), count=int(n)))
    for dim, seed in ((8, 1), (0, 2), (33, 3)):
        r = np.random.default_rng(seed)
        mask = int(r.integers(0, 2**63)) * 2 + 1
        lo, hi = np.float32(r.standard_normal()), np.float32(r.standard_normal())
        vec = r.standard_normal(dim).astype(np.float32)
        msg = (np.uint64(mask).tobytes() + lo.tobytes() + hi.tobytes() + vec.tobytes())
        a, b = socket.socketpair()
        b.sendall(msg)
        m = ctypes.c_uint64()
        flo, fhi = ctypes.c_float(), ctypes.c_float()
        got = np.zeros(max(dim, 1), np.float32)
        st = L.ref_rpc_recv_structured_query(a.fileno(), dim, ctypes.byref(m), ctypes.byref(flo),
                                             ctypes.byref(fhi), got.ctypes.data_as(ref._f32p))
        a.close(), b.close()
        assert st == 0
        out.append(dict(kind="recv_structured_query", dim=dim, wire=msg.hex(), subset_mask=int(m.value),
                        range_min=float(flo.value), range_max=float(fhi.value),
                        vec=got[:dim].astype(np.float64).tolist()))
    return out


def main():
    if not ref.available():
        sys.exit("oracle/_ref/libnitro_ref.so is missing: run `make -C oracle ref` first")
    with open(os.path.join(HERE, "fnv.json"), "w") as f:
        json.dump(make_fnv(), f, indent=0)
    with open(os.path.join(HERE, "block_manager_traces.json"), "w") as f:
        json.dump(make_traces(), f, separators=(",", ":"))
    rec = make_attention()
    with open(os.path.join(HERE, "attention.json"), "w") as f:
        json.dump(rec.meta, f, indent=1)
    np.savez_compressed(os.path.join(HERE, "attention.npz"), **rec.arrays)
    q8_meta, q8_arrays = make_q8()
    with open(os.path.join(HERE, "q8_matmul.json"), "w") as f:
        json.dump(q8_meta, f, indent=1)
    np.savez_compressed(os.path.join(HERE, "q8_matmul.npz"), **q8_arrays)
    blob, m_meta, m_arrays = make_model()
    blob.tofile(os.path.join(HERE, "model_tiny.bin"))
    with open(os.path.join(HERE, "model_forward.json"), "w") as f:
        json.dump(m_meta, f, indent=1)
    np.savez_compressed(os.path.join(HERE, "model_forward.npz"), **m_arrays)
    with open(os.path.join(HERE, "rpc.json"), "w") as f:
        json.dump(make_rpc(), f, indent=0)
    s_meta, s_arrays = make_sched()
    with open(os.path.join(HERE, "sched_traces.json"), "w") as f:
        json.dump(s_meta, f, separators=(",", ":"))
    np.savez_compressed(os.path.join(HERE, "sched_traces.npz"), **s_arrays)
    for fn in ("fnv.json", "block_manager_traces.json", "attention.json", "attention.npz",
               "q8_matmul.json", "q8_matmul.npz", "model_tiny.bin", "model_forward.json",
               "model_forward.npz", "sched_traces.json", "sched_traces.npz", "rpc.json"):
        print(fn, os.path.getsize(os.path.join(HERE, fn)))


if __name__ == "__main__":
    main()
