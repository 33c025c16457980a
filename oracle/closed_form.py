"""fp64 closed-form attention — TEST INFRASTRUCTURE ONLY.

softmax(q K^T / sqrt(hd)) V evaluated in float64 over the rows a block table
resolves to.  This is the textbook definition the reference's loops compute
(src/model_q8.cpp:625-662 two-pass, :485-523 online); it shares no code or
loop structure with the C oracle, so it checks the oracle's indexing (page
lookup, row bound, kv-head mapping, layer offset) and its arithmetic.
"""
from __future__ import annotations

import numpy as np

PAGE = 16


def gather_rows(pool: np.ndarray, layer: int, table, ctx: int) -> np.ndarray:
    """Rows 0..ctx-1 of one sequence: pool[table[t//16], layer, t%16, :] -> [ctx][kv_dim]."""
    t = np.arange(ctx)
    pages = np.asarray(table, dtype=np.int64)[t // PAGE]
    return pool[pages, layer, t % PAGE, :]


def attention_f64(q_heads: np.ndarray, k_rows: np.ndarray, v_rows: np.ndarray, n_heads: int,
                  n_kv_heads: int, head_dim: int) -> np.ndarray:
    """q_heads [H*hd]; k_rows, v_rows [ctx][Hkv*hd] -> out [H*hd] in float64."""
    q = q_heads.astype(np.float64).reshape(n_heads, head_dim)
    k = k_rows.astype(np.float64).reshape(-1, n_kv_heads, head_dim)
    v = v_rows.astype(np.float64).reshape(-1, n_kv_heads, head_dim)
    group = n_heads // n_kv_heads
    out = np.empty((n_heads, head_dim), dtype=np.float64)
    for h in range(n_heads):
        kh = h // group
        s = k[:, kh, :] @ q[h] / np.sqrt(head_dim)
        s = s - s.max()
        p = np.exp(s)
        p /= p.sum()
        out[h] = p @ v[:, kh, :]
    return out.reshape(-1)


def decode_batch_f64(k_pool, v_pool, layer, q, tables, positions, n_heads, n_kv_heads, head_dim):
    out = np.empty(q.shape, dtype=np.float64)
    for b, pos in enumerate(np.asarray(positions)):
        ctx = int(pos) + 1
        out[b] = attention_f64(q[b], gather_rows(k_pool, layer, tables[b], ctx),
                               gather_rows(v_pool, layer, tables[b], ctx), n_heads, n_kv_heads,
                               head_dim)
    return out


def prefill_f64(k_pool, v_pool, layer, q, table, start_pos, n_heads, n_kv_heads, head_dim):
    out = np.empty(q.shape, dtype=np.float64)
    for t in range(q.shape[0]):
        ctx = int(start_pos) + t + 1
        out[t] = attention_f64(q[t], gather_rows(k_pool, layer, table, ctx),
                               gather_rows(v_pool, layer, table, ctx), n_heads, n_kv_heads,
                               head_dim)
    return out


def within_tolerance(got: np.ndarray, want: np.ndarray, atol: float = 1e-4,
                     rtol: float = 1e-3) -> bool:
    """Elementwise |got - want| <= atol + rtol*|want| (the path's parity bar)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    return bool(np.all(np.abs(got - want) <= atol + rtol * np.abs(want)))
