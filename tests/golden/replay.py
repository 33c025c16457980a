"""Rebuilds the pools a golden attention case ran on, for any implementation.

The reference driver filled each pool with counter_pool(seed) before the
recorded call; the call then wrote the K/V rows recorded in the fixture.
Page rows are written here with plain numpy indexing (no oracle code), so the
same rebuilt pool can feed the oracle and the HIP path.
"""
from __future__ import annotations

import hashlib

import numpy as np

from synth import counter_pool


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()[:16]


def write_rows(pool, layer, table, start, rows):
    for t in range(rows.shape[0]):
        pos = start + t
        pool[table[pos // 16], layer, pos % 16, :] = rows[t]


def base_pools(meta):
    kv_dim = meta["Hkv"] * meta["hd"]
    k = counter_pool(meta["pool_seed"], meta["pages"], meta["layers"], kv_dim)
    v = counter_pool(meta["pool_seed"] + 1, meta["pages"], meta["layers"], kv_dim)
    return k, v


def pools_after_call(meta, arr):
    """Pools as the observed attention saw them (observed layer only is exact)."""
    k, v = base_pools(meta)
    layer = meta["layer"]
    kind = meta["kind"]
    if kind in ("decode_batch", "rope_decode"):
        for b, pos in enumerate(arr["positions"]):
            write_rows(k, layer, arr["tables"][b], int(pos), arr["k"][b:b + 1])
            write_rows(v, layer, arr["tables"][b], int(pos), arr["v"][b:b + 1])
    elif kind in ("decode_single", "rope_single"):
        write_rows(k, layer, arr["table"], meta["pos"], arr["k"])
        write_rows(v, layer, arr["table"], meta["pos"], arr["v"])
    elif kind == "prefill":
        starts = arr["chunk_starts"]
        if "earlier_k" in arr:
            write_rows(k, layer, arr["table"], int(starts[0]), arr["earlier_k"])
            write_rows(v, layer, arr["table"], int(starts[0]), arr["earlier_v"])
        write_rows(k, layer, arr["table"], meta["start_pos"], arr["k"])
        write_rows(v, layer, arr["table"], meta["start_pos"], arr["v"])
    elif kind == "prefix_hit":
        write_rows(k, layer, arr["table_a"], 0, arr["k_a"])
        write_rows(v, layer, arr["table_a"], 0, arr["v_a"])
        write_rows(k, layer, arr["table"], meta["start_pos"], arr["k"])
        write_rows(v, layer, arr["table"], meta["start_pos"], arr["v"])
    elif kind == "rope_prefill":
        for ci, st in enumerate(arr["chunk_starts"]):
            write_rows(k, layer, arr["table"], int(st), arr[f"k{ci}"])
            write_rows(v, layer, arr["table"], int(st), arr[f"v{ci}"])
    else:
        raise ValueError(kind)
    return k, v
