"""Decode over shared prefixes (prefix-cache hits) on the GPU.

When sequences of a decode batch begin with the same physical pages, the
launch streams those rows once per set of member sequences (member items) and
each sequence's own rows as usual, then merges the two kinds of partial.  The
reference reads every sequence's pages independently
(src/model_q8.cpp:625-662); the outputs must match the oracle at the parity
bar whichever way the rows are read.  These batches are far below the size
where the library takes the form by itself, so every case forces it
(NITRO_DECODE_PREFIX=2) and also runs with it switched off (=0); the two
results must agree at the same bar, and the launch counts show which form
ran."""
import sys
import zlib

import numpy as np
import pytest

from gpu_helpers import assert_parity, to_gpu
from oracle import attn

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def shared_tables(rng, groups, loners, pages):
    """Tables where each group's members share their first `shared` pages.

    groups: (members, shared pages, own rows low, own rows high); loners: context
    lengths of sequences that share nothing.  Page ids come from one
    permutation of the pool.  Returns (tables, positions)."""
    perm = list(rng.permutation(pages))
    rows, ctx = [], []
    for members, shared, lo, hi in groups:
        common = [perm.pop() for _ in range(shared)]
        for _ in range(members):
            own = int(rng.integers(lo, hi + 1))
            n = shared * 16 + own
            rows.append(common + [perm.pop() for _ in range((n + 15) // 16 - shared)])
            ctx.append(n)
    for n in loners:
        rows.append([perm.pop() for _ in range((n + 15) // 16)])
        ctx.append(n)
    width = max(len(r) for r in rows)
    tables = np.zeros((len(rows), width), np.int32)
    for b, r in enumerate(rows):
        tables[b, :len(r)] = r
    order = rng.permutation(len(rows))  # members of a group are not adjacent in the batch
    return tables[order], (np.asarray(ctx, np.int32) - 1)[order]


CASES = {
    # name: (groups, loners, H, Hkv, hd, pool pages)
    "one_group_12x64": ([(10, 8, 1, 300)], [40, 700, 17], 12, 12, 64, 200),
    "two_groups_odd_sets": ([(5, 4, 20, 90), (7, 13, 1, 200)], [300], 4, 4, 64, 200),
    "big_group_8x128": ([(33, 8, 1, 120)], [64], 8, 8, 128, 400),
    "hd32": ([(6, 16, 5, 400)], [], 4, 4, 32, 200),
    "hd256": ([(5, 4, 1, 64)], [33], 2, 2, 256, 80),
    "padded_hd48": ([(6, 4, 1, 100)], [90], 4, 4, 48, 100),
    "gqa_uses_the_usual_launch": ([(6, 8, 1, 100)], [50], 8, 2, 64, 150),
    "own_rows_just_the_newest": ([(9, 4, 1, 1)], [], 4, 4, 64, 100),
    "list_too_long": ([(180, 4, 100, 400)], [], 2, 2, 64, 5000),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_shared_prefix_decode_matches_oracle(name, monkeypatch):
    import torch

    import nitrorag_amd as na

    groups, loners, H, Hkv, hd, pages = CASES[name]
    say(f"shared-prefix decode {name}")
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    tables, positions = shared_tables(rng, groups, loners, pages)
    kv_dim = Hkv * hd
    k = rng.standard_normal((pages, 1, 16, kv_dim)).astype(np.float32)
    v = rng.standard_normal((pages, 1, 16, kv_dim)).astype(np.float32)
    q = rng.standard_normal((len(positions), H * hd)).astype(np.float32)
    want = attn.decode_batch(k, v, 0, q, tables, positions, H, Hkv, hd)
    dk, dv, dq = to_gpu(k), to_gpu(v), to_gpu(q)
    pool = na.KVPool.wrap(dk, dv)
    pool.upload_decode_batch(tables, positions)
    outs = []
    for prefix in ("2", "0"):
        monkeypatch.setenv("NITRO_DECODE_PREFIX", prefix)
        for rep in range(2):  # twice: the arrival counters are left at zero
            out = torch.full_like(dq, float("nan"))
            pool.decode(0, dq, out, H, Hkv, hd)
            torch.cuda.synchronize()
            assert_parity(out.cpu().numpy(), want, f"{name} prefix={prefix} rep={rep}")
        outs.append(out.cpu().numpy())
    assert_parity(outs[0], outs[1], f"{name}: shared-prefix vs usual launch")
    # GQA runs the usual launch; a list too long for the kernel arguments too
    takes_form = name not in ("gqa_uses_the_usual_launch", "list_too_long")
    assert pool.decode_counts() == (4, 2 if takes_form else 0)
    assert pool.take_device_errors() == 0


@pytest.mark.parametrize("prefix", ["2", "0"])
def test_shared_prefix_decode_append(prefix, monkeypatch):
    """decode_append over a batch with a shared prefix: the appended rows are
    each sequence's own (the shared pages end below every newest row), so the
    append stays fused; the pools hold the reference's appended rows and the
    outputs match the oracle's append + decode."""
    import torch

    import nitrorag_amd as na

    say(f"shared-prefix decode_append prefix={prefix}")
    monkeypatch.setenv("NITRO_DECODE_PREFIX", prefix)
    rng = np.random.default_rng(29)
    H, hd, pages = 6, 64, 150
    kv_dim = H * hd
    tables, positions = shared_tables(rng, [(12, 8, 1, 200)], [77], pages)
    B = len(positions)
    k = rng.standard_normal((pages, 1, 16, kv_dim)).astype(np.float32)
    v = rng.standard_normal((pages, 1, 16, kv_dim)).astype(np.float32)
    q = rng.standard_normal((B, H * hd)).astype(np.float32)
    knew = rng.standard_normal((B, kv_dim)).astype(np.float32)
    vnew = rng.standard_normal((B, kv_dim)).astype(np.float32)
    k2, v2 = k.copy(), v.copy()
    for b in range(B):  # the reference's memcpy of the new row (src/model_q8.cpp:616-623)
        p = int(positions[b])
        page = tables[b, p // 16]
        k2[page, 0, p % 16] = knew[b]
        v2[page, 0, p % 16] = vnew[b]
    want = attn.decode_batch(k2, v2, 0, q, tables, positions, H, H, hd)
    dk, dv = to_gpu(k), to_gpu(v)
    pool = na.KVPool.wrap(dk, dv)
    pool.upload_decode_batch(tables, positions)
    out = torch.full((B, H * hd), float("nan"), device="cuda")
    pool.decode_append(0, to_gpu(q), to_gpu(knew), to_gpu(vnew), out, H, H, hd)
    torch.cuda.synchronize()
    assert_parity(out.cpu().numpy(), want, "shared-prefix decode_append")
    assert pool.decode_counts() == (1, 1 if prefix == "2" else 0)
    assert np.array_equal(dk.cpu().numpy(), k2) and np.array_equal(dv.cpu().numpy(), v2)


def test_shared_prefix_decode_random_groups(monkeypatch):
    """Fifteen seeded random batches of prefix groups (2-40 members sharing 4-40
    pages, own rows 1-300) and loners, MHA at head sizes 32-256: with the form
    forced on and off, each against the oracle at the parity bar, bit-identical
    on a second launch, and the counts show the form ran wherever the list fit
    the kernel arguments."""
    import torch

    import nitrorag_amd as na

    rng = np.random.default_rng(20261204)
    took_form = 0
    for i in range(15):
        hd = int(rng.choice([32, 48, 64, 96, 128, 256]))
        H = int(rng.integers(1, max(2, 1024 // hd // 2) + 1))
        groups = [(int(rng.integers(2, 41)), int(rng.integers(4, 41)), 1, int(rng.integers(1, 301)))
                  for _ in range(int(rng.integers(1, 4)))]
        loners = [int(n) for n in rng.integers(1, 800, size=int(rng.integers(0, 4)))]
        pages = sum(m * ((s * 16 + hi + 15) // 16) for m, s, _, hi in groups) + sum((n + 15) // 16 for n in loners) + 4
        tables, positions = shared_tables(rng, groups, loners, pages)
        say(f"random shared-prefix decode {i}: H={H} hd={hd} groups={[(m, s) for m, s, _, _ in groups]} "
            f"loners={len(loners)}")
        k = rng.standard_normal((pages, 1, 16, H * hd)).astype(np.float32)
        v = rng.standard_normal((pages, 1, 16, H * hd)).astype(np.float32)
        q = rng.standard_normal((len(positions), H * hd)).astype(np.float32)
        want = attn.decode_batch(k, v, 0, q, tables, positions, H, H, hd)
        dq = to_gpu(q)
        pool = na.KVPool.wrap(to_gpu(k), to_gpu(v))
        pool.upload_decode_batch(tables, positions)
        for prefix in ("2", "0"):
            monkeypatch.setenv("NITRO_DECODE_PREFIX", prefix)
            out = torch.full_like(dq, float("nan"))
            pool.decode(0, dq, out, H, H, hd)
            torch.cuda.synchronize()
            first = out.cpu().numpy()
            assert_parity(first, want, f"random shared-prefix {i} prefix={prefix}")
            pool.decode(0, dq, out, H, H, hd)
            torch.cuda.synchronize()
            assert np.array_equal(out.cpu().numpy(), first)
        n, shared = pool.decode_counts()
        assert n == 4 and shared in (0, 2)
        took_form += shared == 2
        assert pool.take_device_errors() == 0
        pool.close()
    assert took_form >= 10, took_form  # the others' lists exceed the kernel arguments
