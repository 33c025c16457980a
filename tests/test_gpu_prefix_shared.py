"""End to end on the GPU: host page bookkeeping -> paged prefill -> paged decode,
with FNV-1a prefix-cache sharing (the prefix-shared decode workload: B=48
sequences whose first 512 tokens map to the same 32 physical pages, then
private suffixes of 64-512 tokens, 12 heads x 64).

Bookkeeping is checked bit-exactly against the Python restatement of the
reference (block tables, reference counts); attention outputs against the CPU
oracle at the parity bar."""
import sys

import numpy as np
import pytest

from gpu_helpers import assert_parity, to_gpu
from oracle import attn
from oracle import paged_memory as pm

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def test_prefix_shared_prefill_then_decode():
    import torch

    import nitrorag_amd as na

    assert torch.cuda.is_available()
    say("prefix-shared end to end")
    rng = np.random.default_rng(0x4E495452)
    B, H, hd, prefix = 48, 12, 64, 512
    kv_dim = H * hd
    suffix = rng.integers(64, 513, size=B)
    suffix[0] = 0
    pages = 32 + int(((suffix + 1 + 15) // 16).sum()) + 16
    shared = rng.integers(1, 32000, size=prefix).tolist()
    prompts = [shared + rng.integers(1, 32000, size=int(s)).tolist() for s in suffix]

    bm = na.BlockManager(pages)
    world = pm.World(pages, B)  # the restatement, driven in lockstep
    seqs = [na.Sequence(b) for b in range(B)]
    for b in range(B):
        world.op(pm.OP_SEQ_NEW, b)

    k = torch.zeros((pages, 1, 16, kv_dim), device="cuda")
    v = torch.zeros_like(k)
    pool = na.KVPool.wrap(k, v)

    # 1) sequence 0 ingests the shared prefix and publishes its pages
    seqs[0].ingest_prompt(prompts[0], bm, True)
    seqs[0].flush_cache(bm)
    world.op(pm.OP_INGEST, 0, 1, toks=prompts[0])
    world.op(pm.OP_SEQ_FLUSH, 0)
    kc = rng.standard_normal((prefix, kv_dim)).astype(np.float32)
    vc = rng.standard_normal((prefix, kv_dim)).astype(np.float32)
    pool.upload_prefill_batch(na.pack_block_tables([seqs[0]]), [0], [prefix])
    pool.kv_append_prefill(0, to_gpu(kc), to_gpu(vc))

    # 2) the other 47 hit all 32 shared pages and prefill only their suffixes
    starts, lens = [], []
    for b in range(1, B):
        n = seqs[b].ingest_prompt(prompts[b], bm, True)
        st, n2 = world.op(pm.OP_INGEST, b, 1, toks=prompts[b])
        assert st == 0 and n2 == n == prefix + suffix[b]
        starts.append(prefix)
        lens.append(int(suffix[b]))
    tables = na.pack_block_tables(seqs[1:])
    for b in range(B):
        assert seqs[b].block_table == world.seqs[b].block_table  # bit-exact bookkeeping
        assert seqs[b].block_table[:32] == seqs[0].block_table[:32]
    for pid in seqs[0].block_table[:32]:
        assert bm.get_block(pid)["ref_count"] == B
        assert world.mem.blocks[pid].ref_count == B
    total = int(sum(lens))
    q = rng.standard_normal((total, H * hd)).astype(np.float32)
    kc2 = rng.standard_normal((total, kv_dim)).astype(np.float32)
    vc2 = rng.standard_normal((total, kv_dim)).astype(np.float32)
    pool.upload_prefill_batch(tables, starts, lens)
    pool.kv_append_prefill(0, to_gpu(kc2), to_gpu(vc2))
    out = torch.empty((total, H * hd), device="cuda")
    pool.prefill(0, to_gpu(q), out, H, H, hd)
    torch.cuda.synchronize()
    kh, vh = k.cpu().numpy(), v.cpu().numpy()
    # oracle on the same pool (the shared rows were written once, by sequence 0)
    want = np.zeros_like(q)
    off = 0
    for i, (s, n) in enumerate(zip(starts, lens)):
        want[off:off + n] = attn.prefill_chunk(kh, vh, 0, q[off:off + n], tables[i], s, H, H, hd)
        off += n
    assert_parity(out.cpu().numpy(), want, "suffix prefill")

    # 3) one decode step for all 48: positions before the append, sequential allocation
    positions = np.array([s.logical_token_count for s in seqs], np.int32)
    for b in range(B):
        seqs[b].allocate_next_token(7, bm)
        world.op(pm.OP_SEQ_APPEND, b, 7)
        assert seqs[b].block_table == world.seqs[b].block_table
    tables = na.pack_block_tables(seqs)
    qd = rng.standard_normal((B, H * hd)).astype(np.float32)
    kn = rng.standard_normal((B, kv_dim)).astype(np.float32)
    vn = rng.standard_normal((B, kv_dim)).astype(np.float32)
    pool.upload_decode_batch(tables, positions)
    pool.kv_append(0, to_gpu(kn), to_gpu(vn))
    od = torch.empty((B, H * hd), device="cuda")
    pool.decode(0, to_gpu(qd), od, H, H, hd)
    torch.cuda.synchronize()
    attn.kv_append_decode(kh, vh, 0, kn, vn, tables, positions)
    assert np.array_equal(k.cpu().numpy(), kh) and np.array_equal(v.cpu().numpy(), vh)
    assert_parity(od.cpu().numpy(), attn.decode_batch(kh, vh, 0, qd, tables, positions, H, H, hd),
                  "prefix-shared decode")
    assert pool.take_device_errors() == 0
