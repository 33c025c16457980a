"""The allocation-free decode entry (nitro_paged_attn_decode_static) through the
C ABI: its outputs match nitro_paged_attn_decode's on the same inputs (the
path's bar, 1e-4 + 1e-3|ref|) and the oracle's, on two calls in a row, the
second with a smaller batch and shorter contexts; both calls split the
contexts, so they use the static workspace (and the second reuses the
counters the first left at zero).  The device's free memory does not change
across the calls."""
import ctypes
import sys

import numpy as np
import pytest

from gpu_helpers import assert_parity, random_tables, to_gpu
from oracle import attn

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def free_device_bytes():
    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def static_decode(pool, layer, q, out, tables_d, pos_d, batch, max_pages, max_context, H, Hkv, hd,
                  pages_private=0):
    from nitrorag_amd import _native as N

    st = N.lib().nitro_paged_attn_decode_static(
        pool.handle, layer, ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(out.data_ptr()),
        ctypes.c_void_p(tables_d.data_ptr()), ctypes.c_void_p(pos_d.data_ptr()), batch, max_pages,
        max_context, H, Hkv, hd, pages_private, None)
    assert st == N.OK, N.last_error()


def test_static_decode_matches_decode_on_two_calls():
    import torch

    import nitrorag_amd as na

    assert torch.cuda.is_available()
    rng = np.random.default_rng(77)
    H, Hkv, hd, pages = 8, 2, 128, 900
    kv_dim = Hkv * hd
    k = rng.standard_normal((pages, 2, 16, kv_dim)).astype(np.float32)
    v = rng.standard_normal((pages, 2, 16, kv_dim)).astype(np.float32)
    dk, dv = to_gpu(k), to_gpu(v)
    pool = na.KVPool.wrap(dk, dv)
    # first call: 3 sequences up to 5000 tokens; second: 2 sequences up to 1800
    for call, ctx in enumerate([np.array([5000, 37, 3100]), np.array([1800, 900])]):
        say(f"static decode call {call}: contexts {ctx.tolist()}")
        B = len(ctx)
        tables = random_tables(rng, ctx, pages)
        positions = (ctx - 1).astype(np.int32)
        q = rng.standard_normal((B, H * hd)).astype(np.float32)
        dq = to_gpu(q)
        # reference entry: uploaded batch, pool-owned workspace
        pool.upload_decode_batch(tables, positions)
        ref = torch.full_like(dq, float("nan"))
        pool.decode(1, dq, ref, H, Hkv, hd)
        torch.cuda.synchronize()
        tables_d = to_gpu(tables)
        pos_d = to_gpu(positions)
        out = torch.full_like(dq, float("nan"))
        torch.cuda.synchronize()
        before = free_device_bytes()
        static_decode(pool, 1, dq, out, tables_d, pos_d, B, tables.shape[1], int(ctx.max()), H, Hkv, hd)
        torch.cuda.synchronize()
        assert free_device_bytes() == before
        got = out.cpu().numpy()
        assert_parity(got, ref.cpu().numpy(), f"call {call} vs nitro_paged_attn_decode")
        assert_parity(got, attn.decode_batch(k, v, 1, q, tables, positions, H, Hkv, hd),
                      f"call {call} vs oracle")
        # repeated launches are bit-identical (the counters were left at zero), and
        # so is the launch with non-temporal K/V loads (these tables share no page)
        for private in (0, 1):
            again = torch.full_like(dq, float("nan"))
            static_decode(pool, 1, dq, again, tables_d, pos_d, B, tables.shape[1], int(ctx.max()), H, Hkv, hd,
                          private)
            torch.cuda.synchronize()
            assert np.array_equal(again.cpu().numpy(), got)
    assert pool.take_device_errors() == 0


def test_static_decode_refuses_what_its_workspace_cannot_hold(monkeypatch):
    """The launch shapes the library picks always fit the 8 MiB workspace; one
    forced to a split per tile (64 x 4096 tokens, 32 heads x 128: 335 MB of
    partials) is refused with an argument error before anything runs, and
    max_context past the table is refused too."""
    import torch

    import nitrorag_amd as na
    from nitrorag_amd import _native as N

    k = torch.zeros((8, 1, 16, 32 * 128), device="cuda")
    pool = na.KVPool.wrap(k, torch.zeros_like(k))
    q = torch.zeros((64, 32 * 128), device="cuda")
    tables = torch.zeros((64, 256), dtype=torch.int32, device="cuda")
    pos = torch.zeros(64, dtype=torch.int32, device="cuda")

    def call(max_pages, max_context):
        return N.lib().nitro_paged_attn_decode_static(
            pool.handle, 0, ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(q.data_ptr()),
            ctypes.c_void_p(tables.data_ptr()), ctypes.c_void_p(pos.data_ptr()), 64, max_pages, max_context,
            32, 32, 128, 0, None)

    monkeypatch.setenv("NITRO_DECODE_SPLIT_TILES", "1")
    assert call(256, 4096) == N.INVALID_ARGUMENT
    assert "static workspace" in N.last_error()
    monkeypatch.delenv("NITRO_DECODE_SPLIT_TILES")
    assert call(256, 4097) == N.INVALID_ARGUMENT  # max_context past the table
    assert N.lib().nitro_paged_attn_decode_static(
        pool.handle, 0, ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(q.data_ptr()),
        ctypes.c_void_p(tables.data_ptr()), ctypes.c_void_p(pos.data_ptr()), 64, 256, 4096,
        32, 32, 128, 2, None) == N.INVALID_ARGUMENT  # pages_private is 0 or 1
    torch.cuda.synchronize()
