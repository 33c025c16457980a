"""GPU parity of the fused RoPE + KV append (then attention) against the CPU
oracle and the reference's golden vectors (recorded with real RoPE tables)."""
import sys

import numpy as np
import pytest

from gpu_helpers import assert_parity, random_tables, to_gpu
from oracle import attn
from replay import base_pools, pools_after_call
from synth import rope_tables

pytestmark = pytest.mark.gpu

# RoPE is two products and a sum per element; the GPU may contract them into an
# FMA where the reference's build did not (or the other way): an ulp or two.
ROPE_TOL = dict(rtol=1e-6, atol=1e-5)


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


@pytest.mark.parametrize("name", ["rope_decode_gqa_hd32", "rope_decode_hd64", "rope_single_hd32"])
def test_rope_decode_matches_reference_golden(golden_attention, name):
    import torch

    import nitrorag_amd as na

    meta, arr = golden_attention[name]
    say(f"golden rope decode {name}")
    H, Hkv, hd = meta["H"], meta["Hkv"], meta["hd"]
    fr, fi = rope_tables(meta["seq_len"], hd, meta["rope_base"])
    if meta["kind"] == "rope_decode":
        tables, positions = arr["tables"], arr["positions"]
    else:
        tables, positions = arr["table"][None, :], np.array([meta["pos"]], np.int32)
    k0, v0 = base_pools(meta)
    dk, dv = to_gpu(k0), to_gpu(v0)
    pool = na.KVPool.wrap(dk, dv)
    pool.upload_decode_batch(tables, positions)
    q, k = to_gpu(arr["q_pre"]), to_gpu(arr["k_pre"])
    pool.rope_kv_append(0, q, k, to_gpu(arr["v"]), to_gpu(fr), to_gpu(fi), H, Hkv, hd)
    out = torch.empty_like(q)
    pool.decode(0, q, out, H, Hkv, hd)
    torch.cuda.synchronize()
    np.testing.assert_allclose(q.cpu().numpy(), arr["q"], **ROPE_TOL)
    np.testing.assert_allclose(k.cpu().numpy(), arr["k"], **ROPE_TOL)
    wk, wv = pools_after_call(meta, arr)  # the reference's pool after its forward pass
    np.testing.assert_allclose(dk.cpu().numpy(), wk, **ROPE_TOL)
    assert np.array_equal(dv.cpu().numpy(), wv)
    assert_parity(out.cpu().numpy()[:, -meta["observed"]:], arr["xb2_obs"], name)
    assert pool.take_device_errors() == 0


def test_rope_prefill_matches_reference_golden(golden_attention):
    import torch

    import nitrorag_amd as na

    meta, arr = golden_attention["rope_prefill_hd32"]
    say("golden rope prefill")
    H, Hkv, hd = meta["H"], meta["Hkv"], meta["hd"]
    fr, fi = to_gpu(rope_tables(meta["seq_len"], hd)[0]), to_gpu(rope_tables(meta["seq_len"], hd)[1])
    k0, v0 = base_pools(meta)
    dk, dv = to_gpu(k0), to_gpu(v0)
    pool = na.KVPool.wrap(dk, dv)
    table = arr["table"][None, :]
    for ci, st in enumerate(arr["chunk_starts"]):
        n = arr[f"q{ci}"].shape[0]
        pool.upload_prefill_batch(table, [int(st)], [n])
        q, k = to_gpu(arr[f"q_pre{ci}"]), to_gpu(arr[f"k_pre{ci}"])
        pool.rope_kv_append_prefill(0, q, k, to_gpu(arr[f"v{ci}"]), fr, fi, H, Hkv, hd)
        out = torch.empty_like(q)
        pool.prefill(0, q, out, H, Hkv, hd)
        torch.cuda.synchronize()
        np.testing.assert_allclose(q.cpu().numpy(), arr[f"q{ci}"], **ROPE_TOL)
        np.testing.assert_allclose(k.cpu().numpy(), arr[f"k{ci}"], **ROPE_TOL)
    assert_parity(out.cpu().numpy()[:, -meta["observed"]:], arr["xb2_obs"], "rope prefill")
    wk, _ = pools_after_call(meta, arr)
    np.testing.assert_allclose(dk.cpu().numpy(), wk, **ROPE_TOL)


@pytest.mark.parametrize("H,Hkv,hd", [(8, 2, 128), (12, 12, 64), (4, 4, 256)])
def test_rope_append_decode_vs_oracle(H, Hkv, hd):
    """Random batch: RoPE + append + decode on the GPU vs the oracle's three steps."""
    import torch

    import nitrorag_amd as na

    say(f"rope decode vs oracle {H}x{Hkv}x{hd}")
    rng = np.random.default_rng(hd + H)
    S, B, pages = 700, 6, 300
    ctx = rng.integers(1, S, size=B)
    tables = random_tables(rng, ctx, pages)
    kv_dim = Hkv * hd
    k0 = rng.standard_normal((pages, 1, 16, kv_dim)).astype(np.float32)
    v0 = rng.standard_normal((pages, 1, 16, kv_dim)).astype(np.float32)
    q = rng.standard_normal((B, H * hd)).astype(np.float32)
    kn = rng.standard_normal((B, kv_dim)).astype(np.float32)
    vn = rng.standard_normal((B, kv_dim)).astype(np.float32)
    fr, fi = rope_tables(S, hd)
    pos = (ctx - 1).astype(np.int32)
    dk, dv = to_gpu(k0), to_gpu(v0)
    pool = na.KVPool.wrap(dk, dv)
    pool.upload_decode_batch(tables, pos)
    dq, dkn = to_gpu(q), to_gpu(kn)
    pool.rope_kv_append(0, dq, dkn, to_gpu(vn), to_gpu(fr), to_gpu(fi), H, Hkv, hd)
    out = torch.empty_like(dq)
    pool.decode(0, dq, out, H, Hkv, hd)
    torch.cuda.synchronize()
    qr, kr = attn.rope(q, kn, pos, fr, fi, hd)
    attn.kv_append_decode(k0, v0, 0, kr, vn, tables, pos)
    np.testing.assert_allclose(dq.cpu().numpy(), qr, **ROPE_TOL)
    np.testing.assert_allclose(dk.cpu().numpy(), k0, **ROPE_TOL)
    assert np.array_equal(dv.cpu().numpy(), v0)
    assert_parity(out.cpu().numpy(), attn.decode_batch(k0, v0, 0, qr, tables, pos, H, Hkv, hd),
                  "rope + decode")


def test_rope_argument_errors():
    import torch

    import nitrorag_amd as na
    from nitrorag_amd import _native as N

    say("rope errors")
    k = torch.zeros((4, 1, 16, 64), device="cuda")
    pool = na.KVPool.wrap(k, torch.zeros_like(k))
    q = torch.zeros((1, 64), device="cuda")
    fr = torch.ones((8, 32), device="cuda")
    with pytest.raises(na.NitroError) as e:
        pool.rope_kv_append(0, q, q.clone(), q.clone(), fr, torch.zeros_like(fr), 1, 1, 64)
    assert e.value.status == N.NO_BATCH
    pool.upload_decode_batch([[0]], [9])
    with pytest.raises(na.NitroError) as e:  # position 9 needs a table of at least 10 rows
        pool.rope_kv_append(0, q, q.clone(), q.clone(), fr, torch.zeros_like(fr), 1, 1, 64)
    assert e.value.status == N.INVALID_ARGUMENT
