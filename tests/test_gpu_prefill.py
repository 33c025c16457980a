"""GPU parity of the causal paged prefill path (KV scatter + attention), through
the C ABI, against the CPU oracle and the reference's golden vectors."""
import sys

import numpy as np
import pytest

from gpu_helpers import assert_parity, to_gpu
from oracle import attn
from replay import base_pools, digest, write_rows

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    import nitrorag_amd  # noqa: F401
    yield
    torch.cuda.synchronize()


@pytest.fixture(params=["x3", "mfma32", "valu"], autouse=True)
def prefill_kernel(request, monkeypatch):
    """Every prefill test runs on the three kernels: bf16 matrix cores with
    three-part splits (default for hd <= 128), fp32 matrix cores
    (NITRO_PREFILL_KERNEL=mfma32) and the VALU one (hd 256, or =valu)."""
    monkeypatch.setenv("NITRO_PREFILL_KERNEL", request.param)
    return request.param


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def run_prefill(k, v, layer, tables, start_pos, lens, q, kc, vc, H, Hkv, hd):
    """GPU: upload the batch, scatter the chunk rows, attend. Returns (out, k_pool, v_pool)."""
    import torch

    import nitrorag_amd as na

    dk, dv = to_gpu(k), to_gpu(v)
    pool = na.KVPool.wrap(dk, dv)
    pool.upload_prefill_batch(tables, start_pos, lens)
    pool.kv_append_prefill(layer, to_gpu(kc), to_gpu(vc))
    dq = to_gpu(q)
    out = torch.full_like(dq, float("nan"))
    pool.prefill(layer, dq, out, H, Hkv, hd)
    torch.cuda.synchronize()
    assert pool.take_device_errors() == 0
    return out.cpu().numpy(), dk.cpu().numpy(), dv.cpu().numpy()


# every paged prefill case of the reference's golden vectors (head sizes 16, 32, 64;
# 16 runs the VALU kernel padded to 32 whichever kernel is asked for)
@pytest.mark.parametrize("name", ["prefill_hd64", "prefill_gqa_hd32_l2", "prefix_hit_hd32",
                                  "prefill_fresh_hd16_l2", "prefill_continued_gqa", "prefix_hit_gqa_l2"])
def test_prefill_matches_reference_golden(golden_attention, name):
    meta, arr = golden_attention[name]
    say(f"golden prefill {name}")
    layer, H, Hkv, hd = meta["layer"], meta["H"], meta["Hkv"], meta["hd"]
    k, v = base_pools(meta)
    if meta["kind"] == "prefix_hit":
        write_rows(k, layer, arr["table_a"], 0, arr["k_a"])
        write_rows(v, layer, arr["table_a"], 0, arr["v_a"])
    elif "earlier_k" in arr:
        write_rows(k, layer, arr["table"], int(arr["chunk_starts"][0]), arr["earlier_k"])
        write_rows(v, layer, arr["table"], int(arr["chunk_starts"][0]), arr["earlier_v"])
    T = arr["q"].shape[0]
    got, gk, gv = run_prefill(k, v, layer, arr["table"][None, :], [meta["start_pos"]], [T],
                              arr["q"], arr["k"], arr["v"], H, Hkv, hd)
    # the GPU scatter leaves the observed layer byte-identical to the reference's pool
    assert digest(gk[:, layer]) == meta["k_pool_digest"]
    assert digest(gv[:, layer]) == meta["v_pool_digest"]
    assert_parity(got[:, -meta["observed"]:], arr["xb2_obs"], name)
    attn.kv_scatter_prefill(k, v, layer, arr["k"], arr["v"], arr["table"], meta["start_pos"])
    want = attn.prefill_chunk(k, v, layer, arr["q"], arr["table"], meta["start_pos"], H, Hkv, hd)
    assert_parity(got, want, name + " (all heads vs oracle)")


def prefill_batch_case(seed, B, lo, hi, H, Hkv, hd, layers=1, layer=0, start_lo=0, start_hi=0,
                       slack=8):
    """Fresh pages from the host block manager (LIFO), random Q/K/V."""
    import nitrorag_amd as na

    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, size=B)
    starts = rng.integers(start_lo, start_hi + 1, size=B)
    pages = int(((starts + lens + 15) // 16).sum()) + slack
    bm = na.BlockManager(pages)
    seqs = []
    for b in range(B):
        s = na.Sequence(b)
        s.ingest_prompt(rng.integers(1, 32000, size=int(starts[b] + lens[b])), bm, False)
        seqs.append(s)
    tables = na.pack_block_tables(seqs)
    kv_dim = Hkv * hd
    k = rng.standard_normal((pages, layers, 16, kv_dim)).astype(np.float32)
    v = rng.standard_normal((pages, layers, 16, kv_dim)).astype(np.float32)
    total = int(lens.sum())
    q = rng.standard_normal((total, H * hd)).astype(np.float32)
    kc = rng.standard_normal((total, kv_dim)).astype(np.float32)
    vc = rng.standard_normal((total, kv_dim)).astype(np.float32)
    return dict(k=k, v=v, tables=tables, starts=starts, lens=lens, q=q, kc=kc, vc=vc, H=H,
                Hkv=Hkv, hd=hd, layer=layer)


def oracle_prefill_batch(c):
    k, v = c["k"].copy(), c["v"].copy()
    out = np.zeros_like(c["q"])
    off = 0
    for b, (s, n) in enumerate(zip(c["starts"], c["lens"])):
        rows = slice(off, off + int(n))
        attn.kv_scatter_prefill(k, v, c["layer"], c["kc"][rows], c["vc"][rows], c["tables"][b],
                                int(s))
        off += int(n)
    off = 0
    for b, (s, n) in enumerate(zip(c["starts"], c["lens"])):
        rows = slice(off, off + int(n))
        out[rows] = attn.prefill_chunk(k, v, c["layer"], c["q"][rows], c["tables"][b], int(s),
                                       c["H"], c["Hkv"], c["hd"])
        off += int(n)
    return out, k, v


CASES = {
    # name: (seed, B, len lo, len hi, H, Hkv, hd, layers, layer, start lo, start hi)
    "prompts_b8_12x64": (1, 8, 128, 1024, 12, 12, 64, 1, 0, 0, 0),
    "continued_chunks_gqa_8x2_hd128": (2, 4, 1, 200, 8, 2, 128, 2, 1, 1, 300),
    "short_chunks_hd32": (3, 6, 1, 70, 4, 4, 32, 1, 0, 0, 40),
    "mha_hd256": (4, 2, 30, 150, 2, 2, 256, 1, 0, 0, 20),
    "single_token_chunks": (5, 5, 1, 1, 4, 4, 64, 1, 0, 0, 100),
    # keys past the 2048 block-table entries a workgroup keeps in LDS (32k
    # tokens): the rest of the table is read from global memory
    "beyond_lds_table_hd64": (6, 2, 5, 40, 2, 2, 64, 1, 0, 33000, 33100),
    "beyond_lds_table_gqa_hd128": (7, 2, 5, 150, 2, 1, 128, 1, 0, 33000, 33100),
    # head sizes other than 32/64/128/256 (multiples of 4): the VALU kernel with
    # the head padded to the next kernel width and the extra columns masked
    "hd16_gqa_4x2": (8, 3, 1, 90, 4, 2, 16, 1, 0, 0, 30),
    "hd48": (9, 3, 20, 140, 3, 3, 48, 2, 1, 0, 17),
    "hd80_gqa_6x2": (10, 2, 1, 120, 6, 2, 80, 1, 0, 5, 40),
    "hd96": (11, 2, 30, 100, 2, 2, 96, 1, 0, 0, 0),
    "hd4": (12, 2, 1, 60, 2, 1, 4, 1, 0, 0, 20),
    "hd200": (13, 2, 10, 80, 2, 2, 200, 1, 0, 0, 9),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_prefill_batch_vs_oracle(name):
    say(f"prefill vs oracle {name}")
    seed, B, lo, hi, H, Hkv, hd, layers, layer, slo, shi = CASES[name]
    c = prefill_batch_case(seed, B, lo, hi, H, Hkv, hd, layers, layer, slo, shi)
    got, gk, gv = run_prefill(c["k"], c["v"], layer, c["tables"], c["starts"], c["lens"], c["q"],
                              c["kc"], c["vc"], H, Hkv, hd)
    want, wk, wv = oracle_prefill_batch(c)
    assert np.array_equal(gk, wk) and np.array_equal(gv, wv)  # scatter is bit-exact
    assert_parity(got, want, name)


@pytest.mark.parametrize("hd", [32, 64, 128])
def test_prefill_rising_and_falling_scores(hd):
    """Scores that climb by ~17 (log2 units) per 16-key block for four blocks,
    climb by ~5 per block for twelve, or fall: the running max moves every
    block, lags the true max by up to 2^8 in the weights, or never moves after
    the first keys.  Ranges stay within ~70 log2 units (|q.k| ~ 500), where
    fp32 summation order alone keeps any two implementations within the bar."""
    say(f"prefill score profiles hd={hd}")
    H = Hkv = 2
    c = prefill_batch_case(7, 3, 250, 400, H, Hkv, hd, 1, 0, 0, 0)
    rng = np.random.default_rng(70 + hd)
    u = rng.standard_normal((Hkv, hd)).astype(np.float32)
    u /= np.linalg.norm(u, axis=1, keepdims=True)
    # q = a*u: q.k_t / sqrt(hd) * log2(e) = a * c_t * log2(e) / sqrt(hd)
    a = 6.0 * np.sqrt(hd) / 8.0
    per_log2 = a * np.log2(np.e) / np.sqrt(hd)  # log2 units per unit of c_t
    off = 0
    for b, n in enumerate(c["lens"]):
        n = int(n)
        t = np.arange(n, dtype=np.float64)
        # log2-unit score of key t for an aligned query
        s2 = [17.0 / 16 * np.minimum(t, 64), 5.0 / 16 * np.minimum(t, 200),
              np.minimum(60.0, 3.0 / 16 * (n - t))][b]
        ct = s2 / per_log2
        for kh in range(Hkv):
            cols = slice(kh * hd, (kh + 1) * hd)
            noise = 0.05 * rng.standard_normal((n, hd))
            c["kc"][off:off + n, cols] = (ct[:, None] * u[kh] + noise).astype(np.float32)
        for h in range(H):
            qn = 0.05 * rng.standard_normal((n, hd))
            c["q"][off:off + n, h * hd:(h + 1) * hd] = (a * u[h // (H // Hkv)] + qn).astype(np.float32)
        off += n
    got, _, _ = run_prefill(c["k"], c["v"], 0, c["tables"], c["starts"], c["lens"], c["q"],
                            c["kc"], c["vc"], H, Hkv, hd)
    want, _, _ = oracle_prefill_batch(c)
    assert np.isfinite(got).all()
    assert_parity(got, want, f"score profiles hd={hd}")


def test_prefill_errors():
    import torch

    import nitrorag_amd as na
    from nitrorag_amd import _native as N

    say("prefill errors")
    k = torch.zeros((4, 1, 16, 64), device="cuda")
    pool = na.KVPool.wrap(k, torch.zeros_like(k))
    q = torch.zeros((1, 64), device="cuda")
    with pytest.raises(na.NitroError) as e:
        pool.prefill(0, q, torch.zeros_like(q), 1, 1, 64)
    assert e.value.status == N.NO_BATCH
    with pytest.raises(na.NitroError) as e:
        pool.upload_prefill_batch([[0, 1]], [20], [13])  # last position 32 needs a third page
    assert e.value.status == N.BAD_BLOCK_TABLE
    with pytest.raises(na.NitroError) as e:
        pool.upload_prefill_batch([[0, 4]], [0], [20])  # page 4 outside a 4-page pool
    assert e.value.status == N.BAD_BLOCK_TABLE
    with pytest.raises(na.NitroError) as e:
        pool.upload_prefill_batch([[0]], [0], [0])  # nothing to do
    assert e.value.status == N.INVALID_ARGUMENT


def test_prefill_random_shapes():
    """Twelve seeded random prefill batches on each kernel: 1-5 chunks of 1-300
    tokens starting at positions 0-400 (continued chunks attend their earlier
    rows), MHA and GQA, head sizes that are any multiple of 4 up to 256, 1-2
    layers; the scatter bit-exact and the attention at the parity bar against
    the oracle."""
    rng = np.random.default_rng(20261203)
    for i in range(12):
        B = int(rng.integers(1, 6))
        kv_mul = int(rng.choice([1, 1, 2, 4]))
        hd = 4 * int(rng.integers(1, 65))
        Hkv = int(rng.integers(1, max(2, min(4, 512 // hd)) + 1))
        layers = int(rng.integers(1, 3))
        layer = int(rng.integers(0, layers))
        say(f"random prefill {i}: B={B} H={Hkv * kv_mul} Hkv={Hkv} hd={hd} layers={layers}")
        c = prefill_batch_case(int(rng.integers(1 << 30)), B, 1, 300, Hkv * kv_mul, Hkv, hd, layers, layer, 0, 400)
        got, gk, gv = run_prefill(c["k"], c["v"], layer, c["tables"], c["starts"], c["lens"], c["q"],
                                  c["kc"], c["vc"], c["H"], Hkv, hd)
        want, wk, wv = oracle_prefill_batch(c)
        assert np.array_equal(gk, wk) and np.array_equal(gv, wv)
        assert_parity(got, want, f"random prefill {i}")
