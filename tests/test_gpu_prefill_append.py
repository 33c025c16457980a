"""GPU: the prefill step with the KV scatter inside the attention launch
(nitro_paged_attn_prefill_append) against the scatter and the attention as two
launches (src/model_q8.cpp:473-484 then :485-523) and against the oracle.  The
one-launch form reads a chunk's keys from the new rows instead of the pool (and
keys cached before the chunk from the pool), the same floats in the same order,
so the output and both pools must be bit-identical to the two-launch form's.
It runs when no page a chunk row lands on is named by another table entry;
other batches run the two launches behind the same call."""
import sys

import numpy as np
import pytest

from gpu_helpers import assert_parity, to_gpu
from test_gpu_prefill import CASES, oracle_prefill_batch, prefill_batch_case

pytestmark = pytest.mark.gpu


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


def run(c, fused):
    """(out, k pool, v pool, prefill_counts) after one step of case c."""
    import torch

    import nitrorag_amd as na

    dk, dv = to_gpu(c["k"]), to_gpu(c["v"])
    pool = na.KVPool.wrap(dk, dv)
    pool.upload_prefill_batch(c["tables"], c["starts"], c["lens"])
    dq, kc, vc = to_gpu(c["q"]), to_gpu(c["kc"]), to_gpu(c["vc"])
    out = torch.full_like(dq, float("nan"))
    if fused:
        pool.prefill_append(c["layer"], dq, kc, vc, out, c["H"], c["Hkv"], c["hd"])
    else:
        pool.kv_append_prefill(c["layer"], kc, vc)
        pool.prefill(c["layer"], dq, out, c["H"], c["Hkv"], c["hd"])
    torch.cuda.synchronize()
    assert pool.take_device_errors() == 0
    counts = pool.prefill_counts()
    return out.cpu().numpy(), dk.cpu().numpy(), dv.cpu().numpy(), counts


def check(c, one_launch, name):
    got, gk, gv, counts = run(c, True)
    assert counts == (1, 1 if one_launch else 0), (name, counts)
    want, wk, wv, _ = run(c, False)
    assert np.array_equal(gk, wk) and np.array_equal(gv, wv), name
    assert np.array_equal(got, want), name
    ref, rk, rv = oracle_prefill_batch(c)
    assert np.array_equal(gk, rk) and np.array_equal(gv, rv), name
    assert_parity(got, ref, name)


FRESH = {
    # name: (seed, B, len lo, len hi, H, Hkv, hd, layers, layer, start lo, start hi)
    "fresh_gqa_8x2_hd128": (2, 4, 1, 200, 8, 2, 128, 2, 1, 0, 0),
    "fresh_hd32": (3, 6, 1, 70, 4, 4, 32, 1, 0, 0, 0),
    "fresh_single_tokens_hd64": (5, 5, 1, 1, 4, 4, 64, 1, 0, 0, 0),
    "fresh_gqa_16x4_hd64_long": (14, 2, 900, 2100, 16, 4, 64, 1, 0, 0, 0),
    "fresh_gqa_8x2_hd128_long": (15, 2, 2500, 4000, 8, 2, 128, 1, 0, 0, 0),
    # chunks after cached keys (random starts: tiles and V groups straddle them)
    "continued_12x64": (17, 5, 1, 300, 12, 12, 64, 2, 1, 1, 700),
    "continued_gqa_16x4_hd64": (18, 3, 100, 900, 16, 4, 64, 1, 0, 500, 1500),
    # the reference scheduler's 256-token chunks (src/pagedMemory.hpp:360-379)
    "chunk_256_after_512_hd64": (19, 4, 256, 256, 12, 12, 64, 1, 0, 512, 512),
    "chunk_256_after_256_hd128": (20, 3, 200, 256, 8, 8, 128, 1, 0, 256, 256),
}


# fresh prompts and chunks after cached keys at head sizes 32, 64, 128 take the
# one-launch form; head size 256 and padded sizes, and keys past the LDS copy of
# the table (32k tokens) run the two launches behind the same call
@pytest.mark.parametrize("name,one_launch", [
    ("prompts_b8_12x64", True),
    ("fresh_gqa_8x2_hd128", True),
    ("fresh_hd32", True),
    ("fresh_single_tokens_hd64", True),
    ("fresh_gqa_16x4_hd64_long", True),
    ("fresh_gqa_8x2_hd128_long", True),
    ("continued_chunks_gqa_8x2_hd128", True),
    ("short_chunks_hd32", True),
    ("single_token_chunks", True),
    ("continued_12x64", True),
    ("continued_gqa_16x4_hd64", True),
    ("chunk_256_after_512_hd64", True),
    ("chunk_256_after_256_hd128", True),
    ("mha_hd256", False),
    ("hd48", False),
    ("beyond_lds_table_hd64", False),
])
def test_append_matches_two_launches(name, one_launch):
    say(f"prefill append {name}")
    seed, B, lo, hi, H, Hkv, hd, layers, layer, slo, shi = (FRESH.get(name) or CASES[name])
    check(prefill_batch_case(seed, B, lo, hi, H, Hkv, hd, layers, layer, slo, shi), one_launch, name)


def test_append_prompt_near_the_table_limit():
    """One fresh 32,000-token prompt at hd 64 (2,000 pages, just below the
    2,048 table entries a workgroup keeps in LDS): the one-launch form leaves
    the output and both pools bit-identical to the two launches, and sampled
    query rows (first, last, and 30 in between) match the oracle, each row
    computed as a one-row chunk at its position over the written pool (a row's
    output depends only on keys 0..pos)."""
    from oracle import attn

    say("prefill append, 32000-token prompt at hd 64")
    c = prefill_batch_case(16, 1, 32000, 32000, 2, 2, 64, 1, 0, 0, 0)
    got, gk, gv, counts = run(c, True)
    assert counts == (1, 1)
    want, wk, wv, _ = run(c, False)
    assert np.array_equal(gk, wk) and np.array_equal(gv, wv)
    assert np.array_equal(got, want)
    k, v = c["k"].copy(), c["v"].copy()
    attn.kv_scatter_prefill(k, v, 0, c["kc"], c["vc"], c["tables"][0], 0)
    assert np.array_equal(gk, k) and np.array_equal(gv, v)
    rng = np.random.default_rng(16)
    for t in sorted({0, 31999, *rng.integers(1, 31999, size=30).tolist()}):
        ref = attn.prefill_chunk(k, v, 0, c["q"][t:t + 1], c["tables"][0], t, 2, 2, 64)
        assert_parity(got[t:t + 1], ref, f"row {t}")


def test_append_random_batches():
    """Sixteen seeded random batches at head sizes 32, 64 and 128: 1-6 chunks
    of 1-300 tokens, fresh prompts in half of them and chunks after 1-400
    cached keys in the other half, MHA and GQA, 1-2 layers; all one launch."""
    rng = np.random.default_rng(20261204)
    for i in range(16):
        B = int(rng.integers(1, 7))
        kv_mul = int(rng.choice([1, 2, 4]))
        hd = int(rng.choice([32, 64, 128]))
        Hkv = int(rng.integers(1, 4))
        layers = int(rng.integers(1, 3))
        layer = int(rng.integers(0, layers))
        slo, shi = (0, 0) if i % 2 == 0 else (1, 400)
        name = f"random append {i}: B={B} H={Hkv * kv_mul} Hkv={Hkv} hd={hd} starts {slo}..{shi}"
        say(name)
        c = prefill_batch_case(int(rng.integers(1 << 30)), B, 1, 300, Hkv * kv_mul, Hkv, hd, layers,
                               layer, slo, shi)
        check(c, True, name)


def test_append_chunks_after_shared_cached_pages():
    """Two sequences whose cached keys sit on the same two pages (prefix-cache
    hits) each prefill a chunk onto pages of their own: the one-launch form
    runs (the shared pages are only read) and matches the two launches bit for
    bit and the oracle."""
    rng = np.random.default_rng(8)
    H, Hkv, hd = 4, 2, 64
    kv_dim = Hkv * hd
    tables = np.array([[0, 1, 2, 4], [0, 1, 3, 5]], dtype=np.int32)
    starts = np.array([32, 40])   # the second chunk starts inside its page 2 (id 3)
    lens = np.array([30, 21])
    total = int(lens.sum())
    c = dict(k=rng.standard_normal((6, 1, 16, kv_dim)).astype(np.float32),
             v=rng.standard_normal((6, 1, 16, kv_dim)).astype(np.float32),
             tables=tables, starts=starts, lens=lens,
             q=rng.standard_normal((total, H * hd)).astype(np.float32),
             kc=rng.standard_normal((total, kv_dim)).astype(np.float32),
             vc=rng.standard_normal((total, kv_dim)).astype(np.float32),
             H=H, Hkv=Hkv, hd=hd, layer=0)
    say("prefill append after shared cached pages")
    check(c, True, "shared cached pages")


def test_append_page_read_by_another_sequence():
    """A page that one sequence's chunk writes and another reads as cached keys:
    the scatter runs first (two launches), as the step requires."""
    rng = np.random.default_rng(7)
    H = Hkv = 2
    hd = 64
    kv_dim = Hkv * hd
    pages = 6
    # sequence 0: cached 0..31 on pages 0, 1; its chunk 32..47 lands on page 2.
    # sequence 1: cached 0..31 on pages 3, 2 (page 2 holds its keys 16..31); chunk on page 4.
    tables = np.array([[0, 1, 2], [3, 2, 4]], dtype=np.int32)
    starts = np.array([32, 32])
    lens = np.array([16, 5])
    total = int(lens.sum())
    c = dict(k=rng.standard_normal((pages, 1, 16, kv_dim)).astype(np.float32),
             v=rng.standard_normal((pages, 1, 16, kv_dim)).astype(np.float32),
             tables=tables, starts=starts, lens=lens,
             q=rng.standard_normal((total, H * hd)).astype(np.float32),
             kc=rng.standard_normal((total, kv_dim)).astype(np.float32),
             vc=rng.standard_normal((total, kv_dim)).astype(np.float32),
             H=H, Hkv=Hkv, hd=hd, layer=0)
    check(c, False, "page shared across sequences")


def test_append_other_kernels_run_two_launches(monkeypatch):
    """NITRO_PREFILL_KERNEL=valu / mfma32 have no appending form."""
    seed, B, lo, hi, H, Hkv, hd, layers, layer, slo, shi = CASES["short_chunks_hd32"]
    c = prefill_batch_case(seed, B, lo, hi, H, Hkv, hd, layers, layer, slo, shi)
    for kern in ("valu", "mfma32"):
        monkeypatch.setenv("NITRO_PREFILL_KERNEL", kern)
        say(f"prefill append on {kern}")
        check(c, False, kern)


def test_append_page_written_twice_runs_two_launches():
    """Fresh prompts whose tables name one page twice: the call runs the two
    launches (which rows land there is the scatter's order, as in the
    reference's loop)."""
    import torch

    import nitrorag_amd as na

    rng = np.random.default_rng(9)
    kv_dim, hd, H = 64, 64, 1
    k = torch.zeros((4, 1, 16, kv_dim), dtype=torch.float32, device="cuda")
    v = torch.zeros_like(k)
    pool = na.KVPool.wrap(k, v)
    pool.upload_prefill_batch(np.array([[0, 1], [2, 1]], dtype=np.int32), np.array([0, 0]), np.array([20, 20]))
    q, kc, vc = (torch.from_numpy(rng.standard_normal((40, w)).astype(np.float32)).cuda() for w in (H * hd, kv_dim, kv_dim))
    out = torch.empty_like(q)
    pool.prefill_append(0, q, kc, vc, out, H, 1, hd)
    torch.cuda.synchronize()
    assert pool.take_device_errors() == 0
    assert pool.prefill_counts() == (1, 0)
    assert torch.isfinite(out).all().item()
