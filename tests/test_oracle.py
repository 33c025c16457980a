"""Pins the CPU oracle: golden vectors recorded from the reference's own
compiled code, FNV-1a specification vectors, fp64 closed forms and invariants.
"""
import numpy as np
import pytest

from oracle import attn, closed_form as cf, paged_memory as pm
from replay import base_pools, digest, pools_after_call
from synth import counter_pool, rope_tables

# The oracle is a restatement compiled with the reference's flags; against the
# reference build it must agree far inside the path's 1e-4/1e-3 parity bar.
TIGHT = dict(atol=1e-6, rtol=1e-5)


def run_oracle_case(meta, arr, k, v):
    H, Hkv, hd, layer = meta["H"], meta["Hkv"], meta["hd"], meta["layer"]
    kind = meta["kind"]
    if kind == "decode_batch":
        return attn.decode_batch(k, v, layer, arr["q"], arr["tables"], arr["positions"], H, Hkv, hd)
    if kind == "decode_single":
        return attn.decode_single_avx2(k, v, layer, arr["q"][0], arr["table"], meta["pos"], H,
                                       Hkv, hd)[None, :]
    if kind in ("prefill", "prefix_hit"):
        return attn.prefill_chunk(k, v, layer, arr["q"], arr["table"], meta["start_pos"], H, Hkv,
                                  hd)
    raise ValueError(kind)


def closed_form_case(meta, arr, k, v):
    H, Hkv, hd, layer = meta["H"], meta["Hkv"], meta["hd"], meta["layer"]
    kind = meta["kind"]
    if kind == "decode_batch":
        return cf.decode_batch_f64(k, v, layer, arr["q"], arr["tables"], arr["positions"], H, Hkv,
                                   hd)
    if kind == "decode_single":
        return cf.decode_batch_f64(k, v, layer, arr["q"], arr["table"][None, :],
                                   [meta["pos"]], H, Hkv, hd)
    return cf.prefill_f64(k, v, layer, arr["q"], arr["table"], meta["start_pos"], H, Hkv, hd)


PAGED_CASES = ["decode_mha_hd16_l2", "decode_gqa_h8kv2_hd16", "decode_hd64", "decode_hd128",
               "single_hd32_l2", "single_gqa_hd64", "single_pos0", "prefill_fresh_hd16_l2",
               "prefill_continued_gqa", "prefill_hd64", "prefix_hit_gqa_l2",
               "decode_gqa_h4kv2_hd32", "prefill_gqa_hd32_l2", "prefix_hit_hd32"]


@pytest.mark.parametrize("name", PAGED_CASES)
def test_oracle_matches_reference_golden(golden_attention, name):
    meta, arr = golden_attention[name]
    k, v = pools_after_call(meta, arr)
    assert digest(k[:, meta["layer"]]) == meta["k_pool_digest"]
    assert digest(v[:, meta["layer"]]) == meta["v_pool_digest"]
    out = run_oracle_case(meta, arr, k, v)
    obs = meta["observed"]
    np.testing.assert_allclose(out[:, -obs:], arr["xb2_obs"], **TIGHT)
    # The reference's outputs also sit on the fp64 closed form at the parity bar.
    f64 = closed_form_case(meta, arr, k, v)
    assert cf.within_tolerance(arr["xb2_obs"], f64[:, -obs:])
    assert cf.within_tolerance(out, f64, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("name", ["decode_mha_hd16_l2", "decode_gqa_h8kv2_hd16", "decode_hd64",
                                  "decode_hd128", "single_hd32_l2", "single_pos0"])
def test_oracle_kv_append_matches_reference_pool(golden_attention, name):
    meta, arr = golden_attention[name]
    k, v = base_pools(meta)
    layer = meta["layer"]
    if meta["kind"] == "decode_batch":
        attn.kv_append_decode(k, v, layer, arr["k"], arr["v"], arr["tables"], arr["positions"])
    else:
        attn.kv_append_decode(k, v, layer, arr["k"], arr["v"], arr["table"][None, :],
                              np.array([meta["pos"]], np.int32))
    assert digest(k[:, layer]) == meta["k_pool_digest"]
    assert digest(v[:, layer]) == meta["v_pool_digest"]


@pytest.mark.parametrize("name", ["prefill_fresh_hd16_l2", "prefill_continued_gqa",
                                  "prefill_hd64", "prefix_hit_gqa_l2"])
def test_oracle_kv_scatter_matches_reference_pool(golden_attention, name):
    meta, arr = golden_attention[name]
    k, v = base_pools(meta)
    layer = meta["layer"]
    if meta["kind"] == "prefix_hit":
        attn.kv_scatter_prefill(k, v, layer, arr["k_a"], arr["v_a"], arr["table_a"], 0)
        assert np.array_equal(arr["table"][:meta["hits"]], arr["table_a"][:meta["hits"]])
    elif "earlier_k" in arr:
        attn.kv_scatter_prefill(k, v, layer, arr["earlier_k"], arr["earlier_v"], arr["table"],
                                int(arr["chunk_starts"][0]))
    attn.kv_scatter_prefill(k, v, layer, arr["k"], arr["v"], arr["table"], meta["start_pos"])
    assert digest(k[:, layer]) == meta["k_pool_digest"]
    assert digest(v[:, layer]) == meta["v_pool_digest"]


@pytest.mark.parametrize("name", ["contiguous_hd16", "contiguous_gqa_hd32"])
def test_oracle_contiguous_matches_reference_golden(golden_attention, name):
    meta, arr = golden_attention[name]
    H, Hkv, hd, pos = meta["H"], meta["Hkv"], meta["hd"], meta["pos"]
    kv_dim = Hkv * hd
    kc = np.zeros((1, 256, kv_dim), np.float32)
    vc = np.zeros((1, 256, kv_dim), np.float32)
    kc[0, :pos + 1] = arr["key_rows"]
    vc[0, :pos + 1] = arr["value_rows"]
    out = attn.contiguous_attention(kc, vc, 0, arr["q"][0], pos, H, Hkv, hd)
    np.testing.assert_allclose(out, arr["xb2_obs"][0], **TIGHT)
    # paged == contiguous: the same rows behind a shuffled block table
    pages = (pos + 16) // 16
    rng = np.random.default_rng(pos)
    table = rng.permutation(pages + 3)[:pages].astype(np.int32)
    kp = np.zeros((pages + 3, 1, 16, kv_dim), np.float32)
    vp = np.zeros_like(kp)
    for t in range(pos + 1):
        kp[table[t // 16], 0, t % 16] = arr["key_rows"][t]
        vp[table[t // 16], 0, t % 16] = arr["value_rows"][t]
    paged = attn.decode_batch(kp, vp, 0, arr["q"], table[None, :], np.array([pos], np.int32), H,
                              Hkv, hd)
    np.testing.assert_allclose(paged[0], out, **TIGHT)


def test_softmax_closed_form():
    rng = np.random.default_rng(5)
    for n in (1, 2, 17, 1000):
        x = (rng.standard_normal(n) * 4).astype(np.float32)
        y = attn.softmax(x)
        e = np.exp(x.astype(np.float64) - x.max())
        np.testing.assert_allclose(y, e / e.sum(), rtol=2e-6, atol=1e-9)
    # all-equal scores -> uniform; one dominant score -> one-hot
    np.testing.assert_allclose(attn.softmax(np.full(8, 3.0, np.float32)), np.full(8, 0.125))
    y = attn.softmax(np.array([0, 0, 200, 0], np.float32))
    assert y[2] == 1.0 and np.all(y[[0, 1, 3]] == 0)


def random_paged_case(rng, B, H, Hkv, hd, pages, layers, max_ctx):
    kv_dim = Hkv * hd
    k = rng.standard_normal((pages, layers, 16, kv_dim)).astype(np.float32)
    v = rng.standard_normal((pages, layers, 16, kv_dim)).astype(np.float32)
    ctx = rng.integers(1, max_ctx + 1, size=B)
    max_pages = int((ctx.max() + 15) // 16)
    perm = rng.permutation(pages).astype(np.int32)
    tables = np.zeros((B, max_pages), np.int32)
    used = 0
    for b in range(B):
        n = int((ctx[b] + 15) // 16)
        tables[b, :n] = perm[used:used + n]
        used += n
    q = rng.standard_normal((B, H * hd)).astype(np.float32)
    return k, v, q, tables, (ctx - 1).astype(np.int32)


@pytest.mark.parametrize("H,Hkv,hd", [(4, 4, 64), (8, 2, 32), (2, 2, 128)])
def test_decode_batch_vs_closed_form(H, Hkv, hd):
    rng = np.random.default_rng(hd + H)
    k, v, q, tables, pos = random_paged_case(rng, 6, H, Hkv, hd, 64, 2, 150)
    out = attn.decode_batch(k, v, 1, q, tables, pos, H, Hkv, hd)
    f64 = cf.decode_batch_f64(k, v, 1, q, tables, pos, H, Hkv, hd)
    assert np.max(np.abs(out - f64)) < 1e-5


def test_decode_invariants():
    rng = np.random.default_rng(9)
    H, Hkv, hd = 4, 2, 64
    k, v, q, tables, pos = random_paged_case(rng, 5, H, Hkv, hd, 48, 1, 120)
    base = attn.decode_batch(k, v, 0, q, tables, pos, H, Hkv, hd)
    # consistent permutation of physical page ids leaves outputs bit-identical
    perm = rng.permutation(48).astype(np.int32)
    k2 = np.empty_like(k)
    v2 = np.empty_like(v)
    k2[perm] = k
    v2[perm] = v
    out = attn.decode_batch(k2, v2, 0, q, perm[tables], pos, H, Hkv, hd)
    assert np.array_equal(out, base)
    # constant V rows -> output equals that constant
    vc = np.broadcast_to(rng.standard_normal(Hkv * hd).astype(np.float32), v.shape).copy()
    out = attn.decode_batch(k, vc, 0, q, tables, pos, H, Hkv, hd)
    expect = np.repeat(vc[0, 0, 0].reshape(Hkv, hd), H // Hkv, axis=0).reshape(-1)
    np.testing.assert_allclose(out, np.broadcast_to(expect, out.shape), rtol=1e-5, atol=1e-6)
    # ctx = 1 -> output is v_0 of the sequence's first page
    p0 = np.zeros(5, np.int32)
    out = attn.decode_batch(k, v, 0, q, tables, p0, H, Hkv, hd)
    for b in range(5):
        row = v[tables[b, 0], 0, 0].reshape(Hkv, hd)
        np.testing.assert_allclose(out[b].reshape(H, hd), np.repeat(row, H // Hkv, axis=0),
                                   rtol=1e-6)
    # q = lambda * k_j for a large lambda -> attention collapses onto row j
    b, j = 2, int(pos[2]) // 2
    kj = k[tables[b, j // 16], 0, j % 16].reshape(Hkv, hd)
    qs = q.copy()
    qs[b] = (np.repeat(kj, H // Hkv, axis=0) * 50).reshape(-1)
    out = attn.decode_batch(k, v, 0, qs, tables, pos, H, Hkv, hd)
    vj = v[tables[b, j // 16], 0, j % 16].reshape(Hkv, hd)
    np.testing.assert_allclose(out[b].reshape(H, hd), np.repeat(vj, H // Hkv, axis=0), atol=1e-4)


def test_single_avx2_matches_batched():
    rng = np.random.default_rng(13)
    H, Hkv, hd = 12, 12, 64
    k, v, q, tables, pos = random_paged_case(rng, 1, H, Hkv, hd, 64, 12, 256)
    a = attn.decode_single_avx2(k, v, 5, q[0], tables[0], int(pos[0]), H, Hkv, hd)
    b = attn.decode_batch(k, v, 5, q, tables, pos, H, Hkv, hd)[0]
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-6)


def test_prefill_online_vs_two_pass_and_closed_form():
    rng = np.random.default_rng(17)
    H, Hkv, hd = 4, 4, 64
    pages, T, start = 16, 70, 21
    kv_dim = Hkv * hd
    k = rng.standard_normal((pages, 1, 16, kv_dim)).astype(np.float32)
    v = rng.standard_normal((pages, 1, 16, kv_dim)).astype(np.float32)
    table = rng.permutation(pages).astype(np.int32)
    q = rng.standard_normal((T, H * hd)).astype(np.float32)
    out = attn.prefill_chunk(k, v, 0, q, table, start, H, Hkv, hd)
    # each query row t attends 0..start+t: the two-pass decode over the same rows agrees
    tables = np.repeat(table[None, :], T, axis=0)
    two_pass = attn.decode_batch(k, v, 0, q, tables, np.arange(start, start + T, dtype=np.int32),
                                 H, Hkv, hd)
    assert cf.within_tolerance(out, two_pass, atol=1e-5, rtol=1e-4)
    f64 = cf.prefill_f64(k, v, 0, q, table, start, H, Hkv, hd)
    assert np.max(np.abs(out - f64)) < 1e-5


def test_counter_pool_is_exact_and_reproducible():
    a = counter_pool(7, 3, 2, 8)
    b = counter_pool(7, 3, 2, 8)
    assert a.dtype == np.float32 and np.array_equal(a, b)
    assert a.min() >= -1 and a.max() < 1
    # every value is a multiple of 2^-23 (24 random bits, exact in fp32)
    assert np.all((a.astype(np.float64) * 2 ** 23) % 1 == 0)


ROPE_CASES = ["rope_decode_gqa_hd32", "rope_decode_hd64", "rope_single_hd32", "rope_prefill_hd32"]


def rope_rows(meta, arr):
    """(q_pre, k_pre, positions, q_post, k_post) of every recorded row."""
    if meta["kind"] == "rope_decode":
        return arr["q_pre"], arr["k_pre"], arr["positions"], arr["q"], arr["k"]
    if meta["kind"] == "rope_single":
        return arr["q_pre"], arr["k_pre"], np.array([meta["pos"]], np.int32), arr["q"], arr["k"]
    qs, ks, ps, qo, ko = [], [], [], [], []
    for ci, st in enumerate(arr["chunk_starts"]):
        n = arr[f"q{ci}"].shape[0]
        qs.append(arr[f"q_pre{ci}"])
        ks.append(arr[f"k_pre{ci}"])
        ps.append(np.arange(st, st + n, dtype=np.int32))
        qo.append(arr[f"q{ci}"])
        ko.append(arr[f"k{ci}"])
    return (np.concatenate(qs), np.concatenate(ks), np.concatenate(ps), np.concatenate(qo),
            np.concatenate(ko))


@pytest.mark.parametrize("name", ROPE_CASES)
def test_oracle_rope_matches_reference_golden(golden_attention, name):
    meta, arr = golden_attention[name]
    fr, fi = rope_tables(meta["seq_len"], meta["hd"], meta["rope_base"])
    q_pre, k_pre, pos, q_post, k_post = rope_rows(meta, arr)
    q, k = attn.rope(q_pre, k_pre, pos, fr, fi, meta["hd"])
    # contraction of the two products into FMAs may differ by an ulp or two
    np.testing.assert_allclose(q, q_post, rtol=1e-6, atol=1e-5)
    np.testing.assert_allclose(k, k_post, rtol=1e-6, atol=1e-5)
    # a plausible slip (cos/sin swapped, pair order, position off by one) is far outside that
    q_bad, _ = attn.rope(q_pre, k_pre, pos + 1, fr, fi, meta["hd"])
    assert np.max(np.abs(q_bad - q_post)) > 1e-2


@pytest.mark.parametrize("name", ROPE_CASES)
def test_oracle_attention_after_rope_matches_reference(golden_attention, name):
    meta, arr = golden_attention[name]
    k, v = pools_after_call(meta, arr)
    assert digest(k[:, 0]) == meta["k_pool_digest"] and digest(v[:, 0]) == meta["v_pool_digest"]
    H, Hkv, hd = meta["H"], meta["Hkv"], meta["hd"]
    if meta["kind"] == "rope_decode":
        out = attn.decode_batch(k, v, 0, arr["q"], arr["tables"], arr["positions"], H, Hkv, hd)
    elif meta["kind"] == "rope_single":
        out = attn.decode_single_avx2(k, v, 0, arr["q"][0], arr["table"], meta["pos"], H, Hkv,
                                      hd)[None, :]
    else:
        last = meta["chunks"] - 1
        out = attn.prefill_chunk(k, v, 0, arr[f"q{last}"], arr["table"],
                                 int(arr["chunk_starts"][last]), H, Hkv, hd)
    np.testing.assert_allclose(out[:, -meta["observed"]:], arr["xb2_obs"], **TIGHT)


def test_rope_closed_form():
    """Each pair rotates by its angle: norms kept, position 0 is the identity,
    and rotating by the table equals multiplying by exp(i*angle) in fp64."""
    rng = np.random.default_rng(2)
    H, Hkv, hd, S = 4, 2, 64, 300
    fr, fi = rope_tables(S, hd)
    q = rng.standard_normal((5, H * hd)).astype(np.float32)
    k = rng.standard_normal((5, Hkv * hd)).astype(np.float32)
    pos = np.array([0, 1, 17, 150, 299], np.int32)
    qr, kr = attn.rope(q, k, pos, fr, fi, hd)
    np.testing.assert_array_equal(qr[0], q[0])
    np.testing.assert_array_equal(kr[0], k[0])
    for x, xr, heads in ((q, qr, H), (k, kr, Hkv)):
        z = (x[:, 0::2] + 1j * x[:, 1::2]).astype(np.complex128)
        ang = fr.astype(np.float64)[pos][:, None, :] + 1j * fi.astype(np.float64)[pos][:, None, :]
        want = (z.reshape(5, heads, hd // 2) * ang).reshape(5, -1)
        np.testing.assert_allclose(xr[:, 0::2], want.real, atol=2e-6)
        np.testing.assert_allclose(xr[:, 1::2], want.imag, atol=2e-6)
