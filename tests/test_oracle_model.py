"""CPU pins of the model-level oracle (oracle/model_oracle.c, oracle/model.py):
Q8 products against the reference build's golden vectors (bit-exact) and
closed forms, and the quantizer restatement against known answers and the
invariants scripts/quantize.py implies."""
import numpy as np
import pytest

from oracle import model as om
from oracle import ref


def dequant(w, n, d):
    scale, q = om.unpack_q8(w, n, d)
    return (q.astype(np.float64).reshape(d, n // 32, 32) * scale.astype(np.float64)[:, :, None]).reshape(d, n)


def test_q8_oracle_matches_reference_golden(golden_q8):
    for name, (m, a) in golden_q8.items():
        n, d = m["n"], m["d"]
        assert np.array_equal(om.q8_matmul(a["w"], a["x"], n, d), a["full"]), name
        assert np.array_equal(om.q8_matmul_bulk(a["w"], a["x"], n, d), a["bulk"]), name


def test_q8_golden_against_fp64_closed_form(golden_q8):
    """matmul = x . dequant(w)^T; matmul_bulk = the same over the last 32 columns only."""
    for name, (m, a) in golden_q8.items():
        n, d = m["n"], m["d"]
        W = dequant(a["w"], n, d)
        x = a["x"].astype(np.float64)
        np.testing.assert_allclose(a["full"], x @ W.T, rtol=1e-5, atol=1e-5, err_msg=name)
        np.testing.assert_allclose(a["bulk"], x[:, -32:] @ W[:, -32:].T, rtol=1e-5, atol=1e-5,
                                   err_msg=name)
        if n > 32:  # the quirk is observable: full and bulk differ
            assert not np.allclose(a["full"], a["bulk"])


def test_q8_oracle_random_shapes_closed_form():
    rng = np.random.default_rng(5)
    for n, d, B in [(32, 1, 1), (768, 40, 2), (2048, 24, 3), (160, 17, 4)]:
        s, q = om.quantize_q8(rng.standard_normal((d, n)).astype(np.float32) * 0.1)
        w = om.pack_q8(s, q)
        x = rng.standard_normal((B, n)).astype(np.float32)
        W = dequant(w, n, d)
        np.testing.assert_allclose(om.q8_matmul(w, x, n, d), x.astype(np.float64) @ W.T,
                                   rtol=1e-5, atol=2e-5)
        np.testing.assert_allclose(om.q8_matmul_bulk(w, x, n, d),
                                   x[:, -32:].astype(np.float64) @ W[:, -32:].T, rtol=1e-5, atol=2e-5)


def test_quantize_q8_known_answers():
    """scripts/quantize.py:12-20 by hand: scale = max|w|/127, q = round-half-even(w/scale)."""
    block = np.zeros(32, np.float32)
    block[:4] = [2.0, -2.0, 1.0, 0.5]
    s, q = om.quantize_q8(block[None, :])
    assert s[0, 0] == np.float32(2.0) / np.float32(127.0)
    # 1/(2/127) = 63.5 -> 64 (half to even), 0.5/(2/127) = 31.75 -> 32
    assert list(q[0, :4]) == [127, -127, 64, 32]
    zero_s, zero_q = om.quantize_q8(np.zeros((1, 32), np.float32))
    assert zero_s[0, 0] == np.float32(1e-9) and not zero_q.any()


def test_quantize_q8_invariants():
    rng = np.random.default_rng(9)
    W = (rng.standard_normal((13, 256)) * rng.uniform(1e-3, 10, size=(13, 1))).astype(np.float32)
    s, q = om.quantize_q8(W)
    blocks = W.reshape(13, 8, 32)
    deq = q.reshape(13, 8, 32).astype(np.float64) * s[:, :, None]
    assert np.all(np.abs(deq - blocks) <= s[:, :, None] * 0.5 * (1 + 1e-6))
    # the largest-magnitude weight of every block maps to +-127
    idx = np.abs(blocks).argmax(axis=2)
    assert np.all(np.abs(np.take_along_axis(q.reshape(13, 8, 32), idx[:, :, None], 2)) == 127)
    assert np.all(np.abs(q) <= 127)


@pytest.mark.skipif(not ref.available(), reason="reference build not present")
def test_q8_oracle_matches_live_reference():
    rng = np.random.default_rng(17)
    for n, d, B in [(768, 64, 1), (2048, 48, 3), (96, 20, 6)]:
        s, q = om.quantize_q8(rng.standard_normal((d, n)).astype(np.float32) * 0.05)
        w = om.pack_q8(s, q)
        x = rng.standard_normal((B, n)).astype(np.float32)
        want = np.stack([ref.q8_matmul(w, x[b], n, d) for b in range(B)])
        assert np.array_equal(om.q8_matmul(w, x, n, d), want)
        assert np.array_equal(om.q8_matmul_bulk(w, x, n, d), ref.q8_matmul_bulk(w, x, n, d))


def replay_oracle_forward(blob, meta, arrays):
    """Drive oracle.model.OracleModel through the recorded script with this
    library's host bookkeeping; yields (step, logits, want)."""
    import nitrorag_amd as na

    M = om.OracleModel(blob)
    cfg = meta["model"]
    k = np.zeros((cfg["total_blocks"], cfg["n_layers"], 16, M.kv_dim), np.float32)
    v = np.zeros_like(k)
    bm = na.BlockManager(cfg["total_blocks"])
    seqs = {s: na.Sequence(s) for s in range(3)}
    for i, op in enumerate(meta["script"]):
        t = arrays[f"{i}/tokens"]
        slots = op["slots"]
        if op["kind"] == "prefill":
            s = seqs[slots[0]]
            start = s.logical_token_count
            for tok in t:
                s.allocate_next_token(int(tok), bm)
            got = M.forward_prefill_chunk(k, v, na.pack_block_tables([s])[0], start, t)[None, :]
        else:
            batch = [seqs[x] for x in slots]
            pos = [s.logical_token_count for s in batch]
            for s, tok in zip(batch, t):
                s.allocate_next_token(int(tok), bm)
            got = M.forward_decode_batch(k, v, na.pack_block_tables(batch), pos, t,
                                         bulk=op["kind"] != "paged")
        yield i, got, arrays[f"{i}/logits"]


def test_oracle_forward_matches_reference_golden_logits(golden_model):
    """The oracle's composed forward passes against the reference build's
    logits: bit-exact or within fp32 rounding (|logits| reach ~80)."""
    blob, meta, arrays = golden_model
    exact = 0
    for i, got, want in replay_oracle_forward(blob, meta, arrays):
        np.testing.assert_allclose(got, want, rtol=1e-6, atol=2e-5, err_msg=f"step {i}")
        exact += np.array_equal(got, want)
    assert exact >= 3  # the first steps (no accumulated rounding) are bit-exact


def test_model_pieces_closed_form():
    rng = np.random.default_rng(21)
    x = rng.standard_normal((3, 256)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    x64 = x.astype(np.float64)
    want = w * x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-5)
    np.testing.assert_allclose(om.rms_norm(x, w), want, rtol=2e-6, atol=1e-6)
    hb, hb2 = x[0] * 4, x[1]
    np.testing.assert_allclose(om.swiglu(hb, hb2), hb / (1 + np.exp(-hb.astype(np.float64))) * hb2,
                               rtol=2e-6, atol=1e-6)
    W = rng.standard_normal((40, 256)).astype(np.float32)
    for bulk in (False, True):
        np.testing.assert_allclose(om.f32_matmul(W, x, bulk), x64 @ W.T.astype(np.float64),
                                   rtol=1e-5, atol=1e-5)
