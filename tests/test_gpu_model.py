"""GPU parity of the transformer step (nitro_forward_decode_batch /
nitro_forward_prefill over a model loaded from the reference's file layout)
against logits recorded from the reference's own forward_prefill_chunk,
forward_paged and forward_decode_batch on a tiny random model.

The host bookkeeping (BlockManager / Sequence) replays the same script, so
positions and block tables must come out identical.  Logits bar: |gpu - ref|
<= 2e-3 + 1e-3*|ref| (logits reach |80|; every product and reduction of two
layers runs in a different fp32 order)."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LOGIT_ATOL, LOGIT_RTOL = 2e-3, 1e-3


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


def check_logits(got, want, what):
    err = np.abs(got - want)
    bound = LOGIT_ATOL + LOGIT_RTOL * np.abs(want)
    worst = np.unravel_index(np.argmax(err - bound), err.shape)
    assert np.all(err <= bound), (f"{what}: |gpu-ref| {err[worst]:.3g} > {bound[worst]:.3g} at {worst} "
                                  f"(gpu {got[worst]:.6g}, ref {want[worst]:.6g})")
    assert np.array_equal(got.argmax(axis=1), want.argmax(axis=1)), what


def test_model_config_round_trip(golden_model):
    import nitrorag_amd as na

    blob, meta, _ = golden_model
    m = na.Model(blob)
    cfg = meta["model"]
    assert m.config == dict(dim=cfg["n_heads"] * cfg["head_dim"], hidden_dim=cfg["hidden_dim"],
                            n_layers=cfg["n_layers"], n_heads=cfg["n_heads"],
                            n_kv_heads=cfg["n_kv_heads"], vocab_size=cfg["vocab"], seq_len=cfg["seq_len"])


def test_forward_passes_match_reference_golden(golden_model):
    import torch

    import nitrorag_amd as na
    from nitrorag_amd.model import FULL_ROWS, LAST_BLOCK

    blob, meta, arrays = golden_model
    cfg = meta["model"]
    model = na.Model(blob)
    pool = na.KVPool(cfg["total_blocks"], cfg["n_layers"], model.kv_dim)
    bm = na.BlockManager(cfg["total_blocks"])
    seqs = {slot: na.Sequence(slot) for slot in range(3)}
    for i, op in enumerate(meta["script"]):
        toks = arrays[f"{i}/tokens"]
        want = arrays[f"{i}/logits"]
        slots = op["slots"]
        say(f"step {i}: {op['kind']} slots {slots}")
        if op["kind"] == "prefill":
            s = seqs[slots[0]]
            start = s.logical_token_count
            assert start == op["start"]
            for t in toks:  # src/model_q8.cpp:428-430
                s.allocate_next_token(int(t), bm)
            pool.upload_prefill_batch(na.pack_block_tables([s]), [start], [len(toks)])
            got = model.forward_prefill(pool, toks, semantics=LAST_BLOCK)
        else:
            batch = [seqs[x] for x in slots]
            pos = [s.logical_token_count for s in batch]
            assert pos == ([op["pos"]] if op["kind"] == "paged" else op["pos"])
            for s, t in zip(batch, toks):  # in batch order (one reference thread)
                s.allocate_next_token(int(t), bm)
            pool.upload_decode_batch(na.pack_block_tables(batch), pos)
            sem = FULL_ROWS if op["kind"] == "paged" else LAST_BLOCK
            got = model.forward_decode_batch(pool, toks, semantics=sem)
        torch.cuda.synchronize()
        check_logits(got.cpu().numpy(), want, f"step {i} ({op['kind']})")
    assert pool.take_device_errors() == 0
    for slot, table in meta["final_tables"].items():
        assert seqs[int(slot)].block_table == table


def test_model_argument_errors(golden_model):
    import torch

    import nitrorag_amd as na

    blob, meta, _ = golden_model
    with pytest.raises(na.NitroError):
        na.Model(blob[:-4])  # truncated file
    model = na.Model(blob)
    cfg = meta["model"]
    pool = na.KVPool(cfg["total_blocks"], cfg["n_layers"], model.kv_dim)
    with pytest.raises(na.NitroError) as e:
        model.forward_decode_batch(pool, [1])  # no batch uploaded
    assert e.value.status == na._native.NO_BATCH
    bm = na.BlockManager(cfg["total_blocks"])
    s = na.Sequence(0)
    s.allocate_next_token(1, bm)
    pool.upload_decode_batch(na.pack_block_tables([s]), [0])
    with pytest.raises(na.NitroError):
        model.forward_decode_batch(pool, [cfg["vocab"]])  # token outside the vocabulary
    wrong = na.KVPool(cfg["total_blocks"], cfg["n_layers"] + 1, model.kv_dim)
    wrong.upload_decode_batch(na.pack_block_tables([s]), [0])
    with pytest.raises(na.NitroError):
        model.forward_decode_batch(wrong, [1])  # pool geometry differs from the model
    torch.cuda.synchronize()


MODELS = {
    # name: (dim, hidden, layers, heads, kv heads, vocab, seq_len)
    "mha_hd64_l3": (256, 512, 3, 4, 4, 1000, 256),
    "gqa_hd128_l2": (512, 1024, 2, 4, 2, 700, 200),
    "gqa_hd32_l2": (128, 256, 2, 4, 1, 300, 300),
    # rows of >= 2048 k: the flat products with rms_norm, RoPE + K/V append,
    # SwiGLU and residual epilogues (3 decode rows)
    "gqa_hd128_wide_l1": (2048, 2304, 1, 16, 4, 500, 128),
    # head sizes other than 32/64/128/256 (attention on the padded kernels)
    "gqa_hd96_l2": (384, 512, 2, 4, 2, 400, 160),
    "mha_hd80_l1": (320, 384, 1, 4, 4, 300, 160),
    "gqa_hd48_l2": (192, 256, 2, 4, 2, 300, 160),
}


@pytest.mark.parametrize("name", ["mha_hd64_l3", "gqa_hd128_l2", "gqa_hd32_l2", "gqa_hd96_l2"])
def test_full_row_products_over_many_rows(name):
    """Full-row products over more than 4 activation rows take the bf16
    matrix-core kernel over the tile-layout weights, with rms_norm, RoPE + K/V
    append, the residual adds and SwiGLU fused into its launches: a 40-token
    prefill chunk (several launch rows), then decode batches of 6, 20 and 36
    sequences (one and two batch tiles, several launch rows), against the
    oracle composed from full-row matmul."""
    import torch

    import nitrorag_amd as na
    from nitrorag_amd.model import FULL_ROWS, synthetic_model_file
    from oracle import model as om

    dim, hid, L, H, Hkv, V, S = MODELS[name]
    say(f"full rows, many rows: {name}")
    # wo / w2 scaled up so the products, not the embedding carried along the
    # residual stream, decide the logits
    blob = om.scale_residual_outputs(synthetic_model_file(dim, hid, L, H, Hkv, V, S, seed=len(name) + 7), 64.0)
    model, ora = na.Model(blob), om.OracleModel(blob)
    pages = 160
    pool = na.KVPool(pages, L, model.kv_dim)
    k = np.zeros((pages, L, 16, model.kv_dim), np.float32)
    v = np.zeros_like(k)
    bm = na.BlockManager(pages)
    rng = np.random.default_rng(11)
    seqs = [na.Sequence(i) for i in range(36)]
    for i, s in enumerate(seqs):
        n = 40 if i == 0 else int(rng.integers(1, 20))
        toks = rng.integers(0, V, n).astype(np.int32)
        start = s.logical_token_count
        for t in toks:
            s.allocate_next_token(int(t), bm)
        pool.upload_prefill_batch(na.pack_block_tables([s]), [start], [n])
        got = model.forward_prefill(pool, toks, semantics=FULL_ROWS).cpu().numpy()
        want = ora.forward_prefill_chunk(k, v, na.pack_block_tables([s])[0], start, toks, bulk=False)[None, :]
        check_logits(got, want, f"{name} full-row prefill {n}")
    for nb in (6, 20, 36):
        batch = seqs[:nb]
        toks = rng.integers(0, V, nb).astype(np.int32)
        pos = [s.logical_token_count for s in batch]
        for s, t in zip(batch, toks):
            s.allocate_next_token(int(t), bm)
        tables = na.pack_block_tables(batch)
        pool.upload_decode_batch(tables, pos)
        got = model.forward_decode_batch(pool, toks, semantics=FULL_ROWS).cpu().numpy()
        want = ora.forward_decode_batch(k, v, tables, pos, toks, bulk=False)
        check_logits(got, want, f"{name} full-row decode batch {nb}")
    torch.cuda.synchronize()
    assert pool.take_device_errors() == 0


@pytest.mark.parametrize("name,dims", [
    # rows of 2048-2304 k: every product of 1-4 rows takes the flat kernel (x in LDS)
    ("wide", (2048, 2304, 1, 16, 4, 500, 128)),
    # rows of 4608 k: wq/wk/wv and w1/w3 take the flat kernel at 1-3 rows and the
    # row-streaming one at 4 (4 * 4608 floats of x exceed its 16384-float budget);
    # wo (residual epilogue, 39936 floats) stays on the flat kernel at 1-4 rows
    ("wider", (4608, 2304, 1, 36, 4, 300, 64)),
    # w2 over rows of 18944 k (a Qwen2-7B FFN width): 2 rows = 37888 floats of x, the
    # top of the residual flat kernel's budget, where every thread stages 10 float4
    ("ffn18944", (512, 18944, 1, 8, 8, 300, 64)),
    # a classifier larger than the 256 MB Infinity Cache (66000 x 1024 fp32, 270 MB),
    # whose weights the classifier launch reads with non-temporal loads
    ("vocab66000", (1024, 1024, 1, 8, 8, 66000, 64)),
    # w2 over rows of 11008 k (Llama-2-7B): 3 rows = 33024 floats on the flat kernel
    ("ffn11008", (512, 11008, 1, 8, 8, 300, 64)),
])
def test_small_batches_over_long_rows(name, dims):
    """Full-row products of 1-4 activation rows over rows of >= 2048 k, with
    rms_norm, RoPE + K/V append, the residual adds and SwiGLU fused into their
    launches: decode batches of 1, 2, 3 and 4 sequences against the oracle
    composed from full-row matmul."""
    import torch

    import nitrorag_amd as na
    from nitrorag_amd.model import FULL_ROWS, synthetic_model_file
    from oracle import model as om

    dim, hid, L, H, Hkv, V, S = dims
    say(f"small batches over long rows: {name}")
    blob = om.scale_residual_outputs(synthetic_model_file(dim, hid, L, H, Hkv, V, S, seed=len(name) + 3), 64.0)
    model, ora = na.Model(blob), om.OracleModel(blob)
    pages = 32
    pool = na.KVPool(pages, L, model.kv_dim)
    k = np.zeros((pages, L, 16, model.kv_dim), np.float32)
    v = np.zeros_like(k)
    bm = na.BlockManager(pages)
    rng = np.random.default_rng(17)
    seqs = [na.Sequence(i) for i in range(4)]
    for s in seqs:
        n = int(rng.integers(3, 12))
        toks = rng.integers(0, V, n).astype(np.int32)
        start = s.logical_token_count
        for t in toks:
            s.allocate_next_token(int(t), bm)
        pool.upload_prefill_batch(na.pack_block_tables([s]), [start], [n])
        got = model.forward_prefill(pool, toks, semantics=FULL_ROWS).cpu().numpy()
        want = ora.forward_prefill_chunk(k, v, na.pack_block_tables([s])[0], start, toks, bulk=False)[None, :]
        check_logits(got, want, f"{name} prefill {n}")
    for nb in (1, 2, 3, 4):
        say(f"  decode batch {nb}")
        batch = seqs[:nb]
        toks = rng.integers(0, V, nb).astype(np.int32)
        pos = [s.logical_token_count for s in batch]
        for s, t in zip(batch, toks):
            s.allocate_next_token(int(t), bm)
        tables = na.pack_block_tables(batch)
        pool.upload_decode_batch(tables, pos)
        got = model.forward_decode_batch(pool, toks, semantics=FULL_ROWS).cpu().numpy()
        want = ora.forward_decode_batch(k, v, tables, pos, toks, bulk=False)
        check_logits(got, want, f"{name} decode batch {nb}")
    torch.cuda.synchronize()
    assert pool.take_device_errors() == 0


@pytest.mark.parametrize("name", sorted(MODELS))
def test_forward_vs_oracle_on_synthetic_models(name):
    """A synthetic model file through both: the GPU forward passes against the
    oracle's composed restatement (prefill chunks, then batched decode with
    both Q8 semantics), same host bookkeeping."""
    import torch

    import nitrorag_amd as na
    from nitrorag_amd.model import FULL_ROWS, LAST_BLOCK, synthetic_model_file
    from oracle import model as om

    dim, hid, L, H, Hkv, V, S = MODELS[name]
    say(f"synthetic model {name}")
    blob = synthetic_model_file(dim, hid, L, H, Hkv, V, S, seed=len(name))
    model, ora = na.Model(blob), om.OracleModel(blob)
    pages = 64
    pool = na.KVPool(pages, L, model.kv_dim)
    k = np.zeros((pages, L, 16, model.kv_dim), np.float32)
    v = np.zeros_like(k)
    bm = na.BlockManager(pages)
    rng = np.random.default_rng(5)
    seqs = [na.Sequence(i) for i in range(3)]
    for s, n in zip(seqs, (70, 33, 5)):  # prefill each prompt as one chunk
        toks = rng.integers(0, V, n).astype(np.int32)
        start = s.logical_token_count
        for t in toks:
            s.allocate_next_token(int(t), bm)
        pool.upload_prefill_batch(na.pack_block_tables([s]), [start], [n])
        got = model.forward_prefill(pool, toks, semantics=LAST_BLOCK).cpu().numpy()
        want = ora.forward_prefill_chunk(k, v, na.pack_block_tables([s])[0], start, toks)[None, :]
        check_logits(got, want, f"{name} prefill {n}")
    for step, sem in enumerate([LAST_BLOCK, FULL_ROWS, LAST_BLOCK]):
        toks = rng.integers(0, V, 3).astype(np.int32)
        pos = [s.logical_token_count for s in seqs]
        for s, t in zip(seqs, toks):
            s.allocate_next_token(int(t), bm)
        tables = na.pack_block_tables(seqs)
        pool.upload_decode_batch(tables, pos)
        got = model.forward_decode_batch(pool, toks, semantics=sem).cpu().numpy()
        want = ora.forward_decode_batch(k, v, tables, pos, toks, bulk=sem == LAST_BLOCK)
        check_logits(got, want, f"{name} decode step {step}")
    torch.cuda.synchronize()
    assert pool.take_device_errors() == 0
