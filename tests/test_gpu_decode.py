"""GPU parity of the paged-attention decode path and KV append, through the
C ABI, against the CPU oracle (and the reference's golden vectors)."""
import ctypes
import sys
import zlib

import numpy as np
import pytest

from gpu_helpers import DecodeCase, assert_parity, random_tables, to_gpu
from oracle import attn
from replay import pools_after_call

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    import nitrorag_amd  # noqa: F401  (fails loudly without the built library)
    yield
    torch.cuda.synchronize()


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


# every decode case of the reference's golden vectors (head sizes 16, 32, 64, 128)
GOLDEN_DECODE = ["decode_hd64", "decode_hd128", "decode_gqa_h4kv2_hd32", "single_hd32_l2",
                 "single_gqa_hd64", "single_pos0", "decode_mha_hd16_l2", "decode_gqa_h8kv2_hd16"]


@pytest.mark.parametrize("name", GOLDEN_DECODE)
def test_decode_matches_reference_golden(golden_attention, name):
    import torch

    import nitrorag_amd as na

    meta, arr = golden_attention[name]
    say(f"golden decode {name}")
    k, v = pools_after_call(meta, arr)
    if meta["kind"] == "decode_batch":
        tables, positions = arr["tables"], arr["positions"]
    else:
        tables, positions = arr["table"][None, :], np.array([meta["pos"]], np.int32)
    pool = na.KVPool.wrap(to_gpu(k), to_gpu(v))
    pool.upload_decode_batch(tables, positions)
    q = to_gpu(arr["q"])
    out = torch.empty_like(q)
    pool.decode(meta["layer"], q, out, meta["H"], meta["Hkv"], meta["hd"])
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    obs = meta["observed"]
    assert_parity(got[:, -obs:], arr["xb2_obs"], name)
    want = attn.decode_batch(k, v, meta["layer"], arr["q"], tables, positions, meta["H"],
                             meta["Hkv"], meta["hd"])
    assert_parity(got, want, name + " (all heads vs oracle)")
    assert pool.take_device_errors() == 0


SHAPES = {
    # name: (ctx list or (B, lo, hi), H, Hkv, hd, pages, layers, layer)
    "llama110m_single_ctx256": ([256], 12, 12, 64, 64, 12, 7),
    "batched_12x64_b32": ((32, 16, 1024), 12, 12, 64, 2200, 2, 1),
    "gqa_8x2_hd64": ((5, 1, 300), 8, 2, 64, 128, 1, 0),
    "gqa_32x8_hd128": ([1, 700, 2049], 32, 8, 128, 200, 1, 0),
    "mha_hd32": ((4, 1, 500), 4, 4, 32, 140, 1, 0),
    "mha_hd256": ((3, 1, 300), 2, 2, 256, 64, 1, 0),
    "edges_hd128": ([1, 15, 16, 17, 32, 33, 4096], 4, 4, 128, 300, 1, 0),
    "edges_hd64": ([1, 2, 31, 32, 33, 63, 64, 65], 3, 3, 64, 40, 2, 1),
    "gqa_16x2_hd64": ((6, 1, 400), 16, 2, 64, 160, 1, 0),
    "gqa_8x1_hd32": ((4, 1, 900), 8, 1, 32, 240, 2, 1),
    "gqa_4x2_hd256": ((3, 1, 300), 4, 2, 256, 64, 1, 0),
    "gqa_24x4_hd128": ([5, 16, 17, 600], 24, 4, 128, 60, 1, 0),
    # head sizes other than 32/64/128/256: kernels padded to the next width
    "hd16_gqa_8x2": ((5, 1, 700), 8, 2, 16, 260, 1, 0),
    "hd48": ((4, 1, 400), 3, 3, 48, 120, 2, 1),
    "hd80_gqa_10x2": ((3, 1, 500), 10, 2, 80, 110, 1, 0),
    "hd96_gqa_12x4": ([1, 33, 300, 1100], 12, 4, 96, 100, 1, 0),
    "hd112": ((3, 1, 300), 2, 2, 112, 64, 1, 0),
    "hd4": ((3, 1, 200), 4, 1, 4, 40, 1, 0),
    "hd200": ((3, 1, 300), 2, 2, 200, 64, 1, 0),
    "hd252_gqa_4x2": ((2, 1, 200), 4, 2, 252, 32, 1, 0),
}


def make_case(name, seed=0, **kw):
    spec, H, Hkv, hd, pages, layers, layer = SHAPES[name]
    rng = np.random.default_rng(zlib.crc32(name.encode()) + seed)
    if isinstance(spec, tuple):
        B, lo, hi = spec
        ctx = rng.integers(lo, hi + 1, size=B)
    else:
        ctx = np.array(spec)
    return DecodeCase(rng, ctx, H, Hkv, hd, pages, layers, layer, **kw)


@pytest.mark.parametrize("name", sorted(SHAPES))
def test_decode_vs_oracle(name):
    say(f"decode vs oracle {name}")
    c = make_case(name)
    assert_parity(c.run_gpu(), c.run_oracle(), name)
    assert c.pool.take_device_errors() == 0


@pytest.mark.parametrize("tiles,waves", [("1", "4"), ("3", "4"), ("4", "8"), ("8", "16"),
                                         ("100000", "4"), ("100000", "16"), ("", "")])
def test_decode_split_k_partitions_agree(tiles, waves, monkeypatch):
    """Any launch shape (1 tile per split .. one split; 4..16 waves per
    workgroup; the default heuristic) gives the same answer within the bar,
    and repeated launches are bit-identical."""
    say(f"split-K tiles_per_split={tiles} waves={waves}")
    monkeypatch.setenv("NITRO_DECODE_SPLIT_TILES", tiles)
    monkeypatch.setenv("NITRO_DECODE_WAVES", waves)
    c = make_case("edges_hd128")
    want = c.run_oracle()
    first = c.run_gpu()
    assert_parity(first, want, f"tiles={tiles}")
    for _ in range(3):
        again = c.run_gpu()
        assert np.array_equal(again, first)


@pytest.mark.parametrize("name", ["gqa_32x8_hd128", "gqa_8x2_hd64", "batched_12x64_b32", "mha_hd32",
                                  "gqa_16x2_hd64", "gqa_4x2_hd256"])
@pytest.mark.parametrize("stream,remap,tiles", [("0", "0", ""), ("1", "0", ""), ("0", "1", ""),
                                                ("1", "1", ""), ("1", "1", "3"), ("0", "1", "2")])
def test_decode_load_kind_and_work_order_agree(name, stream, remap, tiles, monkeypatch):
    """Non-temporal or plain K/V loads, XCD-grouped or plain work order, with
    and without split-K: every combination matches the oracle."""
    say(f"decode {name} stream={stream} remap={remap} tiles={tiles}")
    monkeypatch.setenv("NITRO_DECODE_STREAM", stream)
    monkeypatch.setenv("NITRO_DECODE_XCD_REMAP", remap)
    monkeypatch.setenv("NITRO_DECODE_SPLIT_TILES", tiles)
    c = make_case(name, seed=3)
    assert_parity(c.run_gpu(), c.run_oracle(), name)
    assert c.pool.take_device_errors() == 0


HEADS_PER_WG = [("gqa_16x2_hd64", q) for q in (1, 2, 4, 8)] + \
    [("gqa_8x1_hd32", q) for q in (1, 2, 4, 8)] + \
    [("gqa_32x8_hd128", q) for q in (1, 2, 4)] + \
    [("gqa_24x4_hd128", q) for q in (1, 2)] + \
    [("gqa_4x2_hd256", q) for q in (1, 2)] + [("gqa_8x2_hd64", 4)]


@pytest.mark.parametrize("name,qh", HEADS_PER_WG)
@pytest.mark.parametrize("waves,tiles", [("", ""), ("8", "2"), ("4", "1")])
def test_decode_heads_per_workgroup_agree(name, qh, waves, tiles, monkeypatch):
    """One workgroup serving 1, 2, 4 or 8 query heads of a KV head (each K/V
    row loaded once for all of them) matches the oracle, with split-K too."""
    say(f"decode {name} heads_per_wg={qh} waves={waves} tiles={tiles}")
    monkeypatch.setenv("NITRO_DECODE_HEADS_PER_WG", str(qh))
    monkeypatch.setenv("NITRO_DECODE_WAVES", waves)
    monkeypatch.setenv("NITRO_DECODE_SPLIT_TILES", tiles)
    c = make_case(name, seed=5)
    want = c.run_oracle()
    first = c.run_gpu()
    assert_parity(first, want, f"{name} qh={qh}")
    assert np.array_equal(c.run_gpu(), first)
    assert c.pool.take_device_errors() == 0


def test_decode_heads_per_workgroup_rejects_bad_override(monkeypatch):
    import nitrorag_amd as na

    for name, qh in [("gqa_16x2_hd64", "3"), ("gqa_24x4_hd128", "4"), ("gqa_4x2_hd256", "4")]:
        monkeypatch.setenv("NITRO_DECODE_HEADS_PER_WG", qh)  # not a divisor of 8 / 6; over the budget
        c = make_case(name)
        with pytest.raises(na.NitroError) as e:
            c.run_gpu()
        assert "NITRO_DECODE_HEADS_PER_WG" in str(e.value)


def test_decode_page_permutation_is_bit_identical():
    """Renaming physical pages consistently leaves the result bit-identical."""
    say("page permutation")
    rng = np.random.default_rng(11)
    c = make_case("batched_12x64_b32")
    base = c.run_gpu()
    perm = rng.permutation(c.k.shape[0]).astype(np.int32)
    k2 = np.empty_like(c.k)
    v2 = np.empty_like(c.v)
    k2[perm] = c.k
    v2[perm] = c.v
    import nitrorag_amd as na

    pool = na.KVPool.wrap(to_gpu(k2), to_gpu(v2))
    pool.upload_decode_batch(perm[c.tables], c.positions)
    import torch

    q = to_gpu(c.q)
    out = torch.empty_like(q)
    pool.decode(c.layer, q, out, c.H, c.Hkv, c.hd)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), base)


def test_decode_constant_v_and_single_key():
    say("constant V / ctx=1")
    import torch

    import nitrorag_amd as na

    rng = np.random.default_rng(5)
    H, hd, pages = 4, 128, 80
    kv_dim = H * hd
    ctx = np.array([1, 17, 600])
    tables = random_tables(rng, ctx, pages)
    k = rng.standard_normal((pages, 1, 16, kv_dim)).astype(np.float32)
    row = rng.standard_normal(kv_dim).astype(np.float32)
    v = np.broadcast_to(row, k.shape).copy()
    q = rng.standard_normal((3, kv_dim)).astype(np.float32)
    pool = na.KVPool.wrap(to_gpu(k), to_gpu(v))
    pool.upload_decode_batch(tables, ctx - 1)
    out = torch.empty_like(to_gpu(q))
    pool.decode(0, to_gpu(q), out, H, H, hd)
    torch.cuda.synchronize()
    np.testing.assert_allclose(out.cpu().numpy(), np.broadcast_to(row, (3, kv_dim)), rtol=1e-5,
                               atol=1e-6)


def test_kv_append_bit_exact_and_then_attended():
    """forward_decode_batch's order: append this step's K/V at pos, then attend 0..pos."""
    say("kv append")
    import torch

    c = make_case("gqa_8x2_hd64")
    B, kv_dim = len(c.ctx), c.Hkv * c.hd
    rng = np.random.default_rng(3)
    knew = rng.standard_normal((B, kv_dim)).astype(np.float32)
    vnew = rng.standard_normal((B, kv_dim)).astype(np.float32)
    c.pool.kv_append(c.layer, to_gpu(knew), to_gpu(vnew))
    got = c.run_gpu()
    attn.kv_append_decode(c.k, c.v, c.layer, knew, vnew, c.tables, c.positions)
    torch.cuda.synchronize()
    assert np.array_equal(c.dk.cpu().numpy(), c.k)
    assert np.array_equal(c.dv.cpu().numpy(), c.v)
    assert_parity(got, c.run_oracle(), "after append")


def test_owned_pool_create_and_layer_offsets():
    """nitro_kvpool_create owns zeroed memory with the reference layout."""
    say("owned pool")
    import torch

    import nitrorag_amd as na

    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    pages, layers, H, hd = 24, 3, 2, 64
    kv_dim = H * hd
    pool = na.KVPool(pages, layers, kv_dim)
    kp, vp = pool.data_ptrs()
    nbytes = pages * layers * 16 * kv_dim * 4
    back = np.ones(pages * layers * 16 * kv_dim, np.float32)
    assert hip.hipMemcpy(back.ctypes.data, kp, nbytes, 2) == 0  # device -> host
    assert not back.any()
    rng = np.random.default_rng(8)
    k = rng.standard_normal((pages, layers, 16, kv_dim)).astype(np.float32)
    v = rng.standard_normal((pages, layers, 16, kv_dim)).astype(np.float32)
    assert hip.hipMemcpy(kp, k.ctypes.data, nbytes, 1) == 0  # host -> device
    assert hip.hipMemcpy(vp, v.ctypes.data, nbytes, 1) == 0
    ctx = np.array([5, 100, 200])
    tables = random_tables(rng, ctx, pages)
    pool.upload_decode_batch(tables, ctx - 1)
    q = rng.standard_normal((3, kv_dim)).astype(np.float32)
    for layer in range(layers):
        out = torch.empty((3, kv_dim), device="cuda")
        pool.decode(layer, to_gpu(q), out, H, H, hd)
        torch.cuda.synchronize()
        assert_parity(out.cpu().numpy(), attn.decode_batch(k, v, layer, q, tables, ctx - 1, H, H,
                                                           hd), f"layer {layer}")
    pool.close()


def test_decode_argument_errors():
    say("argument errors")
    import torch

    import nitrorag_amd as na
    from nitrorag_amd import _native as N

    k = torch.zeros((8, 1, 16, 128), device="cuda")
    v = torch.zeros_like(k)
    pool = na.KVPool.wrap(k, v)
    q = torch.zeros((1, 128), device="cuda")
    out = torch.zeros_like(q)
    with pytest.raises(na.NitroError) as e:
        pool.decode(0, q, out, 1, 1, 128)
    assert e.value.status == N.NO_BATCH
    with pytest.raises(na.NitroError) as e:
        pool.upload_decode_batch([[0, 8]], [17])  # page id 8 outside an 8-page pool
    assert e.value.status == N.BAD_BLOCK_TABLE
    with pytest.raises(na.NitroError) as e:
        pool.upload_decode_batch([[0, 1]], [32])  # pos 32 needs a third page
    assert e.value.status == N.BAD_BLOCK_TABLE
    with pytest.raises(na.NitroError) as e:
        pool.upload_decode_batch([[0, -1]], [20])
    assert e.value.status == N.BAD_BLOCK_TABLE
    pool.upload_decode_batch([[3, 5]], [20])

    def raw(layer, H, Hkv, hd):  # the C entry point itself (no Python-side size checks)
        return N.lib().nitro_paged_attn_decode(pool.handle, layer, ctypes.c_void_p(q.data_ptr()),
                                               ctypes.c_void_p(out.data_ptr()), H, Hkv, hd, None)

    assert raw(0, 1, 1, 126) == N.UNSUPPORTED  # not a multiple of 4
    assert raw(0, 1, 1, 260) == N.UNSUPPORTED  # wider than 256
    assert raw(0, 3, 2, 64) == N.UNSUPPORTED
    assert raw(1, 1, 1, 128) == N.INVALID_ARGUMENT  # layer outside a 1-layer pool
    assert raw(0, 2, 1, 64) == N.INVALID_ARGUMENT   # kv_dim mismatch (1*64 != 128)
    assert raw(0, 1, 1, 128) == N.OK
    torch.cuda.synchronize()
    assert pool.take_device_errors() == 0


def test_full_size_b64_ctx4096_32x128_subset_vs_oracle():
    """The benchmark's call at its real size (B=64, ctx 4096, 32 heads x 128,
    20k-page pool): append + attend in one launch (decode_append).  All 64
    appended K/V rows read back bit-exact from their pages; four sequences
    checked against the oracle on host copies of just their pages (the new
    rows included); the launch equals the separate append + decode launches
    bit for bit; all outputs finite, and the batch is invariant to the order
    of sequences."""
    import torch

    import nitrorag_amd as na

    say("full-size B=64 ctx=4096 32x128")
    B, H, hd, ctx, pages = 64, 32, 128, 4096, 20000
    kv_dim = H * hd
    g = torch.Generator(device="cuda")
    g.manual_seed(0x4E4954525005)
    k = torch.randn((pages, 1, 16, kv_dim), device="cuda", generator=g)
    v = torch.randn((pages, 1, 16, kv_dim), device="cuda", generator=g)
    q = torch.randn((B, kv_dim), device="cuda", generator=g)
    knew = torch.randn((B, kv_dim), device="cuda", generator=g)
    vnew = torch.randn((B, kv_dim), device="cuda", generator=g)
    rng = np.random.default_rng(5)
    tables = random_tables(rng, np.full(B, ctx), pages)
    positions = np.full(B, ctx - 1, np.int32)
    pool = na.KVPool.wrap(k, v)
    pool.upload_decode_batch(tables, positions)
    out = torch.empty_like(q)
    pool.decode_append(0, q, knew, vnew, out, H, H, hd)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.all(np.isfinite(got))
    new_pages = torch.from_numpy(tables[np.arange(B), positions >> 4].astype(np.int64)).cuda()
    rows = torch.from_numpy((positions & 15).astype(np.int64)).cuda()
    assert torch.equal(k[new_pages, 0, rows], knew) and torch.equal(v[new_pages, 0, rows], vnew)
    # the separate launches (append, then attend over the pool) give the same bits
    sep = torch.empty_like(q)
    pool.kv_append(0, knew, vnew)
    pool.decode(0, q, sep, H, H, hd)
    torch.cuda.synchronize()
    assert np.array_equal(sep.cpu().numpy(), got)
    for b in (0, 17, 42, 63):
        idx = torch.from_numpy(tables[b].astype(np.int64)).cuda()
        kb = k.index_select(0, idx).cpu().numpy()
        vb = v.index_select(0, idx).cpu().numpy()
        local = np.arange(tables.shape[1], dtype=np.int32)[None, :]
        want = attn.decode_batch(kb, vb, 0, q[b:b + 1].cpu().numpy(), local, positions[b:b + 1],
                                 H, H, hd)
        assert_parity(got[b:b + 1], want, f"sequence {b}")
    order = rng.permutation(B)
    pool.upload_decode_batch(tables[order], positions[order])
    out2 = torch.empty_like(q)
    pool.decode(0, q[torch.from_numpy(order).cuda()].contiguous(), out2, H, H, hd)
    torch.cuda.synchronize()
    assert np.array_equal(out2.cpu().numpy(), got[order])
    assert pool.take_device_errors() == 0
    del k, v
    torch.cuda.empty_cache()


def test_long_context_decode_splits_past_the_lds_table_slice():
    """Contexts past 1,022 pages per split (16,352 tokens) force split-K whatever
    the launch heuristic picks (each split's block-table slice is staged in
    LDS): two sequences at 20,000 and 33,000 tokens beside a short one."""
    say("long-context decode (ctx 20000 / 33000)")
    rng = np.random.default_rng(21)
    c = DecodeCase(rng, np.array([20000, 7, 33000]), 4, 4, 64, 3400, 1, 0)
    assert_parity(c.run_gpu(), c.run_oracle(), "long context")
    assert c.pool.take_device_errors() == 0


def test_oversized_pool_reports_device_alloc():
    """A pool larger than the GPU's memory fails with NITRO_ERR_DEVICE_ALLOC (the
    reference exits at src/pagedMemory.hpp:96) and leaves later launches working."""
    say("oversized pool")
    import nitrorag_amd as na
    from nitrorag_amd import _native as N

    h = ctypes.c_void_p()
    # 1.2M pages x 16 x 4096 floats = 314 GB per pool, above the 288 GB of HBM
    st = N.lib().nitro_kvpool_create(1_200_000, 1, 4096, ctypes.byref(h))
    assert st == N.DEVICE_ALLOC and not h.value, N.last_error()
    c = make_case("mha_hd32")
    assert_parity(c.run_gpu(), c.run_oracle(), "after a failed allocation")


def test_prefill_scatter_of_more_rows_than_a_grid_dimension():
    """KV scatter of a prefill batch of 72,000 rows (72 chunks of 1,000 tokens at
    non-page-aligned starts), more than the 65,535 workgroups one grid dimension
    holds: the pools match the oracle's scatter (src/model_q8.cpp:473-484) bit
    for bit."""
    say("prefill scatter of 72,000 rows")
    import torch

    import nitrorag_amd as na

    rng = np.random.default_rng(33)
    B, T, kv_dim = 72, 1000, 32
    starts = rng.integers(0, 40, size=B).astype(np.int32)
    lens = np.full(B, T, np.int32)
    need = (starts + lens + 15) // 16
    pages = int(need.sum())
    perm = rng.permutation(pages).astype(np.int32)
    tables = np.zeros((B, int(need.max())), np.int32)
    off = 0
    for b in range(B):
        tables[b, :need[b]] = perm[off:off + need[b]]
        off += need[b]
    k = rng.standard_normal((pages, 1, 16, kv_dim)).astype(np.float32)
    v = rng.standard_normal((pages, 1, 16, kv_dim)).astype(np.float32)
    kc = rng.standard_normal((B * T, kv_dim)).astype(np.float32)
    vc = rng.standard_normal((B * T, kv_dim)).astype(np.float32)
    dk, dv = to_gpu(k), to_gpu(v)
    pool = na.KVPool.wrap(dk, dv)
    pool.upload_prefill_batch(tables, starts, lens)
    pool.kv_append_prefill(0, to_gpu(kc), to_gpu(vc))
    torch.cuda.synchronize()
    for b in range(B):
        attn.kv_scatter_prefill(k, v, 0, kc[b * T:(b + 1) * T], vc[b * T:(b + 1) * T], tables[b],
                                int(starts[b]))
    assert np.array_equal(dk.cpu().numpy(), k)
    assert np.array_equal(dv.cpu().numpy(), v)
    assert pool.take_device_errors() == 0


@pytest.mark.parametrize("name", ["batched_12x64_b32", "gqa_32x8_hd128", "hd96_gqa_12x4", "edges_hd64"])
@pytest.mark.parametrize("tiles,waves,worklist", [("2", "4", "1"), ("2", "4", "0"), ("3", "8", "1"),
                                                  ("1", "16", "1"), ("", "", "1"), ("", "", "0")])
def test_decode_work_list_and_implied_items_agree(name, tiles, waves, worklist, monkeypatch):
    """Sequences split into runs of `tiles` tiles, handed out by a work list
    (only real items, full ones first) or implied by the block id (workgroups
    past a sequence's last split exit): both match the oracle, and repeated
    launches are bit-identical (the split merge runs in split order whichever
    workgroup arrives last)."""
    say(f"decode {name} tiles={tiles} waves={waves} work_list={worklist}")
    monkeypatch.setenv("NITRO_DECODE_SPLIT_TILES", tiles)
    monkeypatch.setenv("NITRO_DECODE_WAVES", waves)
    monkeypatch.setenv("NITRO_DECODE_WORK_LIST", worklist)
    c = make_case(name, seed=9)
    want = c.run_oracle()
    first = c.run_gpu()
    assert_parity(first, want, f"{name} tiles={tiles} list={worklist}")
    for _ in range(3):
        assert np.array_equal(c.run_gpu(), first)
    assert c.pool.take_device_errors() == 0


@pytest.mark.parametrize("name", ["llama110m_single_ctx256", "batched_12x64_b32", "gqa_32x8_hd128",
                                  "gqa_8x2_hd64", "edges_hd128", "hd48", "mha_hd256"])
@pytest.mark.parametrize("tiles", ["", "2"])
def test_decode_append_equals_append_then_decode(name, tiles, monkeypatch):
    """nitro_paged_attn_decode_append (the new row read from k/v and written by
    the decode launch itself) leaves the same pools, byte for byte, and the
    same outputs, bit for bit, as nitro_kv_append then nitro_paged_attn_decode;
    both match the oracle's append + decode (src/model_q8.cpp:616-662)."""
    import torch

    import nitrorag_amd as na

    say(f"decode_append {name} tiles={tiles}")
    monkeypatch.setenv("NITRO_DECODE_SPLIT_TILES", tiles)
    c = make_case(name, seed=13)
    B, kv_dim = len(c.ctx), c.Hkv * c.hd
    rng = np.random.default_rng(17)
    knew = rng.standard_normal((B, kv_dim)).astype(np.float32)
    vnew = rng.standard_normal((B, kv_dim)).astype(np.float32)
    q = to_gpu(c.q)
    # fused
    out1 = torch.full_like(q, float("nan"))
    c.pool.decode_append(c.layer, q, to_gpu(knew), to_gpu(vnew), out1, c.H, c.Hkv, c.hd)
    torch.cuda.synchronize()
    k1, v1 = c.dk.cpu().numpy(), c.dv.cpu().numpy()
    # separate, on a fresh copy of the original pools
    dk2, dv2 = to_gpu(c.k), to_gpu(c.v)
    pool2 = na.KVPool.wrap(dk2, dv2)
    pool2.upload_decode_batch(c.tables, c.positions)
    pool2.kv_append(c.layer, to_gpu(knew), to_gpu(vnew))
    out2 = torch.full_like(q, float("nan"))
    pool2.decode(c.layer, q, out2, c.H, c.Hkv, c.hd)
    torch.cuda.synchronize()
    assert np.array_equal(k1, dk2.cpu().numpy()) and np.array_equal(v1, dv2.cpu().numpy())
    assert np.array_equal(out1.cpu().numpy(), out2.cpu().numpy())
    attn.kv_append_decode(c.k, c.v, c.layer, knew, vnew, c.tables, c.positions)
    assert np.array_equal(k1, c.k) and np.array_equal(v1, c.v)
    assert_parity(out1.cpu().numpy(), c.run_oracle(), f"decode_append {name}")
    assert c.pool.take_device_errors() == 0


def test_decode_append_when_rows_share_the_appended_page():
    """Rows of one sequence at consecutive positions (a short prefill chunk run
    as decode rows) read the page the others append to: decode_append then
    appends every row before attending, as the reference does, and row i sees
    the rows appended before it."""
    import torch

    import nitrorag_amd as na

    say("decode_append with a shared appended page")
    rng = np.random.default_rng(23)
    H, hd, pages = 4, 64, 40
    kv_dim = H * hd
    start, n = 37, 6  # positions 37..42 share page 2 of the table
    table = rng.permutation(pages)[:4].astype(np.int32)
    tables = np.repeat(table[None, :], n, axis=0)
    positions = np.arange(start, start + n, dtype=np.int32)
    k = rng.standard_normal((pages, 1, 16, kv_dim)).astype(np.float32)
    v = rng.standard_normal((pages, 1, 16, kv_dim)).astype(np.float32)
    q = rng.standard_normal((n, kv_dim)).astype(np.float32)
    knew = rng.standard_normal((n, kv_dim)).astype(np.float32)
    vnew = rng.standard_normal((n, kv_dim)).astype(np.float32)
    dk, dv = to_gpu(k), to_gpu(v)
    pool = na.KVPool.wrap(dk, dv)
    pool.upload_decode_batch(tables, positions)
    out = torch.full_like(to_gpu(q), float("nan"))
    pool.decode_append(0, to_gpu(q), to_gpu(knew), to_gpu(vnew), out, H, H, hd)
    torch.cuda.synchronize()
    attn.kv_append_decode(k, v, 0, knew, vnew, tables, positions)
    assert np.array_equal(dk.cpu().numpy(), k) and np.array_equal(dv.cpu().numpy(), v)
    assert_parity(out.cpu().numpy(), attn.decode_batch(k, v, 0, q, tables, positions, H, H, hd),
                  "shared appended page")


@pytest.mark.parametrize("name,tiles", [("llama110m_single_ctx256", ""), ("batched_12x64_b32", "2"),
                                        ("gqa_32x8_hd128", "2"), ("edges_hd64", "1")])
def test_decode_graph_replays_match_eager(name, tiles, monkeypatch):
    """decode_append captured into a HIP graph (after an eager call has sized
    the workspace) replays to the eager outputs and pools bit for bit, replay
    after replay, with eager launches on the same pool in between: the launch
    records no memset (the split-merge counters are reset by the kernel)."""
    import torch

    say(f"decode_append graph replays {name} tiles={tiles}")
    monkeypatch.setenv("NITRO_DECODE_SPLIT_TILES", tiles)
    c = make_case(name, seed=29)
    B, kv_dim = len(c.ctx), c.Hkv * c.hd
    rng = np.random.default_rng(31)
    knew = rng.standard_normal((B, kv_dim)).astype(np.float32)
    vnew = rng.standard_normal((B, kv_dim)).astype(np.float32)
    q, kn, vn = to_gpu(c.q), to_gpu(knew), to_gpu(vnew)
    want = torch.full_like(q, float("nan"))
    c.pool.decode_append(c.layer, q, kn, vn, want, c.H, c.Hkv, c.hd)
    torch.cuda.synchronize()
    k_after, v_after = c.dk.clone(), c.dv.clone()
    attn.kv_append_decode(c.k, c.v, c.layer, knew, vnew, c.tables, c.positions)
    assert np.array_equal(k_after.cpu().numpy(), c.k) and np.array_equal(v_after.cpu().numpy(), c.v)
    assert_parity(want.cpu().numpy(), c.run_oracle(), f"graph case {name} (eager)")

    out = torch.full_like(q, float("nan"))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        c.pool.decode_append(c.layer, q, kn, vn, out, c.H, c.Hkv, c.hd,
                             torch.cuda.current_stream())
    torch.cuda.synchronize()
    for i in range(4):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i}"
        assert torch.equal(c.dk, k_after) and torch.equal(c.dv, v_after), f"pools after replay {i}"
        eager = torch.full_like(q, float("nan"))
        c.pool.decode_append(c.layer, q, kn, vn, eager, c.H, c.Hkv, c.hd)
        torch.cuda.synchronize()
        assert torch.equal(eager, want), f"eager call after replay {i}"
    del graph
    assert c.pool.take_device_errors() == 0


@pytest.mark.parametrize("max_context_split", [False, True])
def test_decode_counts_and_skips_page_ids_outside_the_pool(max_context_split):
    """Tables handed to the kernel directly (nitro_paged_attn_decode_static
    takes device tables, with no host validation) may hold page ids outside
    the pool: the kernel counts them (nitro_kvpool_take_device_errors) and
    skips their rows without reading them.  The other sequences' outputs are
    bit-identical to a launch with clean tables, and the damaged sequence
    attends exactly its rows on valid pages (fp64 closed form).  With
    max_context_split the launch splits, so the skipped rows fall in split
    partials that are merged."""
    import torch

    import nitrorag_amd as na
    from nitrorag_amd import _native as N
    from oracle import closed_form as cf

    say(f"bad page ids, split={max_context_split}")
    rng = np.random.default_rng(91)
    H, Hkv, hd, pages = 4, 4, 64, 600
    ctx = np.array([50, 37, 64] if not max_context_split else [3000, 2100, 64])
    tables = random_tables(rng, ctx, pages)
    positions = (ctx - 1).astype(np.int32)
    k = rng.standard_normal((pages, 1, 16, Hkv * hd)).astype(np.float32)
    v = rng.standard_normal((pages, 1, 16, Hkv * hd)).astype(np.float32)
    q = rng.standard_normal((len(ctx), H * hd)).astype(np.float32)
    pool = na.KVPool.wrap(to_gpu(k), to_gpu(v))
    dq, pos_d = to_gpu(q), to_gpu(positions)

    def run(tab):
        out = torch.full_like(dq, float("nan"))
        tab_d = to_gpu(tab)
        st = N.lib().nitro_paged_attn_decode_static(
            pool.handle, 0, ctypes.c_void_p(dq.data_ptr()), ctypes.c_void_p(out.data_ptr()),
            ctypes.c_void_p(tab_d.data_ptr()), ctypes.c_void_p(pos_d.data_ptr()), len(ctx),
            tab.shape[1], int(ctx.max()), H, Hkv, hd, 0, None)
        assert st == N.OK, N.last_error()
        torch.cuda.synchronize()
        return out.cpu().numpy()

    clean = run(tables)
    assert pool.take_device_errors() == 0
    bad = tables.copy()
    bad[1, 1] = pages + 7  # past the pool
    bad[1, 2] = -3         # negative
    got = run(bad)
    assert pool.take_device_errors() > 0
    assert np.array_equal(got[0], clean[0]) and np.array_equal(got[2], clean[2])
    rows = np.arange(ctx[1])
    keep = rows[(rows // 16 != 1) & (rows // 16 != 2)]
    pg = tables[1][keep // 16].astype(np.int64)
    want = cf.attention_f64(q[1], k[pg, 0, keep % 16], v[pg, 0, keep % 16], H, Hkv, hd)
    assert_parity(got[1:2], want[None, :].astype(np.float32), "sequence with bad page ids")
    # a device position below 0: that sequence attends nothing and its output
    # rows are zeros (counted once per sequence); the others are unchanged
    say(f"negative device position, split={max_context_split}")
    neg = positions.copy()
    neg[1], neg[2] = -1, -9
    pos_d = to_gpu(neg)
    got = run(tables)
    assert pool.take_device_errors() == 2
    assert np.array_equal(got[0], clean[0])
    assert np.all(got[1:] == 0.0)


def test_decode_random_shapes():
    """Thirty seeded random batches: 1-9 sequences of 1-2500 tokens, MHA and GQA
    (groups of 1-8 query heads), head sizes that are any multiple of 4 up to
    256, 1-2 layers; every one against the oracle at the parity bar, and a
    second launch bit-identical to the first."""
    rng = np.random.default_rng(20261202)
    for i in range(30):
        B = int(rng.integers(1, 10))
        kv_mul = int(rng.choice([1, 1, 2, 3, 4, 8]))
        hd = 4 * int(rng.integers(1, 65))
        Hkv = int(rng.integers(1, max(2, min(8, 1024 // hd)) + 1))
        layers = int(rng.integers(1, 3))
        ctx = rng.integers(1, 2501, size=B)
        pages = int(((ctx + 15) // 16).sum()) + int(rng.integers(0, 9))
        say(f"random decode {i}: B={B} H={Hkv * kv_mul} Hkv={Hkv} hd={hd} layers={layers} "
            f"ctx={ctx.min()}..{ctx.max()}")
        c = DecodeCase(rng, ctx, Hkv * kv_mul, Hkv, hd, pages, layers, int(rng.integers(0, layers)))
        first = c.run_gpu()
        assert_parity(first, c.run_oracle(), f"random decode {i}")
        assert np.array_equal(c.run_gpu(), first)
        assert c.pool.take_device_errors() == 0
