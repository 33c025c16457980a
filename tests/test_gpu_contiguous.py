"""GPU parity of forward's non-paged attention (src/model_q8.cpp:189-222),
served by the paged kernels over a view of its contiguous caches
(nitro_kvpool_wrap_contiguous: [layers][seq_len][kv_dim], page p of a layer =
its rows 16p..16p+15, identity block table).  Checked against the reference's
own forward (golden vectors) and the oracle's contiguous restatement."""
import ctypes
import sys

import numpy as np
import pytest

from gpu_helpers import assert_parity, to_gpu
from oracle import attn

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


def identity_table(pos):
    return np.arange(pos // 16 + 1, dtype=np.int32)[None, :]


@pytest.mark.parametrize("layers,layer", [(1, 0), (3, 2), (4, 1)])
@pytest.mark.parametrize("name", ["contiguous_hd16", "contiguous_gqa_hd32"])
def test_contiguous_matches_reference_golden(golden_attention, name, layers, layer):
    """The reference forward's cache rows 0..pos placed in one layer of a
    multi-layer contiguous cache (random rows everywhere else, including past
    pos in the same page); decode over the view reproduces its attention output
    and the oracle's contiguous attention for every head."""
    import torch

    import nitrorag_amd as na

    meta, arr = golden_attention[name]
    H, Hkv, hd, pos = meta["H"], meta["Hkv"], meta["hd"], meta["pos"]
    say(f"contiguous golden {name} layers={layers} layer={layer}")
    kv_dim, seq_len = Hkv * hd, 256
    rng = np.random.default_rng(pos * 10 + layers)
    kc = rng.standard_normal((layers, seq_len, kv_dim)).astype(np.float32)
    vc = rng.standard_normal((layers, seq_len, kv_dim)).astype(np.float32)
    kc[layer, :pos + 1] = arr["key_rows"]
    vc[layer, :pos + 1] = arr["value_rows"]
    pool = na.KVPool.wrap_contiguous(to_gpu(kc), to_gpu(vc))
    pool.upload_decode_batch(identity_table(pos), [pos])
    q = to_gpu(arr["q"])
    out = torch.full_like(q, float("nan"))
    pool.decode(layer, q, out, H, Hkv, hd)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert_parity(got[:, -meta["observed"]:], arr["xb2_obs"], name)
    want = attn.contiguous_attention(kc, vc, layer, arr["q"][0], pos, H, Hkv, hd)
    assert_parity(got[0], want, name + " (all heads vs oracle)")
    assert pool.take_device_errors() == 0


@pytest.mark.parametrize("H,Hkv,hd,seq_len,layers", [(8, 2, 64, 64, 3), (4, 4, 128, 48, 2),
                                                     (12, 12, 64, 32, 12)])
def test_contiguous_session_writes_then_attends(H, Hkv, hd, seq_len, layers):
    """forward's per-layer order over a whole session, positions 0..seq_len-1:
    write this token's k/v at row pos of the layer (src/model_q8.cpp:189-191),
    then attend rows 0..pos (:193-222).  Alternate layers take the separate
    append + decode calls and the fused decode_append; every output matches
    the oracle, and the caches end bit-identical to the host's writes."""
    import torch

    import nitrorag_amd as na

    say(f"contiguous session H={H} Hkv={Hkv} hd={hd} seq_len={seq_len} layers={layers}")
    kv_dim = Hkv * hd
    rng = np.random.default_rng(H * 1000 + hd + seq_len)
    kc = np.zeros((layers, seq_len, kv_dim), np.float32)
    vc = np.zeros_like(kc)
    dk, dv = to_gpu(kc), to_gpu(vc)
    pool = na.KVPool.wrap_contiguous(dk, dv)
    out = torch.empty((1, H * hd), device="cuda")
    for pos in range(seq_len):
        pool.upload_decode_batch(identity_table(pos), [pos])
        for layer in range(layers):
            q = rng.standard_normal((1, H * hd)).astype(np.float32)
            k = rng.standard_normal((1, kv_dim)).astype(np.float32)
            v = rng.standard_normal((1, kv_dim)).astype(np.float32)
            out.fill_(float("nan"))
            if (pos + layer) % 2:
                pool.kv_append(layer, to_gpu(k), to_gpu(v))
                pool.decode(layer, to_gpu(q), out, H, Hkv, hd)
            else:
                pool.decode_append(layer, to_gpu(q), to_gpu(k), to_gpu(v), out, H, Hkv, hd)
            torch.cuda.synchronize()
            kc[layer, pos], vc[layer, pos] = k[0], v[0]
            want = attn.contiguous_attention(kc, vc, layer, q[0], pos, H, Hkv, hd)
            assert_parity(out.cpu().numpy()[0], want, f"pos {pos} layer {layer}")
    assert np.array_equal(dk.cpu().numpy(), kc)
    assert np.array_equal(dv.cpu().numpy(), vc)
    assert pool.take_device_errors() == 0


def test_contiguous_view_argument_errors():
    """seq_len not a whole number of pages is refused (UNSUPPORTED), a
    non-positive one is an argument error, and a table entry past the layer's
    seq_len/16 pages is rejected at upload like any page outside a pool."""
    import torch

    import nitrorag_amd as na
    from nitrorag_amd import _native as N

    say("contiguous view argument errors")
    buf = torch.zeros(2 * 40 * 64, device="cuda")
    h = ctypes.c_void_p()
    p = ctypes.c_void_p(buf.data_ptr())
    assert N.lib().nitro_kvpool_wrap_contiguous(p, p, 40, 2, 64, ctypes.byref(h)) == N.UNSUPPORTED
    assert not h.value
    assert N.lib().nitro_kvpool_wrap_contiguous(p, p, 0, 2, 64, ctypes.byref(h)) == N.INVALID_ARGUMENT
    assert N.lib().nitro_kvpool_wrap_contiguous(None, None, 32, 2, 64, ctypes.byref(h)) == N.INVALID_ARGUMENT
    kc = torch.zeros((2, 32, 64), device="cuda")
    pool = na.KVPool.wrap_contiguous(kc, kc.clone())
    with pytest.raises(na.NitroError) as e:
        pool.upload_decode_batch([[0, 1, 2]], [40])  # page 2 is past a 32-row layer
    assert e.value.status == N.BAD_BLOCK_TABLE
    pool.upload_decode_batch([[0, 1]], [31])
