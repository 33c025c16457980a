"""GPU parity of the Q8_0 matrix product (nitro_q8_matmul) against the
reference's golden vectors and the CPU oracle, both semantics (matmul and
matmul_bulk).  Bar: |gpu - cpu| <= 1e-4 + 1e-3*|cpu| (fp32 products and
accumulation in a different summation order)."""
import sys

import numpy as np
import pytest

from gpu_helpers import assert_parity, to_gpu
from oracle import model as om

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


def run_gpu(w, x, d, semantics):
    import torch

    import nitrorag_amd as na

    dw = torch.from_numpy(np.ascontiguousarray(w, dtype=np.uint8)).cuda()
    dx = to_gpu(x)
    out = torch.full((x.shape[0], d), float("nan"), device="cuda")
    na.q8_matmul(dw, dx, out, semantics)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_q8_matches_reference_golden(golden_q8):
    from nitrorag_amd.q8 import FULL_ROWS, LAST_BLOCK

    for name, (m, a) in golden_q8.items():
        say(f"q8 golden {name}")
        assert_parity(run_gpu(a["w"], a["x"], m["d"], FULL_ROWS), a["full"], name + " full rows")
        assert_parity(run_gpu(a["w"], a["x"], m["d"], LAST_BLOCK), a["bulk"], name + " last block")


SHAPES = [
    # n, d, batch: Llama-2-110M projections (768x768, 2048x768, 768x2048), batch
    # tiles of 16 (1, 15, 16, 17, 64, 65), rows not a multiple of 16, odd blocks per row
    (768, 768, 1), (768, 2048, 3), (2048, 768, 16), (768, 768, 17), (2048, 768, 64),
    (768, 200, 65), (96, 40, 100), (32, 7, 5), (4096, 48, 2),
    # rows of >= 2048 k with 1-4 activation rows whose x fits 16384 floats take
    # the flat kernel (x in LDS): a last chunk of one block, 7 rows, more row
    # units than workgroups, batch x n at the limit
    (2048, 40, 1), (2304, 96, 2), (2080, 7, 3), (4096, 4100, 4), (4128, 16400, 1), (16384, 20, 1),
    # larger batch x n: the row-streaming kernel, 1024-k chunks split over two
    # k halves (odd and even chunk counts), tiles of 16 rows not filling the matrix
    (11008, 64, 3), (6144, 40, 4), (8224, 4100, 2),
    # long rows with 5..64 activation rows (bf16 matrix-core kernel): a partial
    # 16-row batch tile, row tiles not filling the matrix, 344 blocks per row
    (4096, 4100, 8), (11008, 80, 33), (4096, 48, 5),
]


@pytest.mark.parametrize("n,d,batch", SHAPES)
def test_q8_vs_oracle(n, d, batch):
    from nitrorag_amd.q8 import FULL_ROWS, LAST_BLOCK

    say(f"q8 vs oracle n={n} d={d} batch={batch}")
    rng = np.random.default_rng(n * 7 + d * 3 + batch)
    s, q = om.quantize_q8((rng.standard_normal((d, n)) * 0.05).astype(np.float32))
    w = om.pack_q8(s, q)
    x = rng.standard_normal((batch, n)).astype(np.float32)
    assert_parity(run_gpu(w, x, d, FULL_ROWS), om.q8_matmul(w, x, n, d), f"full {n}x{d}x{batch}")
    assert_parity(run_gpu(w, x, d, LAST_BLOCK), om.q8_matmul_bulk(w, x, n, d), f"last {n}x{d}x{batch}")


def test_q8_repeat_is_bit_identical():
    from nitrorag_amd.q8 import FULL_ROWS

    say("q8 repeat")
    rng = np.random.default_rng(3)
    s, q = om.quantize_q8((rng.standard_normal((768, 2048)) * 0.05).astype(np.float32))
    w = om.pack_q8(s, q)
    x = rng.standard_normal((9, 2048)).astype(np.float32)
    first = run_gpu(w, x, 768, FULL_ROWS)
    assert np.array_equal(run_gpu(w, x, 768, FULL_ROWS), first)


def test_q8_argument_errors():
    import torch

    import nitrorag_amd as na
    from nitrorag_amd import _native as N

    say("q8 errors")
    w = torch.zeros(36 * 4, dtype=torch.uint8, device="cuda")
    x = torch.zeros((1, 32), device="cuda")
    out = torch.zeros((1, 4), device="cuda")
    with pytest.raises(na.NitroError):
        na.q8_matmul(w[:-1], x, out)  # wrong byte count
    with pytest.raises(na.NitroError):
        na.q8_matmul(w, torch.zeros((1, 33), device="cuda"), out)  # n not a multiple of 32
    lib = N.lib()
    st = lib.nitro_q8_matmul(w.data_ptr(), x.data_ptr(), out.data_ptr(), 1, 32, 4, 2, None)
    assert st == N.INVALID_ARGUMENT  # unknown semantics
    st = lib.nitro_q8_matmul(w.data_ptr(), x.data_ptr() + 4, out.data_ptr(), 1, 32, 4, 0, None)
    assert st == N.INVALID_ARGUMENT  # x not 16-byte aligned


def test_q8_random_shapes():
    """Twenty-five seeded random products over every kernel the shape selects
    (slab, flat, row-streaming, bf16 matrix cores): rows of 32-12288 k, 1-2100
    output rows, 1-40 activation rows, weights at random scales; both
    semantics against the oracle."""
    from nitrorag_amd.q8 import FULL_ROWS, LAST_BLOCK

    rng = np.random.default_rng(20261205)
    for i in range(25):
        n = 32 * int(rng.integers(1, 385))
        d = int(rng.integers(1, 2101))
        batch = int(rng.choice([1, 2, 3, 4, int(rng.integers(5, 41))]))
        say(f"q8 random {i}: n={n} d={d} batch={batch}")
        s, q = om.quantize_q8((rng.standard_normal((d, n)) * float(rng.choice([0.01, 0.05, 0.3]))).astype(np.float32))
        w = om.pack_q8(s, q)
        x = rng.standard_normal((batch, n)).astype(np.float32)
        assert_parity(run_gpu(w, x, d, FULL_ROWS), om.q8_matmul(w, x, n, d), f"random full {i}")
        assert_parity(run_gpu(w, x, d, LAST_BLOCK), om.q8_matmul_bulk(w, x, n, d), f"random last {i}")
