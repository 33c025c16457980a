"""Shared helpers of the GPU parity tests (host data, device copies, the bar)."""
from __future__ import annotations

import numpy as np

# The path's parity bar: |gpu - cpu| <= 1e-4 + 1e-3 * |cpu| elementwise (fp32).
ATOL = 1e-4
RTOL = 1e-3


def assert_parity(got, want, what=""):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - want) - (ATOL + RTOL * np.abs(want))
    worst = np.unravel_index(np.argmax(err), err.shape)
    assert err[worst] <= 0, (f"{what}: |gpu-cpu| exceeds 1e-4 + 1e-3|cpu| at {worst}: "
                             f"gpu={got[worst]} cpu={want[worst]}")


def to_gpu(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def random_tables(rng, ctx, pages):
    """Block tables from one permutation of the pool, consumed sequentially."""
    ctx = np.asarray(ctx)
    need = (ctx + 15) // 16
    max_pages = int(need.max())
    assert need.sum() <= pages
    perm = rng.permutation(pages).astype(np.int32)
    tables = np.zeros((len(ctx), max_pages), np.int32)
    used = 0
    for b, n in enumerate(need):
        tables[b, :n] = perm[used:used + n]
        used += n
    return tables


class DecodeCase:
    """Random pool + tables + q on the host, mirrored on the GPU."""

    def __init__(self, rng, ctx, n_heads, n_kv_heads, head_dim, pages, layers=1, layer=0,
                 scale=1.0):
        import nitrorag_amd as na

        self.H, self.Hkv, self.hd, self.layer = n_heads, n_kv_heads, head_dim, layer
        kv_dim = n_kv_heads * head_dim
        self.ctx = np.asarray(ctx)
        self.positions = (self.ctx - 1).astype(np.int32)
        self.tables = random_tables(rng, self.ctx, pages)
        shape = (pages, layers, 16, kv_dim)
        self.k = (rng.standard_normal(shape) * scale).astype(np.float32)
        self.v = rng.standard_normal(shape).astype(np.float32)
        self.q = (rng.standard_normal((len(ctx), n_heads * head_dim)) * scale).astype(np.float32)
        self.dk, self.dv = to_gpu(self.k), to_gpu(self.v)
        self.pool = na.KVPool.wrap(self.dk, self.dv)
        self.pool.upload_decode_batch(self.tables, self.positions)

    def run_gpu(self):
        import torch

        q = to_gpu(self.q)
        out = torch.full_like(q, float("nan"))
        self.pool.decode(self.layer, q, out, self.H, self.Hkv, self.hd)
        torch.cuda.synchronize()
        return out.cpu().numpy()

    def run_oracle(self):
        from oracle import attn

        return attn.decode_batch(self.k, self.v, self.layer, self.q, self.tables, self.positions,
                                 self.H, self.Hkv, self.hd)
