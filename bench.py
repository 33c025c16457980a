"""Benchmark of the MI355X paged-attention path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Default workload (the headline line): batched paged-attention decode at the
Llama-2-7B attention shape — B=64 sequences, 32 query heads = 32 KV heads,
head_dim 128, context 4096 tokens each (256 pages of 16 tokens), fp32 K/V ~
N(0,1) in a 20,000-page pool with block tables drawn from one seeded
permutation of the pool, one layer.  A step is what forward_decode_batch does
per layer for attention (src/model_q8.cpp:616-662): append this step's K/V row
of every sequence at its position, then attend over positions 0..4095.
Inputs are resident in HBM before timing starts.

Reported:
  value / unit      algorithmic GB/s of the whole step (append + decode)
  roofline          the dominant kernel alone: algorithmic bytes per launch /
                    mean launch time from HIP events on the launch stream,
                    against MI355X's 8 TB/s HBM peak; `traffic` is the HBM bytes
                    per launch measured with rocprofv3 (profiles/)
  cpu_baseline      the CPU oracle (C restatement of the reference's OpenMP
                    loops, all host cores) on a sample of the same workload
  parity            after the timed steps, the first and the last sequence's
                    outputs against the oracle (1e-4 + 1e-3|cpu|) and all 64
                    appended K/V rows bit for bit; a mismatch ends the run with
                    exit status 3 and no line
  configs           the four other configurations of the metric, each measured
                    in this process the way its own --workload run measures it,
                    with its roofline and its own oracle check (no CPU baseline):
                    decode-single-110m, decode-b32-mixed, prefill-b8-12x64,
                    decode-prefix-shared (--no-configs leaves them out)
Algorithmic bytes per decode launch (append fused): sum_b ctx_b*Hkv*hd*4*2 (K
and V, the new row read from the appended k/v) + B*H*hd*4*2 (q in, out) +
sum_b ceil(ctx_b/16)*4 (block-table entries) + B*Hkv*hd*4*2 (the new rows
written into their pages).

Other workloads (the other paged-attention shapes, the model step around the path,
Q8 products and the serving loop):
  decode-single-110m     1 sequence, 12 layers x 12 heads x 64, ctx 256, 64-page pool;
                         a step is one token through all 12 layers' append + attention,
                         the 12 launches replayed as one HIP graph (decode-single-110m-
                         flushed: eager, 1 GiB read before each layer's launch, only the
                         launches timed)
  decode-b32-mixed       B=32, 12x64, ctx ~ U[16,1024], 4096-page pool of 12 layers; a step
                         is the 12 layers' launches, one HIP graph
  decode-prefix-shared   B=48, 12x64, 512 shared prefix tokens (32 pages, FNV-1a cache
                         hits) + private suffixes ~ U[64,512], 12 layers, one HIP graph
  decode-long-131072-32x128  one sequence of 131072 tokens, 32x128 (a long retrieved context)
  prefill-long-16384-32x128  one 16384-token prompt, 32x128 (its CPU baseline runs the whole
                         prompt: minutes; --no-cpu-baseline skips it)
  prefill-chunks-b8-256-12x64  8 chunks of 256 tokens after 256-768 cached tokens each
                         (the reference scheduler's chunked prefill), 12x64, one launch
  prefill-b8-12x64       B=8 prompts, lengths ~ U[128,1024], 12x64, KV scattered into
                         fresh pages then attended causally, in one launch; 12 such
                         steps per HIP graph; FLOPs = sum 2*H*hd*L(L+1)
  q8-gemv-7b-ffn         Q8_0 product, W 11008 x 4096 BlockQ8, 1 activation row
  q8-matmul-110m-b32     Q8_0 product, W 2048 x 768 BlockQ8, 32 activation rows
  model-110m-decode-b32  one decode step of a 110M-shaped Q8 model, B=32 at context 512
  model-7b-decode-bN     one decode step of a Llama-2-7B-shaped Q8 model, N = 1, 2 or 8
                         sequences at context 1024
  serve-110m-uN          the reference's continuous-batching experiment, N users
Short launches are timed as HIP graphs of a step's launches: K replays back to
back under the wall clock, then K more between one pair of events (kernel time
= their time / launches).  One layer of the mixed-length or prefix-shared batch
fits in the 256 MB Infinity Cache, but a step's 12 layers are 1.1-1.2 GB of
distinct rows, so every launch reads rows the cache no longer holds.  The
prefill step's graph holds 12 steps over the same prompts: their q/k/v stay in
the caches, as the q/k/v product just before the attention leaves them.  Long
launches (the headline) run K steps back to back under the wall clock, then K
more with an event pair around every launch.  The -flushed single-sequence form
reads 1 GiB before every launch and times each launch between its own events.
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

# The CPU baseline's OpenMP threads stay on neighbouring cores (set before
# anything in this process initialises the OpenMP runtime).
os.environ.setdefault("OMP_PROC_BIND", "close")

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
FP32_PEAK_TFLOPS = 157.3
METRIC = "paged-attn decode GB/s (% HBM peak) + tokens/s at B=64 ctx4096"
DEFAULT_WORKLOAD = "decode-b64-ctx4096"


def decode_bytes(ctx, B: int, H: int, Hkv: int, hd: int) -> int:
    ctx = np.asarray(ctx, dtype=np.int64)
    return int((ctx * Hkv * hd * 4 * 2).sum() + B * H * hd * 4 * 2 + ((ctx + 15) // 16 * 4).sum())


def append_bytes(B: int, Hkv: int, hd: int) -> int:
    """The new K and V row of every sequence written into its page."""
    return B * Hkv * hd * 4 * 2


def seeded_tables(ctx, pages: int, seed: int) -> np.ndarray:
    """Block tables consumed sequentially from one seeded permutation of the pool."""
    ctx = np.asarray(ctx)
    need = (ctx + 15) // 16
    assert need.sum() <= pages
    perm = np.random.default_rng(seed).permutation(pages).astype(np.int32)
    t = np.zeros((len(ctx), int(need.max())), np.int32)
    off = 0
    for b, n in enumerate(need):
        t[b, :n] = perm[off:off + n]
        off += n
    return t


def measured_traffic(path: str):
    """HBM bytes per decode launch recorded from rocprofv3 FETCH_SIZE + WRITE_SIZE
    runs (calibrated against a copy of known size) in the profile summary, or None."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def time_cpu(fn, seconds: float, warmup: int = 2, min_reps: int = 5):
    """Median seconds per call over at least min_reps timed calls (and about
    `seconds` of them), after `warmup` untimed ones; returns (median, reps,
    elapsed)."""
    for _ in range(warmup):
        fn()
    times, t0 = [], time.perf_counter()
    while len(times) < min_reps or time.perf_counter() - t0 < seconds:
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    return float(np.median(times)), len(times), time.perf_counter() - t0


class ParityError(AssertionError):
    pass


def check_parity(got, want, what):
    """|gpu - cpu| <= 1e-4 + 1e-3 |cpu| elementwise (the path's fp32 bar); raises ParityError."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    if got.shape != want.shape or not np.all(np.isfinite(got)):
        raise ParityError(f"{what}: shape {got.shape} vs {want.shape}, or non-finite output")
    excess = np.abs(got - want) - (1e-4 + 1e-3 * np.abs(want))
    if excess.max() > 0:
        i = np.unravel_index(np.argmax(excess), excess.shape)
        raise ParityError(f"{what}: |gpu-cpu| exceeds 1e-4 + 1e-3|cpu| at {i}: gpu={got[i]} cpu={want[i]}")


class DecodeWorkload:
    """Paged decode: per layer, append every sequence's new K/V row, then attend."""

    bound = "hbm"
    graph = False

    def __init__(self, name, B, H, Hkv, hd, pages, layers, steps_layers, ctx, flush, seed,
                 tables=None, shared_pages=False, describe=""):
        self.name, self.B, self.H, self.Hkv, self.hd = name, B, H, Hkv, hd
        self.pages, self.layers, self.steps_layers = pages, layers, steps_layers
        self.ctx = np.asarray(ctx, dtype=np.int64)
        self.positions = (self.ctx - 1).astype(np.int32)
        self.flush, self.seed, self.describe = flush, seed, describe
        self.tables = seeded_tables(self.ctx, pages, seed) if tables is None else tables
        self.shared_pages = shared_pages
        # K/V rows the launch reads, each (page, row) slot counted once however
        # many sequences' tables hold its page
        rows = np.concatenate([self.tables[b, np.arange(c) >> 4].astype(np.int64) * 16 + (np.arange(c) & 15)
                               for b, c in enumerate(self.ctx)])
        self.unique_rows = int(np.unique(rows).size)

    def setup(self, dev, g):
        import torch

        import nitrorag_amd as na

        kv_dim = self.Hkv * self.hd
        self.k = torch.randn((self.pages, self.layers, 16, kv_dim), device=dev, generator=g)
        self.v = torch.randn((self.pages, self.layers, 16, kv_dim), device=dev, generator=g)
        L = len(self.steps_layers)
        self.q = torch.randn((L, self.B, self.H * self.hd), device=dev, generator=g)
        self.knew = torch.randn((L, self.B, kv_dim), device=dev, generator=g)
        self.vnew = torch.randn((L, self.B, kv_dim), device=dev, generator=g)
        self.out = torch.empty((L, self.B, self.H * self.hd), device=dev)
        self.pool = na.KVPool.wrap(self.k, self.v)
        self.pool.upload_decode_batch(self.tables, self.positions)
        # 1 GiB read before each timed launch evicts the 256 MB Infinity Cache and the
        # L2s with clean lines (a write would leave dirty lines draining during the launch)
        self.scratch = torch.ones(2**28, device=dev) if self.flush else None
        self.flush_out = torch.empty((), device=dev)

    def step(self, stream, events=None):
        import torch

        for i, layer in enumerate(self.steps_layers):
            if self.scratch is not None:
                torch.sum(self.scratch, dim=0, out=self.flush_out)
            if events is not None:
                events[i][0].record(stream)
            # append + attend (one launch: no other sequence reads a page being appended to)
            self.pool.decode_append(layer, self.q[i], self.knew[i], self.vnew[i], self.out[i], self.H,
                                    self.Hkv, self.hd, stream)
            if events is not None:
                events[i][1].record(stream)

    def launches_per_step(self):
        return len(self.steps_layers)

    def work_per_launch(self):
        # the launch also writes each sequence's new K/V row into its page
        return decode_bytes(self.ctx, self.B, self.H, self.Hkv, self.hd) + append_bytes(self.B, self.Hkv, self.hd)

    def hbm_bytes_per_launch(self):
        """Bytes the launch must move through HBM: a page that several sequences'
        tables share is counted once (the logical bytes count it per sequence)."""
        kv_row = self.Hkv * self.hd * 4 * 2
        return self.work_per_launch() - (int(self.ctx.sum()) - self.unique_rows) * kv_row

    def tokens_per_step(self):
        return self.B

    def check(self):
        import torch

        assert torch.isfinite(self.out).all().item(), "non-finite decode output"

    def check_graph_replay(self):
        """The graph's replays recompute the eager step's outputs bit for bit."""
        import torch

        torch.cuda.synchronize()
        assert torch.equal(self.out, self.eager_out), "graph replay differs from the eager step"

    def verify(self, sample=None, layers=None):
        """After the timed steps: the outputs of `sample` sequences (all by
        default) in the step's layers `layers` (all by default) against the
        oracle at the parity bar, over host copies of just their pages, and
        every sampled sequence's appended K/V row in its page bit for bit."""
        import torch

        from oracle import attn

        sel = np.arange(self.B) if sample is None else np.asarray(sample)
        steps = range(len(self.steps_layers)) if layers is None else layers
        n_pages = self.tables.shape[1]
        idx = torch.from_numpy(self.tables[sel].reshape(-1).astype(np.int64)).to(self.k.device)
        local = np.arange(len(sel) * n_pages, dtype=np.int32).reshape(len(sel), n_pages)
        pos = self.positions[sel]
        new_page = local[np.arange(len(sel)), pos >> 4]
        for i in steps:
            layer = self.steps_layers[i]
            kh = self.k[:, layer].index_select(0, idx).cpu().numpy()[:, None]
            vh = self.v[:, layer].index_select(0, idx).cpu().numpy()[:, None]
            for pool, new, what in ((kh, self.knew, "K"), (vh, self.vnew, "V")):
                if not np.array_equal(pool[new_page, 0, pos & 15], new[i, torch.from_numpy(sel)].cpu().numpy()):
                    raise ParityError(f"{self.name} layer {layer}: an appended {what} row differs from its input")
            want = attn.decode_batch(kh, vh, 0, self.q[i, torch.from_numpy(sel)].cpu().numpy(), local, pos,
                                     self.H, self.Hkv, self.hd)
            check_parity(self.out[i, torch.from_numpy(sel)].cpu().numpy(), want, f"{self.name} layer {layer}")
        return (f"{len(sel)} of {self.B} sequences x {len(steps)} of {len(self.steps_layers)} layers vs the "
                f"oracle within 1e-4 + 1e-3|cpu|; their appended K/V rows bit-exact")

    def release(self):
        self.pool.close()
        for name in ("k", "v", "q", "knew", "vnew", "out", "scratch", "eager_out"):
            if hasattr(self, name):
                delattr(self, name)

    def cpu_baseline(self, seconds, sample):
        """Oracle append + decode on `sample` sequences (their pages copied to a compact pool)."""
        import torch

        from oracle import attn

        sample = min(sample, self.B)
        n_pages = self.tables.shape[1]
        sel = self.tables[:sample]
        idx = torch.from_numpy(sel.reshape(-1).astype(np.int64)).to(self.k.device)
        kh = self.k.index_select(0, idx).cpu().numpy()
        vh = self.v.index_select(0, idx).cpu().numpy()
        local = np.arange(sample * n_pages, dtype=np.int32).reshape(sample, n_pages)
        q = self.q[:, :sample].cpu().numpy()
        kn = self.knew[:, :sample].cpu().numpy()
        vn = self.vnew[:, :sample].cpu().numpy()
        pos = self.positions[:sample]
        threads = attn.max_threads()

        def run():
            for i, layer in enumerate(self.steps_layers):
                attn.kv_append_decode(kh, vh, layer, kn[i], vn[i], local, pos)
                attn.decode_batch(kh, vh, layer, q[i], local, pos, self.H, self.Hkv, self.hd,
                                  threads)

        per_rep, reps, el = time_cpu(run, seconds)
        nbytes = decode_bytes(pos + 1, sample, self.H, self.Hkv, self.hd) * len(self.steps_layers)
        return {
            "value": round(nbytes / per_rep / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": (f"{sample} of the {self.B} sequences of this workload, append + batched "
                       f"decode over {len(self.steps_layers)} layer(s), median of {reps} runs in {el:.1f} s; "
                       f"{sample / per_rep:.1f} tokens/s"),
            "tokens_per_s": round(sample / per_rep, 3),
        }

    def extra(self, kernel_s):
        if not self.shared_pages:
            return {}
        ub = self.unique_rows * self.Hkv * self.hd * 4 * 2
        return {"unique_kv_bytes_per_launch": int(ub),
                "logical_bytes_per_launch": self.work_per_launch(),
                "logical_gbps": round(self.work_per_launch() / kernel_s / 1e9, 2)}


class PrefillWorkload:
    """Causal paged prefill: the scatter of the chunk's K/V rows into the pool and
    the attention, in one launch (nitro_paged_attn_prefill_append).  A chunk of
    lens[b] tokens starts at position starts[b] (0: a fresh prompt; otherwise the
    keys before it are cached in the pool).  Rates are the algorithmic fp32 FLOPs
    (QK^T and PV over keys 0..pos of every chunk row) against the fp32 matrix-core
    peak; the default kernel reaches fp32 accuracy on the bf16 matrix cores
    (split operands)."""

    bound = "mfma"
    flush = False

    def __init__(self, name, B, H, Hkv, hd, lens, seed, describe, layers=1, starts=None):
        import nitrorag_amd as na

        self.name, self.B, self.H, self.Hkv, self.hd = name, B, H, Hkv, hd
        # a step runs the prefill of every layer of the pool, each with its own q/k/v
        self.layers = layers
        self.graph = layers > 1
        self.lens = np.asarray(lens, dtype=np.int64)
        self.starts = np.zeros(B, np.int64) if starts is None else np.asarray(starts, dtype=np.int64)
        self.seed, self.describe = seed, describe
        self.pages = int(((self.starts + self.lens + 15) // 16).sum())
        bm = na.BlockManager(self.pages)  # fresh pool: LIFO page ids, as the reference hands out
        seqs = []
        rng = np.random.default_rng(seed)
        for b in range(B):
            s = na.Sequence(b)
            s.ingest_prompt(rng.integers(1, 32000, size=int(self.starts[b] + self.lens[b])), bm, False)
            seqs.append(s)
        self.tables = na.pack_block_tables(seqs)

    def setup(self, dev, g):
        import torch

        import nitrorag_amd as na

        kv_dim = self.Hkv * self.hd
        total = int(self.lens.sum())
        L = self.layers
        # the cached keys before each chunk (random; fresh prompts have none)
        self.k = torch.randn((self.pages, L, 16, kv_dim), device=dev, generator=g)
        self.v = torch.randn((self.pages, L, 16, kv_dim), device=dev, generator=g)
        self.q = torch.randn((L, total, self.H * self.hd), device=dev, generator=g)
        self.kc = torch.randn((L, total, kv_dim), device=dev, generator=g)
        self.vc = torch.randn((L, total, kv_dim), device=dev, generator=g)
        self.out = torch.empty_like(self.q)
        self.pool = na.KVPool.wrap(self.k, self.v)
        self.pool.upload_prefill_batch(self.tables, self.starts, self.lens)

    def step(self, stream, events=None):
        for layer in range(self.layers):
            if events is not None:
                events[layer][0].record(stream)
            self.pool.prefill_append(layer, self.q[layer], self.kc[layer], self.vc[layer], self.out[layer],
                                     self.H, self.Hkv, self.hd, stream)
            if events is not None:
                events[layer][1].record(stream)

    def launches_per_step(self):
        return self.layers

    def check_graph_replay(self):
        import torch

        torch.cuda.synchronize()
        assert torch.equal(self.out, self.eager_out), "graph replay differs from the eager step"

    def verify(self, sample=None, layers=None):
        """After the timed steps: every prompt's K/V rows in its pages bit for
        bit (all layers), and the attention outputs of `sample` prompts (all by
        default) in `layers` (the last layer by default) against the oracle's
        causal prefill at the parity bar."""
        from oracle import attn

        sel = range(self.B) if sample is None else sample
        layers = [self.layers - 1] if layers is None else layers
        off = np.concatenate([[0], np.cumsum(self.lens)])
        k, v = self.k.cpu().numpy(), self.v.cpu().numpy()
        kc, vc = self.kc.cpu().numpy(), self.vc.cpu().numpy()
        for b in range(self.B):
            t = int(self.starts[b]) + np.arange(int(self.lens[b]))
            pg = self.tables[b][t >> 4]
            rows = slice(int(off[b]), int(off[b + 1]))
            if not (np.array_equal(k[pg, :, t & 15].transpose(1, 0, 2), kc[:, rows]) and
                    np.array_equal(v[pg, :, t & 15].transpose(1, 0, 2), vc[:, rows])):
                raise ParityError(f"{self.name}: prompt {b}'s K/V rows in its pages differ from its input")
        for layer in layers:
            q, out = self.q[layer].cpu().numpy(), self.out[layer].cpu().numpy()
            for b in sel:
                rows = slice(int(off[b]), int(off[b + 1]))
                want = attn.prefill_chunk(k, v, layer, q[rows], self.tables[b], int(self.starts[b]), self.H,
                                          self.Hkv, self.hd)
                check_parity(out[rows], want, f"{self.name} prompt {b} layer {layer}")
        return (f"{len(sel)} of {self.B} prompts x {len(layers)} of {self.layers} layer(s) vs the oracle "
                f"within 1e-4 + 1e-3|cpu|; every prompt's K/V rows in its pages bit-exact")

    def release(self):
        self.pool.close()
        for name in ("k", "v", "q", "kc", "vc", "out", "eager_out"):
            if hasattr(self, name):
                delattr(self, name)

    def work_per_launch(self):
        # sum over chunk rows at positions s..s+n-1 of 4*H*hd*(pos+1)
        n, s = self.lens, self.starts
        return int((2 * self.H * self.hd * n * (2 * s + n + 1)).sum())

    def tokens_per_step(self):
        return int(self.lens.sum())

    def check(self):
        import torch

        assert torch.isfinite(self.out).all().item(), "non-finite prefill output"
        calls, one_launch = self.pool.prefill_counts()
        if os.environ.get("NITRO_PREFILL_APPEND", "1") != "0":
            assert one_launch == calls, "a prefill step ran the scatter as a launch of its own"

    def cpu_baseline(self, seconds, sample):
        from oracle import attn

        sample = min(sample, self.B)
        k = self.k[:, :1].cpu().numpy()
        v = self.v[:, :1].cpu().numpy()
        q = self.q[0].cpu().numpy()
        kc, vc = self.kc[0].cpu().numpy(), self.vc[0].cpu().numpy()
        off = np.concatenate([[0], np.cumsum(self.lens)])
        threads = attn.max_threads()

        def run():
            for b in range(sample):
                rows = slice(int(off[b]), int(off[b + 1]))
                s = int(self.starts[b])
                attn.kv_scatter_prefill(k, v, 0, kc[rows], vc[rows], self.tables[b], s)
                attn.prefill_chunk(k, v, 0, q[rows], self.tables[b], s, self.H, self.Hkv,
                                   self.hd, threads)

        per_rep, reps, el = time_cpu(run, seconds)
        n, s = self.lens[:sample], self.starts[:sample]
        flops = float((2 * self.H * self.hd * n * (2 * s + n + 1)).sum())
        toks = int(self.lens[:sample].sum())
        return {"value": round(flops / per_rep / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
                "kind": "port",
                "sample": (f"prompts 0..{sample - 1} of the {self.B} ({toks} tokens), scatter + "
                           f"causal prefill, median of {reps} runs in {el:.1f} s; {toks / per_rep:.1f} tokens/s"),
                "tokens_per_s": round(toks / per_rep, 3)}

    def extra(self, kernel_s):
        return {}


class Q8Workload:
    """One Q8_0 matrix product, out[B][d] = x[B][n] . W[d][n]^T with W in the
    reference's BlockQ8 layout (36 bytes per 32 weights).  Algorithmic bytes
    per launch: d*(n/32)*36 (weights) + B*n*4 (x) + B*d*4 (out)."""

    bound = "hbm"
    flush = True

    def __init__(self, name, n, d, B, seed, describe):
        self.name, self.n, self.d, self.B, self.seed, self.describe = name, n, d, B, seed, describe

    def setup(self, dev, g):
        import torch

        nb = self.n // 32
        q = torch.randint(-127, 128, (self.d, nb, 32), device=dev, generator=g, dtype=torch.int32)
        scale = torch.rand((self.d, nb, 1), device=dev, generator=g) * 0.01 + 0.005
        self.w = torch.cat([scale.view(torch.uint8), q.to(torch.int8).view(torch.uint8)],
                           dim=2).contiguous().view(-1)
        self.x = torch.randn((self.B, self.n), device=dev, generator=g)
        self.out = torch.empty((self.B, self.d), device=dev)
        self.scratch = torch.ones(2**28, device=dev)  # 1 GiB read evicts L2 and MALL
        self.flush_out = torch.empty((), device=dev)

    def step(self, stream, events=None):
        import torch

        import nitrorag_amd as na

        torch.sum(self.scratch, dim=0, out=self.flush_out)
        if events is not None:
            events[0][0].record(stream)
        na.q8_matmul(self.w, self.x, self.out, 0, stream)
        if events is not None:
            events[0][1].record(stream)

    def launches_per_step(self):
        return 1

    def work_per_launch(self):
        return self.d * (self.n // 32) * 36 + self.B * self.n * 4 + self.B * self.d * 4

    def tokens_per_step(self):
        return self.B

    def kernel(self):
        if self.B <= 4:
            if self.n < 2048:
                return "q8_gemv_kernel (VALU)"
            return "q8_flat_kernel (VALU, x in LDS)" if self.B * self.n <= 16384 else "q8_rowdot_kernel (VALU)"
        return "q8_mma_kernel (bf16 matrix cores, x split in three exact parts)"

    def config(self):
        return {"workload": self.describe, "batch": self.B, "n": self.n, "d": self.d,
                "parallelism": "single GPU"}

    def check(self):
        import torch

        assert torch.isfinite(self.out).all().item(), "non-finite Q8 product"

    def device_errors(self):
        return 0

    def cpu_baseline(self, seconds, sample):
        """The oracle's AVX2 restatement of the reference's matmul on all host cores."""
        from oracle import attn
        from oracle import model as om

        w = self.w.cpu().numpy()
        x = self.x.cpu().numpy()
        threads = attn.max_threads()
        rows = min(sample, self.B)
        per_rep, reps, el = time_cpu(lambda: om.q8_matmul(w, x[:rows], self.n, self.d, threads),
                                     seconds)
        nbytes = self.d * (self.n // 32) * 36 * rows + rows * (self.n + self.d) * 4
        return {"value": round(nbytes / per_rep / 1e9, 3), "unit": "GB/s", "cores": threads,
                "kind": "port",
                "sample": (f"{rows} of the {self.B} activation rows of this workload, one matmul "
                           f"(src/model_q8.cpp:92-125) per row over the full matrix, median of "
                           f"{reps} runs in {el:.1f} s")}

    def extra(self, kernel_s):
        return {}


class ModelDecodeWorkload:
    """One decode step of the whole model (nitro_forward_decode_batch, full-row
    Q8 products): embedding, n_layers x (rms_norm, wq/wk/wv, RoPE + KV append,
    paged attention, wo, residual, rms_norm, w1/w3, SwiGLU, w2, residual), final
    rms_norm and the fp32 classifier, for B sequences at context ctx.  Synthetic
    model file in the reference's layout (nitrorag_amd.model.synthetic_model_file).
    Algorithmic bytes per step: every weight once + K/V rows read by attention +
    K/V rows written + activations in/out (logits)."""

    bound = "hbm"
    flush = False

    def __init__(self, name, cfg, B, ctx, seed, describe):
        self.name, self.cfg, self.B, self.ctx, self.seed, self.describe = name, cfg, B, ctx, seed, describe
        dim, hid, L, H, Hkv, V, S = cfg
        self.H, self.Hkv, self.hd, self.L, self.V = H, Hkv, dim // H, L, V
        self.kv_dim = Hkv * (dim // H)
        self.pages = B * ((ctx + 15) // 16) + 16
        self.tables = seeded_tables(np.full(B, ctx), self.pages, seed)
        self.positions = np.full(B, ctx - 1, np.int32)

    def setup(self, dev, g):
        import torch

        import nitrorag_amd as na
        from nitrorag_amd.model import synthetic_model_file

        self.blob = synthetic_model_file(*self.cfg, seed=self.seed)
        self.model = na.Model(self.blob)
        shape = (self.pages, self.L, 16, self.kv_dim)
        self.k = torch.randn(shape, device=dev, generator=g)
        self.v = torch.randn(shape, device=dev, generator=g)
        self.pool = na.KVPool.wrap(self.k, self.v)
        self.pool.upload_decode_batch(self.tables, self.positions)
        self.tokens = np.random.default_rng(self.seed).integers(0, self.V, self.B).astype(np.int32)
        self.logits = torch.empty((self.B, self.V), device=dev)

    def step(self, stream, events=None):
        from nitrorag_amd.model import FULL_ROWS

        if events is not None:
            events[0][0].record(stream)
        self.model.forward_decode_batch(self.pool, self.tokens, self.logits, FULL_ROWS, stream)
        if events is not None:
            events[0][1].record(stream)

    def launches_per_step(self):
        return 1

    def work_per_launch(self):
        dim, hid, L, H, Hkv, V, S = self.cfg
        q8 = lambda r, c: r * (c // 32) * 36
        weights = (V * dim * 4 + L * (q8(dim, dim) * 2 + q8(self.kv_dim, dim) * 2 + q8(hid, dim) * 2
                                      + q8(dim, hid) + 2 * dim * 4) + dim * 4)
        kv = L * self.B * self.ctx * self.kv_dim * 8 + L * self.B * self.kv_dim * 8
        return int(weights + kv + self.B * V * 4)

    def tokens_per_step(self):
        return self.B

    def kernel(self):
        return "forward_decode_batch step (all kernels)"

    def config(self):
        dim, hid, L, H, Hkv, V, S = self.cfg
        return {"workload": self.describe, "batch": self.B, "context": self.ctx, "dim": dim,
                "hidden_dim": hid, "n_layers": L, "n_heads": H, "n_kv_heads": Hkv, "vocab": V,
                "parallelism": "single GPU"}

    def check(self):
        import torch

        assert torch.isfinite(self.logits).all().item(), "non-finite logits"

    def cpu_baseline(self, seconds, sample):
        """The oracle's composed forward_paged-style step (full-row matmul, the
        oracle attention) for `sample` of the sequences, their pages copied out."""
        import torch

        from oracle import attn
        from oracle import model as om

        rows = min(sample, self.B)
        ora = om.OracleModel(self.blob)
        n_pages = self.tables.shape[1]
        idx = torch.from_numpy(self.tables[:rows].reshape(-1).astype(np.int64)).to(self.k.device)
        kh = self.k.index_select(0, idx).cpu().numpy()
        vh = self.v.index_select(0, idx).cpu().numpy()
        local = np.arange(rows * n_pages, dtype=np.int32).reshape(rows, n_pages)
        pos = self.positions[:rows]
        toks = self.tokens[:rows]
        per_rep, reps, el = time_cpu(lambda: ora.forward_decode_batch(kh, vh, local, pos, toks, bulk=False),
                                     seconds)
        return {"value": round(rows / per_rep, 2), "unit": "tokens/s", "cores": attn.max_threads(),
                "kind": "port",
                "sample": (f"{rows} of the {self.B} sequences of this workload, one decode step of "
                           f"the oracle's composed forward (src/model_q8.cpp:571-694 with full-row "
                           f"matmul), median of {reps} runs in {el:.1f} s")}

    def device_errors(self):
        return self.pool.take_device_errors()

    def extra(self, kernel_s):
        return {}


class ServeWorkload:
    """The reference's continuous-batching experiment (src/model_q8.cpp:864-908)
    on the device scheduler (nitro_sched_step): `users` requests with the same
    256-token prompt (token 263) submitted together, token budget 256 per
    step, 20 generated tokens each, an 8000-page pool, stepped until every
    request has finished; Llama-2-110M-shaped synthetic model, the
    reference's Q8 products (matmul_bulk semantics).  One bench step = one
    whole run; value = users * 20 / run time (aggregate tokens/s, the
    reference's figure), plus the average time to first token.  Algorithmic
    bytes per run: per scheduler step, the weights the step needs once (the
    fp32 classifier, norms, and the last BlockQ8 of every Q8 row, all that
    matmul_bulk reads) + the K/V rows its attention reads and writes + logits."""

    bound = "hbm"
    flush = False
    event_pass = False
    PROMPT, TOKEN, GEN, BUDGET, PAGES = 256, 263, 20, 256, 8000

    def __init__(self, name, users, seed, describe):
        self.name, self.users, self.seed, self.describe = name, users, seed, describe
        self.cfg = (768, 2048, 12, 12, 12, 32000, 1024)
        dim, hid, L, H, Hkv, V, S = self.cfg
        self.kv_dim, self.L, self.V = Hkv * (dim // H), L, V
        self.ttft_ms = []

    def setup(self, dev, g):
        import nitrorag_amd as na
        from nitrorag_amd.model import synthetic_model_file

        self.blob = synthetic_model_file(*self.cfg, seed=self.seed)
        self.model = na.Model(self.blob)
        self.pool = na.KVPool(self.PAGES, self.L, self.kv_dim)
        self.prompt = [self.TOKEN] * self.PROMPT
        self.sched_steps, self.run_bytes = self._schedule_shape()

    def _schedule_shape(self):
        """Host-only dry run of the same schedule (its shape does not depend
        on the tokens): scheduler steps per run and algorithmic bytes."""
        import nitrorag_amd as na

        dim, hid, L, H, Hkv, V, S = self.cfg
        q8 = lambda r, c: r * 36  # matmul_bulk keeps the last BlockQ8 of each row only
        weights = (V * dim * 4 + L * (q8(dim, dim) * 2 + q8(self.kv_dim, dim) * 2 + q8(hid, dim) * 2
                                      + q8(dim, hid) + 2 * dim * 4) + dim * 4)
        row = L * self.kv_dim * 4 * 2  # one K and one V row over all layers
        bm = na.BlockManager(self.PAGES)
        sch = na.ContinuousScheduler(bm, self.BUDGET, self.GEN)
        for u in range(self.users):
            sch.add_request(u, self.prompt)
        steps, total = 0, 0
        while sch.has_active_requests():
            p = sch.plan()
            rows = len(p.decode_ids) + p.prefill_length
            if rows:
                total += weights
                total += sum(pos + 1 for pos in p.decode_positions) * row  # decode reads
                total += (p.prefill_start + p.prefill_length) * row * (1 if p.prefill_length else 0)
                total += rows * row + (len(p.decode_ids) + p.prefill_finishes) * V * 4
            sch.commit(1 if p.prefill_finishes else 0, [1] * len(p.decode_ids))
            steps += 1
        sch.close()
        return steps, total

    def step(self, stream, events=None):
        import nitrorag_amd as na
        from nitrorag_amd.q8 import LAST_BLOCK

        bm = na.BlockManager(self.PAGES)
        sch = na.ContinuousScheduler(bm, self.BUDGET, self.GEN)
        if events is not None:
            events[0][0].record(stream)
        t0 = time.perf_counter()
        for u in range(self.users):
            sch.add_request(u, self.prompt)
        waiting = set(range(self.users))
        ttft = []
        while sch.has_active_requests():
            sch.step(self.model, self.pool, LAST_BLOCK, stream)
            for u in list(waiting):
                if sch.request_status(u)["is_prefill_done"]:
                    ttft.append((time.perf_counter() - t0) * 1e3)
                    waiting.discard(u)
        if events is not None:
            events[0][1].record(stream)
        self.ttft_ms.append(float(np.mean(ttft)))
        self.generated = sum(len(sch.generated(u)) for u in range(self.users))
        sch.close()

    def launches_per_step(self):
        return 1

    def work_per_launch(self):
        return int(self.run_bytes)

    def tokens_per_step(self):
        return self.users * self.GEN

    def kernel(self):
        return "continuous-scheduler run (all kernels, host plan/commit between steps)"

    def config(self):
        dim, hid, L, H, Hkv, V, S = self.cfg
        return {"workload": self.describe, "users": self.users, "prompt_tokens": self.PROMPT,
                "generated_per_user": self.GEN, "token_budget": self.BUDGET, "pool_pages": self.PAGES,
                "dim": dim, "hidden_dim": hid, "n_layers": L, "n_heads": H, "vocab": V,
                "parallelism": "single GPU"}

    def check(self):
        assert self.generated == self.users * self.GEN, self.generated

    def device_errors(self):
        return self.pool.take_device_errors()

    def headline(self, ms_per_step):
        return {"metric": f"{self.name} aggregate tokens/s", "unit": "tokens/s",
                "value": round(self.users * self.GEN / (ms_per_step * 1e-3), 1)}

    def extra(self, kernel_s):
        return {"avg_ttft_ms": round(float(np.mean(self.ttft_ms[-5:])), 3),
                "scheduler_steps_per_run": self.sched_steps}

    def cpu_baseline(self, seconds, sample):
        """The reference's own scheduler and forward passes (oracle/_ref, built
        from its sources) on the same experiment with `sample` users (at most
        16: with more, two of its OpenMP threads allocate pages at once in
        forward_decode_batch, src/model_q8.cpp:578-582, a data race)."""
        from oracle import ref

        if not ref.available():
            return None
        users = min(sample, 16, self.users)
        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
        dim, hid, L, H, Hkv, V, S = self.cfg
        W = ref.RefWorld.random_model(H, Hkv, dim // H, L, V, S, hid, self.PAGES, max_rows=512,
                                      max_seqs=0, seed=self.seed & 0xffffffff, threads=threads)
        W.sched_create(self.BUDGET)
        t0 = time.perf_counter()
        for u in range(users):
            W.sched_add(u, self.prompt)
        steps = 0
        while W.sched_active():
            assert W.sched_step() == 0
            steps += 1
        el = time.perf_counter() - t0
        W.close()
        return {"value": round(users * self.GEN / el, 2), "unit": "tokens/s", "cores": threads,
                "kind": "reference",
                "sample": (f"{users} users of this experiment through the reference's "
                           f"Continuous_Scheduler and forward passes ({steps} steps, {el:.1f} s, "
                           f"random 110M-shaped weights)")}


def prefix_shared_workload(seed):
    """48 sequences: 512 shared prefix tokens (32 pages via FNV-1a prefix-cache hits),
    private suffixes ~ U[64,512], then one decode token each."""
    import nitrorag_amd as na

    rng = np.random.default_rng(seed)
    B, prefix = 48, 512
    suffix = rng.integers(64, 513, size=B)
    pages = 32 + int(((suffix + 1 + 15) // 16).sum()) + 16
    bm = na.BlockManager(pages)
    shared = rng.integers(1, 32000, size=prefix).tolist()
    seqs = []
    for b in range(B):
        s = na.Sequence(b)
        s.ingest_prompt(shared + rng.integers(1, 32000, size=int(suffix[b])).tolist(), bm, True)
        if b == 0:
            s.flush_cache(bm)
        seqs.append(s)
    positions = np.array([s.logical_token_count for s in seqs], np.int32)
    for s in seqs:
        s.allocate_next_token(7, bm)
    tables = na.pack_block_tables(seqs)
    w = DecodeWorkload("decode-prefix-shared", B, 12, 12, 64, pages, 12, list(range(12)), positions + 1,
                       False, seed, tables=tables, shared_pages=True,
                       describe=(f"prefix-shared decode, B=48, 12 heads x 64, 512 shared tokens "
                                 f"(32 pages, ref_count 48) + private suffixes U[64,512], "
                                 f"{pages}-page pool of 12 layers; a step is one decode token through "
                                 f"the 12 layers (append + attend), one HIP graph"))
    w.graph = True
    return w


def make_workload(name, seed):
    if name == "decode-b64-ctx4096":
        return DecodeWorkload(name, 64, 32, 32, 128, 20000, 1, [0], np.full(64, 4096), False, seed,
                              describe=("paged-attention decode, B=64, ctx=4096, 32 heads x 128 "
                                        "(kv heads 32), 20000-page pool, 16-token pages, one layer, "
                                        "append + attend per step"))
    if name in ("decode-single-110m", "decode-single-110m-flushed"):
        # the 37.7 MB pool stays in the 256 MB Infinity Cache across a decode step,
        # as it does while serving; the -flushed form reads it cold every layer
        flushed = name.endswith("-flushed")
        w = DecodeWorkload(name, 1, 12, 12, 64, 64, 12, list(range(12)), [256], flushed, seed,
                           describe=("single-sequence decode, 12 layers x 12 heads x 64, ctx 256 "
                                     "in a 64-page pool; one token through all 12 layers" +
                                     (", Infinity Cache flushed per launch" if flushed else
                                      ", the 12 launches replayed as one HIP graph")))
        w.graph = not flushed
        return w
    if name == "decode-long-131072-32x128":
        return DecodeWorkload(name, 1, 32, 32, 128, 131072 // 16 + 8, 1, [0], [131072], False, seed,
                              describe=("paged-attention decode of one 131072-token sequence (a long "
                                        "retrieved context), 32 heads x 128, one layer, append + attend "
                                        "per step"))
    if name == "prefill-long-16384-32x128":
        return PrefillWorkload(name, 1, 32, 32, 128, np.array([16384]), seed,
                               describe=("causal prefill of one 16384-token prompt (a long retrieved "
                                         "context), 32 heads x 128, fresh 16-token pages"))
    if name == "decode-b32-mixed":
        rng = np.random.default_rng(seed)
        w = DecodeWorkload(name, 32, 12, 12, 64, 4096, 12, list(range(12)), rng.integers(16, 1025, size=32),
                           False, seed,
                           describe=("batched decode, B=32, 12 heads x 64, ctx ~ U[16,1024], "
                                     "4096-page pool of 12 layers; a step is one decode token through "
                                     "the 12 layers (append + attend), one HIP graph"))
        w.graph = True
        return w
    if name == "decode-prefix-shared":
        return prefix_shared_workload(seed)
    if name == "prefill-b8-12x64":
        rng = np.random.default_rng(seed)
        w = PrefillWorkload(name, 8, 12, 12, 64, rng.integers(128, 1025, size=8), seed,
                            describe=("causal prefill, B=8 prompts, lengths ~ U[128,1024], "
                                      "12 heads x 64, fresh 16-token pages (LIFO ids); a step is one "
                                      "layer's KV scatter + attention (one launch), 12 steps per HIP "
                                      "graph, the prompts' q/k/v left in the caches between them as the "
                                      "q/k/v product before the attention leaves them"))
        w.graph, w.graph_reps = True, 12
        return w
    if name == "prefill-chunks-b8-256-12x64":
        # the reference scheduler's chunked prefill: 256-token chunks
        # (src/pagedMemory.hpp:360-379), here the second to fourth chunk of 8 prompts
        rng = np.random.default_rng(seed)
        w = PrefillWorkload(name, 8, 12, 12, 64, np.full(8, 256), seed,
                            describe=("chunked prefill, B=8 chunks of 256 tokens after 256-768 cached "
                                      "tokens each, 12 heads x 64; a step is one layer's KV scatter + "
                                      "attention (one launch), 12 steps per HIP graph"),
                            starts=256 * rng.integers(1, 4, size=8))
        w.graph, w.graph_reps = True, 12
        return w
    if name == "model-110m-decode-b32":
        return ModelDecodeWorkload(name, (768, 2048, 12, 12, 12, 32000, 1024), 32, 512, seed,
                                   describe=("one decode step of a Llama-2-110M-shaped model "
                                             "(dim 768, hidden 2048, 12 layers, 12 heads x 64, "
                                             "vocab 32000, Q8_0 weights, synthetic), B=32 sequences "
                                             "at context 512, full-row Q8 products"))
    if name.startswith("serve-110m-u"):
        users = int(name.rsplit("u", 1)[1])
        return ServeWorkload(name, users, seed,
                             describe=(f"continuous batching: {users} users x 256-token shared "
                                       f"prompt, 20 generated tokens each, token budget 256, "
                                       f"8000-page pool, Llama-2-110M-shaped Q8_0 model "
                                       f"(synthetic), reference Q8 semantics"))
    if name.startswith("model-7b-decode-b"):
        B = int(name.rsplit("b", 1)[1])
        return ModelDecodeWorkload(name, (4096, 11008, 32, 32, 32, 32000, 4096), B, 1024, seed,
                                   describe=(f"one decode step of a Llama-2-7B-shaped model (dim 4096, "
                                             f"hidden 11008, 32 layers, 32 heads x 128, vocab 32000, "
                                             f"Q8_0 weights, synthetic), B={B} sequences at context 1024, "
                                             f"full-row Q8 products"))
    if name == "q8-gemv-7b-ffn":
        return Q8Workload(name, 4096, 11008, 1, seed,
                          describe=("Q8_0 matrix-vector product at the Llama-2-7B FFN up "
                                    "projection, W 11008 x 4096 (50.7 MB BlockQ8), one activation "
                                    "row, Infinity Cache flushed per launch"))
    if name == "q8-matmul-110m-b32":
        return Q8Workload(name, 768, 2048, 32, seed,
                          describe=("Q8_0 matrix product at the Llama-2-110M FFN up projection, "
                                    "W 2048 x 768 (1.77 MB BlockQ8), 32 activation rows, "
                                    "Infinity Cache flushed per launch"))
    raise ValueError(name)


# rocprofv3 summaries (under profiles/) whose traffic_bytes_per_launch line holds the
# HBM bytes per launch of the workload's dominant kernel
TRAFFIC_PROFILES = {
    "decode-b64-ctx4096": "paged_attn_decode_b64_ctx4096_32x128.md",
    "decode-single-110m": "paged_attn_decode_single_ctx256_12x64.md",
    "decode-single-110m-flushed": "paged_attn_decode_single_ctx256_12x64.md",
    "decode-b32-mixed": "paged_attn_decode_b32_mixed_12x64.md",
    "decode-prefix-shared": "paged_attn_decode_prefix_shared_b48_12x64.md",
    "decode-long-131072-32x128": "paged_attn_decode_long_131072_32x128.md",
    "prefill-b8-12x64": "paged_attn_prefill_b8_12x64.md",
    "prefill-chunks-b8-256-12x64": "paged_attn_prefill_chunks_b8_256_12x64.md",
    "prefill-long-16384-32x128": "paged_attn_prefill_long_16384_32x128.md",
    "model-7b-decode-b1": "model_7b_decode_b1.md",
}

WORKLOADS = ["decode-b64-ctx4096", "decode-single-110m", "decode-single-110m-flushed", "decode-b32-mixed",
             "decode-prefix-shared", "decode-long-131072-32x128", "prefill-b8-12x64", "prefill-chunks-b8-256-12x64",
             "prefill-long-16384-32x128", "q8-gemv-7b-ffn", "q8-matmul-110m-b32",
             "model-110m-decode-b32", "model-7b-decode-b1", "model-7b-decode-b2", "model-7b-decode-b8", "serve-110m-u1", "serve-110m-u4", "serve-110m-u8",
             "serve-110m-u16", "serve-110m-u32"]


def kernel_name(w) -> str:
    if hasattr(w, "kernel"):
        return w.kernel()
    if w.bound == "hbm":
        # <head_dim, query heads per workgroup, non-temporal K/V loads>: the
        # library streams K/V unless pages are shared or a KV head has several
        # workgroups; every workload here is MHA (one query head per workgroup).
        kv_mul = w.H // w.Hkv
        qh = 1
        while qh * 2 <= (8 if w.hd <= 64 else 4 if w.hd == 128 else 2) and kv_mul % (qh * 2) == 0:
            qh *= 2
        if w.shared_pages and qh == 1:
            # shared prefixes: member items first in the list, the own rows
            # streamed (its pages are read once each)
            return (f"paged_attn_decode_kernel<{w.hd}, 1, true, true, true> "
                    "(append fused; shared prefixes read once per member set)")
        stream = qh == kv_mul and not w.shared_pages
        return f"paged_attn_decode_kernel<{w.hd}, {qh}, {str(stream).lower()}, true, false> (append fused)"
    kern = os.environ.get("NITRO_PREFILL_KERNEL")
    if w.hd == 256 or kern == "valu":
        return f"paged_attn_prefill_kernel<{w.hd}> (VALU)"
    if kern == "mfma32":
        return f"paged_attn_prefill_mfma_kernel<{w.hd}> (fp32 matrix cores)"
    append = os.environ.get("NITRO_PREFILL_APPEND", "1") != "0"
    cached = bool((w.starts > 0).any())
    return (f"paged_attn_prefill_x3_kernel<{w.hd}> (bf16 matrix cores, three-part splits"
            + ((", KV scatter inside the launch" + (", cached keys from the pool)" if cached else ")"))
               if append else "; the scatter as a launch of its own)"))


def host_cpu():
    """The host's CPU model, sockets and logical CPUs as lscpu reports them
    (/proc/cpuinfo where lscpu is missing), and whether it runs AVX-512."""
    from oracle import attn

    info = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for ln in out.splitlines():
            key, _, val = ln.partition(":")
            info[key.strip()] = val.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    model, sockets = info.get("Model name"), info.get("Socket(s)")
    if model is None:
        ids = set()
        try:
            with open("/proc/cpuinfo") as f:
                for ln in f:
                    key, _, val = ln.partition(":")
                    if key.strip() == "model name" and model is None:
                        model = val.strip()
                    elif key.strip() == "physical id":
                        ids.add(val.strip())
        except OSError:
            pass
        sockets = len(ids) or None
    # a guest may see only a generic model name: family, model and cache
    # sizes identify the part
    ident = {k.lower().replace(" ", "_").replace("(s)", "s"): info[k]
             for k in ("CPU family", "Model", "Stepping", "Thread(s) per core", "L2 cache", "L3 cache")
             if k in info}
    return {"cpu_model": model, "sockets": int(sockets) if sockets and str(sockets).isdigit() else sockets,
            "logical_cpus": os.cpu_count(), "avx512": attn.host_has_avx512(),
            "omp_proc_bind": os.environ.get("OMP_PROC_BIND"), **ident}


def spin_cycles(torch, ms: float) -> int:
    """Cycles of torch.cuda._sleep's spin kernel that take about `ms` milliseconds."""
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    cycles = 1 << 20
    a.record()
    torch.cuda._sleep(cycles)
    b.record()
    b.synchronize()
    return int(cycles * ms / max(a.elapsed_time(b), 1e-3))


def capture_step(torch, w):
    """One HIP graph holding the launches of w.graph_reps steps (captured after
    the warm-up, so every buffer the launches use is already allocated)."""
    torch.cuda.synchronize()
    w.step(torch.cuda.current_stream())
    torch.cuda.synchronize()
    w.eager_out = w.out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(getattr(w, "graph_reps", 1)):
            w.step(torch.cuda.current_stream())
    torch.cuda.synchronize()
    return graph


# Configurations of the benchmark's headline metric the default run measures
# beside it, in the order they are listed for it: single-sequence decode,
# batched mixed-length decode, causal prefill, prefix-shared decode (the
# headline itself is the fifth, B=64 at ctx 4096).
CONFIG_WORKLOADS = ["decode-single-110m", "decode-b32-mixed", "prefill-b8-12x64", "decode-prefix-shared"]


# Untimed GPU work before each timed pass of a HIP graph.  The GPU's clocks
# drop while it idles (the host's checks between passes, the one-wave spin
# kernel that lets the host enqueue the replays) and take about 20 ms of
# sustained work to come back: in a kernel trace of 1200 launches of the
# 8-prompt prefill, each pass began at about 55 us per launch and settled at
# 44-45 us.  A pass of short launches (240 launches of ~46 us are 11 ms) would
# otherwise time that ramp rather than the kernel.
WARM_MS = 30.0


def measure(torch, w, dev, g, steps, warmup):
    """Sets the workload up, runs `warmup` untimed steps, then the timed ones.

    Three forms, by workload:
      graph  a step's launches captured as one HIP graph (many short launches):
             a first pass of `steps` replays sizes the warm-up, w.warm_replays
             = enough replays for WARM_MS of GPU work; then that many untimed
             replays and `steps` replays back to back under the wall clock
             (ms_per_step), each checked bit for bit against the eager step;
             then, behind a spin kernel that lets the host enqueue every replay
             first, the warm replays again and another `steps` replays between
             one pair of HIP events on the launch stream: kernel_ms = that time
             / (steps * launches per step)
      flush  a cache flush before every launch, and an event pair around each
             launch (only the launches are timed)
      eager  `steps` steps back to back under the wall clock, then `steps` more
             behind a spin kernel with an event pair around every launch
             (kernel_ms = their mean)
    Returns (ms_per_step, kernel_ms, form)."""
    w.setup(dev, g)
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        w.step(stream)
    torch.cuda.synchronize()
    nl = w.launches_per_step()
    if getattr(w, "graph", False) and not w.flush:
        graph = capture_step(torch, w)
        reps = getattr(w, "graph_reps", 1)
        t0 = time.perf_counter()
        for _ in range(steps):
            graph.replay()
        torch.cuda.synchronize()
        per_replay_ms = (time.perf_counter() - t0) / steps * 1e3
        warm = int(min(4000, max(warmup, np.ceil(WARM_MS / max(per_replay_ms, 1e-3)))))
        w.warm_replays = warm
        for _ in range(warm):
            graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            graph.replay()
        torch.cuda.synchronize()
        ms_per_step = (time.perf_counter() - t0) / (steps * reps) * 1e3
        w.check_graph_replay()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(spin_cycles(torch, 5.0 + 0.05 * (warm + steps)))
        for _ in range(warm):
            graph.replay()
        a.record(stream)
        for _ in range(steps):
            graph.replay()
        b.record(stream)
        torch.cuda.synchronize()
        w.check_graph_replay()
        del graph
        return ms_per_step, a.elapsed_time(b) / (steps * reps * nl), "graph"
    events = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(nl)] for _ in range(steps)]
    if w.flush:
        # the flushes between launches are not part of the step: only the
        # launches, each between its own pair of events, are timed
        for i in range(steps):
            w.step(stream, events[i])
        torch.cuda.synchronize()
        kernel_ms = float(np.mean([a.elapsed_time(b) for ev in events for a, b in ev]))
        return kernel_ms * nl, kernel_ms, "flush"
    if not getattr(w, "event_pass", True):
        # a step that is a whole serving run: its events bracket the run
        t0 = time.perf_counter()
        for i in range(steps):
            w.step(stream, events[i])
        torch.cuda.synchronize()
        ms_per_step = (time.perf_counter() - t0) / steps * 1e3
        return ms_per_step, float(np.mean([a.elapsed_time(b) for ev in events for a, b in ev])), "run"
    t0 = time.perf_counter()
    for _ in range(steps):
        w.step(stream)
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) / steps * 1e3
    spin = spin_cycles(torch, 1.0)
    for i in range(steps):
        torch.cuda._sleep(spin)
        w.step(stream, events[i])
    torch.cuda.synchronize()
    return ms_per_step, float(np.mean([a.elapsed_time(b) for ev in events for a, b in ev])), "eager"


TIMING = {
    "graph": "one HIP graph of {reps} step(s) of {nl} launch(es); kernel_ms = the time of {steps} "
             "back-to-back replays between one event pair on the launch stream / ({steps} x {reps} x {nl} "
             "launches), after {warm} untimed replays (about 30 ms of GPU work, so the clocks are at their "
             "steady state)",
    "flush": "an event pair around each launch, a 1 GiB read before it (not timed)",
    "run": "an event pair around each run",
    "eager": "an event pair around each launch, the launches queued behind a spin kernel",
}


def rates(w, ms_per_step, kernel_ms):
    """(unit, peak, step rate, kernel rate, algorithmic work per launch for the roofline)."""
    work = w.work_per_launch()
    hbm_work = w.hbm_bytes_per_launch() if hasattr(w, "hbm_bytes_per_launch") else work
    if w.bound == "hbm":
        unit, scale, peak = "GB/s", 1e9, HBM_PEAK_GBPS
    else:
        unit, scale, peak = "TFLOP/s", 1e12, FP32_PEAK_TFLOPS
    step_rate = work * w.launches_per_step() / (ms_per_step * 1e-3) / scale
    kernel_rate = hbm_work / (kernel_ms * 1e-3) / scale
    return unit, peak, step_rate, kernel_rate, hbm_work


def config_entry(torch, name, dev, args):
    """One configuration's numbers, measured in this process (no CPU baseline)."""
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed)
    w = make_workload(name, args.seed)
    ms_per_step, kernel_ms, form = measure(torch, w, dev, g, args.steps, args.warmup)
    w.check()
    assert w.pool.take_device_errors() == 0, f"{name}: a kernel saw a page id outside the pool"
    parity = w.verify()
    unit, peak, step_rate, kernel_rate, hbm_work = rates(w, ms_per_step, kernel_ms)
    nl = w.launches_per_step()
    entry = {
        "workload": w.describe,
        "kernel": kernel_name(w),
        "kernel_ms": round(kernel_ms, 5),
        "launches_per_step": nl,
        "ms_per_step": round(ms_per_step, 4),
        ("bytes_per_launch" if w.bound == "hbm" else "flops_per_launch"): hbm_work,
        "achieved": round(kernel_rate, 2 if unit == "GB/s" else 4),
        "peak": peak,
        "unit": unit,
        "frac": round(kernel_rate / peak, 4),
        "traffic": (measured_traffic(os.path.join(ROOT, "profiles", TRAFFIC_PROFILES[name]))
                    if name in TRAFFIC_PROFILES else None),
        "step_rate": round(step_rate, 2 if unit == "GB/s" else 4),
        "tokens_per_s": round(w.tokens_per_step() / (ms_per_step * 1e-3), 1),
        "timing": TIMING[form].format(steps=args.steps, nl=nl, reps=getattr(w, "graph_reps", 1),
                                      warm=getattr(w, "warm_replays", 0)),
        "parity": parity,
    }
    entry.update(w.extra(kernel_ms * 1e-3))
    w.release()
    del w
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return entry


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default=DEFAULT_WORKLOAD, choices=WORKLOADS)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cpu-sample", type=int, default=8,
                    help="sequences (prompts) of the workload the CPU baseline runs")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="default workload only: leave out the other four configurations")
    ap.add_argument("--seed", type=int, default=0x4E49545205)
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="also run a plain device-to-device copy of this many MiB three times "
                         "(the known-size kernel that scales rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--traffic-profile", default=None,
                    help="rocprofv3 summary holding the measured HBM traffic per launch "
                         "(default: the workload's summary under profiles/)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only (the paged-attention path shards by sequence or "
              "by head with no exchange between GPUs)",
              file=sys.stderr)
        sys.exit(2)

    from oracle import attn

    # the oracle build this process loads (first use below): the one the CPU
    # baseline times, which also checks the outputs after the timed steps
    build = None if args.no_cpu_baseline else attn.use_timing_build()

    import torch

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed)
    w = make_workload(args.workload, args.seed)

    if args.copy_calibration_mib:
        src = torch.randn(args.copy_calibration_mib * 2**18, device=dev, generator=g)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    ms_per_step, kernel_ms, form = measure(torch, w, dev, g, args.steps, args.warmup)
    w.check()
    assert (w.device_errors() if hasattr(w, "device_errors") else w.pool.take_device_errors()) == 0
    default = args.workload == DEFAULT_WORKLOAD
    try:
        # the headline: two sequences (the first and the last) through the oracle
        parity = (w.verify(sample=[0, w.B - 1]) if default else w.verify()) if hasattr(w, "verify") else None
    except ParityError as e:
        print(f"bench.py: parity check failed after the timed steps: {e}", file=sys.stderr, flush=True)
        sys.exit(3)

    nl = w.launches_per_step()
    unit, peak, step_rate, kernel_rate, hbm_work = rates(w, ms_per_step, kernel_ms)
    traffic_profile = args.traffic_profile or (
        os.path.join(ROOT, "profiles", TRAFFIC_PROFILES[args.workload])
        if args.workload in TRAFFIC_PROFILES else None)
    line = {
        "metric": METRIC if default else f"{args.workload} {unit}",
        "value": round(step_rate, 2 if unit == "GB/s" else 4),
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": (w.config() if hasattr(w, "config") else
                   {"workload": w.describe, "batch": w.B, "n_heads": w.H, "n_kv_heads": w.Hkv,
                    "head_dim": w.hd, "pool_pages": w.pages, "parallelism": "single GPU"}),
        "tokens_per_s": round(w.tokens_per_step() / (ms_per_step * 1e-3), 1),
        "roofline": {
            "bound": w.bound,
            "kernel": kernel_name(w),
            "achieved": round(kernel_rate, 2 if unit == "GB/s" else 4),
            "peak": peak,
            "unit": unit,
            "frac": round(kernel_rate / peak, 4),
            "traffic": measured_traffic(traffic_profile) if traffic_profile else None,
            ("bytes_per_launch" if w.bound == "hbm" else "flops_per_launch"): hbm_work,
            "kernel_ms": round(kernel_ms, 5),
            "timing": TIMING[form].format(steps=args.steps, nl=nl, reps=getattr(w, "graph_reps", 1),
                                          warm=getattr(w, "warm_replays", 0)),
        },
        "parity": parity,
        "cpu_baseline": None,
    }
    if hasattr(w, "headline"):
        line.update(w.headline(ms_per_step))
    line.update(w.extra(kernel_ms * 1e-3))
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = w.cpu_baseline(args.cpu_seconds, args.cpu_sample)
        if line["cpu_baseline"]:
            line["cpu_baseline"]["host"] = host_cpu()
            if line["cpu_baseline"].get("kind") == "port":
                line["cpu_baseline"]["build"] = build
            line["cpu_baseline"]["timing"] = "2 warm-up runs, then the median of >= 5 timed runs"
    if default and not args.no_configs:
        if hasattr(w, "release"):
            w.release()
        del w
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        configs = {}
        try:
            for i, name in enumerate(CONFIG_WORKLOADS):
                print(f"bench.py: config {i + 1}: {name}", file=sys.stderr, flush=True)
                configs[name] = {"config": i + 1, **config_entry(torch, name, dev, args)}
        except ParityError as e:
            print(f"bench.py: parity check failed after the timed steps: {e}", file=sys.stderr, flush=True)
            sys.exit(3)
        line["configs"] = configs
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
