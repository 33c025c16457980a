"""Benchmark of the MI355X paged-attention decode path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload decode-b64-ctx4096]

Workload (one GPU): batched paged-attention decode at the Llama-2-7B attention
shape — B=64 sequences, 32 query heads = 32 KV heads, head_dim 128, context
4096 tokens each (256 pages of 16 tokens), fp32 K/V ~ N(0,1) in a 20,000-page
pool with block tables drawn from one seeded permutation of the pool, one
layer.  A step is what forward_decode_batch does per layer for attention
(src/model_q8.cpp:616-662): append this step's K/V row of every sequence at
its position, then attend over positions 0..4095.  Inputs are resident in HBM
before timing starts.

Reported:
  value / unit      algorithmic GB/s of the whole step (append + decode)
  roofline          the decode kernel alone: algorithmic bytes per launch /
                    mean launch time from HIP events on the launch stream,
                    against MI355X's 8 TB/s HBM peak
  cpu_baseline      the CPU oracle (C restatement of the reference's OpenMP
                    loops, all host cores) on a sample of the same workload
Algorithmic bytes per decode launch: sum_b ctx_b*Hkv*hd*4*2 (K and V) +
B*H*hd*4*2 (q in, out) + sum_b ceil(ctx_b/16)*4 (block-table entries).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
METRIC = "paged-attn decode GB/s (% HBM peak) + tokens/s at B=64 ctx4096"

WORKLOADS = {
    # name: (B, ctx, H, Hkv, hd, pool pages, layers)
    "decode-b64-ctx4096": (64, 4096, 32, 32, 128, 20000, 1),
}


def decode_bytes(ctx: np.ndarray, B: int, H: int, Hkv: int, hd: int) -> int:
    ctx = np.asarray(ctx, dtype=np.int64)
    return int((ctx * Hkv * hd * 4 * 2).sum() + B * H * hd * 4 * 2 + ((ctx + 15) // 16 * 4).sum())


def seeded_tables(B: int, ctx: int, pages: int, seed: int) -> np.ndarray:
    perm = np.random.default_rng(seed).permutation(pages).astype(np.int32)
    n = (ctx + 15) // 16
    assert B * n <= pages
    return perm[: B * n].reshape(B, n).copy()


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


def cpu_baseline(k, v, tables, positions, q, knew, vnew, H, Hkv, hd, seconds=10.0,
                 sample=8):
    """Times the CPU oracle (append + batched decode, all host cores) on the
    first `sample` sequences, their pages copied to a compact host pool."""
    import torch

    from oracle import attn

    n_pages = tables.shape[1]
    sel = tables[:sample]
    idx = torch.from_numpy(sel.reshape(-1).astype(np.int64)).to(k.device)
    kh = k.index_select(0, idx).cpu().numpy()
    vh = v.index_select(0, idx).cpu().numpy()
    local = np.arange(sample * n_pages, dtype=np.int32).reshape(sample, n_pages)
    qh = q[:sample].cpu().numpy()
    kn = knew[:sample].cpu().numpy()
    vn = vnew[:sample].cpu().numpy()
    pos = positions[:sample]
    threads = attn.max_threads()
    attn.kv_append_decode(kh, vh, 0, kn, vn, local, pos)
    attn.decode_batch(kh, vh, 0, qh, local, pos, H, Hkv, hd, threads)  # warm-up
    reps, t0 = 0, time.perf_counter()
    while True:
        attn.kv_append_decode(kh, vh, 0, kn, vn, local, pos)
        attn.decode_batch(kh, vh, 0, qh, local, pos, H, Hkv, hd, threads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    per_rep = el / reps
    b = decode_bytes(pos + 1, sample, H, Hkv, hd)
    return {
        "value": round(b / per_rep / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{sample} of the {len(positions)} sequences (same shape, ctx {int(pos[0]) + 1}, "
                   f"{H}x{hd}), append + batched decode, {reps} reps in {el:.1f} s; "
                   f"{sample / per_rep:.1f} tokens/s"),
        "tokens_per_s": round(sample / per_rep, 3),
        "ms_per_rep": round(per_rep * 1e3, 3),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="decode-b64-ctx4096", choices=sorted(WORKLOADS))
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--seed", type=int, default=0x4E49545205)
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="also run a plain device-to-device copy of this many MiB three times "
                         "(the known-size kernel that scales rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--traffic-profile",
                    default=os.path.join(ROOT, "profiles", "paged_attn_decode_b64_ctx4096_32x128.md"),
                    help="rocprofv3 summary holding the measured HBM traffic per decode launch")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the paged-attention path shards by sequence or "
              "by head with no exchange, and multi-GPU runs are not part of this build",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import nitrorag_amd as na

    B, ctx, H, Hkv, hd, pages, layers = WORKLOADS[args.workload]
    kv_dim = Hkv * hd
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed)
    k = torch.randn((pages, layers, 16, kv_dim), device=dev, generator=g)
    v = torch.randn((pages, layers, 16, kv_dim), device=dev, generator=g)
    q = torch.randn((B, H * hd), device=dev, generator=g)
    knew = torch.randn((B, kv_dim), device=dev, generator=g)
    vnew = torch.randn((B, kv_dim), device=dev, generator=g)
    out = torch.empty_like(q)
    tables = seeded_tables(B, ctx, pages, args.seed)
    positions = np.full(B, ctx - 1, np.int32)

    if args.copy_calibration_mib:
        src = torch.randn(args.copy_calibration_mib * 2**18, device=dev, generator=g)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    stream = torch.cuda.current_stream()
    pool = na.KVPool.wrap(k, v)
    pool.upload_decode_batch(tables, positions, stream)

    def step(ev=None):
        pool.kv_append(0, knew, vnew, stream)
        if ev is not None:
            ev[0].record(stream)
        pool.decode(0, q, out, H, Hkv, hd, stream)
        if ev is not None:
            ev[1].record(stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(events[i])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    kernel_ms = float(np.mean([a.elapsed_time(b) for a, b in events]))
    assert torch.isfinite(out).all().item(), "non-finite decode output"
    assert pool.take_device_errors() == 0

    ms_per_step = elapsed / args.steps * 1e3
    nbytes = decode_bytes(positions + 1, B, H, Hkv, hd)
    step_gbps = nbytes / (ms_per_step * 1e-3) / 1e9
    kernel_gbps = nbytes / (kernel_ms * 1e-3) / 1e9

    line = {
        "metric": METRIC,
        "value": round(step_gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": (f"paged-attention decode, B={B}, ctx={ctx}, {H} heads x {hd} "
                         f"(kv heads {Hkv}), {pages}-page pool, 16-token pages, one layer, "
                         "append + attend per step"),
            "batch": B, "context": ctx, "n_heads": H, "n_kv_heads": Hkv, "head_dim": hd,
            "pool_pages": pages, "parallelism": "single GPU",
        },
        "tokens_per_s": round(B / (ms_per_step * 1e-3), 1),
        "hbm_fraction_step": round(step_gbps / HBM_PEAK_GBPS, 4),
        "roofline": {
            "bound": "hbm",
            "kernel": "paged_attn_decode_kernel<128>",
            "achieved": round(kernel_gbps, 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(kernel_gbps / HBM_PEAK_GBPS, 4),
            "traffic": measured_traffic(args.traffic_profile),
            "bytes_per_launch": nbytes,
            "kernel_ms": round(kernel_ms, 4),
        },
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(k, v, tables, positions, q, knew, vnew, H, Hkv, hd,
                                            seconds=args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
