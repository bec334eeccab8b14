"""Shared pieces of the benchmark scripts: impls, timers, arguments, CSV output."""
import argparse
import csv
import os
import time

import numpy as np
import torch

from streamtopk_sae.ops import topk_sae_cpu, topk_sae_cuda_approx, topk_sae_cuda_exact


def baseline_eager(X, W_enc, b_enc, k):
    """The dense path (reference: streamtopk_sae/baselines.py:13-17): matmul in
    the input dtype (hipBLASLt), the fp32 bias added, fp32 top-k.  It
    materialises the (B, F) score matrix."""
    preacts = (X @ W_enc.T + b_enc).float()
    values, indices = torch.topk(preacts, k, dim=-1)
    return values, indices.to(torch.int32)


def gaussian_inputs(B, d, F, dtype, seed=0, device="cuda"):
    """The reference harness's gaussian inputs (streamtopk_sae/utils.py:50-54,
    its STREAMTOPK_DATA=gaussian branch): X and W_enc drawn N(0, 1) directly in
    `dtype` from one seeded CPU generator (W_enc rows not normalised), b_enc
    zero."""
    rng = torch.Generator()
    rng.manual_seed(seed)
    X = torch.randn(B, d, dtype=dtype, generator=rng)
    W = torch.randn(F, d, dtype=dtype, generator=rng)
    b = torch.zeros(F, dtype=torch.float32)
    return X.to(device), W.to(device), b.to(device)


# impl name -> fn(X, W, b, k); cuda_approx uses c = max(16, k) as the reference does
IMPL_FNS = {
    "eager": baseline_eager,
    "cpu": topk_sae_cpu,
    "cuda_exact": topk_sae_cuda_exact,
    "cuda_approx": lambda X, W, b, k: topk_sae_cuda_approx(X, W, b, k, max(16, k)),
}


def time_gpu(fn, X, W, b, k, warmup, iters):
    """Per-iteration times in microseconds: a HIP event pair on torch's current
    stream around each call (the ops launch on that stream)."""
    for _ in range(warmup):
        fn(X, W, b, k)
    torch.cuda.synchronize()
    times = []
    for _ in range(iters):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        fn(X, W, b, k)
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) * 1000.0)
    return times


def time_cpu(fn, X, W, b, k, warmup, iters):
    """Per-iteration wall times in microseconds (time.perf_counter)."""
    for _ in range(warmup):
        fn(X, W, b, k)
    times = []
    for _ in range(iters):
        t0 = time.perf_counter()
        fn(X, W, b, k)
        times.append((time.perf_counter() - t0) * 1e6)
    return times


def stats_us(times):
    return {
        "median_us": float(np.median(times)),
        "p10_us": float(np.percentile(times, 10)),
        "p90_us": float(np.percentile(times, 90)),
        "min_us": float(np.min(times)),
        "max_us": float(np.max(times)),
    }


def parse_ints(s):
    return [int(x) for x in s.split(",")]


def parse_strs(s):
    return [x.strip() for x in s.split(",")]


def add_grid_filters(parser):
    parser.add_argument("--B", type=parse_ints, default=None, metavar="B,...")
    parser.add_argument("--d", type=parse_ints, default=None, metavar="d,...")
    parser.add_argument("--F", type=parse_ints, default=None, metavar="F,...")
    parser.add_argument("--k", type=parse_ints, default=None, metavar="k,...")
    parser.add_argument("--dtype", type=parse_strs, default=None, metavar="dtype,...")


def new_parser(doc, out):
    parser = argparse.ArgumentParser(description=doc)
    parser.add_argument("--out", default=out)
    parser.add_argument("--dry-run", action="store_true", help="one cell per impl; nothing is written")
    return parser


def error_status(exc):
    """The status column for a failed cell (reference: "OOM" or "ERR:<message>")."""
    if isinstance(exc, torch.cuda.OutOfMemoryError):
        return "OOM"
    return f"ERR:{exc}"


def write_csv(path, fieldnames, rows):
    os.makedirs(os.path.dirname(path) or ".", exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=fieldnames, extrasaction="ignore")
        w.writeheader()
        w.writerows(rows)
    print(f"\nWrote {len(rows)} rows to {path}")


def finish(args, fieldnames, rows):
    if args.dry_run:
        print(f"\nDry-run complete ({len(rows)} row(s)) -- results NOT written to disk")
        return
    write_csv(args.out, fieldnames, rows)


def free_cache():
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
