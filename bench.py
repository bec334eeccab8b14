#!/usr/bin/env python3
"""Benchmark of the streaming fused top-k SAE encoder on one MI355X.

Default workload (the headline): exact encode, bf16 X and
W_enc, fp32 b_enc, B=128, d=2048, F=262144, k=64.  One step = one call of
topk_sae_cuda_exact over the resident batch.  Prints ONE JSON line.

  python bench.py [--steps K] [--warmup W] [--workload NAME] [--no-cpu]

Workloads: c2_bf16 (default), c2_fp16, c2_fp32, c1_bf16, c3_approx_c{16,32,64,128},
c3_cand_c{16,32,64,128} (the approximate op with its candidate buffer),
c4_bf16, c4_bf16_heavy.  Only --gpus 1 is supported (one GPU per box).
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "streamtopk-sae_amd")
for _p in (PKG_DIR, ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, 8 TB/s
MFMA_PEAK_TFLOPS = {"bf16": 2500.0, "fp16": 2500.0, "fp32": 157.3}
METRIC = "rows/s + % of HBM-or-MFMA roofline, bf16 exact B=128 d=2048 F=262144 k=64"

WORKLOADS = {
    "c1_bf16": dict(B=128, d=768, F=65536, k=32, dtype="bf16", op="exact", label="BASELINE config 1"),
    "c2_bf16": dict(B=128, d=2048, F=262144, k=64, dtype="bf16", op="exact", label="BASELINE config 2 (headline)"),
    "c2_fp16": dict(B=128, d=2048, F=262144, k=64, dtype="fp16", op="exact", label="BASELINE config 2, fp16"),
    "c2_fp32": dict(B=128, d=2048, F=262144, k=64, dtype="fp32", op="exact", label="BASELINE config 2, fp32"),
    "c4_bf16": dict(B=1024, d=4096, F=262144, k=128, dtype="bf16", op="exact", label="BASELINE config 4"),
    "c4_bf16_heavy": dict(B=1024, d=4096, F=262144, k=128, dtype="bf16", op="exact", heavy=True,
                          label="BASELINE config 4, heavy-tailed W_enc"),
}
for _c in (16, 32, 64, 128):
    # the approximate op requires k <= c (streamtopk_approx.cu:248): c=16 runs at k=16
    WORKLOADS[f"c3_approx_c{_c}"] = dict(B=128, d=2048, F=1048576, k=min(32, _c), c=_c, dtype="bf16",
                                         op="approx", label=f"BASELINE config 3, c={_c}, k={min(32, _c)}")
    # the same with the per-group candidate buffer requested (group_kernel + cand_kernel)
    WORKLOADS[f"c3_cand_c{_c}"] = dict(B=128, d=2048, F=1048576, k=min(32, _c), c=_c, dtype="bf16",
                                       op="approx_cand",
                                       label=f"BASELINE config 3, c={_c}, k={min(32, _c)}, candidate buffer")


def _cpu_cores():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_baseline(X, W, b, k, seconds):
    """Times the oracle's restatement of the reference CPU kernel (OpenMP over
    rows, each row streaming all of W) over whole passes of the same batch,
    repeated until about `seconds` of CPU work has been done."""
    import numpy as np
    import oracle
    cores = _cpu_cores()
    Xf = np.ascontiguousarray(X.float().cpu().numpy())
    Wf = np.ascontiguousarray(W.float().cpu().numpy())
    bf = np.ascontiguousarray(b.float().cpu().numpy())
    passes, rows, t = 0, 0, 0.0
    while t < seconds:
        t0 = time.perf_counter()
        oracle.cpu_stream(Xf, Wf, bf, k, nthreads=cores)
        t += time.perf_counter() - t0
        passes += 1
        rows += Xf.shape[0]
    return {"value": rows / t, "unit": "rows/s", "cores": cores, "kind": "port",
            "sample": f"{passes} passes over the same {Xf.shape[0]}-row batch (full F and d, fp32 upcast "
                      f"inputs), {t:.1f} s; oracle/stk_oracle_cpu.c, the reference streamtopk_cpu.cpp restated"}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_c0_baseline():
    """BASELINE config 0 (fp32 B=32 d=768 F=16384 k=32) on the product's own
    OpenMP CPU encoder (stk_cpu_forward, the topk_sae_cpu path): 1 warmup call,
    then the median of 5, on one thread (the reference CPU kernel is serial)
    and on all of this process's cores."""
    import ctypes
    import statistics
    import torch
    from streamtopk_sae import _lib, make_inputs
    lib = _lib.load()
    B, d, F, k = 32, 768, 16384, 32
    X, W, b = make_inputs(B, d, F, dtype=torch.float32, seed=0, device="cpu")
    V = torch.empty(B, k, dtype=torch.float32)
    I = torch.empty(B, k, dtype=torch.int32)
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())
    res = {}
    for nt in sorted({1, _cpu_cores()}):
        times = []
        for it in range(6):
            t0 = time.perf_counter()
            _lib.check(lib.stk_cpu_forward(ptr(X), ptr(W), ptr(b), ptr(V), ptr(I), B, d, F, k, nt))
            if it:
                times.append(time.perf_counter() - t0)
        res[str(nt)] = round(1e3 * statistics.median(times), 3)
    return {"config": "c0: fp32 B=32 d=768 F=16384 k=32", "op": "topk_sae_cpu (stk_cpu_forward)",
            "median_ms_by_threads": res,
            "rows_per_s_by_threads": {n: round(B / (ms * 1e-3), 1) for n, ms in res.items()},
            "cpu_model": _cpu_model()}


def copy_calibration(nbytes, steps):
    """Plain elementwise copy of `nbytes` fp32 bytes (torch's vectorised
    elementwise kernel: reads nbytes, writes nbytes), timed with HIP events.
    Run under `rocprofv3 --pmc FETCH_SIZE` / `WRITE_SIZE` it gives the factor
    that turns those counters into HBM bytes on this part."""
    import torch
    dev = torch.device("cuda:0")
    n = nbytes // 4
    src = torch.randn(n, device=dev)
    dst = torch.empty_like(src)
    for _ in range(2):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        torch.mul(src, 1.0, out=dst)
    e1.record()
    torch.cuda.synchronize()
    us = 1e3 * e0.elapsed_time(e1) / steps
    print(json.dumps({"copy_calibration": {"read_bytes": 4 * n, "write_bytes": 4 * n, "avg_us": round(us, 2),
                                           "GBps_rw": round(8 * n / (us * 1e-6) / 1e9, 1)}}), flush=True)


def traffic_from_profile(kernel, workload):
    """HBM bytes per launch of the streaming kernel, as recorded by the
    calibrated PMC summary profiles/<kernel>_<workload>_hbm_traffic.md (a line
    `traffic_bytes_per_launch: N`), or None when no such summary exists."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_{workload}_hbm_traffic.md")
    try:
        with open(path) as fh:
            for line in fh:
                line = line.strip().strip("`")
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip())
    except OSError:
        return None
    return None


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--workload", default="c2_bf16", choices=sorted(WORKLOADS))
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--settle", type=float, default=0.5, metavar="SECONDS",
                    help="untimed calls of the step for this long before the warmup steps")
    ap.add_argument("--copy-calib", type=int, default=0, metavar="BYTES",
                    help="only run the PMC calibration copy of BYTES bytes, --steps times")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}, WORLD_SIZE {world}); "
              "the encoder would shard F across GPUs with one small all-gather of (B, k) candidates, "
              "which is not built here.", file=sys.stderr)
        sys.exit(2)

    if args.copy_calib:
        copy_calibration(args.copy_calib, args.steps)
        return

    import torch
    from streamtopk_sae import _lib, make_inputs, topk_sae_cuda_approx, topk_sae_cuda_exact

    wl = WORKLOADS[args.workload]
    B, d, F, k, dtn = wl["B"], wl["d"], wl["F"], wl["k"], wl["dtype"]
    dtype = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[dtn]
    es = 4 if dtn == "fp32" else 2
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    X, W, b = make_inputs(B, d, F, dtype, seed=args.seed, device=dev, heavy_tail=wl.get("heavy", False))
    # A W smaller than ~3x the 256 MiB MALL (config 1: 96 MiB) would be served
    # from the MALL on every step after the first: successive steps rotate over
    # copies of W (same values) totalling at least 768 MiB, so that each step
    # streams its W from HBM.
    w_bytes_all = W.numel() * W.element_size()
    n_copies = max(1, -(-768 * 2**20 // w_bytes_all))
    W_copies = [W] + [W.clone() for _ in range(n_copies - 1)]
    rot = [0]

    def next_w():
        w = W_copies[rot[0] % n_copies]
        rot[0] += 1
        return w
    torch.cuda.synchronize()
    lib = _lib.load()

    if wl["op"] == "exact":
        def step():
            return topk_sae_cuda_exact(X, next_w(), b, k)
        main_name = "main_kernel"
    elif wl["op"] == "approx":
        c = wl["c"]

        def step():
            return topk_sae_cuda_approx(X, next_w(), b, k, c)
        main_name = "main_kernel"
    else:
        c = wl["c"]
        cand = torch.empty((B, (F + 127) // 128, c), dtype=torch.float32, device=dev)

        def step():
            return topk_sae_cuda_approx(X, next_w(), b, k, c, candidate_buffer=cand)
        main_name = "group_kernel"

    # The plain-read ceiling: a read stream over W's bytes, timed with the same
    # in-packet events as the streaming kernel (rotating over the copies too).
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    stream_ptr = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def probe():
        _lib.check(lib.stk_read_probe(ctypes.c_void_p(next_w().data_ptr()), w_bytes_all,
                                      ctypes.c_void_p(sink.data_ptr()), stream_ptr))

    for _ in range(20):
        probe()
    torch.cuda.synchronize()
    _lib.check(lib.stk_profile_enable(1))
    for _ in range(20):
        probe()
    torch.cuda.synchronize()
    probe_rec = ctypes.c_double(0)
    probe_n = ctypes.c_int64(0)
    _lib.check(lib.stk_profile_read(b"read_probe", ctypes.byref(probe_rec), ctypes.byref(probe_n)))
    probe_us = 1e3 * probe_rec.value / probe_n.value
    _lib.check(lib.stk_profile_enable(0))

    # Memory: everything the op allocates from its first call on, the workspace
    # it keeps per stream included, over the resident inputs.
    torch.cuda.synchronize()
    base_mem = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()

    # Device settle: untimed calls of the step for --settle seconds before the
    # W warmup steps.  Short runs that start from another load (or from idle)
    # come out 5-20 % slower on this part until its clocks have adjusted to the
    # workload's sustained power draw; the settle keeps that transient out of
    # the K timed steps however small W is.
    t_settle = time.perf_counter()
    settle_steps = 0
    while time.perf_counter() - t_settle < args.settle:
        for _ in range(10):
            step()
        settle_steps += 10
        torch.cuda.synchronize()
    settle_s = time.perf_counter() - t_settle

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # timed region: the K steps alone, no event in any kernel's packet
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        V, I = step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    peak_extra = torch.cuda.max_memory_allocated() - base_mem

    # kernel-timing pass, right after and as long: the same K steps with a
    # start/stop event pair in the streaming kernel's own dispatch packet
    # (profile mode 2), on the stream it is launched on; its average launch
    # duration is the roofline's.  The pass's own step time shows what the
    # events cost.
    _lib.check(lib.stk_profile_enable(2))
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall_ev = time.perf_counter() - t1

    def read_profile(names):
        out = {}
        for name in names:
            tot = ctypes.c_double(0)
            n = ctypes.c_int64(0)
            _lib.check(lib.stk_profile_read(name.encode(), ctypes.byref(tot), ctypes.byref(n)))
            if n.value:
                out[name] = {"avg_us": 1e3 * tot.value / n.value, "launches": n.value}
        return out

    kern = read_profile((main_name,))
    # untimed breakdown pass: events around every kernel of the pipeline
    _lib.check(lib.stk_profile_enable(1))
    for _ in range(min(args.steps, 50)):
        step()
    torch.cuda.synchronize()
    breakdown = read_profile(("sample_kernel", "thr_kernel", "main_kernel", "merge_kernel", "group_kernel",
                              "cand_kernel"))
    _lib.check(lib.stk_profile_enable(0))

    recall = None
    if wl["op"] != "exact":
        # recall@k of the approximate op (bench/run_recall.py:74-91 measures it
        # against the dense reference), untimed, on this workload's own inputs
        from streamtopk_sae import reference_topk_sae
        from streamtopk_sae.utils import recall_per_row
        _, I_ap = step()
        _, I_ex = topk_sae_cuda_exact(X, W, b, k)
        _, I_dense = reference_topk_sae(X, W, b, k)
        r_ex, r_dense = recall_per_row(I_ap, I_ex), recall_per_row(I_ap, I_dense)
        recall = {"recall_at_k_vs_exact": round(float(r_ex.mean()), 6),
                  "min_row_vs_exact": round(float(r_ex.min()), 6),
                  "recall_at_k_vs_dense_reference": round(float(r_dense.mean()), 6),
                  "min_row_vs_dense_reference": round(float(r_dense.min()), 6),
                  "rows": B, "k": k, "c": wl["c"],
                  "note": "against topk_sae_cuda_exact and against reference_topk_sae (fp32 dense "
                          "scores + torch.topk); the two references may differ on near-tied scores"}
        del I_dense
        torch.cuda.empty_cache()

    ms_per_step = 1e3 * wall / args.steps
    rows_per_s = B * args.steps / wall
    w_bytes = F * d * es
    alg_main = w_bytes + B * d * es + 4 * F                 # W + X + b streamed by main_kernel
    if main_name == "group_kernel":
        alg_main += 8 * B * ((F + 127) // 128) * wl["c"]    # + the candidate values and indices written
    alg_total = alg_main + 8 * B * k                        # + V, I (bench/run_bandwidth.py:73-77)
    flops = 2.0 * B * d * F
    main_us = kern[main_name]["avg_us"]
    bw_main = alg_main / (main_us * 1e-6) / 1e9
    tflops_main = flops / (main_us * 1e-6) / 1e12
    ai = flops / alg_total
    ridge = MFMA_PEAK_TFLOPS[dtn] * 1e12 / (HBM_PEAK_GBS * 1e9)
    if ai < ridge:
        roof = {"bound": "hbm", "achieved": round(bw_main, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(bw_main / HBM_PEAK_GBS, 4)}
    else:
        roof = {"bound": "mfma", "achieved": round(tflops_main, 2), "peak": MFMA_PEAK_TFLOPS[dtn],
                "unit": "TFLOP/s", "frac": round(tflops_main / MFMA_PEAK_TFLOPS[dtn], 4)}
    # batches of 512 rows or more run the large-batch kernel (mainl_kernel);
    # both are timed under the profile name main_kernel
    kname = main_name if main_name != "main_kernel" else "mainl_kernel" if B >= 512 else "main_kernel"
    roof["kernel"] = kname
    roof["traffic"] = traffic_from_profile(kname, args.workload)
    roof["alg_bytes_per_launch"] = alg_main
    roof["avg_launch_us"] = round(main_us, 2)
    roof["timing"] = ("in-packet HIP start/stop events of the streaming kernel on its launch stream, over "
                      "K steps run right after the timed region")
    # measured read ceiling: the W bytes through a plain coalesced read kernel
    stream_gbs = w_bytes_all / (probe_us * 1e-6) / 1e9
    roof["measured_read_stream_GBs"] = round(stream_gbs, 1)
    if roof["bound"] == "hbm":
        roof["frac_of_measured_stream"] = round(bw_main / stream_gbs, 4)

    out = {
        "metric": METRIC if args.workload == "c2_bf16" else f"rows/s, {wl['label']}",
        "value": round(rows_per_s, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "ms_per_step_kernel_timing_pass": round(1e3 * wall_ev / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtn,
        "data": f"synthetic: X~N(0,1), W_enc rows N(0,1/d) then L2-normalised, b_enc~N(0,0.1^2); seed {args.seed}",
        "config": {"workload": f"{args.workload}: {wl['label']}", "op": wl["op"], "B": B, "d": d, "F": F,
                   "k": k, **({"c": wl["c"]} if "c" in wl else {}),
                   **({"W_copies_rotated": n_copies} if n_copies > 1 else {})},
        "roofline": roof,
        "pipeline": {"W_GBps_effective": round(w_bytes / (ms_per_step * 1e-3) / 1e9, 1),
                     "alg_bytes_per_step": alg_total,
                     "hbm_frac_per_step": round(alg_total / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "tflops_per_step": round(flops / (ms_per_step * 1e-3) / 1e12, 2),
                     "kernels_us": {n: round(v["avg_us"], 2) for n, v in breakdown.items()}},
        "device_settle": {"seconds": round(settle_s, 3), "steps": settle_steps,
                          "note": "untimed calls of the step before the warmup steps (sustained clocks)"},
        "memory": {"peak_extra_bytes": int(peak_extra), "BxF_fp32_bytes": B * F * 4,
                   "note": "peak allocation over the resident inputs, from the first call on (the "
                           "workspace the op keeps per stream, the outputs in flight)"},
        **({"recall": recall} if recall is not None else {}),
        "reference_published": "A5000: ~60 rows/s on this config read off results/report/roofline.png "
                               "(not tabulated; BASELINE.json published is empty)",
    }
    if not args.no_cpu and wl["op"] == "exact":
        out["cpu_baseline"] = cpu_baseline(X, W, b, k, args.cpu_seconds)
        out["cpu_c0"] = cpu_c0_baseline()
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
