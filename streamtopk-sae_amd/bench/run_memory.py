"""Peak device memory per (impl, B, d, F, k, dtype) cell
(reference: bench/run_memory.py; same columns and grid).

Each GPU cell runs in a child process of its own (``--_measure``), so the
caching allocator starts empty: baseline_mem is the memory the inputs hold,
peak_mem the peak during one call, working_mem = peak - baseline - the (B, k)
outputs.  (The reference reads the allocator's peak after making the inputs
as the baseline, which also counts the input generator's fp32 temporaries and
can push working_mem below zero; this reads what stays allocated.)  The library allocates nothing itself (the ops take their
workspace from torch), so torch's counters see all of it.  The cpu impl
reports the growth of the process's peak RSS.

  python -m bench.run_memory --impl cuda_exact,eager,cuda_approx --out results/memory.csv
  python -m bench.run_memory --dry-run
"""
import json
import os
import subprocess
import sys

from bench import common
from bench.grid import BENCH_GRID, BENCH_GRID_CPU, dry_run_cell, filter_cells, iter_grid

FIELDS = ["impl", "B", "d", "F", "k", "dtype", "baseline_mem_mb", "peak_mem_mb", "working_mem_mb", "status"]
_HERE = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def measure_gpu_cell(impl_name, cell):
    """One cell in this process (called in a fresh child process)."""
    import torch
    from streamtopk_sae.inputs import make_inputs
    from streamtopk_sae.utils import str_to_dtype
    B, d, F, k, dt = cell["B"], cell["d"], cell["F"], cell["k"], cell["dtype"]
    key = {"impl": impl_name, "B": B, "d": d, "F": F, "k": k, "dtype": dt}
    try:
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats()
        X, W, b = make_inputs(B, d, F, dtype=str_to_dtype(dt), device="cuda")
        torch.cuda.synchronize()
        base = torch.cuda.memory_allocated()   # the resident inputs
        torch.cuda.reset_peak_memory_stats()
        common.IMPL_FNS[impl_name](X, W, b, k)
        torch.cuda.synchronize()
        peak = torch.cuda.max_memory_allocated()
        work = peak - base - B * k * 8
        return {**key, "baseline_mem_mb": base / 1e6, "peak_mem_mb": peak / 1e6,
                "working_mem_mb": work / 1e6, "status": "ok"}
    except Exception as e:
        return {**key, "status": common.error_status(e)}


def measure_gpu_cell_isolated(impl_name, cell, timeout=300):
    cmd = [sys.executable, "-m", "bench.run_memory", "--_measure", impl_name,
           str(cell["B"]), str(cell["d"]), str(cell["F"]), str(cell["k"]), cell["dtype"]]
    key = {"impl": impl_name, **cell}
    try:
        res = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout, cwd=_HERE)
    except subprocess.TimeoutExpired:
        return {**key, "status": "TIMEOUT"}
    if res.returncode != 0:
        return {**key, "status": "ERR:" + res.stderr[-300:].strip()}
    return json.loads(res.stdout.strip().splitlines()[-1])


def measure_cpu_cell(cell):
    import resource
    import torch
    from streamtopk_sae.inputs import make_inputs
    from streamtopk_sae.ops import topk_sae_cpu
    B, d, F, k = cell["B"], cell["d"], cell["F"], cell["k"]
    before = resource.getrusage(resource.RUSAGE_SELF).ru_maxrss
    X, W, b = make_inputs(B, d, F, dtype=torch.float32, device="cpu")
    topk_sae_cpu(X, W, b, k)
    after = resource.getrusage(resource.RUSAGE_SELF).ru_maxrss
    return {"impl": "cpu", "B": B, "d": d, "F": F, "k": k, "dtype": "fp32",
            "working_mem_mb": (after - before) / 1024, "status": "ok"}


def main(argv=None):
    parser = common.new_parser(__doc__, "results/memory.csv")
    parser.add_argument("--impl", default="cuda_exact,eager,cuda_approx")
    common.add_grid_filters(parser)
    parser.add_argument("--_measure", nargs=6, metavar=("IMPL", "B", "d", "F", "k", "DTYPE"),
                        help="(internal) measure one GPU cell in this process and print it as JSON")
    args = parser.parse_args(argv)

    if args._measure:
        impl_name, B, d, F, k, dt = args._measure
        row = measure_gpu_cell(impl_name, {"B": int(B), "d": int(d), "F": int(F), "k": int(k), "dtype": dt})
        print(json.dumps(row), flush=True)
        return [row]

    rows = []
    for impl_name in common.parse_strs(args.impl):
        grid = BENCH_GRID_CPU if impl_name == "cpu" else BENCH_GRID
        cells = [dry_run_cell(grid)] if args.dry_run else list(filter_cells(iter_grid(grid), args))
        for cell in cells:
            row = measure_cpu_cell(cell) if impl_name == "cpu" else measure_gpu_cell_isolated(impl_name, cell)
            rows.append(row)
            print(row, flush=True)
    common.finish(args, FIELDS, rows)
    return rows


if __name__ == "__main__":
    main()
