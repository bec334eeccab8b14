"""Latency per (impl, B, d, F, k, dtype) cell: median, p10, p90, min, max in us
(reference: bench/run_runtime.py; same columns, grid, randomized cell order).

  python -m bench.run_runtime --impl cpu,cuda_exact,cuda_approx,eager \\
      --warmup 10 --iters 100 --out results/runtime.csv
  python -m bench.run_runtime --dry-run
"""
import random

import torch

from bench import common
from bench.grid import BENCH_GRID, BENCH_GRID_CPU, dry_run_cell, filter_cells, iter_grid
from streamtopk_sae.inputs import make_inputs
from streamtopk_sae.utils import str_to_dtype

FIELDS = ["impl", "B", "d", "F", "k", "dtype", "device",
          "median_us", "p10_us", "p90_us", "min_us", "max_us", "status"]


def bench_cell(impl_name, cell, warmup, iters):
    B, d, F, k, dt = cell["B"], cell["d"], cell["F"], cell["k"], cell["dtype"]
    key = {"impl": impl_name, "B": B, "d": d, "F": F, "k": k, "dtype": dt}
    is_cpu = impl_name == "cpu"
    try:
        X, W, b = make_inputs(B, d, F, dtype=str_to_dtype(dt), device="cpu" if is_cpu else "cuda")
        fn = common.IMPL_FNS[impl_name]
        times = (common.time_cpu if is_cpu else common.time_gpu)(fn, X, W, b, k, warmup, iters)
        device = "cpu" if is_cpu else torch.cuda.get_device_name(0)
        return {**key, "device": device, **common.stats_us(times), "status": "ok"}
    except Exception as e:   # OOM or an argument error: recorded, the sweep goes on
        return {**key, "status": common.error_status(e)}


def main(argv=None):
    parser = common.new_parser(__doc__, "results/runtime.csv")
    parser.add_argument("--impl", default=",".join(common.IMPL_FNS))
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--iters", type=int, default=100)
    parser.add_argument("--seed", type=int, default=None, help="seed of the cell shuffle")
    common.add_grid_filters(parser)
    args = parser.parse_args(argv)

    rng = random.Random(args.seed)
    rows = []
    for impl_name in common.parse_strs(args.impl):
        if impl_name not in common.IMPL_FNS:
            raise SystemExit(f"unknown impl {impl_name!r}; choose from {list(common.IMPL_FNS)}")
        grid = BENCH_GRID_CPU if impl_name == "cpu" else BENCH_GRID
        if args.dry_run:
            cells = [dry_run_cell(grid)]
        else:
            cells = list(filter_cells(iter_grid(grid), args))
            rng.shuffle(cells)
        warmup, iters = (2, 3) if args.dry_run else (args.warmup, args.iters)
        for cell in cells:
            if impl_name == "cpu" and cell["dtype"] != "fp32":
                continue
            row = bench_cell(impl_name, cell, warmup, iters)
            rows.append(row)
            print(row, flush=True)
            common.free_cache()
    common.finish(args, FIELDS, rows)
    return rows


if __name__ == "__main__":
    main()
