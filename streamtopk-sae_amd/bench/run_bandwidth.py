"""Achieved bandwidth and arithmetic intensity on representative cells
(reference: bench/run_bandwidth.py; same cells and columns).

bytes_moved = B*d*s + F*d*s + 4F + 8Bk, flops = 2*B*d*F, runtime = median of
HIP-event-timed calls.

  python -m bench.run_bandwidth --out results/bandwidth.csv
  python -m bench.run_bandwidth --dry-run
"""
import numpy as np

from bench import common
from streamtopk_sae.inputs import make_inputs
from streamtopk_sae.utils import str_to_dtype

REPRESENTATIVE_CELLS = [
    dict(B=128, d=768, F=2**16, k=32, dtype="bf16"),
    dict(B=128, d=2048, F=2**18, k=64, dtype="bf16"),
    dict(B=512, d=2048, F=2**16, k=32, dtype="bf16"),
    dict(B=32, d=4096, F=2**14, k=16, dtype="bf16"),
]

IMPLS = ["eager", "cuda_exact", "cuda_approx"]

FIELDS = ["impl", "B", "d", "F", "k", "dtype", "runtime_s", "bytes_moved", "flops",
          "bandwidth_GBs", "arithmetic_intensity", "status"]


def traffic(B, d, F, k, dtype):
    s = 4 if dtype == "fp32" else 2
    return B * d * s + F * d * s + F * 4 + B * k * 8, 2 * B * d * F


def main(argv=None):
    parser = common.new_parser(__doc__, "results/bandwidth.csv")
    parser.add_argument("--impl", default=",".join(IMPLS))
    args = parser.parse_args(argv)
    cells = REPRESENTATIVE_CELLS[:1] if args.dry_run else REPRESENTATIVE_CELLS
    warmup, iters = (2, 3) if args.dry_run else (5, 20)
    rows = []
    for cell in cells:
        B, d, F, k, dt = cell["B"], cell["d"], cell["F"], cell["k"], cell["dtype"]
        moved, flops = traffic(B, d, F, k, dt)
        for impl_name in common.parse_strs(args.impl):
            key = {"impl": impl_name, "B": B, "d": d, "F": F, "k": k, "dtype": dt}
            try:
                X, W, b = make_inputs(B, d, F, dtype=str_to_dtype(dt), device="cuda")
                times = common.time_gpu(common.IMPL_FNS[impl_name], X, W, b, k, warmup, iters)
                t = float(np.median(times)) * 1e-6
                row = {**key, "runtime_s": t, "bytes_moved": moved, "flops": flops,
                       "bandwidth_GBs": moved / t / 1e9, "arithmetic_intensity": flops / moved,
                       "status": "ok"}
            except Exception as e:
                row = {**key, "status": common.error_status(e)}
            rows.append(row)
            print(row, flush=True)
            common.free_cache()
    common.finish(args, FIELDS, rows)
    return rows


if __name__ == "__main__":
    main()
