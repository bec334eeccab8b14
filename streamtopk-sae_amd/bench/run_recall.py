"""Recall@k of the approximate kernel against the dense reference
(reference: bench/run_recall.py; same grid, c snapping and columns).

c = k * c_multiplier snapped to the nearest supported c (ties to the smaller),
then raised to the smallest supported c >= k.  Per-row recall |pred & true| / k.

--oracle picks the dense reference the recall is scored against:
  upcast   the scores of the upcast fp32 inputs (streamtopk_sae.reference, the
           quantity the kernels compute; default);
  rounded  the reference's own formula (reference.py:17): the matmul in the
           input dtype, so bf16/fp16 scores are rounded before the fp32 bias
           is added and top-k picks among the rounded values.
--data picks the inputs: ours (streamtopk_sae.inputs.make_inputs, unit-norm
W_enc rows, b_enc ~ N(0, 0.1^2)) or gaussian (the reference harness's gaussian
branch, bench.common.gaussian_inputs: X, W_enc ~ N(0, 1), b_enc = 0).

  python -m bench.run_recall --out results/recall.csv
  python -m bench.run_recall --oracle rounded --data gaussian --B 128 --d 2048
  python -m bench.run_recall --dry-run
"""
import numpy as np

from bench import common
from bench.grid import RECALL_GRID, dry_run_cell, filter_cells, iter_grid
from streamtopk_sae.inputs import make_inputs
from streamtopk_sae.ops import topk_sae_cuda_approx
from streamtopk_sae.reference import reference_topk_sae
from streamtopk_sae.utils import recall_per_row, str_to_dtype

SUPPORTED_C = [16, 32, 64, 128]

FIELDS = ["B", "d", "F", "k", "c", "c_multiplier", "dtype",
          "recall_mean", "recall_std", "recall_min", "recall_p10", "recall_p50", "recall_p90", "status"]


def snap_c(k, c_mult):
    c = min(SUPPORTED_C, key=lambda s: (abs(s - k * c_mult), s))
    if c < k:
        c = min(s for s in SUPPORTED_C if s >= k)
    return c


def main(argv=None):
    parser = common.new_parser(__doc__, "results/recall.csv")
    common.add_grid_filters(parser)
    parser.add_argument("--oracle", choices=["upcast", "rounded"], default="upcast")
    parser.add_argument("--data", choices=["ours", "gaussian"], default="ours")
    args = parser.parse_args(argv)
    oracle = reference_topk_sae if args.oracle == "upcast" else common.baseline_eager
    gen = make_inputs if args.data == "ours" else common.gaussian_inputs
    cells = [dry_run_cell(RECALL_GRID)] if args.dry_run else list(filter_cells(iter_grid(RECALL_GRID), args))
    rows = []
    for cell in cells:
        B, d, F, k, dt, cm = cell["B"], cell["d"], cell["F"], cell["k"], cell["dtype"], cell["c_multiplier"]
        c = snap_c(k, cm)
        key = {"B": B, "d": d, "F": F, "k": k, "c": c, "c_multiplier": cm, "dtype": dt}
        try:
            X, W, b = gen(B, d, F, dtype=str_to_dtype(dt), device="cuda")
            _, ref_i = oracle(X, W, b, k)
            _, pred_i = topk_sae_cuda_approx(X, W, b, k, c)
            r = recall_per_row(pred_i, ref_i).numpy()
            row = {**key, "recall_mean": float(np.mean(r)), "recall_std": float(np.std(r)),
                   "recall_min": float(np.min(r)), "recall_p10": float(np.percentile(r, 10)),
                   "recall_p50": float(np.median(r)), "recall_p90": float(np.percentile(r, 90)),
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
