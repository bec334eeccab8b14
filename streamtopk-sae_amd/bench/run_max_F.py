"""Largest F (a power of two, 2^14 .. 2^22) whose call fits in device memory,
by binary search (reference: bench/run_max_F.py; same configs, range and
columns).  A cell that fails for any reason counts as not fitting.

  python -m bench.run_max_F --out results/max_F.csv
  python -m bench.run_max_F --dry-run
  python -m bench.run_max_F --configs 1 --max-pow 28   # past the reference's 2^22 cap

The reference's range (2^22 at most) was sized for a 24 GB card; on a 288 GB
MI355X every implementation reaches it at these configs, so --max-pow extends
the search to show where each one actually stops.
"""
import torch

from bench import common
from streamtopk_sae.inputs import make_inputs
from streamtopk_sae.utils import str_to_dtype

CONFIGS = [
    dict(B=128, d=768, k=32, dtype="bf16"),
    dict(B=2048, d=768, k=32, dtype="bf16"),
]
IMPLS = ["eager", "cuda_exact", "cuda_approx"]
F_MIN_POW, F_MAX_POW = 14, 22
FIELDS = ["impl", "B", "d", "k", "dtype", "max_F"]


def fits(impl_name, B, d, F, k, dtype):
    ok = False
    try:
        torch.cuda.empty_cache()
        X, W, b = make_inputs(B, d, F, dtype=dtype, device="cuda")
        common.IMPL_FNS[impl_name](X, W, b, k)
        torch.cuda.synchronize()
        ok = True
    except Exception:
        ok = False
    finally:
        X = W = b = None
        torch.cuda.empty_cache()
    print(f"# {impl_name} B={B} d={d} F={F}: {'fits' if ok else 'does not fit'}", flush=True)
    return ok


def max_F(impl_name, B, d, k, dtype, lo=F_MIN_POW, hi=F_MAX_POW):
    best = None
    while lo <= hi:
        mid = (lo + hi) // 2
        if fits(impl_name, B, d, 2 ** mid, k, dtype):
            best, lo = 2 ** mid, mid + 1
        else:
            hi = mid - 1
    return best


def main(argv=None):
    parser = common.new_parser(__doc__, "results/max_F.csv")
    parser.add_argument("--impl", default=",".join(IMPLS))
    parser.add_argument("--configs", default=None, help="indices into CONFIGS, e.g. 1 or 0,1")
    parser.add_argument("--max-pow", type=int, default=F_MAX_POW, help="largest log2(F) searched")
    args = parser.parse_args(argv)
    rows = []
    cfgs = CONFIGS if args.configs is None else [CONFIGS[int(i)] for i in common.parse_strs(args.configs)]
    for cfg in (CONFIGS[:1] if args.dry_run else cfgs):
        B, d, k, dt = cfg["B"], cfg["d"], cfg["k"], cfg["dtype"]
        for impl_name in common.parse_strs(args.impl):
            if args.dry_run:
                F = 2 ** F_MIN_POW
                m = F if fits(impl_name, B, d, F, k, str_to_dtype(dt)) else None
            else:
                m = max_F(impl_name, B, d, k, str_to_dtype(dt), hi=args.max_pow)
            row = {"impl": impl_name, "B": B, "d": d, "k": k, "dtype": dt,
                   "max_F": m if m is not None else "OOM"}
            rows.append(row)
            print(row, flush=True)
    common.finish(args, FIELDS, rows)
    return rows


if __name__ == "__main__":
    main()
