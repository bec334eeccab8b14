"""Benchmark harness with the reference's CSV schemas.

Run from the ``streamtopk-sae_amd`` directory, as the reference runs its own
from the repository root (reference bench/run_*.py usage lines):

    python -m bench.run_runtime   --impl cpu,cuda_exact,cuda_approx,eager --out results/runtime.csv
    python -m bench.run_bandwidth --out results/bandwidth.csv
    python -m bench.run_recall    --out results/recall.csv
    python -m bench.run_memory    --impl cuda_exact,eager,cuda_approx --out results/memory.csv
    python -m bench.run_max_F     --out results/max_F.csv

Every script takes ``--dry-run`` (one cell per impl, nothing written).  The
column sets, grids and per-cell statistics are the reference's, so a CSV of
published A5000 rows and a CSV of MI355X rows line up column for column.  The
impls are this build's: ``cpu`` (OpenMP), ``cuda_exact`` and ``cuda_approx``
(the gfx950 kernels, on torch's current HIP stream) and ``eager`` (the dense
torch path: matmul in the input dtype, fp32 top-k).  The reference's
``compiled`` and ``triton`` baselines are not part of this build.
"""
