"""The benchmark harness under streamtopk-sae_amd/bench: the reference's CSV
schemas (bench/run_runtime.py:169-170, run_bandwidth.py:112-114,
run_recall.py:109-111, run_memory.py:182-183, run_max_F.py:98), grids
(bench/grid.py:5-29) and c snapping (run_recall.py:66-70).

The scripts run as ``python -m bench.<script>`` from the package directory,
as a user runs them; the repository's own bench.py shares the module name, so
they are not imported into the test process.
"""
import ast
import csv
import importlib.util
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "streamtopk-sae_amd")

# Column lists as the reference writes them.
RUNTIME_FIELDS = ["impl", "B", "d", "F", "k", "dtype", "device",
                  "median_us", "p10_us", "p90_us", "min_us", "max_us", "status"]
BANDWIDTH_FIELDS = ["impl", "B", "d", "F", "k", "dtype", "runtime_s", "bytes_moved", "flops",
                    "bandwidth_GBs", "arithmetic_intensity", "status"]
RECALL_FIELDS = ["B", "d", "F", "k", "c", "c_multiplier", "dtype", "recall_mean", "recall_std",
                 "recall_min", "recall_p10", "recall_p50", "recall_p90", "status"]
MEMORY_FIELDS = ["impl", "B", "d", "F", "k", "dtype", "baseline_mem_mb", "peak_mem_mb",
                 "working_mem_mb", "status"]


def run_script(module, *args, timeout=110):
    res = subprocess.run([sys.executable, "-m", f"bench.{module}", *args], cwd=PKG_DIR,
                         capture_output=True, text=True, timeout=timeout)
    assert res.returncode == 0, res.stderr[-2000:]
    return res.stdout


def printed_rows(stdout):
    return [ast.literal_eval(line) for line in stdout.splitlines() if line.startswith("{")]


def read_csv(path):
    with open(path, newline="") as f:
        r = csv.DictReader(f)
        return r.fieldnames, list(r)


def load_grid():
    spec = importlib.util.spec_from_file_location("stk_bench_grid", os.path.join(PKG_DIR, "bench", "grid.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_grids_are_the_reference_grids():
    g = load_grid()
    assert g.BENCH_GRID == {"B": [32, 128, 512, 2048], "d": [768, 2048, 4096],
                            "F": [16384, 65536, 262144, 1048576, 4194304], "k": [16, 32, 64, 128],
                            "dtype": ["fp16", "bf16", "fp32"]}
    assert g.BENCH_GRID_CPU == {"B": [32, 128, 512], "d": [768, 2048], "F": [16384, 65536, 262144],
                                "k": [16, 32, 64], "dtype": ["fp32"]}
    assert g.RECALL_GRID["c_multiplier"] == [1, 2, 4, 8, 16]
    cells = list(g.iter_grid(g.BENCH_GRID))
    assert len(cells) == 4 * 3 * 5 * 4 * 3
    assert len({tuple(c.values()) for c in cells}) == len(cells)
    # last key varies fastest, as itertools.product over the keys in order
    assert cells[0] == dict(B=32, d=768, F=16384, k=16, dtype="fp16") == g.dry_run_cell(g.BENCH_GRID)
    assert cells[1]["dtype"] == "bf16" and cells[3]["k"] == 32


def test_recall_c_snapping():
    # c = k * multiplier, snapped to the nearest of {16, 32, 64, 128} (ties to the
    # smaller), then at least k.  Worked by hand from the rule: 32*8 = 256 -> 128,
    # 64*2 = 128, 16*3 = 48 is 16 away from both 32 and 64 -> 32.
    code = ("from bench.run_recall import snap_c; "
            "print([snap_c(k, m) for k, m in [(32, 1), (32, 2), (32, 4), (32, 8), (32, 16), "
            "(64, 1), (64, 2), (64, 16), (16, 1), (16, 3), (128, 1)]])")
    res = subprocess.run([sys.executable, "-c", code], cwd=PKG_DIR, capture_output=True, text=True, timeout=110)
    assert res.returncode == 0, res.stderr[-2000:]
    assert ast.literal_eval(res.stdout.strip()) == [32, 64, 128, 128, 128, 64, 128, 128, 16, 32, 128]


def test_runtime_cpu_cells_csv(tmp_path):
    out = tmp_path / "runtime.csv"
    run_script("run_runtime", "--impl", "cpu", "--B", "32", "--d", "768", "--F", "16384", "--k", "16,32",
               "--warmup", "1", "--iters", "2", "--seed", "3", "--out", str(out))
    fields, rows = read_csv(out)
    assert fields == RUNTIME_FIELDS
    assert sorted(int(r["k"]) for r in rows) == [16, 32]
    for r in rows:
        assert r["status"] == "ok" and r["device"] == "cpu" and r["dtype"] == "fp32"
        assert 0 < float(r["min_us"]) <= float(r["median_us"]) <= float(r["max_us"])


def test_runtime_rejects_unknown_impl():
    res = subprocess.run([sys.executable, "-m", "bench.run_runtime", "--impl", "triton", "--dry-run"],
                         cwd=PKG_DIR, capture_output=True, text=True, timeout=110)
    assert res.returncode != 0 and "unknown impl" in (res.stdout + res.stderr)


def test_memory_cpu_dry_run():
    rows = printed_rows(run_script("run_memory", "--impl", "cpu", "--dry-run"))
    assert len(rows) == 1 and rows[0]["status"] == "ok" and rows[0]["impl"] == "cpu"
    assert set(rows[0]) <= set(MEMORY_FIELDS)


@pytest.mark.gpu
def test_runtime_gpu_cells_csv(cuda_dev, tmp_path):
    out = tmp_path / "runtime.csv"
    run_script("run_runtime", "--impl", "cuda_exact,cuda_approx,eager", "--B", "32", "--d", "768",
               "--F", "16384", "--k", "16", "--dtype", "bf16", "--warmup", "2", "--iters", "5", "--out", str(out))
    fields, rows = read_csv(out)
    assert fields == RUNTIME_FIELDS
    assert sorted(r["impl"] for r in rows) == ["cuda_approx", "cuda_exact", "eager"]
    for r in rows:
        assert r["status"] == "ok" and r["device"] and float(r["median_us"]) > 0


@pytest.mark.gpu
def test_bandwidth_dry_run(cuda_dev):
    rows = printed_rows(run_script("run_bandwidth", "--dry-run"))
    assert [r["impl"] for r in rows] == ["eager", "cuda_exact", "cuda_approx"]
    for r in rows:
        assert r["status"] == "ok" and set(r) == set(BANDWIDTH_FIELDS)
        # cell 0: B=128 d=768 F=2^16 k=32 bf16
        assert r["bytes_moved"] == 128 * 768 * 2 + 65536 * 768 * 2 + 65536 * 4 + 128 * 32 * 8
        assert r["flops"] == 2 * 128 * 768 * 65536
        assert r["bandwidth_GBs"] == pytest.approx(r["bytes_moved"] / r["runtime_s"] / 1e9)


@pytest.mark.gpu
def test_recall_csv(cuda_dev, tmp_path):
    out = tmp_path / "recall.csv"
    run_script("run_recall", "--B", "128", "--d", "2048", "--F", "65536", "--k", "32", "--out", str(out))
    fields, rows = read_csv(out)
    assert fields == RECALL_FIELDS
    assert [int(r["c"]) for r in rows] == [32, 64, 128, 128, 128]
    for r in rows:
        # k <= c: the union of the per-group top-c holds the exact top-k, so recall
        # against the dense reference is 1 up to fp32 near-ties
        assert r["status"] == "ok" and float(r["recall_mean"]) >= 0.99


@pytest.mark.gpu
def test_recall_rounded_oracle_gaussian(cuda_dev, tmp_path):
    """The reference's published recall setting: its gaussian inputs (X, W_enc
    ~ N(0, 1) in bf16, b_enc = 0) scored against its own dense formula, which
    rounds the bf16 scores (|score| ~ 200 here, a bf16 step of 1.0) before
    top-k.  The approximate op returns the exact fp32 top-k, so its recall
    against that oracle is the exact op's, below 1 where the rounding ties or
    reorders latents near the k-th score."""
    import torch
    out = tmp_path / "recall.csv"
    run_script("run_recall", "--B", "128", "--d", "2048", "--F", "262144", "--k", "32", "--oracle", "rounded",
               "--data", "gaussian", "--out", str(out))
    fields, rows = read_csv(out)
    assert fields == RECALL_FIELDS
    assert all(r["status"] == "ok" for r in rows)
    rec = {float(r["recall_mean"]) for r in rows}
    assert len(rec) == 1   # the same latents for every c (k <= c)
    from streamtopk_sae import recall_at_k, topk_sae_cuda_exact
    # the same inputs (bench.common.gaussian_inputs, seed 0) and oracle
    # (bench.common.baseline_eager) in this process
    rng = torch.Generator()
    rng.manual_seed(0)
    X = torch.randn(128, 2048, dtype=torch.bfloat16, generator=rng).to(cuda_dev)
    W = torch.randn(262144, 2048, dtype=torch.bfloat16, generator=rng).to(cuda_dev)
    b = torch.zeros(262144, dtype=torch.float32, device=cuda_dev)
    _, I_ex = topk_sae_cuda_exact(X, W, b, 32)
    I_rd = torch.topk((X @ W.T + b).float(), 32, dim=-1).indices
    assert float(rows[0]["recall_mean"]) == pytest.approx(recall_at_k(I_ex, I_rd), abs=1e-9)
    assert float(rows[0]["recall_mean"]) < 1.0


@pytest.mark.gpu
def test_memory_gpu_cells(cuda_dev, tmp_path):
    out = tmp_path / "memory.csv"
    # at the headline F the (B, F) fp32 scores (134 MB) outweigh the streaming
    # path's workspace, which does not grow with F
    B, F = 128, 262144
    run_script("run_memory", "--impl", "cuda_exact,eager", "--B", str(B), "--d", "768", "--F", str(F),
               "--k", "16", "--dtype", "bf16", "--out", str(out))
    fields, rows = read_csv(out)
    assert fields == MEMORY_FIELDS
    by = {r["impl"]: r for r in rows}
    assert by["cuda_exact"]["status"] == "ok" and by["eager"]["status"] == "ok"
    score_matrix_mb = B * F * 4 / 1e6
    # the dense path materialises the (B, F) scores; the streaming path does not
    assert float(by["eager"]["working_mem_mb"]) >= score_matrix_mb
    assert float(by["cuda_exact"]["working_mem_mb"]) < score_matrix_mb


@pytest.mark.gpu
def test_max_F_dry_run(cuda_dev):
    rows = printed_rows(run_script("run_max_F", "--dry-run"))
    assert [r["impl"] for r in rows] == ["eager", "cuda_exact", "cuda_approx"]
    assert all(r["max_F"] == 16384 for r in rows)
