"""A seeded sweep of shapes across the encoder's boundaries, every case
checked against the oracle's float64 scores on a row subset:

* B around one 32-row block, four blocks (128) and the large-batch kernel's
  threshold (512), and 1024;
* F around the 256-latent tile, the 128-latent group, the sampling
  threshold (16384) and the larger sample's (131072);
* d ragged (a partial last 128-byte step) and a multiple of it;
* k from 1 to 128, every dtype, the exact op and the approximate op (with and
  without a candidate buffer).

The cases are drawn once from a fixed generator, so the sweep is the same on
every run; one workspace per stream is reused across all of them (the op's
cache), which also exercises growing and reusing it between shapes.
"""
import numpy as np
import pytest
import torch

import oracle
from parity import check_against_scores, tol_of
from streamtopk_sae import make_inputs, topk_sae_cuda_approx, topk_sae_cuda_exact

pytestmark = pytest.mark.gpu

_DT = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}


def _cases():
    rng = np.random.default_rng(2026)
    Bs = [1, 31, 33, 96, 97, 127, 128, 129, 255, 511, 512, 520, 1024]
    Fs = [100, 255, 257, 1000, 4096, 16383, 16384, 16385, 40000, 70001, 131073]
    ds = [8, 64, 72, 200, 256, 768, 1000]
    ks = [1, 2, 4, 8, 16, 32, 64, 128]
    out = []
    for i in range(84):
        B = int(rng.choice(Bs))
        F = int(rng.choice(Fs))
        d = int(rng.choice(ds))
        dt = str(rng.choice(["bf16", "fp16", "fp32"]))
        if dt == "fp32" and d % 4:
            d += 4 - d % 4
        k = int(rng.choice([x for x in ks if x <= F]))
        op = ["exact", "approx", "approx_cand"][i % 3]
        out.append((i, op, dt, B, d, F, k))
    return out


def _np(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"{c[0]}-{c[1]}-{c[2]}-B{c[3]}-d{c[4]}-F{c[5]}-k{c[6]}")
def test_sweep(cuda_dev, case):
    i, op, dt, B, d, F, k = case
    print(f"case sweep {case}", flush=True)
    X, W, b = make_inputs(B, d, F, _DT[dt], seed=100 + i, device=cuda_dev)
    if op == "exact":
        V, I = topk_sae_cuda_exact(X, W, b, k)
    else:
        c = min(x for x in (16, 32, 64, 128) if x >= k)
        cb = None
        if op == "approx_cand":
            cb = torch.empty((B, (F + 127) // 128, c), dtype=torch.float32, device=cuda_dev)
        V, I = topk_sae_cuda_approx(X, W, b, k, c, candidate_buffer=cb)
    torch.cuda.synchronize()
    rows = np.unique(np.linspace(0, B - 1, num=min(B, 12)).astype(np.int64))
    S = oracle.scores_f64(_np(X[rows]), _np(W), _np(b))
    ties = check_against_scores(V[rows].cpu().numpy(), I[rows].cpu().numpy(), S, k, tol_of(dt), f"sweep {case}")
    if ties:
        print(f"[ties] sweep {case}: {ties} row(s)")
