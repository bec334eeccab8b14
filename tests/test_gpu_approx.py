"""GPU parity of the approximate encoder (topk_sae_cuda_approx).

Without a candidate buffer the result must equal the exact top-k (with k <= c
every exact top-k latent is inside its group's top-c).  With a candidate
buffer the per-group top-c values are compared with the oracle's candidates
(streamtopk_approx.cu:118-166 semantics) and the final top-k with the
oracle's approx result.  Recall tests mirror the reference's
tests/test_recall.py:22-96.
"""
import numpy as np
import pytest
import torch

import oracle
from parity import check_against_scores
from streamtopk_sae import make_inputs, recall_at_k, topk_sae_cuda_approx, topk_sae_cuda_exact

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("c", [16, 32, 64, 128])
def test_approx_equals_exact(cuda_dev, c):
    print(f"case approx==exact c={c}", flush=True)
    X, W, b = make_inputs(32, 256, 20000, torch.bfloat16, seed=21, device=cuda_dev)
    k = 16
    Va, Ia = topk_sae_cuda_approx(X, W, b, k, c)
    Ve, Ie = topk_sae_cuda_exact(X, W, b, k)
    assert torch.equal(Va, Ve) and torch.equal(Ia, Ie)
    assert recall_at_k(Ia, Ie) == 1.0


@pytest.mark.parametrize("c", [16, 32, 64, 128])
@pytest.mark.parametrize("F", [256, 1000])
def test_approx_candidate_buffer(cuda_dev, c, F):
    print(f"case approx candidates c={c} F={F}", flush=True)
    B, d, k = 8, 64, min(16, c)
    X, W, b = make_inputs(B, d, F, torch.bfloat16, seed=22, device=cuda_dev)
    nt = (F + 127) // 128
    cb = torch.empty((B, nt, c), dtype=torch.float32, device=cuda_dev)
    V, I = topk_sae_cuda_approx(X, W, b, k, c, candidate_buffer=cb)
    Vo, Io, cvo, cio = oracle.approx(_np(X), _np(W), _np(b), k, c, with_candidates=True)
    cbn = cb.cpu().numpy()
    pad = cio < 0
    assert np.array_equal(cbn[pad], cvo[pad])
    err = np.abs(cbn[~pad] - cvo[~pad]) / np.maximum(np.abs(cvo[~pad]), 1.0)
    assert err.max() <= 2e-3
    S = oracle.scores_f64(_np(X), _np(W), _np(b))
    check_against_scores(V.cpu().numpy(), I.cpu().numpy(), S, k, 2e-3, f"approx c={c}")


def test_approx_candidate_buffer_final_matches_exact(cuda_dev):
    X, W, b = make_inputs(16, 128, 5000, torch.bfloat16, seed=23, device=cuda_dev)
    nt = (5000 + 127) // 128
    cb = torch.empty((16, nt, 32), dtype=torch.float32, device=cuda_dev)
    Va, Ia = topk_sae_cuda_approx(X, W, b, 32, 32, candidate_buffer=cb)
    Ve, Ie = topk_sae_cuda_exact(X, W, b, 32)
    assert torch.equal(Va, Ve) and torch.equal(Ia, Ie)


@pytest.mark.parametrize("shape", [dict(B=32, d=256, F=1024, k=16), dict(B=32, d=256, F=2048, k=32)])
def test_recall_monotonicity(cuda_dev, shape):
    X, W, b = make_inputs(shape["B"], shape["d"], shape["F"], torch.bfloat16, seed=0, device=cuda_dev)
    k = shape["k"]
    _, ref_i = topk_sae_cuda_exact(X, W, b, k)
    recalls = [recall_at_k(topk_sae_cuda_approx(X, W, b, k, c)[1], ref_i) for c in (16, 32, 64, 128) if c >= k]
    for r0, r1 in zip(recalls, recalls[1:]):
        assert r1 >= r0 - 0.02
    assert all(r == 1.0 for r in recalls)


def test_approx_errors(cuda_dev):
    X, W, b = make_inputs(4, 64, 256, torch.bfloat16, seed=24, device=cuda_dev)
    with pytest.raises(RuntimeError, match="k must be <= c"):
        topk_sae_cuda_approx(X, W, b, 32, 16)
    with pytest.raises(RuntimeError, match="unsupported c=48"):
        topk_sae_cuda_approx(X, W, b, 8, 48)
    with pytest.raises(RuntimeError, match="candidate_buffer shape mismatch"):
        topk_sae_cuda_approx(X, W, b, 8, 16, candidate_buffer=torch.empty(4, 3, 16, device=cuda_dev))


@pytest.mark.parametrize("with_buffer", [False, True])
def test_approx_known_answers(cuda_dev, with_buffer):
    from golden.make_golden import load as load_golden
    for X, W, b, k, Vk, Ik in load_golden():
        c = max(16, k)
        Xt = torch.from_numpy(X).to(cuda_dev).bfloat16()
        Wt = torch.from_numpy(W).to(cuda_dev).bfloat16()
        bt = torch.from_numpy(b).to(cuda_dev)
        cb = None
        if with_buffer:
            cb = torch.empty((X.shape[0], (W.shape[0] + 127) // 128, c), dtype=torch.float32, device=cuda_dev)
        V, I = topk_sae_cuda_approx(Xt, Wt, bt, k, c, candidate_buffer=cb)
        assert np.array_equal(V.cpu().numpy(), Vk) and np.array_equal(I.cpu().numpy(), Ik)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("B,F,c", [(100, 5000, 32), (40, 3000, 128), (5, 2000, 16), (130, 1280, 64)])
def test_approx_candidates_shapes(cuda_dev, dtype, B, F, c):
    """Ragged batches (one, two and four 32-row blocks; a partial second row
    block), F not a multiple of the 256-latent tile, every dtype: per-group
    candidates against the oracle's, in descending order, and the final top-k
    equal to the exact kernel's."""
    print(f"case approx candidates {dtype} B={B} F={F} c={c}", flush=True)
    d, k = 128, min(16, c)
    tol = 1e-5 if dtype == torch.float32 else 2e-3
    X, W, b = make_inputs(B, d, F, dtype, seed=25, device=cuda_dev)
    nt = (F + 127) // 128
    cb = torch.empty((B, nt, c), dtype=torch.float32, device=cuda_dev)
    V, I = topk_sae_cuda_approx(X, W, b, k, c, candidate_buffer=cb)
    _, _, cvo, cio = oracle.approx(_np(X), _np(W), _np(b), k, c, with_candidates=True)
    cbn = cb.cpu().numpy()
    pad = cio < 0
    assert np.array_equal(cbn[pad], cvo[pad])
    err = np.abs(cbn[~pad] - cvo[~pad]) / np.maximum(np.abs(cvo[~pad]), 1.0)
    assert err.max() <= tol
    assert np.all(np.diff(cbn, axis=2) <= 0)
    Ve, Ie = topk_sae_cuda_exact(X, W, b, k)
    assert torch.equal(V, Ve) and torch.equal(I, Ie)


@pytest.mark.parametrize("dtype,d,F,c", [(torch.bfloat16, 64, 100, 128), (torch.float32, 32, 700, 16)])
def test_approx_candidates_small(cuda_dev, dtype, d, F, c):
    """F below one group (one tile, mostly padding) and the narrowest fp32 row
    (one d-step)."""
    print(f"case approx candidates small {dtype} d={d} F={F} c={c}", flush=True)
    B, k = 3, 16
    tol = 1e-5 if dtype == torch.float32 else 2e-3
    X, W, b = make_inputs(B, d, F, dtype, seed=27, device=cuda_dev)
    nt = (F + 127) // 128
    cb = torch.empty((B, nt, c), dtype=torch.float32, device=cuda_dev)
    V, I = topk_sae_cuda_approx(X, W, b, k, c, candidate_buffer=cb)
    _, _, cvo, cio = oracle.approx(_np(X), _np(W), _np(b), k, c, with_candidates=True)
    cbn = cb.cpu().numpy()
    pad = cio < 0
    # padded slots per row: c minus the real latents of each group, where negative none
    assert pad.sum() == B * sum(max(0, c - min(128, F - 128 * g)) for g in range(nt))
    assert np.array_equal(cbn[pad], cvo[pad])
    err = np.abs(cbn[~pad] - cvo[~pad]) / np.maximum(np.abs(cvo[~pad]), 1.0)
    assert err.max() <= tol
    Ve, Ie = topk_sae_cuda_exact(X, W, b, k)
    assert torch.equal(V, Ve) and torch.equal(I, Ie)


def test_approx_candidates_equal_scores(cuda_dev):
    """All scores equal (X = 0, constant b_enc): ties go to the lower index, and
    the groups that reach the row bound hold more candidates than one
    selection buffer, so the final selection compacts and resumes."""
    print("case approx candidates equal scores", flush=True)
    B, d, F, k, c = 4, 64, 51200, 32, 32
    X = torch.zeros((B, d), dtype=torch.bfloat16, device=cuda_dev)
    _, W, _ = make_inputs(B, d, F, torch.bfloat16, seed=26, device=cuda_dev)
    b = torch.full((F,), 0.5, dtype=torch.float32, device=cuda_dev)
    cb = torch.empty((B, F // 128, c), dtype=torch.float32, device=cuda_dev)
    V, I = topk_sae_cuda_approx(X, W, b, k, c, candidate_buffer=cb)
    assert torch.equal(I.cpu(), torch.arange(k, dtype=torch.int32).expand(B, k))
    assert bool((V == 0.5).all()) and bool((cb == 0.5).all())


@pytest.mark.parametrize("dtype,B,d,F", [
    (torch.bfloat16, 128, 200, 150000),   # ragged last d-step; 3 tiles per workgroup, the last one 1
    (torch.bfloat16, 128, 256, 200000),   # 4 tiles per workgroup, the last one 2
    (torch.float32, 160, 36, 70000),      # fp32, a partial second d-step; a partial second row block
    (torch.float16, 128, 64, 3000),       # one d-step: every tile's sort takes extra intervals
])
def test_candidates_full_row_blocks(cuda_dev, dtype, B, d, F):
    """Full 128-row blocks (four 32-row blocks per workgroup) with several tiles
    per workgroup (odd and even counts), ragged and one-step d, every dtype:
    per-group candidates against the oracle's, and the final top-k against f64
    scores."""
    print(f"case candidates full row blocks {dtype} B={B} d={d} F={F}", flush=True)
    c, k = 32, 16
    tol = 1e-5 if dtype == torch.float32 else 2e-3
    X, W, b = make_inputs(B, d, F, dtype, seed=31, device=cuda_dev)
    nt = (F + 127) // 128
    cb = torch.empty((B, nt, c), dtype=torch.float32, device=cuda_dev)
    V, I = topk_sae_cuda_approx(X, W, b, k, c, candidate_buffer=cb)
    _, _, cvo, cio = oracle.approx(_np(X), _np(W), _np(b), k, c, with_candidates=True)
    cbn = cb.cpu().numpy()
    pad = cio < 0
    assert np.array_equal(cbn[pad], cvo[pad])
    err = np.abs(cbn[~pad] - cvo[~pad]) / np.maximum(np.abs(cvo[~pad]), 1.0)
    assert err.max() <= tol
    assert np.all(np.diff(cbn, axis=2) <= 0)
    # the final top-k against f64 scores on a row subset (the exact kernel
    # scores sampled latents through summed d-splits, so its values can differ
    # from these in the last bit once F is large enough to be sampled)
    rows = slice(0, 16)
    S = oracle.scores_f64(_np(X[rows]), _np(W), _np(b))
    check_against_scores(V[rows].cpu().numpy(), I[rows].cpu().numpy(), S, k, tol, "full row blocks")


def _tie_heavy_inputs(B, d, F, seed):
    """fp32 inputs whose scores are chosen exactly: X[r] is the unit vector
    e_(r % d) and b_enc is 0, so score[r, f] = W[f, r % d] with no rounding.
    Each (group, column) gets one of five patterns: 128 distinct values inside
    one 2^-16 relative bucket (every ordered word equal once its low 7 bits
    are dropped), a few such buckets, exact duplicates, negatives inside one
    bucket, and plain Gaussian values."""
    rng = np.random.default_rng(seed)
    X = np.zeros((B, d), dtype=np.float32)
    X[np.arange(B), np.arange(B) % d] = 1.0
    W = np.empty((F, d), dtype=np.float32)
    ulp = np.float32(2.0 ** -23)
    for g0 in range(0, F, 128):
        n = min(128, F - g0)
        for j in range(d):
            kind = rng.integers(0, 5)
            if kind == 0:
                v = 1 + rng.permutation(128)[:n].astype(np.float32) * ulp
            elif kind == 1:
                v = 1 + (rng.integers(0, 3, n) * 128 + rng.permutation(128)[:n]).astype(np.float32) * ulp
            elif kind == 2:
                v = 1 + rng.integers(0, 24, n).astype(np.float32) * ulp * 128
            elif kind == 3:
                v = -(1 + rng.permutation(128)[:n].astype(np.float32) * ulp)
            else:
                v = rng.standard_normal(n).astype(np.float32)
            W[g0:g0 + n, j] = v
    return X, W, np.zeros(F, dtype=np.float32)


@pytest.mark.parametrize("c", [16, 32, 64, 128])
def test_approx_candidates_truncated_ties(cuda_dev, c):
    """Per-group selection where the scores tie once truncated to 25 bits
    (and some tie exactly): the candidates must equal the oracle's bit for bit
    (values identify the latents here), and the final top-k exactly."""
    print(f"case approx candidates truncated ties c={c}", flush=True)
    B, d, F = 40, 32, 1280 + 77
    k = min(16, c)
    Xn, Wn, bn = _tie_heavy_inputs(B, d, F, seed=40 + c)
    X, W, b = (torch.from_numpy(a).to(cuda_dev) for a in (Xn, Wn, bn))
    nt = (F + 127) // 128
    cb = torch.empty((B, nt, c), dtype=torch.float32, device=cuda_dev)
    V, I = topk_sae_cuda_approx(X, W, b, k, c, candidate_buffer=cb)
    Vo, Io, cvo, cio = oracle.approx(Xn, Wn, bn, k, c, with_candidates=True)
    assert np.array_equal(cb.cpu().numpy(), cvo)
    assert np.array_equal(V.cpu().numpy(), Vo) and np.array_equal(I.cpu().numpy(), Io)


def test_candidate_heads_across_workgroup_runs(cuda_dev):
    """group_kernel collects each row's group heads in LDS over windows of 8
    aligned tiles and writes a window when it ends or when the workgroup's
    run of tiles does.  Here a run is 11 tiles on a 256-CU device (windows
    straddle the runs), the group count is odd and the last group partial.
    Two calls on one stream with different inputs: a head the flush missed
    would be the first call's, and cand_kernel, which skips groups by their
    heads, would then miss top-k latents of the second."""
    B, d, k, c = 40, 64, 16, 16
    G = 5621                          # 2811 tiles: 11 per workgroup over 256 workgroups
    F = G * 128 - 50
    print(f"case approx heads across runs B={B} F={F}", flush=True)
    nt = (F + 127) // 128
    for seed in (41, 42):
        X, W, b = make_inputs(B, d, F, torch.bfloat16, seed=seed, device=cuda_dev)
        cb = torch.empty((B, nt, c), dtype=torch.float32, device=cuda_dev)
        V, I = topk_sae_cuda_approx(X, W, b, k, c, candidate_buffer=cb)
        Ve, Ie = topk_sae_cuda_exact(X, W, b, k)
        assert torch.equal(V, Ve) and torch.equal(I, Ie), f"seed {seed}"
    _, _, cvo, cio = oracle.approx(_np(X), _np(W), _np(b), k, c, with_candidates=True)
    cbn = cb.cpu().numpy()
    pad = cio < 0
    assert np.array_equal(cbn[pad], cvo[pad])
    err = np.abs(cbn[~pad] - cvo[~pad]) / np.maximum(np.abs(cvo[~pad]), 1.0)
    assert err.max() <= 2e-3
