"""GPU parity at the BASELINE configurations that the per-kernel suites leave
out, and the approximate op's less common arguments.

* Config 3 at full size (bf16, B=128, d=2048, F=2^20; k=32, k=16 at c=16),
  every c in {16, 32, 64, 128}: the default path (no candidate buffer) and the
  candidate-buffer path (group_kernel + cand_kernel) against float64 scores
  computed on the GPU, the per-group top-c of sampled rows against the same
  scores, and recall@k against the exact kernel (reference
  tests/test_recall.py:22-96, bench/run_recall.py:77-92).
* Config 0's shape (fp32, B=32, d=768, F=16384, k=32) on the device path
  against the C oracle (reference tests/test_correctness.py:127-152 checks the
  CPU path at this shape; tests/test_cpu_op.py does that here).
* The large-batch regime at B=2048 (reference bench/run_max_F.py CONFIGS:
  B=2048, d=768, k=32, bf16).
* topk_sae_cuda_approx with k not a power of two and with d > 4096, which the
  approximate op accepts (streamtopk_approx.cu:243-259 has neither limit).
"""
import numpy as np
import pytest
import torch

import oracle
from parity import check_against_scores, term_magnitudes
from streamtopk_sae import make_inputs, recall_at_k, topk_sae_cuda_approx, topk_sae_cuda_exact

pytestmark = pytest.mark.gpu

C3 = dict(B=128, d=2048, F=1 << 20)


def _np(t):
    return t.detach().float().cpu().numpy()


def _scores_f64(X, W, b, chunk=1 << 16, magnitudes=False):
    """float64 scores X @ W.T + b on the GPU, F-chunk by F-chunk, as a host
    array; with magnitudes, also |X| @ |W|.T + |b| (parity.term_magnitudes)."""
    out = np.empty((X.shape[0], W.shape[0]), dtype=np.float64)
    mag = np.empty_like(out) if magnitudes else None
    Xd = X.double()
    for f0 in range(0, W.shape[0], chunk):
        f1 = min(W.shape[0], f0 + chunk)
        out[:, f0:f1] = (Xd @ W[f0:f1].double().T + b[f0:f1].double()).cpu().numpy()
        if magnitudes:
            mag[:, f0:f1] = term_magnitudes(X, W[f0:f1], b[f0:f1])
    return (out, mag) if magnitudes else out


@pytest.fixture(scope="module")
def c3(cuda_dev):
    print("case config3 inputs", flush=True)
    X, W, b = make_inputs(C3["B"], C3["d"], C3["F"], torch.bfloat16, seed=0, device=cuda_dev)
    S, A = _scores_f64(X, W, b, magnitudes=True)
    exact = {k: topk_sae_cuda_exact(X, W, b, k) for k in (16, 32)}
    return X, W, b, S, A, exact


def _k_of(c):
    # the approximate op requires k <= c (streamtopk_approx.cu:248)
    return min(32, c)


@pytest.mark.parametrize("c", [16, 32, 64, 128])
def test_config3_default_path(c3, c):
    X, W, b, S, A, exact = c3
    k = _k_of(c)
    print(f"case config3 default c={c} k={k}", flush=True)
    V, I = topk_sae_cuda_approx(X, W, b, k, c)
    ties = check_against_scores(V.cpu().numpy(), I.cpu().numpy(), S, k, 2e-3, f"config3 c={c}",
                                A=A, d=C3["d"], max_tie_frac=0.02)
    if ties:
        print(f"[ties] config3 c={c}: {ties} row(s)")
    # k <= c: the union of the per-group top-c holds the exact top-k
    Ve, Ie = exact[k]
    assert torch.equal(V, Ve) and torch.equal(I, Ie)
    assert recall_at_k(I, Ie) == 1.0


def _check_group_candidates(cv, ci, S_row, c, tol, name, A_row=None, d=None):
    """One row's (G, c) candidates against its float64 scores: each group's
    top-c (value descending, near-ties allowed), padded past F; with A_row,
    values held to the fp32 accumulation bound."""
    G = cv.shape[0]
    F = S_row.size
    Sg = np.full((G, 128), -np.inf)
    Sg.reshape(-1)[:F] = S_row
    Ag = None
    if A_row is not None:
        Ag = np.zeros((G, 128))
        Ag.reshape(-1)[:F] = A_row
    assert np.all(np.diff(cv, axis=1) <= 0), f"{name}: candidates not descending"
    real = ci >= 0
    assert np.all(cv[~real] == np.float32(-3.402823466e38)), f"{name}: padding value"
    n_real = np.minimum(128, F - 128 * np.arange(G))
    assert np.array_equal(real.sum(axis=1), np.minimum(c, n_real)), f"{name}: padding count"
    g_of = np.where(real, ci // 128, np.arange(G)[:, None])
    assert np.all(g_of == np.arange(G)[:, None]), f"{name}: candidate outside its group"
    full = n_real >= c
    local = np.where(real, ci - 128 * np.arange(G)[:, None], 0)
    return check_against_scores(cv[full], local[full], Sg[full], c, tol, name,
                                A=None if Ag is None else Ag[full], d=d)


@pytest.mark.parametrize("c", [16, 32, 64, 128])
def test_config3_candidate_buffer(c3, c):
    X, W, b, S, A, exact = c3
    k = _k_of(c)
    G = C3["F"] // 128
    print(f"case config3 candidates c={c} k={k}", flush=True)
    cb = torch.empty((C3["B"], G, c), dtype=torch.float32, device=X.device)
    V, I = topk_sae_cuda_approx(X, W, b, k, c, candidate_buffer=cb)
    check_against_scores(V.cpu().numpy(), I.cpu().numpy(), S, k, 2e-3, f"config3 cand c={c}",
                         A=A, d=C3["d"], max_tie_frac=0.02)
    # the same latents as the exact kernel; values to fp32 rounding (the exact
    # path scores its sampled latents in d ranges, summed in another order)
    # (a latent tied with the k-th to within that rounding may trade places)
    Ve, Ie = exact[k]
    assert recall_at_k(I, Ie) >= 0.999
    assert torch.allclose(V, Ve, rtol=1e-5, atol=1e-5)
    # the per-group top-c, read back with their indices through the native op
    # (approx_forward returns the index buffer the public op keeps internal)
    from streamtopk_sae.ops import approx_forward
    _, _, cv, ci = approx_forward(X, W, b, k, c, candidates=True)
    assert torch.equal(cv, cb)
    cvn, cin = cv.cpu().numpy(), ci.cpu().numpy()
    for r in (0, 61, 127):
        ties = _check_group_candidates(cvn[r], cin[r], S[r], c, 2e-3, f"config3 c={c} row {r}",
                                       A_row=A[r], d=C3["d"])
        if ties:
            print(f"[ties] config3 c={c} row {r}: {ties} group(s)")


def test_config3_recall_per_c(c3):
    """recall@k of the approximate op against the exact kernel for every c
    (run_recall.py:77-92 statistics): non-decreasing in c, and 1 because
    k <= c (reference test_recall.py:22-96 asks for > 0.9 at c=128)."""
    X, W, b, S, A, exact = c3
    rec = []
    for c in (16, 32, 64, 128):
        k = _k_of(c)
        _, I = topk_sae_cuda_approx(X, W, b, k, c)
        rec.append(recall_at_k(I, exact[k][1]))
    print(f"[recall] config3 c=16,32,64,128: {rec}")
    assert all(r1 >= r0 for r0, r1 in zip(rec, rec[1:]))
    assert rec[-1] > 0.9 and all(r == 1.0 for r in rec)


def test_config0_shape_device_fp32(cuda_dev):
    """Config 0's shape and dtype (fp32 B=32 d=768 F=16384 k=32) on the device
    path, against the C oracle's float64 scores at the fp32 tolerance."""
    print("case config0 shape fp32 device", flush=True)
    X, W, b = make_inputs(32, 768, 16384, torch.float32, seed=0, device=cuda_dev)
    V, I = topk_sae_cuda_exact(X, W, b, 32)
    S = oracle.scores_f64(_np(X), _np(W), _np(b))
    check_against_scores(V.cpu().numpy(), I.cpu().numpy(), S, 32, 1e-5, "config0 device")
    Vo, Io = oracle.exact(_np(X), _np(W), _np(b), 32)
    assert np.abs(V.cpu().numpy() - Vo).max() <= 1e-5 * max(1.0, float(np.abs(Vo).max()))


def test_large_batch_b2048(cuda_dev):
    """B=2048 (the reference's max-F configuration, bench/run_max_F.py:18-21:
    d=768, k=32, bf16) at F=131072: eight 256-row blocks of the large-batch
    kernel and the 8192-latent sample."""
    print("case B=2048 d=768 F=131072 k=32", flush=True)
    X, W, b = make_inputs(2048, 768, 131072, torch.bfloat16, seed=5, device=cuda_dev)
    V, I = topk_sae_cuda_exact(X, W, b, 32)
    S, A = _scores_f64(X, W, b, magnitudes=True)
    ties = check_against_scores(V.cpu().numpy(), I.cpu().numpy(), S, 32, 2e-3, "B=2048",
                                A=A, d=768, max_tie_frac=0.02)
    if ties:
        print(f"[ties] B=2048: {ties} row(s)")


@pytest.mark.parametrize("k,c", [(3, 16), (20, 32), (5, 128)])
@pytest.mark.parametrize("with_buffer", [False, True])
def test_approx_k_not_power_of_two(cuda_dev, k, c, with_buffer):
    """The approximate op accepts any 1 <= k <= c; the default path runs the
    exact pipeline with that k, the buffer path selects k from the groups."""
    print(f"case approx k={k} c={c} buffer={with_buffer}", flush=True)
    B, d, F = 40, 128, 20000
    X, W, b = make_inputs(B, d, F, torch.bfloat16, seed=50 + k, device=cuda_dev)
    cb = torch.empty((B, (F + 127) // 128, c), dtype=torch.float32, device=cuda_dev) if with_buffer else None
    V, I = topk_sae_cuda_approx(X, W, b, k, c, candidate_buffer=cb)
    S = oracle.scores_f64(_np(X), _np(W), _np(b))
    check_against_scores(V.cpu().numpy(), I.cpu().numpy(), S, k, 2e-3, f"approx k={k} c={c}")
    Vo, Io, cvo, cio = oracle.approx(_np(X), _np(W), _np(b), k, c, with_candidates=True)
    if with_buffer:
        cbn = cb.cpu().numpy()
        err = np.abs(cbn - cvo) / np.maximum(np.abs(cvo), 1.0)
        assert err.max() <= 2e-3


@pytest.mark.parametrize("with_buffer", [False, True])
def test_approx_d_above_4096(cuda_dev, with_buffer):
    """d = 4160 (> the exact op's D_MAX=4096, which the approximate op does not
    impose) on both approximate paths."""
    print(f"case approx d=4160 buffer={with_buffer}", flush=True)
    B, d, F, k, c = 16, 4160, 5000, 16, 32
    X, W, b = make_inputs(B, d, F, torch.bfloat16, seed=60, device=cuda_dev)
    cb = torch.empty((B, (F + 127) // 128, c), dtype=torch.float32, device=cuda_dev) if with_buffer else None
    V, I = topk_sae_cuda_approx(X, W, b, k, c, candidate_buffer=cb)
    S = oracle.scores_f64(_np(X), _np(W), _np(b))
    check_against_scores(V.cpu().numpy(), I.cpu().numpy(), S, k, 2e-3, f"approx d=4160")


def test_approx_candidate_buffer_misaligned(cuda_dev):
    """A contiguous candidate_buffer view at a storage offset that is not
    16-byte aligned (the kernel writes 16-byte vectors) is filled correctly."""
    print("case approx misaligned candidate buffer", flush=True)
    B, d, F, k, c = 8, 64, 1000, 16, 16
    X, W, b = make_inputs(B, d, F, torch.bfloat16, seed=61, device=cuda_dev)
    nt = (F + 127) // 128
    store = torch.full((B * nt * c + 1,), 7.0, dtype=torch.float32, device=cuda_dev)
    cb = store[1:].view(B, nt, c)
    assert cb.data_ptr() % 16 != 0 and cb.is_contiguous()
    V, I = topk_sae_cuda_approx(X, W, b, k, c, candidate_buffer=cb)
    _, _, cvo, _ = oracle.approx(_np(X), _np(W), _np(b), k, c, with_candidates=True)
    err = np.abs(cb.cpu().numpy() - cvo) / np.maximum(np.abs(cvo), 1.0)
    assert err.max() <= 2e-3
    assert float(store[0]) == 7.0
