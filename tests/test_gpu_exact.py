"""GPU parity of the exact encoder (topk_sae_cuda_exact -> stk_exact_forward).

Small and medium shapes are checked against the C oracle's float64 scores;
larger shapes against float64 scores computed on the GPU with torch (the same
quantity, cross-checked against the oracle in test_torch_f64_scores_match_oracle);
the full headline configuration through size-independent properties.
Shapes and edge cases follow the reference's tests/test_correctness.py:16-293.
"""
import numpy as np
import pytest
import torch

import oracle
from hooks import hooks
from parity import check_against_scores, term_magnitudes, tol_of
from streamtopk_sae import make_inputs, topk_sae_cuda_exact

pytestmark = pytest.mark.gpu

DT = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}


def _np(t):
    return t.detach().float().cpu().numpy()


def _oracle_scores(X, W, b):
    return oracle.scores_f64(_np(X), _np(W), _np(b))


def _gpu_scores_f64(X, W, b):
    return (X.double() @ W.double().T + b.double()).cpu().numpy()


def _run_check(X, W, b, k, dtype_name, scores="oracle", name="", max_tie_frac=None):
    """The op against float64 scores: values within the fp32 accumulation
    bound of each score's terms (parity.fp32_sum_bound), index sets equal up
    to near-ties of the k-th score (logged, optionally bounded)."""
    V, I = topk_sae_cuda_exact(X, W, b, k)
    torch.cuda.synchronize()
    assert V.dtype == torch.float32 and I.dtype == torch.int32
    assert V.device == X.device and I.device == X.device
    if scores == "oracle":
        S = _oracle_scores(X, W, b)
        A = term_magnitudes(_np(X), _np(W), _np(b))
    else:
        S = _gpu_scores_f64(X, W, b)
        A = term_magnitudes(X, W, b)
    ties = check_against_scores(V.cpu().numpy(), I.cpu().numpy(), S, k, tol_of(dtype_name), name,
                                A=A, d=X.shape[1], max_tie_frac=max_tie_frac)
    if ties:
        print(f"[ties] {name}: {ties} row(s) with near-tie index differences")
    return V, I


SHAPES = {
    "small": dict(B=4, d=64, F=256, k=8),
    "medium": dict(B=32, d=512, F=4096, k=32),
    "sampled": dict(B=64, d=256, F=20000, k=64),
}


@pytest.mark.parametrize("shape", list(SHAPES))
@pytest.mark.parametrize("dtype_name", ["fp32", "fp16", "bf16"])
def test_exact_shapes(cuda_dev, shape, dtype_name):
    c = SHAPES[shape]
    print(f"case exact {shape} {dtype_name} {c}", flush=True)
    X, W, b = make_inputs(c["B"], c["d"], c["F"], DT[dtype_name], seed=42, device=cuda_dev)
    _run_check(X, W, b, c["k"], dtype_name, name=f"{shape}/{dtype_name}")


@pytest.mark.parametrize("k", [1, 2, 4, 8, 16, 32, 64, 128])
def test_exact_k_sweep(cuda_dev, k):
    print(f"case k-sweep k={k}", flush=True)
    X, W, b = make_inputs(16, 128, 512, torch.bfloat16, seed=3, device=cuda_dev)
    _run_check(X, W, b, k, "bf16", name=f"k={k}")


@pytest.mark.parametrize("k", [1, 32, 64, 128])
def test_exact_k_sweep_sampled(cuda_dev, k):
    """F >= 16384 turns on the sampled threshold seed; every k through it."""
    print(f"case k-sweep sampled k={k}", flush=True)
    X, W, b = make_inputs(40, 256, 16384 + 37, torch.bfloat16, seed=4, device=cuda_dev)
    _run_check(X, W, b, k, "bf16", name=f"sampled k={k}")


@pytest.mark.parametrize("B", [1, 31, 33, 97, 130, 300])
def test_exact_ragged_batch(cuda_dev, B):
    print(f"case ragged B={B}", flush=True)
    X, W, b = make_inputs(B, 128, 3000, torch.bfloat16, seed=5, device=cuda_dev)
    _run_check(X, W, b, 16, "bf16", name=f"B={B}")


def test_exact_k128_many_rows(cuda_dev):
    """k=128 uses 64-row workgroups; B=200 spans several row chunks."""
    X, W, b = make_inputs(200, 192, 20000, torch.bfloat16, seed=6, device=cuda_dev)
    _run_check(X, W, b, 128, "bf16", name="k128 B200")


def test_exact_ragged_d(cuda_dev):
    """d not a multiple of 8 (fp16/bf16) or 4 (fp32): the op pads X and W_enc
    with zero columns."""
    X, W, b = make_inputs(8, 100, 600, torch.bfloat16, seed=7, device=cuda_dev)
    _run_check(X, W, b, 16, "bf16", name="d=100")
    X, W, b = make_inputs(8, 30, 600, torch.float32, seed=7, device=cuda_dev)
    _run_check(X, W, b, 8, "fp32", name="d=30 fp32")


# d a multiple of 16 bytes but not of one 128-byte d-step: the kernels mask
# the partial last step themselves (no copy of W_enc).  Every streaming kernel
# and the sample passes (F >= 16384), with row blocks past B.
RAGGED_D = [
    dict(B=40, d=200, F=20000, k=32, dtype_name="bf16"),      # main_kernel + sample_kernel
    dict(B=7, d=8, F=3000, k=8, dtype_name="fp16"),           # one partial step only
    dict(B=100, d=1000, F=17000, k=64, dtype_name="fp32"),    # fp32: 32-element steps, 8 valid in the last
    dict(B=600, d=200, F=20000, k=64, dtype_name="bf16"),     # mainl_kernel + its sample mode
    dict(B=520, d=36, F=3000, k=16, dtype_name="fp32"),       # mainl_kernel, one partial step per tile row
]


@pytest.mark.parametrize("shape", RAGGED_D, ids=lambda s: f"B{s['B']}-d{s['d']}-{s['dtype_name']}")
def test_exact_ragged_d_in_kernel(cuda_dev, shape):
    c = shape
    print(f"case ragged d in kernel {c}", flush=True)
    X, W, b = make_inputs(c["B"], c["d"], c["F"], DT[c["dtype_name"]], seed=8, device=cuda_dev)
    nb = ctypes_workspace_bytes(c)
    assert nb > 0   # accepted by the C ABI as is (no padding in the op)
    _run_check(X, W, b, c["k"], c["dtype_name"], scores="torch64", name=f"ragged d {c}")


def ctypes_workspace_bytes(c):
    import ctypes
    from streamtopk_sae import _lib
    dt = {"fp32": _lib.STK_DTYPE_F32, "fp16": _lib.STK_DTYPE_F16, "bf16": _lib.STK_DTYPE_BF16}[c["dtype_name"]]
    nb = ctypes.c_size_t(0)
    _lib.check(_lib.load().stk_exact_workspace_bytes(c["B"], c["d"], c["F"], c["k"], dt, ctypes.byref(nb)))
    return nb.value


@pytest.mark.parametrize("c", [16, 128])
def test_approx_ragged_d_in_kernel(cuda_dev, c):
    """The candidate-buffer kernel with a partial last d-step (d = 200 bf16)."""
    print(f"case approx ragged d c={c}", flush=True)
    B, d, F, k = 40, 200, 3000, 16
    X, W, b = make_inputs(B, d, F, torch.bfloat16, seed=9, device=cuda_dev)
    cb = torch.empty((B, (F + 127) // 128, c), dtype=torch.float32, device=cuda_dev)
    from streamtopk_sae import topk_sae_cuda_approx
    V, I = topk_sae_cuda_approx(X, W, b, k, c, candidate_buffer=cb)
    _, _, cvo, cio = oracle.approx(_np(X), _np(W), _np(b), k, c, with_candidates=True)
    err = np.abs(cb.cpu().numpy() - cvo) / np.maximum(np.abs(cvo), 1.0)
    assert err.max() <= 2e-3
    S = _oracle_scores(X, W, b)
    check_against_scores(V.cpu().numpy(), I.cpu().numpy(), S, k, 2e-3, "approx ragged d")


def test_edge_k_equals_F(cuda_dev):
    X, W, b = make_inputs(4, 64, 16, torch.float32, seed=8, device=cuda_dev)
    V, I = _run_check(X, W, b, 16, "fp32", name="k=F")
    for i in range(4):
        assert sorted(I[i].tolist()) == list(range(16))


def test_edge_k_equals_1(cuda_dev):
    X, W, b = make_inputs(8, 64, 256, torch.bfloat16, seed=9, device=cuda_dev)
    V, I = _run_check(X, W, b, 1, "bf16", name="k=1")
    S = _oracle_scores(X, W, b)
    assert np.array_equal(I.cpu().numpy()[:, 0], np.argmax(S, axis=1))


def test_edge_F_not_multiple_of_tile(cuda_dev):
    X, W, b = make_inputs(8, 128, 300, torch.bfloat16, seed=10, device=cuda_dev)
    _run_check(X, W, b, 16, "bf16", name="F=300")


def test_edge_all_zero_X(cuda_dev):
    """Scores are exactly b: the result is the top-k of b, bit for bit."""
    for F in (128, 20011):
        X = torch.zeros(4, 64, dtype=torch.bfloat16, device=cuda_dev)
        _, W, b = make_inputs(4, 64, F, torch.bfloat16, seed=11, device=cuda_dev)
        V, I = topk_sae_cuda_exact(X, W, b, 8)
        bv = b.cpu().numpy()
        order = np.lexsort((np.arange(F), -bv.astype(np.float64)))[:8]
        for i in range(4):
            assert np.array_equal(I[i].cpu().numpy(), order)
            assert np.array_equal(V[i].cpu().numpy(), bv[order])


def test_edge_large_bias(cuda_dev):
    """One bias entry at +1e4 must be rank 0 in every row."""
    X, W, b = make_inputs(16, 64, 20000, torch.bfloat16, seed=12, device=cuda_dev)
    b[12345] = 1e4
    V, I = _run_check(X, W, b, 8, "bf16", name="bias 1e4")
    assert torch.all(I[:, 0] == 12345)


def test_edge_batch_zero(cuda_dev):
    X, W, b = make_inputs(1, 64, 256, torch.bfloat16, seed=13, device=cuda_dev)
    V, I = topk_sae_cuda_exact(X[:0], W, b, 8)
    assert V.shape == (0, 8) and I.shape == (0, 8)


@pytest.mark.parametrize("F", [8000, 20480])
def test_increasing_scores_adversarial(cuda_dev, F):
    """Scores increase along F, so every later latent beats the running
    threshold: exercises the queue-compaction path on every tile (F=8000 has
    no sampled seed; F=20480 does)."""
    B, d, k = 8, 64, 64
    X = torch.ones(B, d, dtype=torch.float32, device=cuda_dev)
    W = torch.zeros(F, d, dtype=torch.float32, device=cuda_dev)
    b = torch.arange(F, dtype=torch.float32, device=cuda_dev) * 1e-3
    _run_check(X, W, b, k, "fp32", name="increasing")
    V, I = topk_sae_cuda_exact(X, W, b, k)
    assert np.array_equal(I[0].cpu().numpy(), np.arange(F - 1, F - 1 - k, -1))


def test_exact_ties_lower_index_first(cuda_dev):
    """All scores equal: the k lowest indices, in order."""
    X = torch.zeros(3, 64, dtype=torch.bfloat16, device=cuda_dev)
    W = torch.zeros(5000, 64, dtype=torch.bfloat16, device=cuda_dev)
    b = torch.full((5000,), 0.5, dtype=torch.float32, device=cuda_dev)
    V, I = topk_sae_cuda_exact(X, W, b, 32)
    assert torch.all(I == torch.arange(32, device=cuda_dev, dtype=torch.int32))
    assert torch.all(V == 0.5)


def test_torch_f64_scores_match_oracle(cuda_dev):
    X, W, b = make_inputs(16, 256, 2048, torch.bfloat16, seed=14, device=cuda_dev)
    S1 = _oracle_scores(X, W, b)
    S2 = _gpu_scores_f64(X, W, b)
    assert np.max(np.abs(S1 - S2)) < 1e-9


@pytest.mark.parametrize("dtype_name", ["bf16", "fp16", "fp32"])
def test_exact_config1_shape(cuda_dev, dtype_name):
    """BASELINE config 1 shape (B=128 d=768 F=65536 k=32)."""
    print(f"case config1 {dtype_name}", flush=True)
    X, W, b = make_inputs(128, 768, 65536, DT[dtype_name], seed=0, device=cuda_dev)
    _run_check(X, W, b, 32, dtype_name, scores="torch64", name=f"config1/{dtype_name}")


def test_exact_deterministic(cuda_dev):
    X, W, b = make_inputs(64, 512, 40000, torch.bfloat16, seed=15, device=cuda_dev)
    V1, I1 = topk_sae_cuda_exact(X, W, b, 64)
    V2, I2 = topk_sae_cuda_exact(X, W, b, 64)
    assert torch.equal(V1, V2) and torch.equal(I1, I2)


@pytest.mark.parametrize("dtype_name", ["fp32", "fp16", "bf16"])
def test_exact_known_answers(cuda_dev, dtype_name):
    """Scores exact in every dtype: values bit-exact and indices identical,
    lower index first among equal scores (tests/golden/make_golden.py)."""
    from golden.make_golden import load as load_golden
    for X, W, b, k, Vk, Ik in load_golden():
        Xt = torch.from_numpy(X).to(cuda_dev).to(DT[dtype_name])
        Wt = torch.from_numpy(W).to(cuda_dev).to(DT[dtype_name])
        bt = torch.from_numpy(b).to(cuda_dev)
        V, I = topk_sae_cuda_exact(Xt, Wt, bt, k)
        assert np.array_equal(V.cpu().numpy(), Vk), f"{dtype_name} {X.shape} {W.shape} k={k}"
        assert np.array_equal(I.cpu().numpy(), Ik), f"{dtype_name} {X.shape} {W.shape} k={k}"


# BASELINE config 2 (headline) at full size: B=128 d=2048 F=262144 k=64, and
# its edge cases (F=262143, k=1, all-zero X, one b_enc entry at +1e4).
C2 = dict(B=128, d=2048, F=262144, k=64)


@pytest.mark.parametrize("dtype_name", ["bf16", "fp16", "fp32"])
def test_exact_headline_config(cuda_dev, dtype_name):
    print(f"case headline {dtype_name}", flush=True)
    X, W, b = make_inputs(C2["B"], C2["d"], C2["F"], DT[dtype_name], seed=0, device=cuda_dev)
    _run_check(X, W, b, C2["k"], dtype_name, scores="torch64", name=f"headline/{dtype_name}", max_tie_frac=0.02)


def test_exact_headline_F_not_multiple_of_tile(cuda_dev):
    print("case headline F=262143", flush=True)
    X, W, b = make_inputs(C2["B"], C2["d"], C2["F"] - 1, torch.bfloat16, seed=1, device=cuda_dev)
    V, I = _run_check(X, W, b, C2["k"], "bf16", scores="torch64", name="headline/F=262143")
    assert int(I.max()) < C2["F"] - 1 and int(I.min()) >= 0


def test_exact_headline_k1(cuda_dev):
    print("case headline k=1", flush=True)
    X, W, b = make_inputs(C2["B"], C2["d"], C2["F"], torch.bfloat16, seed=2, device=cuda_dev)
    V, I = _run_check(X, W, b, 1, "bf16", scores="torch64", name="headline/k=1")
    # k=1 is the row argmax: its value must be the row maximum of the float64 scores
    Smax = (X.double() @ W.double().T + b.double()).max(dim=1).values.float()
    assert torch.allclose(V[:, 0], Smax, rtol=2e-3, atol=2e-3)


def test_exact_headline_zero_X(cuda_dev):
    """All-zero X: every row's result is the top-k of b_enc, bit-exact, lower index first."""
    print("case headline zero X", flush=True)
    _, W, b = make_inputs(C2["B"], C2["d"], C2["F"], torch.bfloat16, seed=3, device=cuda_dev)
    X = torch.zeros(C2["B"], C2["d"], dtype=torch.bfloat16, device=cuda_dev)
    V, I = topk_sae_cuda_exact(X, W, b, C2["k"])
    bn = b.cpu().numpy()
    order = np.lexsort((np.arange(bn.size), -bn.astype(np.float64)))[:C2["k"]]
    assert np.array_equal(I.cpu().numpy(), np.broadcast_to(order.astype(np.int32), (C2["B"], C2["k"])))
    assert np.array_equal(V.cpu().numpy(), np.broadcast_to(bn[order], (C2["B"], C2["k"])))


def test_exact_headline_large_bias(cuda_dev):
    """One b_enc entry at +1e4: that latent is rank 0 of every row."""
    print("case headline large bias", flush=True)
    X, W, b = make_inputs(C2["B"], C2["d"], C2["F"], torch.bfloat16, seed=4, device=cuda_dev)
    j = 123457
    b[j] = 1e4
    V, I = _run_check(X, W, b, C2["k"], "bf16", scores="torch64", name="headline/bias")
    assert torch.all(I[:, 0] == j)


# Large batches (B >= 512) run the 256-row streaming kernel with per-workgroup
# queue segments in global memory.
LARGE = {
    "large_sampled": dict(B=512, d=256, F=20000, k=128),
    "large_unsampled_ragged": dict(B=600, d=128, F=3000, k=16),
    "large_k64": dict(B=1024, d=512, F=40000, k=64),
    "large_sample8k": dict(B=520, d=128, F=70001, k=128),   # F >= 65536: 8192 sampled latents
    # d not a multiple of the kernel's 64-element (fp32: 32) d-step: the
    # instances built for a partial last step, with the exchange and with the
    # sample pass
    "large_tail_d200": dict(B=512, d=200, F=20000, k=64),
    "large_tail_sampled_d72": dict(B=520, d=72, F=70001, k=128),
    # the d-step loop runs steps in pairs, each step also finishing the
    # previous one's last MFMAs: an odd step count (a padded step of zeros),
    # a single step (fp16/bf16), and a single partial step
    "large_odd_steps_d192": dict(B=520, d=192, F=20000, k=64),
    "large_one_step_d64": dict(B=512, d=64, F=5000, k=32),
    "large_one_partial_step_d40": dict(B=512, d=40, F=3000, k=16),
}


@pytest.mark.parametrize("shape", list(LARGE))
@pytest.mark.parametrize("dtype_name", ["fp32", "fp16", "bf16"])
def test_exact_large_batch(cuda_dev, shape, dtype_name):
    c = LARGE[shape]
    print(f"case large {shape} {dtype_name} {c}", flush=True)
    X, W, b = make_inputs(c["B"], c["d"], c["F"], DT[dtype_name], seed=31, device=cuda_dev)
    _run_check(X, W, b, c["k"], dtype_name, scores="torch64", name=f"{shape}/{dtype_name}")


@pytest.mark.parametrize("k", [1, 2, 4, 8, 16, 32, 64, 128])
def test_exact_large_batch_k_sweep(cuda_dev, k):
    print(f"case large k-sweep k={k}", flush=True)
    X, W, b = make_inputs(513, 128, 16384 + 300, torch.bfloat16, seed=32, device=cuda_dev)
    _run_check(X, W, b, k, "bf16", scores="torch64", name=f"large k={k}")


@pytest.mark.parametrize("F", [8000, 20480])
def test_large_batch_increasing_scores_adversarial(cuda_dev, F):
    """Scores increase along F: every segment overflows and is compacted on
    every tile, in the large-batch kernel."""
    print(f"case large increasing F={F}", flush=True)
    B, d, k = 512, 64, 128
    X = torch.ones(B, d, dtype=torch.float32, device=cuda_dev)
    W = torch.zeros(F, d, dtype=torch.float32, device=cuda_dev)
    b = torch.arange(F, dtype=torch.float32, device=cuda_dev) * 1e-3
    V, I = topk_sae_cuda_exact(X, W, b, k)
    want = np.arange(F - 1, F - 1 - k, -1)
    In = I.cpu().numpy()
    assert all(np.array_equal(In[i], want) for i in range(B))
    assert np.array_equal(V[0].cpu().numpy(), b.cpu().numpy()[want])


@pytest.mark.parametrize("heavy", [False, True])
def test_exact_config4_shape(cuda_dev, heavy):
    """BASELINE config 4 at full size (B=1024 d=4096 F=262144 k=128), with and
    without the heavy-tailed W_enc (1% of rows scaled 5x)."""
    print(f"case config4 heavy={heavy}", flush=True)
    X, W, b = make_inputs(1024, 4096, 262144, torch.bfloat16, seed=0, device=cuda_dev, heavy_tail=heavy)
    _run_check(X, W, b, 128, "bf16", scores="torch64", name=f"config4/heavy={heavy}", max_tie_frac=0.02)


@pytest.mark.parametrize("B,F,k", [(64, 20480, 64), (512, 8000, 128)])
def test_retry_bound_marks_output(cuda_dev, B, F, k):
    """The streaming kernels' spill-and-retry loops are bounded.  With the
    bound forced down from the host (the max_rounds test hook, which the
    library reads at each call), scores that rise along F overflow every tile and
    reach it: the call then marks its output (indices -1, values NaN) rather
    than returning a result with candidates missing.  With the default bounds
    the same inputs give the exact answer.  B=64 runs main_kernel, B=512
    mainl_kernel."""
    print(f"case retry bound B={B} F={F} k={k}", flush=True)
    d = 64
    X = torch.ones(B, d, dtype=torch.float32, device=cuda_dev)
    W = torch.zeros(F, d, dtype=torch.float32, device=cuda_dev)
    b = torch.arange(F, dtype=torch.float32, device=cuda_dev) * 1e-3
    with hooks(max_rounds=0):
        V, I = topk_sae_cuda_exact(X, W, b, k)
    assert bool((I == -1).all()) and bool(torch.isnan(V).all())
    V, I = topk_sae_cuda_exact(X, W, b, k)
    want = np.arange(F - 1, F - 1 - k, -1)
    assert all(np.array_equal(r, want) for r in I.cpu().numpy())
    assert np.array_equal(V[0].cpu().numpy(), b.cpu().numpy()[want])
