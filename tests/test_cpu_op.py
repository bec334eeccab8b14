"""topk_sae_cpu (the OpenMP CPU encoder of libstreamtopk_hip.so) against the
oracle, on the shapes of the reference's tests/test_correctness.py:127-152,
287-293."""
import numpy as np
import pytest
import torch

import oracle
from golden.make_golden import load as load_golden
from parity import check_against_scores
from streamtopk_sae import topk_sae_cpu


def _inputs(B, d, F, seed):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(B, d, generator=g)
    W = torch.randn(F, d, generator=g) / d ** 0.5
    b = 0.1 * torch.randn(F, generator=g)
    return X, W, b


@pytest.mark.parametrize("B,d,F,k", [(4, 64, 256, 8), (32, 512, 4096, 32), (1024, 128, 512, 16),
                                     (16, 128, 512, 128), (3, 40, 16, 16)])
def test_cpu_op_vs_oracle(B, d, F, k):
    X, W, b = _inputs(B, d, F, B + F)
    V, I = topk_sae_cpu(X, W, b, k)
    assert V.dtype == torch.float32 and I.dtype == torch.int32 and V.shape == (B, k)
    S = oracle.scores_f64(X.numpy(), W.numpy(), b.numpy())
    check_against_scores(V.numpy(), I.numpy(), S, k, 1e-5, "cpu op")


def test_cpu_op_config0_shape():
    """BASELINE config 0 at its own shape and inputs (fp32 B=32 d=768 F=16384
    k=32, the seeded generator of the benchmark) against the oracle at the
    fp32 tolerance (reference tests/test_correctness.py:127-152)."""
    from streamtopk_sae import make_inputs
    X, W, b = make_inputs(32, 768, 16384, torch.float32, seed=0, device="cpu")
    V, I = topk_sae_cpu(X, W, b, 32)
    S = oracle.scores_f64(X.numpy(), W.numpy(), b.numpy())
    check_against_scores(V.numpy(), I.numpy(), S, 32, 1e-5, "cpu config0")
    Vo, Io = oracle.exact(X.numpy(), W.numpy(), b.numpy(), 32, nthreads=4)
    assert np.abs(V.numpy() - Vo).max() <= 1e-5 * max(1.0, float(np.abs(Vo).max()))


@pytest.mark.parametrize("k", [16, 32, 64])
def test_cpu_op_k(k):
    X, W, b = _inputs(16, 128, 512, k)
    V, I = topk_sae_cpu(X, W, b, k)
    S = oracle.scores_f64(X.numpy(), W.numpy(), b.numpy())
    check_against_scores(V.numpy(), I.numpy(), S, k, 1e-5, "cpu op k")


def test_cpu_op_upcasts_bf16():
    X, W, b = _inputs(8, 64, 300, 1)
    V, I = topk_sae_cpu(X.bfloat16(), W.bfloat16(), b, 8)
    S = oracle.scores_f64(X.bfloat16().float().numpy(), W.bfloat16().float().numpy(), b.numpy())
    check_against_scores(V.numpy(), I.numpy(), S, 8, 1e-5, "cpu bf16")


def test_cpu_op_known_answers():
    for X, W, b, k, Vk, Ik in load_golden():
        V, I = topk_sae_cpu(torch.from_numpy(X), torch.from_numpy(W), torch.from_numpy(b), k)
        assert np.array_equal(V.numpy(), Vk) and np.array_equal(I.numpy(), Ik)


def test_cpu_op_errors():
    X, W, b = _inputs(2, 16, 32, 0)
    with pytest.raises(RuntimeError, match="unsupported k=3"):
        topk_sae_cpu(X, W, b, 3)
    with pytest.raises(RuntimeError, match="k out of range"):
        topk_sae_cpu(X, W, b, 64)
    with pytest.raises(RuntimeError, match="W_enc d-dim mismatch"):
        topk_sae_cpu(X, W[:, :8], b, 4)
