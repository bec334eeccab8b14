"""streamtopk_sae_native: the reference's native-module surface over the C ABI.

The calls below are the ones the reference's ops.py makes on its native module
(streamtopk_sae/ops.py:40, 57, 75-81), including its Python-side finish of the
approximate path, and must agree with the package's own ops.
"""
import numpy as np
import pytest
import torch

import oracle
import streamtopk_sae_native as native
from parity import check_against_scores
from streamtopk_sae import make_inputs, topk_sae_cuda_approx, topk_sae_cuda_exact


def test_cpu_forward_matches_oracle():
    X, W, b = make_inputs(8, 96, 1000, torch.float32, seed=21, device="cpu")
    V, I = native.streamtopk_cpu_forward(X, W, b, 16)
    assert V.dtype == torch.float32 and I.dtype == torch.int32 and V.shape == (8, 16)
    S = oracle.scores_f64(X.numpy(), W.numpy(), b.numpy())
    check_against_scores(V.numpy(), I.numpy(), S, 16, 1e-5, "native cpu")


@pytest.mark.parametrize("which", ["X", "W_enc", "b_enc"])
def test_cpu_forward_requires_contiguous(which):
    X, W, b = make_inputs(4, 64, 256, torch.float32, seed=22, device="cpu")
    t = {"X": X, "W_enc": W, "b_enc": b}
    t[which] = torch.cat([t[which], t[which]], dim=-1)[..., ::2]   # same values, strided
    with pytest.raises(RuntimeError, match=f"{which} must be contiguous"):
        native.streamtopk_cpu_forward(t["X"], t["W_enc"], t["b_enc"], 8)


def test_cpu_forward_requires_fp32():
    X, W, b = make_inputs(4, 64, 256, torch.float32, seed=23, device="cpu")
    with pytest.raises(RuntimeError, match="X must be fp32"):
        native.streamtopk_cpu_forward(X.half(), W, b, 8)
    with pytest.raises(RuntimeError, match="b_enc must be fp32"):
        native.streamtopk_cpu_forward(X, W, b.double(), 8)


@pytest.mark.gpu
def test_cuda_exact_forward_matches_op(cuda_dev):
    X, W, b = make_inputs(64, 256, 20000, torch.bfloat16, seed=24, device=cuda_dev)
    V1, I1 = native.streamtopk_cuda_exact_forward(X, W, b, 32)
    V2, I2 = topk_sae_cuda_exact(X, W, b, 32)
    assert torch.equal(V1, V2) and torch.equal(I1, I2)
    with pytest.raises(RuntimeError, match="X must be contiguous"):
        native.streamtopk_cuda_exact_forward(X.t().contiguous().t(), W, b, 32)


@pytest.mark.gpu
@pytest.mark.parametrize("c", [16, 128])
def test_cuda_approx_forward_reference_flow(cuda_dev, c):
    """The reference's ops.py finish (torch.topk over the flat candidates, then
    gather) gives the same values as the device-side finish, and the same
    indices wherever the candidates hold no tied values."""
    B, d, F, k = 32, 256, 3000, 16
    X, W, b = make_inputs(B, d, F, torch.float16, seed=25, device=cuda_dev)
    flat_vals, flat_idxs, cand_vals, cand_idxs = native.streamtopk_cuda_approx_forward(X, W, b, k, c, None)
    nt = (F + 127) // 128
    assert flat_vals.shape == (B, nt * c) and flat_idxs.dtype == torch.int32
    assert cand_vals.shape == (B, nt, c) and flat_vals.data_ptr() == cand_vals.data_ptr()
    top_vals, top_pos = torch.topk(flat_vals, k, dim=-1)
    top_idxs = flat_idxs.gather(1, top_pos).to(torch.int32)
    V, I = topk_sae_cuda_approx(X, W, b, k, c)
    assert torch.equal(top_vals, V)
    S = (X.double() @ W.double().T + b.double()).cpu().numpy()
    check_against_scores(top_vals.cpu().numpy(), top_idxs.cpu().numpy(), S, k, 2e-3, "reference flow")
    same = (top_idxs == I).all(dim=1).cpu().numpy()
    vals = V.cpu().numpy()
    tied = np.array([len(set(r.tolist())) < k for r in vals])
    assert np.all(same | tied)
