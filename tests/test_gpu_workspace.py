"""The op's workspace cache (streamtopk_sae.ops): one workspace per (device,
stream), reused by later calls on the stream and grown when a call needs more.

* consecutive calls on one stream share the workspace and give the same
  results as a call with a fresh one;
* a call on another stream gets a workspace of its own;
* a larger problem grows the stream's workspace, and a smaller problem after
  it runs in the larger workspace; every result is checked against the
  oracle's f64 scores.
"""
import pytest
import torch

import oracle
from parity import check_against_scores, tol_of
from streamtopk_sae import clear_workspace_cache, make_inputs, ops, topk_sae_cuda_approx, topk_sae_cuda_exact

pytestmark = pytest.mark.gpu


def _scores(X, W, b):
    return oracle.scores_f64(X.float().cpu().numpy(), W.float().cpu().numpy(), b.cpu().numpy())


def _key(dev, stream):
    return (dev.index, int(stream.cuda_stream))


def test_workspace_reused_per_stream(cuda_dev):
    print("case workspace reuse B=64 d=256 F=32768 k=32 bf16", flush=True)
    clear_workspace_cache()
    X, W, b = make_inputs(64, 256, 32768, torch.bfloat16, seed=11, device=cuda_dev)
    S = _scores(X, W, b)
    main = torch.cuda.current_stream(cuda_dev)
    V0, I0 = topk_sae_cuda_exact(X, W, b, 32)
    ws0 = ops._WS[_key(cuda_dev, main)]
    V1, I1 = topk_sae_cuda_exact(X, W, b, 32)
    assert ops._WS[_key(cuda_dev, main)].data_ptr() == ws0.data_ptr()
    torch.cuda.synchronize()
    assert torch.equal(V0, V1) and torch.equal(I0, I1)
    check_against_scores(V1.cpu().numpy(), I1.cpu().numpy(), S, 32, tol_of("bf16"), "reuse")

    side = torch.cuda.Stream(cuda_dev)
    side.wait_stream(main)
    with torch.cuda.stream(side):
        V2, I2 = topk_sae_cuda_exact(X, W, b, 32)
    main.wait_stream(side)
    ws_side = ops._WS[_key(cuda_dev, side)]
    assert ws_side.data_ptr() != ws0.data_ptr()
    torch.cuda.synchronize()
    assert torch.equal(V0, V2) and torch.equal(I0, I2)


def test_workspace_grows_then_serves_smaller(cuda_dev):
    print("case workspace growth: F=16384 k=16, F=262144 k=64, back to F=16384", flush=True)
    clear_workspace_cache()
    main = torch.cuda.current_stream(cuda_dev)
    small = make_inputs(32, 512, 16384, torch.bfloat16, seed=12, device=cuda_dev)
    big = make_inputs(128, 512, 262144, torch.bfloat16, seed=13, device=cuda_dev)
    Vs0, Is0 = topk_sae_cuda_exact(*small, 16)
    n_small = ops._WS[_key(cuda_dev, main)].numel()
    Vb, Ib = topk_sae_cuda_exact(*big, 64)
    n_big = ops._WS[_key(cuda_dev, main)].numel()
    assert n_big > n_small
    Vs1, Is1 = topk_sae_cuda_exact(*small, 16)
    # the approximate op (exact pipeline without a candidate buffer) shares it too
    Va, Ia = topk_sae_cuda_approx(*small, 16, 16)
    assert ops._WS[_key(cuda_dev, main)].numel() == n_big
    torch.cuda.synchronize()
    assert torch.equal(Vs0, Vs1) and torch.equal(Is0, Is1)
    assert torch.equal(Vs0, Va) and torch.equal(Is0, Ia)
    check_against_scores(Vs1.cpu().numpy(), Is1.cpu().numpy(), _scores(*small), 16, tol_of("bf16"), "small")
    rows = slice(0, 16)
    Xb, Wb, bb = big
    S = _scores(Xb[rows], Wb, bb)
    check_against_scores(Vb[rows].cpu().numpy(), Ib[rows].cpu().numpy(), S, 64, tol_of("bf16"), "big")
