"""F-sharding on one GPU: W_enc split into shards, each encoded with a global
index offset (stk_exact_forward_shard), the per-shard top-k results combined
by stk_topk_merge.  This is the per-GPU part of an F-sharded encoder (no
counterpart in the reference, which runs one device); the shards run one
after another on the one GPU here.  Checked against the C oracle's float64
scores of the whole dictionary, to the same bar as the unsharded encoder."""
import numpy as np
import pytest
import torch

import oracle
from parity import check_against_scores, tol_of
from streamtopk_sae import make_inputs, merge_topk_shards, topk_sae_cuda_exact

pytestmark = pytest.mark.gpu

DT = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}


def _np(t):
    return t.detach().float().cpu().numpy()


def _sharded(X, W, b, k, cuts):
    Vs, Is = [], []
    for lo, hi in zip(cuts[:-1], cuts[1:]):
        V, I = topk_sae_cuda_exact(X, W[lo:hi], b[lo:hi], k, f_offset=lo)
        Vs.append(V)
        Is.append(I)
    return merge_topk_shards(Vs, Is, k), (Vs, Is)


@pytest.mark.parametrize("B,d,F,k,dtype_name,cuts", [
    (64, 512, 32768, 32, "bf16", [0, 16384, 32768]),
    (64, 512, 32768, 32, "bf16", [0, 8192, 16384, 24576, 32768]),
    (33, 256, 30001, 16, "fp16", [0, 7001, 19000, 30001]),        # uneven shards, ragged B
    (16, 128, 20000, 8, "fp32", [0, 12345, 20000]),
    (512, 256, 16384, 16, "bf16", [0, 9000, 16384]),              # large-batch kernel
    (8, 128, 4096, 1, "bf16", [0, 1000, 2500, 4096]),             # k = 1
])
def test_shards_match_oracle(cuda_dev, B, d, F, k, dtype_name, cuts):
    X, W, b = make_inputs(B, d, F, DT[dtype_name], seed=11, device=cuda_dev)
    (V, I), (Vs, Is) = _sharded(X, W, b, k, cuts)
    torch.cuda.synchronize()
    S = oracle.scores_f64(_np(X), _np(W), _np(b))
    ties = check_against_scores(V.cpu().numpy(), I.cpu().numpy(), S, k, tol_of(dtype_name),
                                f"shards {cuts}")
    print(f"B={B} d={d} F={F} k={k} {dtype_name} shards={len(cuts) - 1}: near-ties {ties}")
    # every shard's own result is that shard's top-k, with global indices
    for (lo, hi), Vp, Ip in zip(zip(cuts[:-1], cuts[1:]), Vs, Is):
        Ip = Ip.cpu().numpy()
        assert np.all((Ip >= lo) & (Ip < hi))
        sub = np.full_like(S, -np.inf)
        sub[:, lo:hi] = S[:, lo:hi]
        check_against_scores(Vp.cpu().numpy(), Ip, sub, k, tol_of(dtype_name), f"shard {lo}:{hi}")
    # the unsharded encoder gives the same top-k up to near-ties
    V1, I1 = topk_sae_cuda_exact(X, W, b, k)
    torch.cuda.synchronize()
    rtol = tol_of(dtype_name)
    assert np.all(np.abs(V.cpu().numpy() - V1.cpu().numpy()) <= rtol * np.maximum(np.abs(V1.cpu().numpy()), 1.0))


def test_merge_single_part_is_identity(cuda_dev):
    X, W, b = make_inputs(32, 256, 8192, torch.bfloat16, seed=3, device=cuda_dev)
    V, I = topk_sae_cuda_exact(X, W, b, 16)
    V2, I2 = merge_topk_shards([V], [I], 16)
    torch.cuda.synchronize()
    assert torch.equal(V, V2) and torch.equal(I, I2)


def test_merge_orders_equal_values_by_index(cuda_dev):
    # two parts, k = 2; equal values across parts come out lower index first
    Vp = torch.tensor([[[1.0, 0.5]], [[1.0, 0.7]]], device=cuda_dev)
    Ip = torch.tensor([[[10, 20]], [[5, 30]]], dtype=torch.int32, device=cuda_dev)
    V, I = merge_topk_shards(Vp, Ip, 2)
    torch.cuda.synchronize()
    assert V.cpu().tolist() == [[1.0, 1.0]]
    assert I.cpu().tolist() == [[5, 10]]


def test_merge_many_parts(cuda_dev):
    # 40 parts x k=128 = 5120 candidates per row: the 8192-slot chunk variant
    g = torch.Generator(device="cpu").manual_seed(5)
    nparts, B, k = 40, 8, 128
    vals = torch.randn(nparts * k * B, generator=g).reshape(B, nparts * k)
    idx = torch.randperm(nparts * k * B, generator=g).reshape(B, nparts * k).to(torch.int32)
    top = torch.topk(vals, k, dim=1)
    Vp = vals.reshape(B, nparts, k).permute(1, 0, 2).contiguous().to(cuda_dev)
    Ip = idx.reshape(B, nparts, k).permute(1, 0, 2).contiguous().to(cuda_dev)
    V, I = merge_topk_shards(Vp, Ip, k)
    torch.cuda.synchronize()
    assert torch.equal(V.cpu(), top.values)
    assert torch.equal(I.cpu(), torch.gather(idx, 1, top.indices))


def test_shard_offset_beyond_int32_rejected(cuda_dev):
    X, W, b = make_inputs(4, 64, 256, torch.bfloat16, seed=0, device=cuda_dev)
    with pytest.raises(RuntimeError, match="int32 index range"):
        topk_sae_cuda_exact(X, W, b, 8, f_offset=2**31 - 100)


def test_merge_repeated_parts_keep_every_copy(cuda_dev):
    """Parts that repeat a latent (the same shard passed twice) give equal keys;
    they take consecutive ranks, so every output slot is written: each of the
    top k/2 latents appears twice, in order."""
    X, W, b = make_inputs(16, 256, 8192, torch.bfloat16, seed=4, device=cuda_dev)
    V, I = topk_sae_cuda_exact(X, W, b, 32)
    V2, I2 = merge_topk_shards([V, V], [I, I], 32)
    torch.cuda.synchronize()
    want_v = V[:, :16].repeat_interleave(2, dim=1)
    want_i = I[:, :16].repeat_interleave(2, dim=1)
    assert torch.equal(V2, want_v) and torch.equal(I2, want_i)
