"""Seeded synthetic inputs of the benchmark configurations.

X ~ N(0, 1) of shape (B, d); W_enc ~ N(0, 1/d) of shape (F, d) with every row
then L2-normalised; b_enc ~ N(0, 0.1^2) fp32 of shape (F,) ("N(0, 0.1)" read
as standard deviation 0.1).  X and W_enc are generated in fp32 and then cast to
`dtype`; b_enc stays fp32.  `heavy_tail` scales a seeded 1% of the W_enc rows
by 5 after normalisation.  W_enc is generated on `device` in row chunks with a
per-chunk seed, so the same (seed, shape) gives the same tensors on any device
type that torch's generator supports there.
"""
import torch


def make_inputs(B, d, F, dtype=torch.bfloat16, seed=0, device="cuda", heavy_tail=False,
                chunk=65536):
    dev = torch.device(device)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    X = torch.randn(B, d, generator=g, device=dev, dtype=torch.float32).to(dtype)
    b = (0.1 * torch.randn(F, generator=g, device=dev, dtype=torch.float32)).contiguous()
    W = torch.empty(F, d, device=dev, dtype=dtype)
    for i, f0 in enumerate(range(0, F, chunk)):
        f1 = min(F, f0 + chunk)
        gc = torch.Generator(device=dev)
        gc.manual_seed(seed * 1000003 + 17 + i)
        w = torch.randn(f1 - f0, d, generator=gc, device=dev, dtype=torch.float32) * d ** -0.5
        w = w / w.norm(dim=1, keepdim=True).clamp_min(1e-30)
        W[f0:f1] = w.to(dtype)
    if heavy_tail and F > 0:
        gh = torch.Generator(device=dev)
        gh.manual_seed(seed * 7919 + 5)
        n = max(1, F // 100)
        rows = torch.randperm(F, generator=gh, device=dev)[:n]
        W[rows] = (W[rows].float() * 5.0).to(dtype)
    return X.contiguous(), W.contiguous(), b
