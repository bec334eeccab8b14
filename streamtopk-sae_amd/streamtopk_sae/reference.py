"""Dense reference encoder (reference: streamtopk_sae/reference.py:9-19).

``reference_topk_sae`` materialises the full (B, F) score matrix, so it is a
baseline for small and medium shapes, not the streaming path.  Unlike the
reference, which multiplies in the input dtype and so rounds bf16/fp16 scores
before the bias is added (reference.py:17), the scores here are formed from
the upcast fp32 inputs -- the quantity the streaming kernels compute.  Values
are sorted descending; indices are int32 (reference.py:18-19).
"""
import torch


def reference_topk_sae(X, W_enc, b_enc, k):
    """X (B, d), W_enc (F, d), b_enc (F,) -> values (B, k) fp32, indices (B, k) int32."""
    preacts = X.float() @ W_enc.float().T + b_enc.float()
    values, indices = torch.topk(preacts, k, dim=-1)
    return values, indices.to(torch.int32)
