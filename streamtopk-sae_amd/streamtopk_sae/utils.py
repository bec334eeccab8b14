"""Helpers of the op surface (reference: streamtopk_sae/utils.py).

``recall_at_k`` follows utils.py:23-36 (mean over rows of |pred & true| / k),
computed with tensor ops instead of a Python loop over rows.
"""
import torch

DTYPE_MAP = {
    "fp16": torch.float16,
    "bf16": torch.bfloat16,
    "fp32": torch.float32,
}


def str_to_dtype(s):
    if s not in DTYPE_MAP:
        raise ValueError(f"Unknown dtype '{s}'. Choose from: {list(DTYPE_MAP)}")
    return DTYPE_MAP[s]


def recall_per_row(pred_idxs, true_idxs):
    """Per-row recall |pred & true| / k as a float64 CPU tensor of shape (B,)."""
    pred = torch.as_tensor(pred_idxs).to("cpu", torch.int64)
    true = torch.as_tensor(true_idxs).to("cpu", torch.int64)
    B, k = true.shape
    if B == 0:
        return torch.zeros(0, dtype=torch.float64)
    hits = (pred.unsqueeze(2) == true.unsqueeze(1)).any(dim=1).sum(dim=1)
    return hits.to(torch.float64) / k


def recall_at_k(pred_idxs, true_idxs):
    """Mean Recall@k over the batch (pred/true: (B, k) int tensors)."""
    r = recall_per_row(pred_idxs, true_idxs)
    return float(r.mean()) if r.numel() else 0.0
