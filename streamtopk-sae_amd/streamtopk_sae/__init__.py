"""StreamTopK-SAE for MI355X: streaming fused top-k SAE encoder on gfx950.

Computes top_k(X @ W_enc.T + b_enc, k) per row without materialising the
(B, F) score matrix.  Op surface as in the reference package
(streamtopk_sae/__init__.py:9-24): the dense Triton/torch.compile baselines
of the reference are not part of this build.
"""
from streamtopk_sae.reference import reference_topk_sae
from streamtopk_sae.ops import (topk_sae_cpu, topk_sae_cuda_exact, topk_sae_cuda_approx, merge_topk_shards,
                                clear_workspace_cache)
from streamtopk_sae.utils import recall_at_k, str_to_dtype
from streamtopk_sae.inputs import make_inputs

__all__ = [
    "reference_topk_sae",
    "topk_sae_cpu",
    "topk_sae_cuda_exact",
    "topk_sae_cuda_approx",
    "merge_topk_shards",
    "clear_workspace_cache",
    "recall_at_k",
    "str_to_dtype",
    "make_inputs",
]
