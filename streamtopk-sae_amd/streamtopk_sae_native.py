"""streamtopk_sae_native -- the reference's native module, over libstreamtopk_hip.so.

The reference's Python layer imports a pybind11 module of this name
(streamtopk_sae/ops.py:9-13, built from streamtopk_sae/csrc/bindings.cpp:28-51)
and calls three functions on it.  This module provides the same three
functions, with the same arguments, checks, error messages and return
conventions, on top of the gfx950 library's C ABI; with the directory that
holds it on sys.path the reference's own ops.py runs unchanged on MI355X.

* streamtopk_cpu_forward(X, W_enc, b_enc, k) -> (V, I)        (bindings.cpp:29)
* streamtopk_cuda_exact_forward(X, W_enc, b_enc, k) -> (V, I)  (bindings.cpp:33)
* streamtopk_cuda_approx_forward(X, W_enc, b_enc, k, c, candidate_buffer)
      -> (flat_vals (B, nt*c), flat_idxs (B, nt*c), cand_vals (B, nt, c),
          cand_idxs (B, nt, c))                                  (bindings.cpp:35)

The approximate forward materialises the per-group candidates because the
reference's ops.py finishes with torch.topk over them (ops.py:75-81); the
package's own streamtopk_sae.ops.topk_sae_cuda_approx does that last step on
the device and skips the candidates.
"""
from streamtopk_sae import ops as _ops

__all__ = ["streamtopk_cpu_forward", "streamtopk_cuda_exact_forward", "streamtopk_cuda_approx_forward"]


def streamtopk_cpu_forward(X, W_enc, b_enc, k):
    return _ops.cpu_forward(X, W_enc, b_enc, k)


def streamtopk_cuda_exact_forward(X, W_enc, b_enc, k):
    return _ops.exact_forward(X, W_enc, b_enc, k)


def streamtopk_cuda_approx_forward(X, W_enc, b_enc, k, c, candidate_buffer=None):
    _, _, cand_vals, cand_idxs = _ops.approx_forward(X, W_enc, b_enc, k, c, candidate_buffer,
                                                     candidates=True)
    B = cand_vals.shape[0]
    return cand_vals.view(B, -1), cand_idxs.view(B, -1), cand_vals, cand_idxs
