"""No (B, F) buffer: the peak device memory one encode call adds on top of its
inputs, at BASELINE configs 1, 2 and 4, measured the way the reference's
bench/run_memory.py:38-60 measures it (torch.cuda.max_memory_allocated around
the call, less what was allocated before it).

The call allocates its outputs and the workspace stk_exact_workspace_bytes
asks for, nothing else (the library itself never allocates).  The bounds:

* below the (B, F) fp32 score matrix at every config;
* at most B * ceil(F / 256) * k * 8 bytes (one k-key list per row and
  256-latent tile, the reference's two-pass temporaries at T=256) wherever
  that exceeds the workspace's F-independent floor, B * #CUs * (k + queue)
  keys: configs 2 and 4.  Config 1 has as many workgroups as tiles (256), so
  its per-workgroup segments of k + lq keys make it 1.4x that figure;
* the workspace is bounded in F.
"""
import ctypes

import pytest
import torch

from streamtopk_sae import _lib, clear_workspace_cache, make_inputs, topk_sae_cuda_exact

pytestmark = pytest.mark.gpu

CONFIGS = {
    "c1": dict(B=128, d=768, F=65536, k=32),
    "c2": dict(B=128, d=2048, F=262144, k=64),
    "c4": dict(B=1024, d=4096, F=262144, k=128),
}


def _peak_extra(X, W, b, k):
    # the op keeps its workspace per stream between calls: released here, so
    # that the measured call allocates it as a first call does
    clear_workspace_cache()
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    V, I = topk_sae_cuda_exact(X, W, b, k)
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated() - base
    del V, I
    return peak


def _workspace(B, d, F, k):
    nb = ctypes.c_size_t(0)
    _lib.check(_lib.load().stk_exact_workspace_bytes(B, d, F, k, _lib.STK_DTYPE_BF16, ctypes.byref(nb)))
    return nb.value


@pytest.mark.parametrize("name", list(CONFIGS))
def test_peak_memory_bound(cuda_dev, name):
    c = CONFIGS[name]
    B, d, F, k = c["B"], c["d"], c["F"], c["k"]
    print(f"case memory {name} {c}", flush=True)
    X, W, b = make_inputs(B, d, F, torch.bfloat16, seed=0, device=cuda_dev)
    topk_sae_cuda_exact(X, W, b, k)          # first call: any one-time set-up
    peak = _peak_extra(X, W, b, k)
    ws = _workspace(B, d, F, k)
    outputs = B * k * 8
    bxf = B * F * 4
    tiles_k = B * ((F + 255) // 256) * k * 8
    print(f"[memory] {name}: peak extra {peak / 1e6:.1f} MB, workspace {ws / 1e6:.1f} MB, "
          f"B*F*4 {bxf / 1e6:.1f} MB, B*tiles*k*8 {tiles_k / 1e6:.1f} MB")
    # the call holds its workspace and outputs, rounded up by the caching allocator
    assert peak <= ws + outputs + 4 * 2**20
    assert peak < bxf
    if name in ("c2", "c4"):
        assert peak <= tiles_k
    else:
        assert peak <= 1.5 * tiles_k


def test_workspace_bounded_in_F(cuda_dev):
    """The workspace is bounded in F: every row keeps one segment per
    workgroup of k keys plus at most the LDS queue's length, however many
    tiles each workgroup streams.  Below 512 rows the queue is sized by the
    survivors a workgroup expects, which grow with its tiles until the queue
    reaches its LDS limit (by F = 2^22 at config 2's shape); large batches
    keep a head and fixed segments."""
    s18 = _workspace(128, 2048, 1 << 18, 64)
    s22 = _workspace(128, 2048, 1 << 22, 64)
    assert s18 <= s22 == _workspace(128, 2048, 1 << 26, 64)
    big_b = _workspace(1024, 4096, 1 << 22, 128)
    assert big_b == _workspace(1024, 4096, 1 << 18, 128)
