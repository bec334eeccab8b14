"""Drop-in op surface of ``streamtopk_sae.ops`` (reference: streamtopk_sae/ops.py).

Same names, arguments, dtype handling and error behaviour as the reference:

* ``topk_sae_cpu(X, W_enc, b_enc, k)``                       (ops.py:23-40)
* ``topk_sae_cuda_exact(X, W_enc, b_enc, k)``                (ops.py:43-57)
* ``topk_sae_cuda_approx(X, W_enc, b_enc, k, c, candidate_buffer=None)``
                                                             (ops.py:60-83)

Each returns ``(values fp32 (B, k), indices int32 (B, k))``, rows sorted by
value descending.  The device ops run the gfx950 kernels of
``libstreamtopk_hip.so`` on the current stream of X's device; outputs and the
workspace are allocated here with torch, so ``torch.cuda.max_memory_allocated``
sees every byte and no (B, F) buffer is ever created.

The workspace (scratch for the duration of one call) is kept per (device,
stream) and reused by later calls on that stream, grown when a call needs more:
calls queued on one stream run one after another, and calls on different
streams get different workspaces.  A new workspace is zero-filled, as the
library requires before a workspace's first use; calls leave it valid for the
next, and a call that fails drops it.  ``clear_workspace_cache()`` releases
them.
"""
import ctypes
import threading

import torch

from . import _lib

_DTYPES = {
    torch.float32: _lib.STK_DTYPE_F32,
    torch.float16: _lib.STK_DTYPE_F16,
    torch.bfloat16: _lib.STK_DTYPE_BF16,
}


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


_WS = {}                      # (device index, stream handle) -> uint8 device tensor
_WS_LOCK = threading.Lock()


def _workspace(device, stream, nbytes):
    """The workspace of `stream` on `device`, at least `nbytes` long.  A
    smaller one is dropped first: the caching allocator hands its block out
    again only in order on the same stream, after the calls queued on it."""
    key = (device.index, int(stream))
    with _WS_LOCK:
        ws = _WS.get(key)
        if ws is None or ws.numel() < nbytes:
            _WS.pop(key, None)
            ws = torch.zeros(max(nbytes, 1), dtype=torch.uint8, device=device)
            _WS[key] = ws
        return ws


def _check_drop(rc, device, stream):
    """_lib.check, dropping the stream's cached workspace on failure: a call
    that failed part-way may not have advanced the workspace's epoch, so its
    words could pass for the next call's; the next call zero-fills a new one."""
    if rc != 0:
        with _WS_LOCK:
            _WS.pop((device.index, int(stream)), None)
    _lib.check(rc)


def clear_workspace_cache():
    """Release every cached workspace (the next call on each stream allocates
    its own again)."""
    with _WS_LOCK:
        _WS.clear()


def _pad_d(X, W_enc, multiple):
    """Zero-pad the reduction axis to `multiple` (exact: zeros add nothing)."""
    d = X.shape[1]
    pad = (-d) % multiple
    if pad == 0:
        return X, W_enc
    X = torch.nn.functional.pad(X, (0, pad))
    W_enc = torch.nn.functional.pad(W_enc, (0, pad))
    return X.contiguous(), W_enc.contiguous()


def _aligned(t):
    """Contiguous tensor whose data pointer is 16-byte aligned."""
    t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


def _device_checks(X, W_enc, b_enc, need_w_device=True):
    # streamtopk_exact.cu:800-812 / streamtopk_approx.cu:246-258
    if not X.is_cuda:
        raise RuntimeError("X must be on CUDA")
    if need_w_device and not W_enc.is_cuda:
        raise RuntimeError("W_enc must be on CUDA")
    if need_w_device and not b_enc.is_cuda:
        raise RuntimeError("b_enc must be on CUDA")
    if W_enc.device != X.device or b_enc.device != X.device:
        raise RuntimeError("X, W_enc and b_enc must be on the same device")
    if b_enc.dtype != torch.float32:
        raise RuntimeError("b_enc must be fp32")
    if X.dtype not in _DTYPES:
        raise RuntimeError("X dtype must be fp32, fp16, or bf16")
    if W_enc.dtype != X.dtype:
        raise RuntimeError("W_enc dtype must match X")
    if X.dim() != 2 or W_enc.dim() != 2 or b_enc.dim() != 1:
        raise RuntimeError("expected X (B, d), W_enc (F, d), b_enc (F,)")
    if W_enc.shape[1] != X.shape[1]:
        raise RuntimeError("W_enc d-dim mismatch")
    if b_enc.shape[0] != W_enc.shape[0]:
        raise RuntimeError("b_enc F-dim mismatch")


def _contiguity_checks(X, W_enc, b_enc):
    # streamtopk_exact.cu:800-802 / streamtopk_approx.cu:243-245
    if not X.is_contiguous():
        raise RuntimeError("X must be contiguous")
    if not W_enc.is_contiguous():
        raise RuntimeError("W_enc must be contiguous")
    if not b_enc.is_contiguous():
        raise RuntimeError("b_enc must be contiguous")


def cpu_forward(X, W_enc, b_enc, k):
    """The native CPU forward (streamtopk_cpu.cpp:81-125): fp32 contiguous CPU
    tensors in, (V fp32 (B,k), I int32 (B,k)) out, rows sorted descending."""
    lib = _lib.load()
    # streamtopk_cpu.cpp:87-99 (plus a device check: the reference would read a
    # device pointer on the host)
    _contiguity_checks(X, W_enc, b_enc)
    if X.dtype != torch.float32:
        raise RuntimeError("X must be fp32")
    if W_enc.dtype != torch.float32:
        raise RuntimeError("W_enc must be fp32")
    if b_enc.dtype != torch.float32:
        raise RuntimeError("b_enc must be fp32")
    if X.is_cuda or W_enc.is_cuda or b_enc.is_cuda:
        raise RuntimeError("topk_sae_cpu expects CPU tensors")
    if W_enc.shape[1] != X.shape[1]:
        raise RuntimeError("W_enc d-dim mismatch")
    if b_enc.shape[0] != W_enc.shape[0]:
        raise RuntimeError("b_enc F-dim mismatch")
    B, d = X.shape
    F = W_enc.shape[0]
    V = torch.empty((B, k), dtype=torch.float32) if k >= 1 else None
    I = torch.empty((B, k), dtype=torch.int32) if k >= 1 else None
    rc = lib.stk_cpu_forward(_ptr(X), _ptr(W_enc), _ptr(b_enc), _ptr(V), _ptr(I),
                             B, d, F, k, 0)
    _lib.check(rc)
    return V, I


def topk_sae_cpu(X, W_enc, b_enc, k):
    """CPU streaming top-k SAE forward (fp32; fp16/bf16 inputs are upcast).

    Returns values (B, k) fp32 and indices (B, k) int32 on the CPU.
    """
    _lib.load()
    if X.dtype != torch.float32:
        X = X.float()
        W_enc = W_enc.float()
    if b_enc.dtype != torch.float32:
        b_enc = b_enc.float()
    return cpu_forward(X.contiguous(), W_enc.contiguous(), b_enc.contiguous(), k)


def _device_inputs(X, W_enc, b_enc):
    """Native-side checks, then 16-byte alignment.  The kernels read rows in
    16-byte chunks and mask a partial last chunk-step themselves, so only a d
    that leaves rows misaligned (not a multiple of 4 fp32 or 8 fp16/bf16
    elements) is zero-padded, which copies W_enc."""
    _contiguity_checks(X, W_enc, b_enc)
    _device_checks(X, W_enc, b_enc)
    multiple = 4 if X.dtype == torch.float32 else 8
    X, W_enc = _pad_d(X, W_enc, multiple)
    return _aligned(X), _aligned(W_enc), b_enc


def exact_forward(X, W_enc, b_enc, k, f_offset=0):
    """The native exact forward (streamtopk_exact.cu:788-833): contiguous device
    tensors, fp32 b_enc; returns (V fp32 (B,k), I int32 (B,k)).  A non-zero
    f_offset marks W_enc / b_enc as latents f_offset .. f_offset+F-1 of a
    larger dictionary (one shard): the indices are global."""
    lib = _lib.load()
    X, W_enc, b_enc = _device_inputs(X, W_enc, b_enc)
    B, d = X.shape
    F = W_enc.shape[0]
    dt = _DTYPES[X.dtype]
    with torch.cuda.device(X.device):
        nbytes = ctypes.c_size_t(0)
        _lib.check(lib.stk_exact_workspace_bytes(B, d, F, k, dt, ctypes.byref(nbytes)))
        V = torch.empty((B, k), dtype=torch.float32, device=X.device)
        I = torch.empty((B, k), dtype=torch.int32, device=X.device)
        stream = torch.cuda.current_stream(X.device).cuda_stream
        ws = _workspace(X.device, stream, nbytes.value)
        if f_offset:
            rc = lib.stk_exact_forward_shard(_ptr(X), _ptr(W_enc), _ptr(b_enc), _ptr(V), _ptr(I),
                                             B, d, F, k, dt, int(f_offset), _ptr(ws), ws.numel(),
                                             ctypes.c_void_p(stream))
        else:
            rc = lib.stk_exact_forward(_ptr(X), _ptr(W_enc), _ptr(b_enc), _ptr(V), _ptr(I),
                                       B, d, F, k, dt, _ptr(ws), ws.numel(), ctypes.c_void_p(stream))
        _check_drop(rc, X.device, stream)
    return V, I


def topk_sae_cuda_exact(X, W_enc, b_enc, k, *, f_offset=0):
    """Exact streaming top-k SAE forward on the GPU (fp16, bf16, fp32; b_enc fp32).

    Returns values (B, k) fp32 and indices (B, k) int32 on X's device.
    ``f_offset`` (keyword only, no counterpart in the reference): W_enc and
    b_enc are latents ``f_offset .. f_offset + F - 1`` of a larger dictionary,
    e.g. one GPU's shard, and the returned indices are global; combine the
    shards' results with :func:`merge_topk_shards`.
    """
    _lib.load()
    if b_enc.dtype != torch.float32:
        b_enc = b_enc.float()
    if f_offset < 0:
        raise RuntimeError("f_offset must be >= 0")
    return exact_forward(X.contiguous(), W_enc.contiguous(), b_enc.contiguous(), k, f_offset=f_offset)


def merge_topk_shards(values, indices, k):
    """Top-k of per-shard top-k results (no counterpart in the reference).

    ``values`` / ``indices``: sequences of (B, k) fp32 / int32 device tensors
    (or stacked (nparts, B, k) tensors) with global latent indices, e.g. the
    outputs of ``topk_sae_cuda_exact(..., f_offset=...)`` over the shards of
    W_enc gathered on one device.  Returns (values (B, k) fp32, indices (B, k)
    int32), rows sorted by value descending, equal values by lower index.
    """
    lib = _lib.load()
    Vp = values if torch.is_tensor(values) else torch.stack(list(values))
    Ip = indices if torch.is_tensor(indices) else torch.stack(list(indices))
    if Vp.dim() != 3 or tuple(Ip.shape) != tuple(Vp.shape):
        raise RuntimeError("expected matching (nparts, B, k) values and indices")
    if Vp.dtype != torch.float32 or Ip.dtype != torch.int32:
        raise RuntimeError("values must be fp32 and indices int32")
    if not Vp.is_cuda or Ip.device != Vp.device:
        raise RuntimeError("values and indices must be on the same CUDA device")
    if Vp.shape[2] != k:
        raise RuntimeError("each part must hold k entries per row")
    Vp, Ip = Vp.contiguous(), Ip.contiguous()
    nparts, B, _ = Vp.shape
    with torch.cuda.device(Vp.device):
        nbytes = ctypes.c_size_t(0)
        _lib.check(lib.stk_topk_merge_workspace_bytes(B, k, nparts, ctypes.byref(nbytes)))
        V = torch.empty((B, k), dtype=torch.float32, device=Vp.device)
        I = torch.empty((B, k), dtype=torch.int32, device=Vp.device)
        stream = torch.cuda.current_stream(Vp.device).cuda_stream
        ws = _workspace(Vp.device, stream, nbytes.value)
        _lib.check(lib.stk_topk_merge(_ptr(Vp), _ptr(Ip), nparts, B, k, _ptr(V), _ptr(I),
                                      _ptr(ws), ws.numel(), ctypes.c_void_p(stream)))
    return V, I


def approx_forward(X, W_enc, b_enc, k, c, candidate_buffer=None, candidates=False):
    """The native approximate forward (streamtopk_approx.cu:234-291) with the
    final top-k done on the device.  Returns (V, I, cand_vals, cand_idxs); the
    candidate tensors, shape (B, ceil(F/128), c), are None unless
    `candidates` is set or a `candidate_buffer` is given."""
    lib = _lib.load()
    X, W_enc, b_enc = _device_inputs(X, W_enc, b_enc)
    B, d = X.shape
    F = W_enc.shape[0]
    dt = _DTYPES[X.dtype]
    nt = (F + 127) // 128
    with torch.cuda.device(X.device):
        with_cand = candidate_buffer is not None or candidates
        cand_vals = cand_idxs = None
        copy_back = None
        if with_cand:
            if candidate_buffer is not None:
                cb = candidate_buffer
                if cb.dim() != 3 or tuple(cb.shape) != (B, nt, c):
                    raise RuntimeError("candidate_buffer shape mismatch")
                if cb.dtype != torch.float32 or cb.device != X.device or not cb.is_contiguous():
                    raise RuntimeError("candidate_buffer must be a contiguous fp32 tensor on X's device")
                if cb.data_ptr() % 16:
                    # the kernel writes 16-byte vectors: fill an aligned buffer, then copy
                    copy_back = cb
                    cb = torch.empty_like(cb)
                cand_vals = cb
            else:
                cand_vals = torch.empty((B, nt, c), dtype=torch.float32, device=X.device)
            cand_idxs = torch.empty((B, nt, c), dtype=torch.int32, device=X.device)
        nbytes = ctypes.c_size_t(0)
        _lib.check(lib.stk_approx_workspace_bytes(B, d, F, k, c, dt, int(with_cand),
                                                  ctypes.byref(nbytes)))
        V = torch.empty((B, k), dtype=torch.float32, device=X.device)
        I = torch.empty((B, k), dtype=torch.int32, device=X.device)
        stream = torch.cuda.current_stream(X.device).cuda_stream
        ws = _workspace(X.device, stream, nbytes.value)
        rc = lib.stk_approx_forward(_ptr(X), _ptr(W_enc), _ptr(b_enc), _ptr(V), _ptr(I),
                                    B, d, F, k, c, dt, _ptr(cand_vals), _ptr(cand_idxs),
                                    _ptr(ws), ws.numel(), ctypes.c_void_p(stream))
        _check_drop(rc, X.device, stream)
        if copy_back is not None:
            copy_back.copy_(cand_vals)
            cand_vals = copy_back
    return V, I, cand_vals, cand_idxs


def topk_sae_cuda_approx(X, W_enc, b_enc, k, c, candidate_buffer=None):
    """Approximate streaming top-k SAE forward: top-c per 128-latent group, then
    top-k of the union.  c must be in {16, 32, 64, 128} and >= k.

    If `candidate_buffer` (fp32, shape (B, ceil(F/128), c)) is given it is
    filled with each group's top-c values, descending, padded with -FLT_MAX.
    Returns values (B, k) fp32 and indices (B, k) int32.
    """
    _lib.load()
    if b_enc.dtype != torch.float32:
        b_enc = b_enc.float()
    V, I, _, _ = approx_forward(X.contiguous(), W_enc.contiguous(), b_enc.contiguous(), k, c,
                                candidate_buffer)
    return V, I
