"""CPU oracle for the streaming top-k SAE encoder -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker.  The product
(the HIP library and the ``streamtopk_sae`` package) never touches it.

Thin ctypes layer over ``liboracle.so`` (built from ``stk_oracle.c`` and
``stk_oracle_cpu.c`` by ``oracle/Makefile``).  Every function takes numpy
float32 arrays (fp16/bf16 inputs are upcast by the caller, which is exact) and
returns numpy arrays.

Functions and the reference code they restate:

* ``scores_f64``  -- ``X @ W.T + b`` in double (streamtopk_sae/reference.py:17).
* ``exact``       -- sorted top-k of the fp32-rounded scores, lower index first
  on equal values (reference.py:17-19).
* ``approx``      -- top-c per 128-latent group, then top-k of the union
  (streamtopk_sae/csrc/cuda/streamtopk_approx.cu:31,118-166; ops.py:80-81).
* ``cpu_stream``  -- the reference CPU kernel's streaming selection
  (streamtopk_sae/csrc/cpu/streamtopk_cpu.cpp:15-67, topk_buffer.hpp:9-72).
* ``buffer_stream`` -- that selection rule alone, on a given score stream.
* ``ref_buffer_stream`` -- the reference's own TopKBuffer driven over a
  stream (``oracle/_ref``), or ``None`` when that harness was not built.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = None
_REF_TRIED = False

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64 = ctypes.c_int64


def build():
    """Compile liboracle.so (and oracle/_ref when the reference is present)."""
    subprocess.run(["make", "-s", "-C", _HERE, "all"], check=True)


def _lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        lib = ctypes.CDLL(path)
        lib.orc_scores_f64.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _i64, _f64p]
        lib.orc_exact.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, _f32p, _i32p, ctypes.c_int]
        lib.orc_topk_scores.argtypes = [_f32p, _i64, _i64, _i64, _f32p, _i32p]
        lib.orc_approx.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, _i64,
                                   _f32p, _i32p, _f32p, _i32p]
        lib.orc_cpu_stream.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, _f32p, _i32p, ctypes.c_int]
        lib.orc_buffer_stream.argtypes = [_f32p, _i64, _i64, _f32p, _i32p]
        _LIB = lib
    return _LIB


def _ref_lib():
    global _REF, _REF_TRIED
    if not _REF_TRIED:
        _REF_TRIED = True
        path = os.path.join(_HERE, "_ref", "libref_topkbuf.so")
        if os.path.exists(path):
            _REF = ctypes.CDLL(path)
            _REF.ref_buffer_stream.argtypes = [_f32p, _i64, _i64, _f32p, _i32p]
    return _REF


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a, t):
    return a.ctypes.data_as(t)


def _inputs(X, W, b):
    X, W, b = _f32(X), _f32(W), _f32(b)
    assert X.ndim == 2 and W.ndim == 2 and b.ndim == 1
    assert X.shape[1] == W.shape[1] and W.shape[0] == b.shape[0]
    return X, W, b


def scores_f64(X, W, b):
    X, W, b = _inputs(X, W, b)
    B, d = X.shape
    F = W.shape[0]
    S = np.empty((B, F), dtype=np.float64)
    _lib().orc_scores_f64(_p(X, _f32p), _p(W, _f32p), _p(b, _f32p), B, d, F, _p(S, _f64p))
    return S


def exact(X, W, b, k, nthreads=1):
    X, W, b = _inputs(X, W, b)
    B, d = X.shape
    F = W.shape[0]
    V = np.empty((B, k), dtype=np.float32)
    I = np.empty((B, k), dtype=np.int32)
    rc = _lib().orc_exact(_p(X, _f32p), _p(W, _f32p), _p(b, _f32p), B, d, F, k,
                          _p(V, _f32p), _p(I, _i32p), nthreads)
    if rc:
        raise ValueError(f"orc_exact failed rc={rc}")
    return V, I


def topk_scores(S, k):
    S = _f32(S)
    B, F = S.shape
    V = np.empty((B, k), dtype=np.float32)
    I = np.empty((B, k), dtype=np.int32)
    rc = _lib().orc_topk_scores(_p(S, _f32p), B, F, k, _p(V, _f32p), _p(I, _i32p))
    if rc:
        raise ValueError(f"orc_topk_scores failed rc={rc}")
    return V, I


def approx(X, W, b, k, c, with_candidates=False):
    X, W, b = _inputs(X, W, b)
    B, d = X.shape
    F = W.shape[0]
    nt = (F + 127) // 128
    V = np.empty((B, k), dtype=np.float32)
    I = np.empty((B, k), dtype=np.int32)
    cv = np.empty((B, nt, c), dtype=np.float32) if with_candidates else None
    ci = np.empty((B, nt, c), dtype=np.int32) if with_candidates else None
    rc = _lib().orc_approx(_p(X, _f32p), _p(W, _f32p), _p(b, _f32p), B, d, F, k, c,
                           _p(V, _f32p), _p(I, _i32p),
                           _p(cv, _f32p) if cv is not None else None,
                           _p(ci, _i32p) if ci is not None else None)
    if rc:
        raise ValueError(f"orc_approx failed rc={rc}")
    if with_candidates:
        return V, I, cv, ci
    return V, I


def cpu_stream(X, W, b, k, nthreads=1):
    X, W, b = _inputs(X, W, b)
    B, d = X.shape
    F = W.shape[0]
    V = np.empty((B, k), dtype=np.float32)
    I = np.empty((B, k), dtype=np.int32)
    rc = _lib().orc_cpu_stream(_p(X, _f32p), _p(W, _f32p), _p(b, _f32p), B, d, F, k,
                               _p(V, _f32p), _p(I, _i32p), nthreads)
    if rc:
        raise ValueError(f"orc_cpu_stream failed rc={rc}")
    return V, I


def buffer_stream(scores, k):
    s = _f32(scores).ravel()
    V = np.empty(k, dtype=np.float32)
    I = np.empty(k, dtype=np.int32)
    rc = _lib().orc_buffer_stream(_p(s, _f32p), s.size, k, _p(V, _f32p), _p(I, _i32p))
    if rc:
        raise ValueError(f"orc_buffer_stream failed rc={rc}")
    return V, I


def ref_buffer_stream(scores, k):
    lib = _ref_lib()
    if lib is None:
        return None
    s = _f32(scores).ravel()
    V = np.empty(k, dtype=np.float32)
    I = np.empty(k, dtype=np.int32)
    rc = lib.ref_buffer_stream(_p(s, _f32p), s.size, k, _p(V, _f32p), _p(I, _i32p))
    if rc:
        raise ValueError(f"ref_buffer_stream: unsupported k={k}")
    return V, I
