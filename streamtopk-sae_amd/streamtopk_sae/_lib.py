"""ctypes binding of ``libstreamtopk_hip.so`` (C ABI in ``include/streamtopk.h``).

Replaces the reference's pybind11 import (streamtopk_sae/ops.py:9-13): the
library is loaded from this package directory and, if it is missing, every op
raises ``RuntimeError`` -- there is no fallback implementation.
"""
import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libstreamtopk_hip.so")

STK_DTYPE_F32 = 0
STK_DTYPE_F16 = 1
STK_DTYPE_BF16 = 2
ABI_VERSION = 1

# Every symbol include/streamtopk.h declares, with its ctypes signature.
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_szp = ctypes.POINTER(ctypes.c_size_t)
SIGNATURES = {
    "stk_abi_version": (_int, []),
    "stk_last_error": (ctypes.c_char_p, []),
    "stk_exact_workspace_bytes": (_int, [_i64, _i64, _i64, _i64, _int, _szp]),
    "stk_exact_forward": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp,
                                 ctypes.c_size_t, _vp]),
    "stk_exact_forward_shard": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _i64,
                                       _vp, ctypes.c_size_t, _vp]),
    "stk_exact_forward_noalloc": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp]),
    "stk_topk_merge_workspace_bytes": (_int, [_i64, _i64, _i64, _szp]),
    "stk_topk_merge": (_int, [_vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, ctypes.c_size_t, _vp]),
    "stk_approx_workspace_bytes": (_int, [_i64, _i64, _i64, _i64, _i64, _int, _int, _szp]),
    "stk_approx_forward": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _int,
                                  _vp, _vp, _vp, ctypes.c_size_t, _vp]),
    "stk_cpu_forward": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int]),
    "stk_read_probe": (_int, [_vp, ctypes.c_size_t, _vp, _vp]),
    "stk_profile_enable": (_int, [_int]),
    "stk_profile_read": (_int, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double),
                                ctypes.POINTER(ctypes.c_int64)]),
}

# Test-only exports (not declared in include/streamtopk.h): hooks that force
# paths real inputs never take, and a window on the no-allocation scratch.
TEST_SIGNATURES = {
    "stk_test_set_hooks": (_int, [_int, _int, _i64]),
    "stk_test_scratch_io": (_int, [ctypes.c_size_t, _vp, ctypes.c_size_t, _int]),
}

_lock = threading.Lock()
_lib = None


def load():
    """Load the library once; raise RuntimeError when it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    "libstreamtopk_hip.so not built (expected at %s). Run: "
                    "make -C streamtopk-sae_amd  (or __graft_entry__.build())" % LIB_PATH)
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in list(SIGNATURES.items()) + list(TEST_SIGNATURES.items()):
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            if lib.stk_abi_version() != ABI_VERSION:
                raise RuntimeError("libstreamtopk_hip.so ABI version %d != %d"
                                   % (lib.stk_abi_version(), ABI_VERSION))
            _lib = lib
    return _lib


def check(rc):
    """Raise RuntimeError carrying the library's message for a non-zero rc."""
    if rc != 0:
        msg = load().stk_last_error().decode("utf-8", "replace")
        raise RuntimeError(msg or ("streamtopk library call failed with code %d" % rc))
