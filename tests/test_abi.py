"""C ABI of libstreamtopk_hip.so, checked without a GPU: the library loads,
exports every function include/streamtopk.h declares, and rejects bad
arguments with the reference's error wording before any device work."""
import ctypes
import os
import re

import numpy as np
import pytest

from streamtopk_sae import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "streamtopk.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(stk_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_version():
    lib = _lib.load()
    assert lib.stk_abi_version() == 1


def test_exports_every_declared_symbol():
    lib = _lib.load()
    names = _declared()
    assert len(names) >= 7
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES)


def _exact(B=4, d=64, F=256, k=8, dtype=2):
    lib = _lib.load()
    return lib.stk_exact_forward(None, None, None, None, None, B, d, F, k, dtype, None, 0, None)


@pytest.mark.parametrize("kw,msg", [
    (dict(k=3), "streamtopk_cuda_exact: unsupported k=3. Supported: 1,2,4,8,16,32,64,128."),
    (dict(k=0), "k out of range"),
    (dict(k=512, F=256), "k out of range"),
    (dict(d=8192), "d exceeds D_MAX=4096"),
    (dict(dtype=7), "X dtype must be fp32, fp16, or bf16"),
    (dict(d=100), "d=100 must be a multiple of 8"),
    (dict(d=30, dtype=0), "d=30 must be a multiple of 4"),
])
def test_exact_argument_errors(kw, msg):
    rc = _exact(**kw)
    assert rc == 1
    assert msg in _lib.load().stk_last_error().decode()


@pytest.mark.parametrize("k,c,msg", [
    (32, 16, "k must be <= c"),
    (8, 48, "streamtopk_cuda_approx: unsupported c=48. Supported: 16,32,64,128."),
    (0, 16, "k must be <= c"),
])
def test_approx_argument_errors(k, c, msg):
    lib = _lib.load()
    rc = lib.stk_approx_forward(None, None, None, None, None, 4, 64, 256, k, c, 2,
                                None, None, None, 0, None)
    assert rc == 1
    assert msg in lib.stk_last_error().decode()


def test_approx_candidate_pointer_checks():
    """Candidate buffers are written as 16-byte vectors: a misaligned pointer,
    or only one of the two, is rejected before any device work (the pointers
    here are never dereferenced)."""
    lib = _lib.load()
    fake = ctypes.c_void_p(0x10000)
    for cv, ci, msg in [(ctypes.c_void_p(0x10004), fake, "must be 16-byte aligned"),
                        (fake, ctypes.c_void_p(0x10008), "must be 16-byte aligned"),
                        (fake, None, "must both be given or both be NULL")]:
        rc = lib.stk_approx_forward(fake, fake, fake, fake, fake, 4, 64, 256, 8, 16, 2,
                                    cv, ci, None, 0, None)
        assert rc == 1
        assert msg in lib.stk_last_error().decode()


def test_cpu_forward_through_abi():
    import oracle
    lib = _lib.load()
    rng = np.random.default_rng(0)
    X = rng.standard_normal((5, 48)).astype(np.float32)
    W = rng.standard_normal((300, 48)).astype(np.float32)
    b = rng.standard_normal(300).astype(np.float32)
    V = np.empty((5, 16), np.float32)
    I = np.empty((5, 16), np.int32)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    assert lib.stk_cpu_forward(p(X), p(W), p(b), p(V), p(I), 5, 48, 300, 16, 2) == 0
    from parity import check_against_scores
    check_against_scores(V, I, oracle.scores_f64(X, W, b), 16, 1e-5, "abi cpu")
    assert lib.stk_cpu_forward(p(X), p(W), p(b), p(V), p(I), 5, 48, 300, 5, 2) == 1
    assert "unsupported k=5" in lib.stk_last_error().decode()


def _shard(f_offset, F=256, k=8):
    lib = _lib.load()
    return lib.stk_exact_forward_shard(None, None, None, None, None, 4, 64, F, k, 2, f_offset, None, 0, None)


@pytest.mark.parametrize("f_offset,F,msg", [
    (-1, 256, "f_offset=-1 out of range"),
    (0x7FFFFFFF - 100, 256, "exceeds the int32 index range"),
])
def test_shard_offset_errors(f_offset, F, msg):
    assert _shard(f_offset, F) == 1
    assert msg in _lib.load().stk_last_error().decode()


def test_merge_workspace_and_errors():
    lib = _lib.load()
    nb = ctypes.c_size_t(0)
    # the 256-byte control line (left to the exact path), dense candidate
    # lists of nparts*k keys per row (256-byte aligned), then one 128-byte
    # count line per row
    assert lib.stk_topk_merge_workspace_bytes(4, 8, 3, ctypes.byref(nb)) == 0
    assert nb.value == 256 + 4 * 24 * 8 + 4 * 32 * 4
    assert lib.stk_topk_merge_workspace_bytes(0, 8, 3, ctypes.byref(nb)) == 0 and nb.value == 0
    for B, k, nparts, msg in [(4, 3, 2, "unsupported k=3"), (4, 8, 0, "nparts=0 out of range"),
                              (4, 128, 9000, "nparts=9000 out of range")]:
        assert lib.stk_topk_merge_workspace_bytes(B, k, nparts, ctypes.byref(nb)) == 1
        assert msg in lib.stk_last_error().decode()
    rc = lib.stk_topk_merge(None, None, 2, 4, 8, None, None, None, 0, None)
    assert rc == 1 and "null tensor pointer" in lib.stk_last_error().decode()
