"""Parity checks shared by the tests (not collected by pytest).

Tolerances follow the target contract: values within 1e-5 relative for fp32
inputs and 2e-3 relative for bf16/fp16 inputs (relative to max(|score|, 1));
index sets identical except where the differing latents' scores are within
that tolerance of the row's k-th score (near-ties, which are counted and
returned so the tests can log them).
"""
import numpy as np

RTOL = {"fp32": 1e-5, "fp16": 2e-3, "bf16": 2e-3}


def tol_of(dtype_name):
    return RTOL[dtype_name]


def check_against_scores(V, I, S, k, rtol, name=""):
    """V, I: (B, k) outputs; S: (B, F) float64 oracle scores.  Returns #near-ties."""
    V = np.asarray(V, dtype=np.float64)
    I = np.asarray(I, dtype=np.int64)
    S = np.asarray(S, dtype=np.float64)
    B, F = S.shape
    assert V.shape == (B, k) and I.shape == (B, k), f"{name}: shape {V.shape} {I.shape}"
    assert np.all((I >= 0) & (I < F)), f"{name}: index out of range"
    part = np.partition(S, F - k, axis=1)[:, F - k:] if k < F else S
    ref = -np.sort(-part, axis=1)
    scale = np.maximum(np.abs(ref), 1.0)
    err = np.abs(V - ref) / scale
    assert np.all(err <= rtol), f"{name}: sorted values differ, max rel err {err.max():.3g}"
    assert np.all(np.diff(V, axis=1) <= 0), f"{name}: values not sorted descending"
    got = np.take_along_axis(S, I, axis=1)
    err2 = np.abs(V - got) / np.maximum(np.abs(got), 1.0)
    assert np.all(err2 <= rtol), f"{name}: value does not match its index's score, {err2.max():.3g}"
    ties = 0
    for i in range(B):
        assert len(set(I[i].tolist())) == k, f"{name}: duplicate index in row {i}"
        kth = ref[i, k - 1]
        above = np.nonzero(S[i] > kth)[0]
        level = np.nonzero(S[i] == kth)[0][:k - above.size]   # lower index first among equals
        want = set(above.tolist()) | set(level.tolist())
        diff = set(I[i].tolist()) ^ want
        if diff:
            for f in diff:
                assert abs(S[i, f] - kth) <= rtol * max(abs(kth), 1.0), (
                    f"{name}: row {i} index {f} (score {S[i, f]!r}) differs beyond a near-tie "
                    f"of the k-th score {kth!r}")
            ties += 1
    return ties
