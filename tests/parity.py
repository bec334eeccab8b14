"""Parity checks shared by the tests (not collected by pytest).

Values.  Given the magnitudes A = |X| @ |W|^T + |b| (float64) of the terms of
each score, a kernel value is held to the error an fp32 sum of those terms
can carry: lambda * sqrt(n) * u * A, with u = 2^-24, n = d + 2 terms (the d
products, their own rounding for fp32 inputs, the bias) and lambda = 10 --
the probabilistic bound of Higham and Mary ("A new approach to probabilistic
rounding error analysis", SIAM J. Sci. Comput. 41(5), 2019, Thm. 3.1), which
holds with probability at least 1 - 2n exp(-lambda^2 / 2) per sum (below
1e-17 here).  Products of bf16/fp16 inputs are exact in fp32, so a kernel
that accumulates in fp32 stays far inside it, while one that rounds scores or
partial sums to bf16 (2^-9 relative, as the reference's dense oracle does)
does not.  Without A, values fall back to the target contract's tolerance:
1e-5 relative for fp32 inputs, 2e-3 for bf16/fp16 (relative to
max(|score|, 1)).

Indices.  Index sets must be identical except where the differing latents'
scores lie within the contract tolerance (rtol) of the row's k-th score:
near-ties.  Every check records its row count and its near-tie rows in
TIE_LOG, which the test session prints at its end and writes as JSON
(conftest.py); a check may also bound the fraction of rows with near-ties
(max_tie_frac).
"""
import math

import numpy as np

RTOL = {"fp32": 1e-5, "fp16": 2e-3, "bf16": 2e-3}
U32 = 2.0 ** -24
LAMBDA = 10.0

TIE_LOG = []   # one dict per check: name, rows, k, tie_rows, value_margin


def tol_of(dtype_name):
    return RTOL[dtype_name]


def fp32_sum_bound(A, d):
    """The error bound of an fp32 sum of d + 2 terms of total magnitude A."""
    return LAMBDA * math.sqrt(d + 2) * U32 * np.asarray(A, dtype=np.float64)


def term_magnitudes(X, W, b):
    """A = |X| @ |W|^T + |b| in float64 (numpy arrays or torch tensors; torch
    tensors are reduced on their device)."""
    try:
        import torch
        if torch.is_tensor(X):
            A = X.double().abs() @ W.double().abs().T + b.double().abs()
            return A.cpu().numpy()
    except ImportError:
        pass
    X = np.asarray(X, dtype=np.float64)
    W = np.asarray(W, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return np.abs(X) @ np.abs(W).T + np.abs(b)


def check_against_scores(V, I, S, k, rtol, name="", A=None, d=None, max_tie_frac=None):
    """V, I: (B, k) outputs; S: (B, F) float64 oracle scores.  A (optional,
    (B, F) term magnitudes) and d: hold values to the fp32 accumulation bound
    instead of rtol.  Returns the number of rows with near-tie index
    differences."""
    V = np.asarray(V, dtype=np.float64)
    I = np.asarray(I, dtype=np.int64)
    S = np.asarray(S, dtype=np.float64)
    B, F = S.shape
    assert V.shape == (B, k) and I.shape == (B, k), f"{name}: shape {V.shape} {I.shape}"
    assert np.all((I >= 0) & (I < F)), f"{name}: index out of range"
    part = np.partition(S, F - k, axis=1)[:, F - k:] if k < F else S
    ref = -np.sort(-part, axis=1)
    got = np.take_along_axis(S, I, axis=1)
    if A is not None:
        assert d is not None, f"{name}: the bound needs d"
        A = np.asarray(A, dtype=np.float64)
        tol_own = fp32_sum_bound(np.take_along_axis(A, I, axis=1), d)
        # the sorted values against the sorted top-k: each sorted position may
        # pair two latents of the row's top k, so the row's largest bound
        top_idx = np.argpartition(-S, k - 1, axis=1)[:, :k] if k < F else np.tile(np.arange(F), (B, 1))
        tol_row = np.maximum(tol_own.max(axis=1),
                             fp32_sum_bound(np.take_along_axis(A, top_idx, axis=1), d).max(axis=1))[:, None]
        tol_row = np.maximum(tol_row, 1e-30)
        tol_own = np.maximum(tol_own, 1e-30)
        err = np.abs(V - ref)
        assert np.all(err <= tol_row), (
            f"{name}: sorted values differ beyond the fp32 accumulation bound, max err/bound "
            f"{(err / tol_row).max():.3g}")
        err2 = np.abs(V - got)
        assert np.all(err2 <= tol_own), (
            f"{name}: a value differs from its index's score beyond the fp32 accumulation bound, "
            f"max err/bound {(err2 / tol_own).max():.3g}")
        margin = float(max((err / tol_row).max(), (err2 / tol_own).max()))
    else:
        scale = np.maximum(np.abs(ref), 1.0)
        err = np.abs(V - ref) / scale
        assert np.all(err <= rtol), f"{name}: sorted values differ, max rel err {err.max():.3g}"
        err2 = np.abs(V - got) / np.maximum(np.abs(got), 1.0)
        assert np.all(err2 <= rtol), f"{name}: value does not match its index's score, {err2.max():.3g}"
        margin = float(max(err.max(), err2.max()) / rtol)
    assert np.all(np.diff(V, axis=1) <= 0), f"{name}: values not sorted descending"
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
    TIE_LOG.append({"name": name, "rows": int(B), "k": int(k), "tie_rows": int(ties),
                    "value_err_over_bound": margin, "bound": "fp32-sum" if A is not None else "rtol"})
    if max_tie_frac is not None:
        assert ties <= max_tie_frac * B, (
            f"{name}: {ties} of {B} rows with near-tie index differences, above {max_tie_frac:.1%}")
    return ties
