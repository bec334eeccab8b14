"""Pins the CPU oracle (oracle/) before it is trusted as the checker.

Each oracle function is checked against something that does not share its
code: numpy float64 brute force, exact-integer known-answer fixtures, closed
forms (zero X, a dominant bias, k=1 argmax, k=F permutation), and the
reference's own CPU TopKBuffer compiled from the reference checkout
(oracle/_ref, when it was built).  A planted mistake in the oracle must be
caught by the parity checker.
"""
import numpy as np
import pytest

import oracle
from golden.make_golden import load as load_golden
from parity import check_against_scores


def _rand(B, d, F, seed):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((B, d)).astype(np.float32)
    W = (rng.standard_normal((F, d)) / np.sqrt(d)).astype(np.float32)
    b = (0.1 * rng.standard_normal(F)).astype(np.float32)
    return X, W, b


def _brute(S32, k):
    """Top-k of fp32 scores: value descending, lower index first."""
    B, F = S32.shape
    I = np.empty((B, k), dtype=np.int32)
    for i in range(B):
        I[i] = np.lexsort((np.arange(F), -S32[i].astype(np.float64)))[:k]
    return np.take_along_axis(S32, I.astype(np.int64), axis=1), I


def test_scores_f64_matches_numpy():
    X, W, b = _rand(5, 37, 70, 1)
    S = oracle.scores_f64(X, W, b)
    ref = X.astype(np.float64) @ W.astype(np.float64).T + b.astype(np.float64)
    assert np.max(np.abs(S - ref)) < 1e-12


@pytest.mark.parametrize("B,d,F,k", [(4, 64, 256, 8), (3, 40, 100, 100), (7, 16, 33, 1), (2, 128, 4096, 64)])
def test_exact_matches_bruteforce(B, d, F, k):
    X, W, b = _rand(B, d, F, B * 1000 + F)
    V, I = oracle.exact(X, W, b, k)
    S32 = (X.astype(np.float64) @ W.astype(np.float64).T + b).astype(np.float32)
    Vb, Ib = _brute(S32, k)
    assert np.array_equal(I, Ib) and np.array_equal(V, Vb)


def test_exact_known_answers():
    for X, W, b, k, Vk, Ik in load_golden():
        V, I = oracle.exact(X, W, b, k)
        assert np.array_equal(V, Vk) and np.array_equal(I, Ik)


def test_exact_closed_forms():
    X, W, b = _rand(3, 32, 500, 7)
    Z = np.zeros_like(X)
    V, I = oracle.exact(Z, W, b, 10)
    want = np.argsort(-b.astype(np.float64), kind="stable")[:10]
    for i in range(3):
        assert np.array_equal(I[i], want) and np.array_equal(V[i], b[want])
    b2 = b.copy()
    b2[123] = 1e4
    _, I = oracle.exact(X, W, b2, 5)
    assert np.all(I[:, 0] == 123)
    _, I = oracle.exact(X, W, b, 1)
    S = oracle.scores_f64(X, W, b)
    assert np.array_equal(I[:, 0], np.argmax(S, axis=1))
    _, I = oracle.exact(X, W[:20], b[:20], 20)
    assert all(sorted(r.tolist()) == list(range(20)) for r in I)


def test_exact_ties_and_nan():
    X = np.zeros((2, 8), dtype=np.float32)
    W = np.zeros((10, 8), dtype=np.float32)
    b = np.array([1, 3, 3, 2, 3, np.nan, 0, 3, -np.inf, 2], dtype=np.float32)
    V, I = oracle.exact(X, W, b, 6)
    # NaN first (torch.topk ranks NaN highest), then equal 3s by lower index
    assert I[0].tolist() == [5, 1, 2, 4, 7, 3]


@pytest.mark.parametrize("B,F,k", [(3, 50, 1), (5, 300, 17), (2, 1000, 128), (4, 64, 64)])
def test_topk_scores_matches_bruteforce(B, F, k):
    """oracle.topk_scores (top-k of given fp32 scores) against a lexsort, with
    many equal values; NaN ranks first, as torch.topk ranks it."""
    rng = np.random.default_rng(B * F + k)
    S = (rng.integers(-40, 40, size=(B, F)) / 3).astype(np.float32)
    S[0, F // 2] = np.nan
    V, I = oracle.topk_scores(S, k)
    key = np.where(np.isnan(S), np.inf, S).astype(np.float64)
    for i in range(B):
        want = np.lexsort((np.arange(F), -key[i]))[:k]
        assert np.array_equal(I[i], want)
        assert np.array_equal(V[i], S[i, want], equal_nan=True)
    assert I[0, 0] == F // 2


@pytest.mark.parametrize("k", [1, 2, 4, 8, 16, 32, 64, 128])
def test_buffer_stream_matches_reference_topkbuffer(k):
    """The selection rule restated in stk_oracle_cpu.c vs the reference's own
    TopKBuffer (topk_buffer.hpp), bit for bit, heap order included."""
    rng = np.random.default_rng(k)
    for trial in range(20):
        n = int(rng.integers(1, 3000))
        s = rng.integers(-50, 50, size=n).astype(np.float32) / 7   # many ties
        ref = oracle.ref_buffer_stream(s, k)
        if ref is None:
            pytest.skip("oracle/_ref not built (reference checkout absent)")
        got = oracle.buffer_stream(s, k)
        assert np.array_equal(got[0], ref[0]) and np.array_equal(got[1], ref[1])


@pytest.mark.parametrize("k", [1, 8, 32, 64])
def test_buffer_stream_is_topk_lower_index_first(k):
    rng = np.random.default_rng(100 + k)
    s = rng.integers(-30, 30, size=2000).astype(np.float32)
    V, I = oracle.buffer_stream(s, k)
    want = np.lexsort((np.arange(s.size), -s.astype(np.float64)))[:k]
    assert np.array_equal(I, want) and np.array_equal(V, s[want])


@pytest.mark.parametrize("k", [16, 32, 64, 128])
def test_cpu_stream_matches_exact(k):
    X, W, b = _rand(6, 96, 3000, 11 + k)
    V, I = oracle.cpu_stream(X, W, b, k, nthreads=2)
    order = np.argsort(-V, axis=1, kind="stable")        # k=128 comes out in heap order
    V = np.take_along_axis(V, order, axis=1)
    I = np.take_along_axis(I, order, axis=1)
    S = oracle.scores_f64(X, W, b)
    check_against_scores(V, I, S, k, 1e-5, "cpu_stream")


def test_cpu_stream_known_answers():
    for X, W, b, k, Vk, Ik in load_golden():
        V, I = oracle.cpu_stream(X, W, b, k)
        if k <= 64:
            assert np.array_equal(V, Vk) and np.array_equal(I, Ik)
            continue
        # k > 64: the reference's min-heap (topk_buffer.hpp:43-60) returns heap
        # order and, when several kept entries tie at the minimum, may evict the
        # lower index first -- so only entries tied with the k-th value may differ.
        o = np.lexsort((I, -V.astype(np.float64)), axis=1)
        V, I = np.take_along_axis(V, o, axis=1), np.take_along_axis(I, o, axis=1)
        assert np.array_equal(V, Vk)
        for i in range(V.shape[0]):
            kth = Vk[i, -1]
            strict = Vk[i] > kth
            assert np.array_equal(I[i][strict], Ik[i][strict])
            S = X[i].astype(np.float64) @ W.astype(np.float64).T + b
            assert np.all(S[I[i][~strict]] == kth)


@pytest.mark.parametrize("c", [16, 32, 64, 128])
def test_approx_candidates_bruteforce(c):
    B, d, F, k = 3, 24, 700, 16
    X, W, b = _rand(B, d, F, 300 + c)
    V, I, cv, ci = oracle.approx(X, W, b, k, c, with_candidates=True)
    S32 = (X.astype(np.float64) @ W.astype(np.float64).T + b).astype(np.float32)
    nt = (F + 127) // 128
    assert cv.shape == (B, nt, c)
    for i in range(B):
        for t in range(nt):
            f0, f1 = 128 * t, min(F, 128 * t + 128)
            seg = S32[i, f0:f1]
            o = np.lexsort((np.arange(f1 - f0), -seg.astype(np.float64)))[:c]
            n = len(o)
            assert np.array_equal(ci[i, t, :n], o + f0)
            assert np.array_equal(cv[i, t, :n], seg[o])
            assert np.all(ci[i, t, n:] == -1) and np.all(cv[i, t, n:] == np.float32(-3.402823466e38))
    # union theorem: with k <= c the approximate top-k is the exact top-k
    Ve, Ie = oracle.exact(X, W, b, k)
    assert np.array_equal(V, Ve) and np.array_equal(I, Ie)


def test_approx_recall_below_one_when_c_small():
    """Sanity of the semantics: the union of per-group top-c can miss exact
    top-k members only when k > c (which the op rejects)."""
    X, W, b = _rand(2, 16, 512, 5)
    # k=16, c=16 -> identical; a planted c smaller than k would not be
    V, I = oracle.approx(X, W, b, 16, 16)
    Ve, Ie = oracle.exact(X, W, b, 16)
    assert np.array_equal(I, Ie)


def test_parity_checker_catches_planted_mistakes():
    X, W, b = _rand(4, 32, 300, 9)
    V, I = oracle.exact(X, W, b, 8)
    S = oracle.scores_f64(X, W, b)
    check_against_scores(V, I, S, 8, 1e-5)
    bad_I = I.copy()
    bad_I[1, 3] = int(np.argmin(S[1]))          # a wrong index
    with pytest.raises(AssertionError):
        check_against_scores(V, bad_I, S, 8, 1e-5)
    bad_V = V.copy()
    bad_V[2, 0] += 1e-3                          # a wrong value
    with pytest.raises(AssertionError):
        check_against_scores(bad_V, I, S, 8, 1e-5)
    dup = I.copy()
    dup[0, 1] = dup[0, 0]                        # a duplicate index
    with pytest.raises(AssertionError):
        check_against_scores(V, dup, S, 8, 1e-5)
