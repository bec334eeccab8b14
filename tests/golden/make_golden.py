"""Writes tests/golden/known_answer.npz: known-answer cases whose scores are
exact in fp32, bf16 and fp16 arithmetic, so every implementation must return
the same values bit for bit and the same indices, tie order included.

X entries are multiples of 1/4 in [-1, 1], W entries multiples of 1/8 in
[-1, 1], b entries multiples of 1/16 in [-1, 1]: every product and partial
sum is a dyadic rational with at most ~12 significant bits, so any summation
order gives the exact score.  The expected top-k is computed here in integer
arithmetic (scores scaled by 32) and ordered by score descending, then lower
latent index first -- the tie rule of the reference's CPU buffer
(streamtopk_sae/csrc/cpu/topk_buffer.hpp:37) and of this build.  The small
integer ranges make equal scores common, so the tie rule is exercised.
Run: python tests/golden/make_golden.py
"""
import os

import numpy as np

CASES = [  # (B, d, F, k)
    (6, 16, 40, 8),
    (5, 64, 300, 16),
    (3, 32, 1000, 128),
    (4, 24, 64, 64),
    (2, 8, 16484, 32),   # F >= 16384: the sampled-seed path of the device op
]


def main():
    rng = np.random.default_rng(20241201)
    out = {}
    for n, (B, d, F, k) in enumerate(CASES):
        xn = rng.integers(-4, 5, size=(B, d)).astype(np.int8)    # X = xn / 4
        wn = rng.integers(-8, 9, size=(F, d)).astype(np.int8)    # W = wn / 8
        bn = rng.integers(-16, 17, size=F).astype(np.int16)      # b = bn / 16
        # score * 32 = xn . wn + 2 * bn   (exact integers)
        s32 = xn.astype(np.int64) @ wn.astype(np.int64).T + 2 * bn.astype(np.int64)[None, :]
        idx = np.empty((B, k), dtype=np.int32)
        for i in range(B):
            order = np.lexsort((np.arange(F), -s32[i]))
            idx[i] = order[:k]
        vals = (np.take_along_axis(s32, idx.astype(np.int64), axis=1) / 32.0).astype(np.float32)
        out[f"c{n}_shape"] = np.array([B, d, F, k], dtype=np.int64)
        out[f"c{n}_xn"] = xn
        out[f"c{n}_wn"] = wn
        out[f"c{n}_bn"] = bn
        out[f"c{n}_V"] = vals
        out[f"c{n}_I"] = idx
    out["ncases"] = np.array(len(CASES))
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "known_answer.npz")
    np.savez_compressed(path, **out)
    print("wrote", path)


def load():
    """Yields (X, W, b, k, V, I) as float32/int32 numpy arrays."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "known_answer.npz")
    z = np.load(path)
    for n in range(int(z["ncases"])):
        B, d, F, k = (int(v) for v in z[f"c{n}_shape"])
        X = z[f"c{n}_xn"].astype(np.float32) / 4
        W = z[f"c{n}_wn"].astype(np.float32) / 8
        b = z[f"c{n}_bn"].astype(np.float32) / 16
        yield X, W, b, k, z[f"c{n}_V"], z[f"c{n}_I"]


if __name__ == "__main__":
    main()
