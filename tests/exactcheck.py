"""Exact whole-matrix check of int32 accumulators (Freivalds' method)."""
import numpy as np


def check_acc_exact(acc, q, t32, seed):
    """Assert acc [M, N] int32 == q [M, K] int8 @ t32 [N, K]^T in every entry.

    Two projections per round, two rounds: acc r == q (t^T r) for a random integer r
    over the output rows with no zero entry (so a single wrong accumulator always
    changes acc r), and l^T acc == t (q^T l) for a random l over the token rows.
    t^T r stays below 2^24 in magnitude (|r| <= 8, N < 2^21), so float32 holds it
    exactly; every other sum is an integer below 2^53, exact in float64."""
    rng = np.random.default_rng(seed)
    assert t32.shape[0] <= (1 << 21)
    a64 = acc.astype(np.float64)
    q64 = q.astype(np.float64)
    for _ in range(2):
        r = (rng.integers(1, 9, size=t32.shape[0]) * rng.choice([-1, 1], size=t32.shape[0])).astype(np.float32)
        v = r @ t32
        assert np.array_equal(a64 @ r.astype(np.float64), q64 @ v.astype(np.float64)), "acc r != q (t^T r)"
        l = (rng.integers(1, 9, size=q.shape[0]) * rng.choice([-1, 1], size=q.shape[0])).astype(np.float64)
        assert np.array_equal(l @ a64, t32.astype(np.float64) @ (l @ q64)), "l^T acc != t (q^T l)"
