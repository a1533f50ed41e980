"""The whole-matrix accumulator check used by the GPU prefill tests, pinned on the
CPU: it accepts the oracle's own accumulators and rejects planted mistakes (one
entry off by one, two entries swapped, a token row computed from the wrong
quantised row, the weights of one output row negated)."""
import numpy as np
import pytest

from datagen import activations, ternary, weights
from exactcheck import check_acc_exact
from oracle import oracle as orc


@pytest.fixture(scope="module")
def case():
    m, k, n = 300, 1088, 700
    x = activations(m, k, seed=1)
    wb, sw = orc.pack(weights(n, k, seed=2))
    _, q, _, acc = orc.forward_i8(x, wb, n, sw)
    t32 = ternary(wb, n * k).reshape(n, k).astype(np.float32)
    return acc, q, t32


def test_accepts_the_oracle_accumulators(case):
    acc, q, t32 = case
    for seed in range(3):
        check_acc_exact(acc, q, t32, seed)


def _planted(acc, q, t32):
    rng = np.random.default_rng(5)
    a = acc.copy()
    i, j = rng.integers(acc.shape[0]), rng.integers(acc.shape[1])
    a[i, j] += 1
    yield a
    a = acc.copy()
    j2 = (j + 1) % acc.shape[1]
    a[i, [j, j2]] = a[i, [j2, j]]
    yield a
    a = acc.copy()
    a[7] = (q[8].astype(np.int64) @ t32.T.astype(np.int64)).astype(np.int32)
    yield a
    a = acc.copy()
    a[:, 11] = -a[:, 11]
    yield a


def test_rejects_planted_mistakes(case):
    acc, q, t32 = case
    for bad in _planted(acc, q, t32):
        assert not np.array_equal(bad, acc)
        for seed in range(3):
            with pytest.raises(AssertionError):
                check_acc_exact(bad, q, t32, seed)
