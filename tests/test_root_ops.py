"""Per-move root operations restated in the C oracle: its own log and exp, gamma and Dirichlet
variates, and move selection with a temperature, pinned by accuracy bounds, moments and the
rule of np.random.choice."""
import math

import numpy as np
import pytest

from oracle.oracle import Oracle, load
from omoknuni_quantum_amd.synthetic import games

ULP = 2.0 ** -52


def test_log_exp_accuracy():
    lib = load()
    rng = np.random.default_rng(0)
    xs = np.concatenate([np.exp(rng.uniform(-700, 700, 20000)), 1 + rng.uniform(-1e-6, 1e-6, 2000),
                         rng.uniform(0.5, 2.0, 5000), [5e-324, 1e-310, 2.2250738585072014e-308,
                                                       1.0, 2.0, 0.5]])
    for x in xs:
        got, ref = lib.orc_log_d(float(x)), math.log(float(x))
        assert abs(got - ref) <= 2 * ULP * max(abs(ref), 1e-300) + 1e-300, (x, got, ref)
    assert lib.orc_log_d(1.0) == 0.0
    for x in np.concatenate([rng.uniform(-745, 709, 20000), rng.uniform(-1, 1, 5000), [0.0]]):
        got, ref = lib.orc_exp_d(float(x)), math.exp(float(x))
        if ref < 2.2250738585072014e-308:
            assert abs(got - ref) <= 2 * 5e-324 + 2 * ULP * ref, (x, got, ref)  # subnormal
        else:
            assert abs(got - ref) <= 2 * ULP * ref, (x, got, ref)
    assert lib.orc_exp_d(0.0) == 1.0 and lib.orc_exp_d(-800.0) == 0.0


@pytest.mark.parametrize("alpha", [0.03, 0.3, 1.0, 2.5])
def test_gamma_moments(alpha):
    lib = load()
    n = 20000
    g = np.array([lib.orc_gamma(alpha, 11, 3, 0, i) for i in range(n)])
    assert np.all(g >= 0) and np.isfinite(g).all()
    # Gamma(alpha, 1): mean alpha, variance alpha; sample-mean standard error sqrt(alpha/n)
    assert abs(g.mean() - alpha) < 5 * math.sqrt(alpha / n), (g.mean(), alpha)
    m4 = 3 * alpha * (alpha + 2)  # fourth central moment of Gamma(alpha)... bound for var error
    assert abs(g.var() - alpha) < 6 * math.sqrt((m4 + 6 * alpha ** 2) / n), (g.var(), alpha)


@pytest.mark.parametrize("alpha,L", [(0.03, 362), (0.3, 225), (1.5, 30)])
def test_dirichlet_rows(alpha, L):
    model = games.go(19) if L == 362 else (games.gomoku(15) if L == 225 else games.gomoku(6))
    T = 400
    A = model.num_actions
    boards = np.zeros((T, model.board_size, model.board_size), np.int8)
    if L == 30:
        boards[:, 0, :6] = 1  # 36 - 6 = 30 legal cells
    legal = games.legal_masks(model, boards, T)
    orc = Oracle(model, T, 4, 8, 8)
    orc.set_roots(games.root_keys(1, T), legal)
    rows = np.stack([orc.root_dirichlet(t, alpha, 5, 9) for t in range(T)])
    assert np.all(rows[:, L:] == 0) and np.all(rows[:, :L] >= 0)
    assert np.allclose(rows.sum(1), 1.0, atol=1e-12)
    x = rows[:, :L].reshape(-1)
    a0 = L * alpha
    mean, var = 1.0 / L, (alpha * (a0 - alpha)) / (a0 * a0 * (a0 + 1))
    assert abs(x.mean() - mean) < 1e-12  # rows sum to one
    assert abs(x.var() - var) < 0.15 * var, (x.var(), var)
    # same moments as numpy's Dirichlet
    ref = np.random.default_rng(0).dirichlet([alpha] * L, T).reshape(-1)
    assert abs(x.var() - ref.var()) < 0.2 * var
    # another counter gives other rows; the same arguments give the same rows
    assert not np.array_equal(rows[0], orc.root_dirichlet(0, alpha, 5, 10))
    assert np.array_equal(rows[3], orc.root_dirichlet(3, alpha, 5, 9))


def _u(seed, counter, t):
    M = (1 << 64) - 1
    sm = games.splitmix64
    base = sm(sm(sm(seed) ^ counter) ^ (((t & 0xFFFFFFFF) << 32) | 0xFFFFFFFF))
    return (sm(base) >> 11) * 2.0 ** -53


def test_sample_action_rule():
    """np.random.choice semantics given the draw u: the first entry of the normalised
    cumulative sums above u; temperature 0 is np.argmax."""
    lib = load()
    rng = np.random.default_rng(7)
    A = 50
    for trial in range(300):
        p = rng.random(A) * (rng.random(A) < 0.4)
        if p.sum() == 0:
            p[3] = 1.0
        p = p / p.sum()
        c = np.ascontiguousarray(p)
        assert lib.orc_sample_action(c.ctypes.data, A, 0.0, 1, trial, 0) == int(np.argmax(p))
        got = lib.orc_sample_action(c.ctypes.data, A, 1.0, 1, trial, 2)
        u = _u(1, trial, 2)
        cdf = np.cumsum(p / p.sum())
        cdf = cdf / cdf[-1]
        want = int(np.searchsorted(cdf, u, side="right"))
        if np.min(np.abs(cdf - u)) > 1e-9:
            assert got == want, (trial, got, want)
        assert p[got] > 0


@pytest.mark.parametrize("temperature", [0.5, 1.0, 2.0])
def test_sample_action_frequencies(temperature):
    lib = load()
    p = np.array([0.5, 0.0, 0.3, 0.15, 0.05])
    c = np.ascontiguousarray(p)
    n = 40000
    picks = np.array([lib.orc_sample_action(c.ctypes.data, 5, temperature, 3, i, 0)
                      for i in range(n)])
    q = p ** (1.0 / temperature)
    q = q / q.sum()
    freq = np.bincount(picks, minlength=5) / n
    assert freq[1] == 0
    assert np.all(np.abs(freq - q) < 5 * np.sqrt(q * (1 - q) / n) + 1e-12), (freq, q)
