"""The sparse model's legal lists are Floyd samples (Bentley & Floyd, CACM 30(9), 1987): step i
of n draws r_i in [0, j_i], j_i = A - n + i, and adds j_i instead when r_i is already in the
set.  The GPU kernel (sparse_legal_list, omq_common.h) settles the steps in parallel by this
rule: step i takes j_i exactly when an earlier step drew the same value, or when r_i is j_k of
an earlier step k that took j_k.  These tests check that rule against the sequential algorithm
on random draws, including chains of replaced steps, and that a rule missing the second clause
fails them."""
import random

import pytest


def floyd_sequential(r, A, n):
    taken, out = set(), []
    for i in range(n):
        t = r[i] if r[i] not in taken else A - n + i
        taken.add(t)
        out.append(t)
    return out


def floyd_parallel(r, A, n, chain_rule=True):
    first = {}
    for i, v in enumerate(r):
        first.setdefault(v, i)
    dup = [first[r[i]] < i for i in range(n)]
    col = dup[:]
    for _ in range(n):
        new = []
        for i in range(n):
            k = r[i] - (A - n)
            new.append(dup[i] or (chain_rule and 0 <= k < i and col[k]))
        if new == col:
            break
        col = new
    return [A - n + i if col[i] else r[i] for i in range(n)]


def _cases(seed, count):
    rng = random.Random(seed)
    for _ in range(count):
        n = rng.randint(1, 64)
        A = n + rng.choice([0, 1, 2, 5, 20, 300, 4672 - 64])
        yield A, n, [rng.randint(0, A - n + i) for i in range(n)]


def test_parallel_rule_equals_sequential_floyd():
    chained = 0
    for A, n, r in _cases(11, 20000):
        seq = floyd_sequential(r, A, n)
        assert floyd_parallel(r, A, n) == seq, (A, n, r)
        assert len(set(seq)) == n and all(0 <= v < A for v in seq)
        chained += any(seq[i] != r[i] and r[i] >= A - n for i in range(n))
    assert chained > 1000  # the chain clause is exercised


def test_rule_without_chain_clause_fails():
    with pytest.raises(AssertionError):
        for A, n, r in _cases(12, 20000):
            assert floyd_parallel(r, A, n, chain_rule=False) == floyd_sequential(r, A, n)


def test_known_chain():
    # A=5, n=3: j = 2, 3, 4.  Step 1 draws 0 again and takes j_1 = 3; step 2 draws 3, which
    # step 1 took, and takes j_2 = 4.
    assert floyd_sequential([0, 0, 3], 5, 3) == [0, 3, 4]
    assert floyd_parallel([0, 0, 3], 5, 3) == [0, 3, 4]
    assert floyd_parallel([0, 0, 3], 5, 3, chain_rule=False) == [0, 3, 3]
