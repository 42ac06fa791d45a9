"""The committed golden fixtures (tests/golden/): the C oracle and the numpy restatement
reproduce them, and the cases with a closed-form answer have it."""
import os

import numpy as np
import pytest

from oracle import golden

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _rows():
    with np.load(os.path.join(HERE, "select_rows.npz")) as z:
        return golden.unpack_crafted(z)


def test_fixture_cases_match_generator():
    """The fixture holds exactly the generator's cases (inputs bit-equal)."""
    got, want = _rows(), golden.crafted_row_cases()
    assert len(got) == len(want)
    for g, w in zip(got, want):
        for key in ("kind", "model", "k", "m", "c", "vl", "N0"):
            assert g[key] == w[key]
        for key in ("N", "W", "P"):
            assert np.array_equal(np.asarray(g[key]).view(np.int32),
                                  np.asarray(w[key]).view(np.int32))


@pytest.mark.parametrize("restatement", ["numpy", "c_oracle"])
def test_select_rows_reproduced(restatement):
    fn = golden.crafted_expected_np if restatement == "numpy" else golden.crafted_expected_oracle
    for i, c in enumerate(_rows()):
        picks, n_after = fn(c)
        assert np.array_equal(picks, c["picks"]), (i, c["kind"], c["k"], c["m"])
        assert np.array_equal(n_after, c["N_after"]), (i, c["kind"])


def test_select_rows_closed_forms():
    """Answers fixed by the rule itself, independent of any restatement."""
    seen = set()
    for c in _rows():
        k, m, picks = c["k"], c["m"], c["picks"]
        vli = int(c["vl"])
        # visit counts: root +VL per simulation, each child +VL per pick
        want = np.concatenate([[c["N0"]], c["N"]]).astype(np.int64)
        want[0] += vli * m
        np.add.at(want, 1 + picks[picks >= 0], vli)
        assert np.array_equal(c["N_after"], want), c["kind"]
        kind = c["kind"]
        seen.add(kind)
        if kind == "ties":
            # identical children: lowest index on ties, and a picked child drops below the rest
            assert np.array_equal(picks, np.arange(m) % k)
        elif kind == "all_unvisited":
            # the first unvisited child wins; virtual loss makes it visited
            assert np.array_equal(picks[:k], np.arange(k))
        elif kind == "late_unvisited":
            assert picks[0] == k - 3 and picks[1] == k - 1
        elif kind == "vl0":
            assert np.all(picks == picks[0]) and picks[0] >= 0
        elif kind == "vl0_np0":
            assert np.all(picks == -1)  # sqrt(0) exploration: the reference returns no child
        elif kind == "single":
            # one simulation: the reference's best child at Np = N0 + VL, computed in float64
            n = c["N"].astype(np.float64)
            if np.any(n == 0):
                assert picks[0] == int(np.flatnonzero(n == 0)[0])
            else:
                s = np.sqrt(c["N0"] + vli)
                sc = c["W"] / (n + c["vl"]) + c["c"] * c["P"].astype(np.float64) * s / (1 + n)
                order = np.argsort(-sc, kind="stable")
                best = order[0]
                if len(sc) > 1 and sc[order[0]] - sc[order[1]] > 1e-5 * abs(sc[order[0]]):
                    assert picks[0] == best
    assert {"ties", "all_unvisited", "late_unvisited", "vl0", "single", "bigQ", "negP", "nanW"} <= seen


@pytest.mark.parametrize("case", golden.SEARCH_CASES, ids=lambda c: c["name"])
def test_search_trees_reproduced(case):
    """The C oracle and the numpy restatement agree on the case (search_expected checks that)
    and both equal the committed fixture."""
    r = golden.search_expected(case)
    with np.load(os.path.join(HERE, "search_trees.npz")) as z:
        for key, v in r.items():
            want = z[f"{case['name']}/{key}"]
            assert np.array_equal(np.asarray(v).view(np.int32) if v.dtype == np.float32 else v,
                                  want.view(np.int32) if want.dtype == np.float32 else want), key


def test_search_trees_invariants():
    """Counts fixed by the rules: the root's count is its initial 1 + the root-expansion
    simulation + every later simulation; the children's counts sum to the simulations that
    passed through them; every node's parent precedes it."""
    with np.load(os.path.join(HERE, "search_trees.npz")) as z:
        for case in golden.SEARCH_CASES:
            g = lambda key: z[f"{case['name']}/{key}"]  # noqa: E731
            N, first, nchild, parent = g("N"), g("first"), g("nchild"), g("parent")
            sims = len(g("path_len")) - 1
            assert N[0] == 2 + sims
            kids = np.arange(first[0] + 1, first[0] + 1 + nchild[0])
            plen = g("path_len")
            assert N[kids].sum() == int((plen[1:] > 1).sum())
            assert np.all(parent[1:] < np.arange(1, len(N)))
