"""The reference's progressive widening (optimized_wave_search.py:394-415, MAX_CHILDREN = 8 of
cython_tree_optimized.pyx:31,239), pinned by its closed form (oracle/golden.py pw_root_count,
written with integer square roots) over a grid of root visit counts and legal-set sizes:

* root:     mc = max(5, min(L, floor(10 sqrt(N0)) + 1, 15)); the chosen set is the top-mc
            priors when L > mc, else all L legal actions; the row is the first min(8, .) of
            the chosen set in ascending action order (the build's order in place of
            np.argpartition's);
* non-root: the top min(3, L) priors.

The C oracle and the numpy restatement both follow it, and each planted misreading of
ref_np.PW_VARIANTS breaks it somewhere on the grid."""
import pytest

from oracle import golden, ref_np


def _grid():
    return [(n0, L) for n0 in golden.PW_GRID_N0 for L in golden.PW_GRID_L]


def test_closed_form_table():
    """Spot values of the rule, by hand."""
    c = golden.pw_root_count
    assert c(1, 25) == (11, 8)    # floor(10*1)+1 = 11 chosen, 8 kept (a search's root)
    assert c(0, 25) == (5, 5)     # floor(0)+1 = 1 -> at least 5
    assert c(2, 25) == (15, 8)    # floor(14.14)+1 = 15
    assert c(4, 25) == (15, 8)    # 21 -> capped at 15
    assert c(1, 3) == (3, 3)      # fewer legal actions than 5: all of them
    assert c(1, 9) == (9, 8)      # L = 9 <= mc = 9 (min(L, 11)): all 9, 8 kept
    assert c(0, 6) == (5, 5)      # L = 6 > mc = 5: the top 5


@pytest.mark.parametrize("seed", [1, 2])
def test_oracle_follows_rule(seed):
    fails = []
    for n0, L in _grid():
        model, board, legal, acts, pol = golden.pw_inputs(L, seed * 1000 + L)
        root, child = golden.pw_oracle_root(n0, L, seed * 1000 + L)
        want = golden.pw_expected(acts, pol, n0)
        if root != want:
            fails.append(f"N0={n0} L={L}: root row {root}, rule {want}")
            continue
        rest = [a for a in acts if a != root[0]]
        want_c = golden.pw_expected(rest, pol, None) if rest else []
        if child != want_c:
            fails.append(f"N0={n0} L={L}: first child's row {child}, rule {want_c}")
    assert not fails, "\n".join(fails[:10])


def _restated(acts, pol, n0, variant=None):
    got, _ = ref_np.choose_children(acts, pol, n0 is not None, "reference_pw",
                                    0 if n0 is None else n0, pw_variant=variant)
    return [int(a) for a in got]


def test_restatement_follows_rule():
    for n0, L in _grid():
        model, board, legal, acts, pol = golden.pw_inputs(L, 7 + L)
        assert _restated(acts, pol, n0) == golden.pw_expected(acts, pol, n0), (n0, L)
        assert _restated(acts, pol, None) == golden.pw_expected(acts, pol, None), L


@pytest.mark.parametrize("variant", ref_np.PW_VARIANTS)
def test_planted_widening_misreading_fails(variant):
    bad = 0
    for n0, L in _grid():
        model, board, legal, acts, pol = golden.pw_inputs(L, 7 + L)
        for root in (n0, None):
            if _restated(acts, pol, root, variant) != golden.pw_expected(acts, pol, root):
                bad += 1
    assert bad > 0, variant
