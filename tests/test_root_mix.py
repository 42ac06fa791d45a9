"""The root Dirichlet mix, pinned against the reference's own numpy expression.

The reference's driver expands the root with (optimized_wave_search.py:377-392, 394-415)

    legal_priors = policy[legal_actions]
    legal_priors = legal_priors / np.sum(legal_priors)
    noise = np.random.dirichlet([alpha] * len(legal_priors))
    legal_priors = (1 - epsilon) * legal_priors + epsilon * noise
    # reference_pw only: top max_children by np.argpartition, then
    legal_priors = legal_priors / np.sum(legal_priors)

and the tree stores ``np.array(priors.tolist(), dtype=np.float32)``
(cython_tree_optimized.pyx:564-572).  Here numpy itself evaluates those lines, so its
promotion rules decide the arithmetic (a float32 array times the Python float 1 - epsilon
stays float32, the float64 noise term makes the sum float64), not a restatement of them.
The C oracle's root priors must equal the result bit for bit on C3-shaped roots (Go 19x19,
250-362 legal root moves, alpha 0.03, epsilon 0.25), under both expansion policies.

Two things the reference leaves open are fixed the build's way:
* np.sum's pairwise order: the policy rows are multiples of 2^-23 summing below 2, so every
  float32 partial sum is exact and any summation order gives the same legal renormalisation.
  The widening's float64 renormalisation of at most 15 noisy priors can differ from the
  canonical order in the last bit of the sum; the quotient's rounding to float32 absorbs that
  (checked: no mismatch on these roots).
* np.argpartition's order inside the chosen set: ascending action order (the rule pinned in
  tests/test_reference_pw.py).

Each planted misreading of ref_np.MIX_VARIANTS fails the comparison somewhere."""
import numpy as np
import pytest

from oracle import ref_np
from oracle.oracle import Oracle
from omoknuni_quantum_amd.synthetic import games

ALPHA, EPS = 0.03, 0.25
NUM_ROOTS = 48


def _roots(seed: int):
    """C3-shaped roots: boards, legal masks and lists, dyadic policy rows, Dirichlet rows."""
    model = games.go(19)
    A = model.num_actions
    boards = games.random_boards(NUM_ROOTS, 19, 112, seed)
    legal_mask = games.legal_masks(model, boards, NUM_ROOTS)
    counts = games.legal_counts(model, legal_mask)
    noise = games.dirichlet_noise(model, counts, ALPHA, seed + 7919)
    rng = np.random.default_rng(seed)
    pol = np.empty((NUM_ROOTS, A), np.float32)
    legal = []
    for t in range(NUM_ROOTS):
        bits = np.unpackbits(legal_mask[t].view(np.uint8), bitorder="little")[:A].astype(bool)
        la = np.flatnonzero(bits)
        legal.append(la)
        logits = rng.normal(0.0, 2.0, la.size)
        p = np.exp(logits - logits.max())
        p /= p.sum()
        m = np.maximum(1, np.round(p * 2.0 ** 23))  # multiples of 2^-23, sum < 2
        row = rng.random(A).astype(np.float32) * 7  # illegal slots hold values never read
        row[la] = (m * 2.0 ** -23).astype(np.float32)
        pol[t] = row
    return model, legal_mask, legal, pol, noise, counts


def _reference_expression(legal_actions, policy, noise_row, policy_kind, root_visits=1):
    """The reference's lines, evaluated by numpy (see the module docstring)."""
    legal_priors = policy[legal_actions]
    assert legal_priors.dtype == np.float32
    legal_priors = legal_priors / np.sum(legal_priors)
    noise = noise_row[:len(legal_priors)]
    scaled = (1 - EPS) * legal_priors
    assert scaled.dtype == np.float32            # the weak Python float keeps float32
    legal_priors = scaled + EPS * noise
    assert legal_priors.dtype == np.float64      # the float64 noise term promotes the sum
    if policy_kind == "reference_pw":
        mc = min(len(legal_actions), int(10.0 * (root_visits ** 0.5)) + 1)
        mc = max(5, min(mc, 15))
        if len(legal_actions) > mc:
            top = np.argpartition(legal_priors, -mc)[-mc:]
            kth = np.sort(legal_priors)[-mc]
            assert np.count_nonzero(legal_priors == kth) == 1  # no tie at the cut
            top = np.sort(top)                   # the build's order within the chosen set
            legal_actions = legal_actions[top]
            legal_priors = legal_priors[top]
            legal_priors = legal_priors / np.sum(legal_priors)
        n = min(len(legal_actions), 8)           # MAX_CHILDREN (cython_tree_optimized.pyx:239)
        legal_actions, legal_priors = legal_actions[:n], legal_priors[:n]
    return legal_actions, np.array(legal_priors.tolist(), dtype=np.float32)


def _oracle_root_rows(model, legal_mask, pol, noise, policy_kind):
    orc = Oracle(model, NUM_ROOTS, 4096, 1, 100)
    orc.set_params(1.4, 3.0, 1 if policy_kind == "reference_pw" else 0, 0, 2.0, EPS)
    orc.set_roots(games.root_keys(5, NUM_ROOTS), legal_mask, noise)
    rows = []
    for t in range(NUM_ROOTS):
        orc.reset_tree(t)
        orc.wave(t, 1, replay_policy=pol[t:t + 1], replay_values=np.zeros(1, np.float32))
        tr = orc.tree(t)
        k = int(tr["nchild"][0])
        rows.append((tr["action"][1:1 + k].copy(), tr["P"][1:1 + k].copy()))
    return rows


def _bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.int32)


@pytest.mark.parametrize("seed", [3, 4])
@pytest.mark.parametrize("policy_kind", ["full", "reference_pw"])
def test_oracle_root_mix_equals_reference_expression(seed, policy_kind):
    model, legal_mask, legal, pol, noise, counts = _roots(seed)
    assert counts.min() >= 250 and counts.max() <= 362
    got = _oracle_root_rows(model, legal_mask, pol, noise, policy_kind)
    for t in range(NUM_ROOTS):
        acts, pri = _reference_expression(legal[t], pol[t], noise[t], policy_kind)
        assert np.array_equal(got[t][0], acts), t
        bad = np.flatnonzero(_bits(got[t][1]) != _bits(pri))
        assert bad.size == 0, (t, bad[:5], got[t][1][bad[:5]], pri[bad[:5]])


@pytest.mark.parametrize("policy_kind", ["full", "reference_pw"])
def test_restatement_root_mix_equals_reference_expression(policy_kind):
    model, legal_mask, legal, pol, noise, counts = _roots(3)
    for t in range(0, NUM_ROOTS, 3):
        acts, pri = _reference_expression(legal[t], pol[t], noise[t], policy_kind)
        ra, rp = ref_np.choose_children(legal[t], pol[t], True, policy_kind, 1, noise[t], EPS)
        assert list(ra) == acts.tolist()
        assert np.array_equal(_bits(rp), _bits(pri)), t


@pytest.mark.parametrize("variant", ref_np.MIX_VARIANTS)
def test_planted_mix_misreadings_fail(variant):
    """Each misreading gives at least one root prior that differs from numpy's evaluation of
    the reference's expression, under one of the two policies."""
    model, legal_mask, legal, pol, noise, counts = _roots(3)
    mismatched = 0
    for policy_kind in ("full", "reference_pw"):
        for t in range(0, NUM_ROOTS, 2):
            acts, pri = _reference_expression(legal[t], pol[t], noise[t], policy_kind)
            ra, rp = ref_np.choose_children(legal[t], pol[t], True, policy_kind, 1, noise[t],
                                            EPS, mix_variant=variant)
            if list(ra) != acts.tolist() or not np.array_equal(_bits(rp), _bits(pri)):
                mismatched += 1
    assert mismatched > 0, variant


def test_mix_has_no_effect_off_the_root():
    """Only the root is mixed (leaf_node == 0): a non-root leaf's priors are the plain
    renormalised policy under either policy."""
    model, legal_mask, legal, pol, noise, counts = _roots(4)
    la = legal[0]
    ra, rp = ref_np.choose_children(la, pol[0], False, "full", 1, noise[0], EPS)
    p = pol[0][la] / np.sum(pol[0][la])
    assert np.array_equal(_bits(rp), _bits(p))
