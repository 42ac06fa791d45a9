"""Pins of the selection rule (cython_tree_optimized.pyx:177-202 select_path, :436-461 the score
of select_best_child_nogil) that do not come from either restatement.

* The pinned rows of oracle/golden.py have their expected picks worked out by hand.  Here they
  are checked in float64 with a stated margin, for the rule and for the misreading each row is
  built against: the two must pick different children, both by a clear margin.  (Both
  restatements reproduce the fixture: tests/test_golden.py.)
* The operand-order row is checked in exact rational arithmetic with binary32 rounding written
  out (round to nearest, ties to even), independently of numpy's float32.
* Every misreading of ref_np.SELECT_VARIANTS, planted into the numpy restatement, fails the
  committed fixture (so the fixture, which the HIP path must reproduce, tells them apart),
  while the restatement without a planted misreading reproduces it.
"""
import math
import os
from fractions import Fraction

import numpy as np
import pytest

from oracle import golden, ref_np

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MARGIN = 0.01  # relative gap between the best and the second-best score, float64


def _rows():
    with np.load(os.path.join(HERE, "select_rows.npz")) as z:
        return golden.unpack_crafted(z)


def _pinned():
    return [c for c in _rows() if c["kind"].startswith("pin_")]


def _scores64(case, variant, Np, n_children):
    """float64 scores of one selection at parent count Np, children counts n_children, under
    the rule (variant None) or a misreading.  None marks an unvisited child taken first."""
    W = np.asarray(case["W"], np.float64)
    P = np.asarray(case["P"], np.float64)
    c, vl = float(case["c"]), float(case["vl"])
    s = math.sqrt(Np + 1 if variant == "sqrt_np_plus1" else Np)
    out = []
    for i, n in enumerate(n_children):
        if n == 0 and variant != "no_unvisited_rule":
            out.append(None)
            continue
        if variant == "q_no_vl":
            q = W[i] / n
        elif n == 0:
            q = 0.0
        else:
            q = W[i] / (n + vl)
        den = n if variant == "denominator_n" else 1 + n
        out.append(q + c * P[i] * s / den)
    return out


def _pick64(scores, ties_highest=False):
    """(pick, relative margin to the runner-up) of float64 scores."""
    for i, s in enumerate(scores):
        if s is None:
            return i, math.inf
    order = sorted(range(len(scores)), key=lambda i: (-scores[i], -i if ties_highest else i))
    best = order[0]
    if len(order) == 1:
        return best, math.inf
    gap = scores[best] - scores[order[1]]
    return best, gap / max(abs(scores[best]), 1e-30)


def _simulate64(case, variant):
    """The case's m simulations in float64: picks, and the smallest margin met."""
    vli = int(case["vl"])
    n = [int(x) for x in case["N"]]
    inflight = [0] * len(n)
    picks, margin = [], math.inf
    for r in range(case["m"]):
        Np = case["N0"] + vli * (r if variant == "np_without_arrival" else r + 1)
        seen = [n[i] - (vli * inflight[i] if variant == "children_no_vl" else 0)
                for i in range(len(n))]
        sc = _scores64(case, variant, Np, seen)
        if variant == "ties_highest" and len(set(sc)) == 1:
            p, g = len(sc) - 1, math.inf
        else:
            p, g = _pick64(sc)
        picks.append(p)
        margin = min(margin, g)
        n[p] += vli
        inflight[p] += 1
    return picks, margin


def test_pinned_rows_present():
    kinds = {c["kind"] for c in _pinned()}
    pinned = {v for c in _pinned() for v in c["pins"]}
    assert pinned == set(ref_np.SELECT_VARIANTS), "every misreading has a row built against it"
    assert len(kinds) == len(_pinned())


@pytest.mark.parametrize("case", _pinned(), ids=lambda c: c["kind"])
def test_pinned_row_by_hand(case):
    """The fixture's picks are the hand-derived ones; in float64 the rule picks them by a
    clear margin (ties and unvisited children aside), and the misreading the row is built
    against picks differently, by a clear margin too."""
    assert list(case["picks"]) == case["expect"]
    if case["kind"] == "pin_op_order":
        return  # an ulp-level row: test_op_order_row_exact
    want, margin = _simulate64(case, None)
    assert want == case["expect"]
    if case["kind"] not in ("pin_ties", "pin_children_vl"):
        assert margin > MARGIN, margin
    for v in case["pins"]:
        got, vmargin = _simulate64(case, v)
        assert got != case["expect"], v
        if v not in ("ties_highest", "children_no_vl"):
            assert vmargin > MARGIN, (v, vmargin)


def _round32(x: Fraction) -> Fraction:
    """x rounded to the nearest binary32 value, ties to even (normal range)."""
    if x == 0:
        return Fraction(0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    ulp = Fraction(2) ** (e - 23)
    q, r = divmod(a, ulp)
    q = int(q)
    if r * 2 > ulp or (r * 2 == ulp and q % 2 == 1):
        q += 1
    return sign * q * ulp


def _f32(x) -> Fraction:
    return Fraction(float(np.float32(x)))


def test_round32_against_ieee():
    """The rounding above agrees with IEEE float32 conversion on random doubles."""
    rng = np.random.default_rng(3)
    for x in rng.uniform(-1e3, 1e3, 2000):
        assert _round32(Fraction(float(x))) == Fraction(float(np.float32(x)))


def test_op_order_row_exact():
    """(c*P)*s and c*(P*s) round apart on the operand-order row; the rule's pick follows
    from exact arithmetic with binary32 rounding after every operation."""
    case = next(c for c in _pinned() if c["kind"] == "pin_op_order")
    c = _f32(case["c"])
    Np = case["N0"] + int(case["vl"])
    # s = sqrtf(Np): the binary32 value nearest to sqrt(Np), checked by squaring
    s = _f32(np.sqrt(np.float32(Np)))
    ulp = Fraction(2) ** (math.frexp(float(s))[1] - 24)
    assert (s - ulp / 2) ** 2 < Np < (s + ulp / 2) ** 2
    n = [int(x) for x in case["N"]]
    W = [_f32(x) for x in case["W"]]
    P = [_f32(x) for x in case["P"]]
    vl = _f32(case["vl"])

    def score(i, alt):
        q = _round32(W[i] / _round32(Fraction(n[i]) + vl))
        num = _round32(c * _round32(P[i] * s)) if alt else _round32(_round32(c * P[i]) * s)
        return _round32(q + _round32(num / (1 + n[i])))

    def pick(alt):
        sc = [score(i, alt) for i in range(len(n))]
        best = 0
        for i in range(1, len(sc)):
            if sc[i] > sc[best]:
                best = i
        return best

    assert _round32(_round32(c * P[1]) * s) != _round32(c * _round32(P[1] * s))
    assert [pick(False)] == case["expect"] == list(case["picks"])
    assert pick(True) != case["expect"][0]


@pytest.mark.parametrize("variant", ref_np.SELECT_VARIANTS)
def test_planted_misreading_fails(variant):
    """The numpy restatement with the misreading planted disagrees with the fixture, at least
    on the pinned row built against it."""
    failed = []
    for c in _rows():
        if c["k"] * c["m"] > 40000:
            continue  # (the widest random rows: slow in pure Python, pinned by the others)
        picks, _ = golden.crafted_expected_np(c, variant=variant)
        if not np.array_equal(picks, c["picks"]):
            failed.append(c["kind"])
    pinned = [c["kind"] for c in _pinned() if variant in c["pins"]]
    assert pinned and set(pinned) <= set(failed), (variant, failed)
