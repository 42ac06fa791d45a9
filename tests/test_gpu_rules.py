"""Gomoku terminal rule on the GPU (omq_gomoku_terminal through the C ABI) against the oracle:
terminal codes, legal counts and whole trees after every wave."""
import numpy as np
import pytest
import torch

from omoknuni_quantum_amd import _lib
from omoknuni_quantum_amd.core.engine import SearchParams, WaveEngine
from omoknuni_quantum_amd.synthetic import games
from omoknuni_quantum_amd.synthetic.evaluator import SyntheticEvaluator
from omoknuni_quantum_amd.synthetic.workloads import get
from oracle.oracle import Oracle
from oracle.parity import compare_wave, run_parity

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rule", [_lib.OMQ_RULE_FREESTYLE, _lib.OMQ_RULE_RENJU])
def test_dense_boards_parity(device, rule):
    wl = get("C2").scaled(name=f"dense9-rule{rule}", model=games.gomoku(9), max_stones=45,
                          num_trees=8, num_simulations=512, wave_size=64, capacity=60_000)
    stats = {}
    assert run_parity(wl, rule=rule, device=device, stats=stats) >= 2
    assert stats["terminal"] > 50


def test_dense_boards_large_wave_parity(device):
    """Waves above OMQ_SELECT_RECORDS_MAX_WAVE: the leaf records come from omq_leaf_info, and the
    terminal check overwrites their legal counts after it."""
    wl = get("C2").scaled(name="dense15-large-wave", model=games.gomoku(15), max_stones=150,
                          num_trees=3, num_simulations=2048, wave_size=1024, capacity=200_000)
    assert wl.wave_size > _lib.OMQ_SELECT_RECORDS_MAX_WAVE
    stats = {}
    assert run_parity(wl, rule=_lib.OMQ_RULE_FREESTYLE, device=device, stats=stats) >= 2
    assert stats["terminal"] > 0


def _planted_boards(T, bs, seed):
    """Root positions with black and white fours with a gap (a move in the gap makes five)
    and black 2+3 split lines (a move in the gap makes an overline of six)."""
    rng = np.random.default_rng(seed)
    boards = np.zeros((T, bs, bs), np.int8)
    for t in range(T):
        b = boards[t]
        r = int(rng.integers(0, bs))
        b[r, 0:2] = 1
        b[r, 3:6] = 1                       # black 11_111: the gap gives six
        r2 = (r + 3) % bs
        b[r2, 1:3] = 2
        b[r2, 4:6] = 2                      # white 22_22: the gap gives five
        c = int(rng.integers(0, bs))
        rows = [x for x in range(bs) if x not in (r, r2)][:4]
        for x in rows:
            if b[x, c] == 0:
                b[x, c] = 1                 # a black column four
        if (b != 0).sum() % 2:
            empties = np.flatnonzero(b.reshape(-1) == 0)
            b.reshape(-1)[empties[int(rng.integers(0, len(empties)))]] = 2
    return boards


@pytest.mark.parametrize("rule", [_lib.OMQ_RULE_FREESTYLE, _lib.OMQ_RULE_RENJU])
def test_planted_overlines_parity(device, rule):
    T, bs, W, cap = 6, 9, 32, 40_000
    model = games.gomoku(bs)
    boards = _planted_boards(T, bs, 40 + rule)
    keys = games.root_keys(99, T)
    legal = games.legal_masks(model, boards, T)
    eng = WaveEngine(model, T, cap, W, 100, device, SearchParams(c_puct=1.4, virtual_loss=3.0))
    eng.set_roots(keys, legal)
    eng.set_gomoku_rules(boards, rule)
    orc = Oracle(model, T, cap, W, 100)
    orc.set_params(1.4, 3.0, 0, 0, 1.0, 0.0)
    orc.set_roots(keys, legal)
    orc.set_gomoku_rules(boards, rule)
    ev = SyntheticEvaluator()
    eng.reset()
    for t in range(T):
        orc.reset_tree(t)
    codes = np.zeros(4, np.int64)
    for i, w in enumerate([1] + [W] * 12):
        eng.run_wave(w, ev)
        for t in range(T):
            orc.wave(t, w)
            u = orc.last_wave(t, w)["uterm"]
            codes += np.bincount(u, minlength=4)
        torch.cuda.synchronize()
        compare_wave(eng, orc, w, f"planted rule {rule} wave {i}")
    assert codes[1] + codes[2] > 0
