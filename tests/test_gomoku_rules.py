"""Gomoku terminal rule: known answers, the numpy restatement against the C oracle on random
dense boards, and small searches with the rule on (C oracle against the numpy restatement)."""
import numpy as np
import pytest

from oracle import ref_np
from oracle.oracle import Oracle, load
from omoknuni_quantum_amd.synthetic import games


def c_terminal(board, renju=False):
    b = np.ascontiguousarray(board, dtype=np.int8)
    return load().orc_gomoku_terminal(b.ctypes.data, b.shape[0], 1 if renju else 0)


def both(board, renju=False):
    a, b = ref_np.gomoku_terminal(board, renju), c_terminal(board, renju)
    assert a == b, (a, b)
    return a


def line(bs, cells, player, board=None):
    b = np.zeros((bs, bs), np.int8) if board is None else board
    for r, c in cells:
        b[r, c] = player
    return b


def test_known_answers():
    """Boards whose answer the rule fixes (fast_terminal_check.py:132-232)."""
    assert both(np.zeros((15, 15), np.int8)) == 0
    # five at each edge and in each direction
    assert both(line(15, [(3, c) for c in range(10, 15)], 2)) == 2
    assert both(line(15, [(r, 0) for r in range(10, 15)], 1)) == 1
    assert both(line(15, [(10 + i, 10 + i) for i in range(5)], 2)) == 2
    assert both(line(15, [(i, 4 - i) for i in range(5)], 1)) == 1
    # four is not enough, also not along a diagonal that runs off the board
    assert both(line(15, [(3, c) for c in range(4)], 1)) == 0
    assert both(line(15, [(i, 3 - i) for i in range(4)], 1)) == 0
    # a broken five
    assert both(line(15, [(7, c) for c in (2, 3, 4, 6, 7)], 1)) == 0
    # overline: wins in freestyle; under renju only for player 2
    six1 = line(15, [(5, c) for c in range(2, 8)], 1)
    assert both(six1) == 1 and both(six1, renju=True) == 0
    six2 = line(15, [(5, c) for c in range(2, 8)], 2)
    assert both(six2, renju=True) == 2
    # exactly five for player 1 under renju wins
    assert both(line(15, [(5, c) for c in range(2, 7)], 1), renju=True) == 1
    # renju: an overline of player 1 at a cell ends that cell's scan, so an exact vertical five
    # starting at the same cell is not seen (the reference's `continue` of its column loop)
    q = line(15, [(5, c) for c in range(2, 8)], 1)
    q = line(15, [(r, 2) for r in range(5, 10)], 1, q)
    assert both(q, renju=True) == 0 and both(q) == 1
    # two fives: the first cell in row-major order decides
    b = line(15, [(2, c) for c in range(5, 10)], 2)
    b = line(15, [(r, 12) for r in range(0, 5)], 1, b)
    assert both(b) == 1
    b = line(15, [(4, c) for c in range(0, 5)], 2)
    b = line(15, [(4 + i, 9 - i) for i in range(5)], 1, b)
    assert both(b) == 2
    # full board without five: draw; a full small board too
    draw = np.array([[1, 1, 2, 2, 1], [2, 2, 1, 1, 2], [1, 1, 2, 2, 1], [2, 2, 1, 1, 2],
                     [1, 1, 2, 2, 1]], np.int8)
    assert both(draw) == 3
    draw[0, 0] = 0
    assert both(draw) == 0
    assert both(np.ones((4, 4), np.int8)) == 3


@pytest.mark.parametrize("renju", [False, True])
def test_random_dense_boards(renju):
    rng = np.random.default_rng(17 + renju)
    wins = draws = 0
    for _ in range(1500):
        bs = int(rng.integers(5, 10))
        fill = rng.uniform(0.4, 1.0)
        b = np.where(rng.random((bs, bs)) < fill, rng.integers(1, 3, (bs, bs)), 0).astype(np.int8)
        r = both(b, renju)
        wins += r in (1, 2)
        draws += r == 3
    assert wins > 300 and draws >= 5


def _rules_pair(seed, bs=7, W=8, sims=120, renju=False, vl=3.0):
    """A search with the rule on, from a root with open fours for both players: the C oracle
    and the numpy restatement must build the same tree, and terminal leaves must occur."""
    model = games.gomoku(bs)
    A = model.num_actions
    rng = np.random.default_rng(seed)
    board = np.zeros((bs, bs), np.int8)
    board[1, 1:5] = 1
    board[5, 2:6] = 2
    board[3, 3] = 1  # player 2 to move (odd stone count)
    extra = [a for a in rng.permutation(A) if board.reshape(-1)[a] == 0][:2]
    board.reshape(-1)[extra] = [2, 1]
    legal = games.legal_masks(model, board[None], 1)
    root_empty = [a for a in range(A) if board.reshape(-1)[a] == 0]
    orc = Oracle(model, 1, 6000, W, 100)
    orc.set_params(1.4, vl, 0, 0, 1.0, 0.0)
    orc.set_roots(games.root_keys(seed, 1), legal, None)
    orc.set_gomoku_rules(board[None], 1 if renju else 0)
    orc.reset_tree(0)
    npt = ref_np.NpTree(6000, 1.4, vl)
    stones = int((board != 0).sum())
    rp = 1 if stones % 2 == 0 else 2

    def terminal_of(pacts):
        b = board.copy().reshape(-1)
        for q, a in enumerate(pacts):
            b[a] = rp if q % 2 == 0 else 3 - rp
        return ref_np.gomoku_terminal(b.reshape(bs, bs), renju) != 0

    legal_of = lambda pacts: ref_np.board_legal(root_empty, pacts)  # noqa: E731
    nterm = 0
    for wi, w in enumerate([1] + [W] * (sims // W)):
        pol = rng.random((W, A)).astype(np.float32) + np.float32(0.01)
        val = (rng.random(W) * 2 - 1).astype(np.float32)
        orc.wave(0, w, replay_policy=pol, replay_values=val)
        ref_np.np_wave(npt, w, 100, legal_of, pol, val, terminal_of=terminal_of)
        lw = orc.last_wave(0, w)
        nterm += int((lw["uterm"] != 0).sum())
        tr = orc.tree(0)
        n = tr["num_nodes"]
        assert n == npt.num_nodes, (wi, n, npt.num_nodes)
        for k in ("N", "parent", "first", "nchild", "action"):
            assert np.array_equal(tr[k], getattr(npt, k)[:n]), (wi, k)
        for k in ("W", "P"):
            assert np.array_equal(tr[k].view(np.int32), getattr(npt, k)[:n].view(np.int32))
    return nterm


@pytest.mark.parametrize("renju", [False, True])
def test_search_with_rules_matches_numpy(renju):
    assert _rules_pair(5, renju=renju) > 5
