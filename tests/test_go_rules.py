"""Go rules of the leaves (omq_go_rules): known answers worked out by hand, the C oracle against
the numpy restatement on random positions, every planted misreading failing a known answer, and
small searches with the rules on (C oracle against the numpy restatement).

The rules (go_kernels.py:17-110, gpu_game_states.py:336-337,373-395,430-441): legal moves are
the empty points, without the root's ko point (inherited by every descendant) and, with the
suicide flag, without the points that have no empty orthogonal neighbour; the pass is always
legal.  A leaf below the root is terminal after two consecutive passes (the root's own trailing
passes counting when the whole path is passes) or when no point is empty."""
import numpy as np
import pytest

from oracle import ref_np
from oracle.oracle import Oracle
from omoknuni_quantum_amd.synthetic import games

KO, SUICIDE = 1, 2
BS = 5
CELLS = BS * BS
PASS = CELLS


def _pt(r, c):
    return r * BS + c


def _board(stones=()):
    b = np.zeros((BS, BS), np.int8)
    for (r, c), p in stones:
        b[r, c] = p
    return b


def _c_rules(board, moves, root_player=None, root_passes=0, ko=-1, flags=KO):
    bs = board.shape[0]
    orc = Oracle(games.go(bs), 1, 64, 1, 8)
    orc.set_go_rules(board[None], flags,
                     root_player=None if root_player is None else [root_player],
                     root_passes=[root_passes], root_ko=[ko])
    legal, term = orc.go_leaf_rules(0, moves)
    return legal, term == 4


def _both(board, moves, **kw):
    a = ref_np.go_rules(board, moves, **kw)
    b = _c_rules(board, moves, **kw)
    assert (list(a[0]), a[1]) == (list(b[0]), b[1]), (a, b)
    return a


def _empty_minus(board, moves, *drop):
    """The empty points of the position after the moves, minus `drop`, plus the pass."""
    taken = {_pt(r, c) for r in range(BS) for c in range(BS) if board[r, c] != 0}
    taken |= {a for a in moves if a != PASS}
    return [a for a in range(CELLS) if a not in taken and a not in drop] + [PASS]


def _known_cases():
    """(name, board, moves, kwargs, legal, terminal), each answer derived by hand."""
    cases = []
    e = _board()
    cases.append(("empty root", e, [], dict(), list(range(CELLS)) + [PASS], False))
    cases.append(("one move", e, [_pt(2, 2)], dict(), _empty_minus(e, [_pt(2, 2)]), False))
    # suicide: the corner (0,0) closed by two stones; (1,1) and the centre (2,2) closed by four
    # stones of both colours each, with their diagonal points empty
    s = _board([((0, 1), 1), ((1, 0), 2), ((1, 2), 1), ((3, 2), 2), ((2, 1), 1), ((2, 3), 2)])
    cases.append(("suicide corner and centre", s, [], dict(flags=SUICIDE),
                  _empty_minus(s, [], _pt(0, 0), _pt(1, 1), _pt(2, 2)), False))
    cases.append(("no suicide flag", s, [], dict(flags=0), _empty_minus(s, []), False))
    # the path's own stones close a point: after (4,3) and (3,4), the corner (4,4) is shut
    cases.append(("suicide from path stones", e, [_pt(4, 3), _pt(3, 4)], dict(flags=SUICIDE),
                  _empty_minus(e, [_pt(4, 3), _pt(3, 4)], _pt(4, 4)), False))
    # ko: excluded at the root and below it; not without the flag
    cases.append(("ko at root", e, [], dict(ko=7), _empty_minus(e, [], 7), False))
    cases.append(("ko below root", e, [_pt(0, 0), _pt(4, 4)], dict(ko=7),
                  _empty_minus(e, [_pt(0, 0), _pt(4, 4)], 7), False))
    cases.append(("ko without flag", e, [_pt(0, 0)], dict(ko=7, flags=0),
                  _empty_minus(e, [_pt(0, 0)]), False))
    # passes
    cases.append(("pass pass", e, [PASS, PASS], dict(), _empty_minus(e, []), True))
    cases.append(("one pass", e, [PASS], dict(), _empty_minus(e, []), False))
    cases.append(("pass after root pass", e, [PASS], dict(root_passes=1),
                  _empty_minus(e, []), True))
    cases.append(("move then pass, root pass", e, [_pt(1, 1), PASS], dict(root_passes=1),
                  _empty_minus(e, [_pt(1, 1)]), False))
    cases.append(("pass move pass", e, [PASS, _pt(1, 1), PASS], dict(),
                  _empty_minus(e, [_pt(1, 1)]), False))
    cases.append(("move pass pass", e, [_pt(1, 1), PASS, PASS], dict(),
                  _empty_minus(e, [_pt(1, 1)]), True))
    cases.append(("root with two passes", e, [], dict(root_passes=2),
                  list(range(CELLS)) + [PASS], False))
    # a full board: the last empty point filled by the path's move
    full = np.where(np.arange(CELLS).reshape(BS, BS) % 2 == 0, 1, 2).astype(np.int8)
    full[4, 4] = 0
    cases.append(("board filled", full, [_pt(4, 4)], dict(), [PASS], True))
    cases.append(("one point left", full, [], dict(), [_pt(4, 4), PASS], False))
    cases.append(("one point left, closed", full, [], dict(flags=SUICIDE), [PASS], False))
    return cases


@pytest.mark.parametrize("case", _known_cases(), ids=lambda c: c[0])
def test_known_answers(case):
    name, board, moves, kw, legal, term = case
    got = _both(board, moves, **kw)
    assert got == (legal, term), name


@pytest.mark.parametrize("variant", ref_np.GO_VARIANTS)
def test_planted_misreading_fails(variant):
    bad = [c[0] for c in _known_cases()
           if ref_np.go_rules(c[1], c[2], variant=variant, **c[3]) != (c[4], c[5])]
    assert bad, variant


def test_random_positions():
    """C oracle = numpy restatement on random positions, paths, flags, ko points and passes."""
    rng = np.random.default_rng(23)
    terms = suicides = 0
    for _ in range(600):
        bs = int(rng.integers(3, 10))
        cells = bs * bs
        fill = rng.uniform(0.0, 0.95)
        b = np.where(rng.random((bs, bs)) < fill, rng.integers(1, 3, (bs, bs)), 0).astype(np.int8)
        empties = np.flatnonzero(b.reshape(-1) == 0).tolist()
        rng.shuffle(empties)
        k = int(rng.integers(0, min(len(empties), 6) + 1))
        moves = empties[:k]
        for _i in range(int(rng.integers(0, 3))):   # passes anywhere, often at the end
            moves.insert(int(rng.integers(len(moves) // 2, len(moves) + 1)), cells)
        ko = int(rng.choice(empties)) if empties and rng.random() < 0.5 else -1
        kw = dict(root_player=int(rng.integers(1, 3)) if rng.random() < 0.5 else None,
                  root_passes=int(rng.integers(0, 3)), ko=ko, flags=int(rng.integers(0, 4)))
        legal, term = _both(b, moves, **kw)
        terms += term
        free = [a for a in range(cells) if b.reshape(-1)[a] == 0 and a not in moves]
        suicides += len(free) - (len(legal) - 1)
    assert terms > 50 and suicides > 100


def _rules_pair(seed, flags, bs=5, W=8, sims=160, vl=3.0):
    """A search with the Go rules on, from a root with closed points, a ko point and a root
    pass: the C oracle and the numpy restatement must build the same tree, and terminal leaves
    must occur."""
    model = games.go(bs)
    A = model.num_actions
    rng = np.random.default_rng(seed)
    board = _board([((0, 1), 1), ((1, 0), 2), ((2, 1), 1), ((2, 3), 2), ((1, 2), 1),
                    ((3, 2), 2)])
    board[4, 0] = 1
    ko, passes = 18, 1
    legal = games.legal_masks(model, board[None], 1)
    orc = Oracle(model, 1, 8000, W, 100)
    orc.set_params(1.4, vl, 0, 0, 1.0, 0.0)
    orc.set_roots(games.root_keys(seed, 1), legal, None)
    orc.set_go_rules(board[None], flags, root_passes=[passes], root_ko=[ko])
    orc.reset_tree(0)
    npt = ref_np.NpTree(8000, 1.4, vl)

    def rules(pacts):
        return ref_np.go_rules(board, pacts, root_passes=passes, ko=ko, flags=flags)

    nterm = 0
    for wi, w in enumerate([1] + [W] * (sims // W)):
        pol = rng.random((W, A)).astype(np.float32) + np.float32(0.01)
        pol[:, A - 1] *= np.float32(4.0)  # passes often enough for two in a row
        val = (rng.random(W) * 2 - 1).astype(np.float32)
        orc.wave(0, w, replay_policy=pol, replay_values=val)
        ref_np.np_wave(npt, w, 100, lambda p: rules(p)[0], pol, val,
                       terminal_of=lambda p: rules(p)[1])
        lw = orc.last_wave(0, w)
        nterm += int((lw["uterm"] == 4).sum())
        tr = orc.tree(0)
        n = tr["num_nodes"]
        assert n == npt.num_nodes, (wi, n, npt.num_nodes)
        for k in ("N", "parent", "first", "nchild", "action"):
            assert np.array_equal(tr[k], getattr(npt, k)[:n]), (wi, k)
        for k in ("W", "P"):
            assert np.array_equal(tr[k].view(np.int32), getattr(npt, k)[:n].view(np.int32))
        assert ko not in tr["action"][1:n].tolist() or not flags & KO
    return nterm


@pytest.mark.parametrize("flags", [KO, KO | SUICIDE])
def test_search_with_rules_matches_numpy(flags):
    assert _rules_pair(9, flags) > 5
