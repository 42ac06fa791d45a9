"""Subtree reuse (CSRTree.shift_root): the C oracle against the numpy restatement, structural
invariants, and searches that continue on the reused tree."""
import numpy as np
import pytest

from oracle import ref_np
from oracle.oracle import Oracle
from omoknuni_quantum_amd.synthetic import games


def _pair_search(seed, bs=5, W=8, sims=160, vl=3.0):
    model = games.gomoku(bs)
    A = model.num_actions
    rng = np.random.default_rng(seed)
    board = np.zeros(A, np.int8)
    board[rng.permutation(A)[:2]] = [1, 2]
    legal = games.legal_masks(model, board.reshape(1, bs, bs), 1)
    root_empty = [a for a in range(A) if board[a] == 0]
    orc = Oracle(model, 1, 8000, W, 100)
    orc.set_params(1.4, vl, 0, 0, 1.0, 0.0)
    orc.set_roots(games.root_keys(seed, 1), legal, None)
    orc.reset_tree(0)
    npt = ref_np.NpTree(8000, 1.4, vl)
    state = {"root_empty": root_empty, "legal": legal, "rng": rng, "model": model}
    _waves(orc, npt, state, [1] + [W] * (sims // W))
    return orc, npt, state


def _waves(orc, npt, st, sizes):
    A = st["model"].num_actions
    legal_of = lambda pacts: ref_np.board_legal(st["root_empty"], pacts)  # noqa: E731
    for w in sizes:
        pol = st["rng"].random((max(sizes), A)).astype(np.float32) + np.float32(0.01)
        val = (st["rng"].random(max(sizes)) * 2 - 1).astype(np.float32)
        orc.wave(0, w, replay_policy=pol, replay_values=val)
        ref_np.np_wave(npt, w, 100, legal_of, pol, val)


def _assert_same(orc, npt, ctx):
    tr = orc.tree(0)
    n = tr["num_nodes"]
    assert n == npt.num_nodes, ctx
    for k in ("N", "parent", "first", "nchild", "action"):
        assert np.array_equal(tr[k], getattr(npt, k)[:n]), (ctx, k)
    for k in ("W", "P"):
        assert np.array_equal(tr[k].view(np.int32), getattr(npt, k)[:n].view(np.int32)), (ctx, k)
    assert np.array_equal(tr["children"], np.arange(1, n, dtype=np.int32)), ctx


def _subtree(tr, r):
    """Old node ids of the subtree of r, depth-first (order-free set)."""
    out, stack = [], [r]
    while stack:
        x = stack.pop()
        out.append(x)
        f, k = tr["first"][x], tr["nchild"][x]
        if f >= 0:
            stack.extend(range(f + 1, f + 1 + k))
    return out


@pytest.mark.parametrize("seed", [3, 4])
def test_shift_matches_numpy_and_keeps_subtree(seed):
    orc, npt, st = _pair_search(seed)
    before = orc.tree(0)
    f0, k0 = before["first"][0], before["nchild"][0]
    kids = np.arange(f0 + 1, f0 + 1 + k0)
    r = int(kids[np.argmax(before["N"][kids])])
    sub = _subtree(before, r)
    kept = orc.shift_root(0, r)
    mapping = npt.shift_root(r)
    assert kept == len(sub) == len(mapping)
    _assert_same(orc, npt, "after shift")
    after = orc.tree(0)
    # the kept nodes carry their statistics; breadth-first numbering keeps rows consecutive
    old_of_new = np.empty(kept, np.int64)
    for o, nw in mapping.items():
        old_of_new[nw] = o
    assert np.array_equal(after["N"], before["N"][old_of_new])
    assert np.array_equal(after["W"].view(np.int32), before["W"][old_of_new].view(np.int32))
    assert after["parent"][0] == -1 and after["action"][0] == -1
    assert np.all(after["parent"][1:] < np.arange(1, kept))
    assert np.array_equal(after["action"][1:], before["action"][old_of_new[1:]])
    # breadth-first: depths never decrease with the new index
    depth = np.zeros(kept, np.int64)
    for i in range(1, kept):
        depth[i] = depth[after["parent"][i]] + 1
    assert np.all(np.diff(depth) >= 0)


def test_search_continues_on_reused_tree():
    """After the shift both restatements search on from the new root (root legal set without
    the played action) and still build the same tree."""
    orc, npt, st = _pair_search(9)
    tr = orc.tree(0)
    f0, k0 = tr["first"][0], tr["nchild"][0]
    kids = np.arange(f0 + 1, f0 + 1 + k0)
    r = int(kids[np.argmax(tr["N"][kids])])
    a = int(tr["action"][r])
    orc.shift_root(0, r)
    npt.shift_root(r)
    st["root_empty"] = [x for x in st["root_empty"] if x != a]
    legal = st["legal"].copy()
    legal[0, a // 32] &= ~np.uint32(1 << (a % 32))
    orc.set_roots(games.root_keys(9, 1), legal, None)
    n0 = int(orc.tree(0)["N"][0])
    _waves(orc, npt, st, [8] * 12)
    _assert_same(orc, npt, "continued")
    assert int(orc.tree(0)["N"][0]) == n0 + 96


def test_shift_to_leaf_and_noop():
    orc, npt, _ = _pair_search(5, sims=16)
    tr = orc.tree(0)
    leaf = int(np.flatnonzero(tr["nchild"] == 0)[-1])
    assert orc.shift_root(0, 0) == 0 and orc.shift_root(0, 10 ** 6) == 0
    assert orc.shift_root(0, leaf) == 1
    npt.shift_root(leaf)
    _assert_same(orc, npt, "leaf")
    t2 = orc.tree(0)
    assert t2["num_nodes"] == 1 and t2["nchild"][0] == 0 and t2["first"][0] == -1
