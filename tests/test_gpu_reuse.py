"""Subtree reuse on the GPU (omq_shift_root through the C ABI) against the oracle's
CSRTree.shift_root restatement: the compacted trees, and searches continued on them."""
import numpy as np
import pytest
import torch

from omoknuni_quantum_amd.core.mcts import MCTS
from omoknuni_quantum_amd.core.mcts_config import GameType, MCTSConfig
from omoknuni_quantum_amd.synthetic import games
from omoknuni_quantum_amd.synthetic.evaluator import SyntheticEvaluator
from omoknuni_quantum_amd.synthetic.workloads import get
from oracle.oracle import Oracle
from oracle.parity import compare_wave, make_pair

pytestmark = pytest.mark.gpu


def _assert_trees(eng, orc, ctx):
    for t in range(eng.T):
        g, o = eng.host_tree(t), orc.tree(t)
        assert g["num_nodes"] == o["num_nodes"], (ctx, t)
        for k in ("N", "parent", "first", "nchild", "action"):
            assert np.array_equal(g[k], o[k]), (ctx, t, k)
        for k in ("W", "P"):
            assert np.array_equal(g[k].view(np.int32), o[k].view(np.int32)), (ctx, t, k)


@pytest.mark.parametrize("name", ["C2", "C4"])
def test_shift_and_continue_matches_oracle(device, name):
    wl = get(name).scaled(num_trees=4, num_simulations=768, wave_size=256, capacity=200_000)
    eng, orc, ev = make_pair(wl, device=device)
    eng.reset()
    for t in range(wl.num_trees):
        orc.reset_tree(t)
    for w in [1] + [256] * 3:
        eng.run_wave(w, ev)
        for t in range(wl.num_trees):
            orc.wave(t, w)
    torch.cuda.synchronize()
    # every tree moves to a different kind of child: most visited, least visited, a leaf child
    keys, legal, _ = wl.root_inputs()
    new_roots, acts = [], []
    for t in range(wl.num_trees):
        tr = orc.tree(t)
        f, k = tr["first"][0], tr["nchild"][0]
        kids = np.arange(f + 1, f + 1 + k)
        pick = [kids[np.argmax(tr["N"][kids])], kids[np.argmin(tr["N"][kids])],
                kids[np.argmax(tr["nchild"][kids] == 0)], kids[len(kids) // 2]][t % 4]
        new_roots.append(int(pick))
        acts.append(int(tr["action"][pick]))
    eng.shift_roots(new_roots)
    for t in range(wl.num_trees):
        assert orc.shift_root(t, new_roots[t]) >= 1
    torch.cuda.synchronize()
    _assert_trees(eng, orc, "after shift")
    # continue from the new roots: child keys, played actions removed from the legal masks
    keys = np.array([games.child_key(int(k), a) for k, a in zip(keys, acts)], np.uint64)
    if wl.model.is_board:
        for t, a in enumerate(acts):
            legal[t, a // 32] &= np.uint32(~(1 << (a % 32)) & 0xFFFFFFFF)
    eng.set_roots(keys, legal)
    orc.set_roots(keys, legal)
    for i in range(3):
        w = 256
        eng.run_wave(w, ev)
        for t in range(wl.num_trees):
            orc.wave(t, w)
        torch.cuda.synchronize()
        compare_wave(eng, orc, w, f"{name} continued wave {i}")


def _cfg(**kw):
    base = dict(num_simulations=384, c_puct=1.4, virtual_loss=3.0, max_wave_size=64,
                dirichlet_epsilon=0.0, max_tree_nodes=120_000, seed=3, board_size=15,
                game_type=GameType.GOMOKU, device="cuda")
    base.update(kw)
    return MCTSConfig(**base)


def test_update_root_reuses_subtree_like_oracle(device):
    cfg = _cfg()
    board = games.random_boards(1, 15, 12, 5, min_stones=12)[0]
    m = MCTS(cfg, SyntheticEvaluator())
    pol = m.search(board)
    a = int(np.argmax(pol))
    model = MCTS._game_model(cfg)
    orc = Oracle(model, 1, cfg.max_tree_nodes, cfg.max_wave_size, cfg.max_depth)
    orc.set_params(cfg.c_puct, cfg.virtual_loss, 0, 0, 1.0, 0.0)
    key0 = games.root_keys(cfg.seed, 1)
    orc.set_roots(key0, games.legal_masks(model, board[None], 1))
    orc.set_gomoku_rules(board[None], 0)
    orc.search(384, 64)
    tr = orc.tree(0)
    kids = np.arange(tr["first"][0] + 1, tr["first"][0] + 1 + tr["nchild"][0])
    child = int(kids[np.flatnonzero(tr["action"][kids] == a)[0]])
    # update_root without a new state: the board follows from the move
    m.update_root(a)
    assert m.stats["tree_reuse_count"] == 1
    kept = orc.shift_root(0, child)
    assert m.stats["tree_reuse_nodes"] == kept
    _assert_trees(m.engine, orc, "api shift")
    nb = board.copy()
    nb.reshape(-1)[a] = 1 if int((board != 0).sum()) % 2 == 0 else 2
    # the next search continues on the reused tree (same board as the one update_root made)
    pol2 = m.search(nb, num_simulations=256)
    orc.set_roots(np.array([games.child_key(int(key0[0]), a)], np.uint64),
                  games.legal_masks(model, nb[None], 1))
    orc.set_gomoku_rules(nb[None], 0)
    for _ in range(4):
        orc.wave(0, 64)
    _assert_trees(m.engine, orc, "api continued")
    assert np.array_equal(pol2, orc.root_policy(0))


def test_update_root_falls_back_to_reset(device):
    """A child below subtree_reuse_min_visits, or an action without a child, resets."""
    cfg = _cfg(num_simulations=64, subtree_reuse_min_visits=10_000)
    m = MCTS(cfg, SyntheticEvaluator())
    board = np.zeros((15, 15), np.int8)
    pol = m.search(board)
    m.update_root(int(np.argmax(pol)))
    assert m.stats["tree_reuse_count"] == 0
    assert int(m.engine.num_nodes[0].item()) == 1
    cfg = _cfg(num_simulations=64)
    m = MCTS(cfg, SyntheticEvaluator())
    board[7, 7] = 1
    m.search(board)
    m.update_root(7 * 15 + 7)  # occupied cell: no such child
    assert m.stats["tree_reuse_count"] == 0 and int(m.engine.num_nodes[0].item()) == 1


def test_shift_large_subtree_matches_oracle(device):
    # a kept subtree whose levels span several chunks of 4096 nodes (C3 rows of ~300 children)
    wl = get("C3").scaled(num_trees=1, num_simulations=4096, wave_size=1024, capacity=1_500_000)
    eng, orc, ev = make_pair(wl, device=device)
    eng.reset()
    orc.reset_tree(0)
    for w in [1] + [1024] * 4:
        eng.run_wave(w, ev)
        orc.wave(0, w)
    torch.cuda.synchronize()
    tr = orc.tree(0)
    f, k = tr["first"][0], tr["nchild"][0]
    kids = np.arange(f + 1, f + 1 + k)
    pick = int(kids[np.argmax(tr["N"][kids])])
    eng.shift_roots([pick])
    kept = orc.shift_root(0, pick)
    torch.cuda.synchronize()
    assert kept > 3 * 4096
    _assert_trees(eng, orc, "after a large shift")


@pytest.mark.parametrize("i", range(12))
def test_random_shift_and_continue_matches_oracle(device, i):
    """Seeded random workloads: after a few waves each tree keeps the subtree of a random root
    child (or stays whole: -1), on the GPU and in the oracle; the compacted trees and two more
    waves on them are compared."""
    _shift_and_continue(device, i, np.random.default_rng(5200 + i), wide=False)


@pytest.mark.parametrize("i", range(6))
def test_random_shift_and_continue_wide_boards(device, i):
    """The same on boards of 289-485 actions (select kernels of five, six and eight slots)."""
    _shift_and_continue(device, i, np.random.default_rng(5400 + i), wide=True)


def _shift_and_continue(device, i, rng, wide):
    kind = ["gomoku", "go"][i % 2] if wide else ["gomoku", "go", "sparse"][i % 3]
    if kind == "gomoku":
        model, base = games.gomoku(int(rng.choice([17, 18, 20, 21, 22]) if wide
                                       else rng.integers(5, 16))), "C2"
    elif kind == "go":
        model, base = games.go(int(rng.choice([17, 20, 21, 22] if wide
                                              else [5, 9, 13, 19]))), "C3"
    else:
        lo = int(rng.integers(1, 30))
        model, base = games.chess_sparse(int(rng.choice([64, 4672])), lo,
                                         lo + int(rng.integers(0, 30))), "C4"
    W = int(rng.choice([16, 64, 256, 600]))
    T = int(rng.integers(1, 5))
    waves = int(rng.integers(1, 4))
    stones = int(rng.integers(0, model.num_actions // 3)) if model.kind != "sparse" else 0
    wl = get(base).scaled(name=f"reuse-random-{i}", model=model, num_trees=T, max_stones=stones,
                          num_simulations=1 + W * (waves + 2), wave_size=W,
                          capacity=1 + W * (waves + 2) * (model.max_legal if model.kind ==
                                                          "sparse" else model.num_actions),
                          dirichlet_epsilon=0.0, seed=int(rng.integers(1, 1 << 30)))
    eng, orc, ev = make_pair(wl, device=device)
    eng.reset()
    for t in range(T):
        orc.reset_tree(t)
    for w in [1] + [W] * waves:
        eng.run_wave(w, ev)
        for t in range(T):
            orc.wave(t, w)
    torch.cuda.synchronize()
    keys, legal, _ = wl.root_inputs()
    new_roots, acts = [], []
    for t in range(T):
        tr = orc.tree(t)
        f, k = tr["first"][0], tr["nchild"][0]
        if k <= 0 or rng.random() < 0.2:
            new_roots.append(-1)
            acts.append(-1)
            continue
        pick = int(f + 1 + rng.integers(0, k))
        new_roots.append(pick)
        acts.append(int(tr["action"][pick]))
    eng.shift_roots(new_roots)
    for t in range(T):
        if new_roots[t] >= 0:
            assert orc.shift_root(t, new_roots[t]) >= 1
    torch.cuda.synchronize()
    _assert_trees(eng, orc, f"random {i} after shift")
    keys = np.array([games.child_key(int(kk), a) if a >= 0 else int(kk)
                     for kk, a in zip(keys, acts)], np.uint64)
    if wl.model.is_board:
        for t, a in enumerate(acts):
            if a >= 0 and not (model.kind == "go" and a == model.num_actions - 1):
                legal[t, a // 32] &= np.uint32(~(1 << (a % 32)) & 0xFFFFFFFF)
    eng.set_roots(keys, legal)
    orc.set_roots(keys, legal)
    for j in range(2):
        eng.run_wave(W, ev)
        for t in range(T):
            orc.wave(t, W)
        torch.cuda.synchronize()
        compare_wave(eng, orc, W, f"random {i} continued wave {j}")
