"""The capacity-full rule of expansion, pinned on tiny capacities.

expand_node (cython_tree_optimized.pyx:232-277) allocates a leaf's n children as one contiguous
run of nodes and edges, and refuses the whole leaf when ``num_nodes + n > max_nodes``
(:242-246).  The driver calls it for every unique leaf of the wave in first-occurrence order
(optimized_wave_search.py:367-438) and goes on after a refusal, so a later leaf with fewer
children can still fit.  A refused leaf stays unexpanded but is backed up like any other
(optimized_wave_search.py:457-483).

The checks below follow from that rule alone, with each leaf's child count taken from the
game model, not from the oracle: 5x5 Gomoku (the root's empty cells less the path's moves, so
counts fall with depth) and the sparse model with 1-10 legal actions per node (a count hashed
from the node's key, so neighbouring leaves differ and later leaves often fit after a refusal):
* ``num_nodes <= capacity`` after every wave;
* walking the wave's unique leaves in first-occurrence order with a running node count, a leaf
  is expanded (with its k children at the running count) exactly when the k fit, and refused
  with no children otherwise;
* a leaf's visit count grows by the number of simulations that ended at it, refused or not,
  and the root's count is 2 + simulations.
The scenarios refuse thousands of leaves and expand dozens after a refusal in the same wave.
The planted first-fail and partial-expansion misreadings (ref_np.CAP_VARIANTS) each break a
check, on the restatement run over a toy model whose counts also vary from leaf to leaf.
"""
import numpy as np
import pytest

from oracle import ref_np
from oracle.oracle import Oracle
from omoknuni_quantum_amd.synthetic import games

BS, WAVE, NWAVES = 5, 16, 12
SCENARIOS = [(stones, cap) for stones in (3, 8, 13, 17) for cap in (30, 55, 80, 130)]
SPARSE_CAPS = tuple(range(24, 200, 4))
SPARSE = games.chess_sparse(64, 1, 10)
EVENTS = ("expanded", "refused", "fit_after_refusal")


def _board(stones: int, seed: int):
    rng = np.random.default_rng(seed)
    board = np.zeros(BS * BS, np.int8)
    board[rng.permutation(BS * BS)[:stones]] = np.where(np.arange(stones) % 2 == 0, 1, 2)
    return board.reshape(1, BS, BS)


def _snapshot(N, nchild, first, expanded, parent, num_nodes):
    n = int(num_nodes)
    return {"N": np.array(N[:n]), "nchild": np.array(nchild[:n]), "first": np.array(first[:n]),
            "expanded": np.array(expanded[:n]).astype(bool), "parent": np.array(parent[:n]),
            "num_nodes": n}


def check_wave(cap, k_of, before, after, paths):
    """Violations of the capacity rule in one wave, and event counts; k_of(path) is the child
    count the game model gives the path's leaf."""
    bad = []
    ev = dict.fromkeys(EVENTS, 0)
    if after["num_nodes"] > cap:
        bad.append(f"num_nodes {after['num_nodes']} > capacity {cap}")
    leaves = [p[-1] for p in paths]
    order = []
    for s, leaf in enumerate(leaves):
        if leaf not in order:
            order.append(leaf)
    path_of = {p[-1]: p for p in paths}
    n = before["num_nodes"]
    refused = False
    for leaf in order:
        if before["expanded"][leaf]:
            continue
        k = k_of(path_of[leaf])
        if k <= 0:
            if after["nchild"][leaf] != 0:
                bad.append(f"leaf {leaf} without legal moves has children")
            continue
        if n + k <= cap:
            if after["nchild"][leaf] != k or not after["expanded"][leaf]:
                bad.append(f"leaf {leaf}: {k} children fit at {n}, got {after['nchild'][leaf]}")
            elif after["first"][leaf] != n - 1 or not np.all(after["parent"][n:n + k] == leaf):
                bad.append(f"leaf {leaf}: row not at the running count {n}")
            ev["expanded"] += 1
            ev["fit_after_refusal"] += refused
            n += k
        else:
            if after["nchild"][leaf] != 0 or after["expanded"][leaf]:
                bad.append(f"leaf {leaf}: {k} children do not fit at {n}, got "
                           f"{after['nchild'][leaf]}")
            ev["refused"] += 1
            refused = True
    if after["num_nodes"] != n:
        bad.append(f"num_nodes {after['num_nodes']}, rule {n}")
    for leaf in order:
        ends = leaves.count(leaf)
        if after["N"][leaf] - before["N"][leaf] != ends:
            bad.append(f"leaf {leaf}: N grew by {after['N'][leaf] - before['N'][leaf]}, "
                       f"{ends} simulations ended there")
    return bad, ev


def _waves(seed, A):
    rng = np.random.default_rng(seed)
    out = []
    for wi in range(NWAVES + 1):
        w = 1 if wi == 0 else WAVE
        out.append((w, rng.random((WAVE, A)).astype(np.float32) + np.float32(0.01),
                    (rng.random(WAVE) * 2 - 1).astype(np.float32)))
    return out


def _run_oracle(model, cap, seed, legal, k_of_tree):
    orc = Oracle(model, 1, cap, WAVE, 100)
    orc.set_params(1.4, 3.0, 0, 0, 1.0, 0.0)
    keys = games.root_keys(seed, 1)
    orc.set_roots(keys, legal, None)
    orc.reset_tree(0)
    bad, ev, sims = [], dict.fromkeys(EVENTS, 0), 0
    for w, pol, val in _waves(seed, model.num_actions):
        tr = orc.tree(0)
        before = _snapshot(tr["N"], tr["nchild"], tr["first"], tr["expanded"], tr["parent"],
                           tr["num_nodes"])
        orc.wave(0, w, replay_policy=pol, replay_values=val)
        tr = orc.tree(0)
        after = _snapshot(tr["N"], tr["nchild"], tr["first"], tr["expanded"], tr["parent"],
                          tr["num_nodes"])
        paths = [list(map(int, p)) for p in orc.last_wave(0, w)["paths"]]
        b, e = check_wave(cap, k_of_tree(tr, int(keys[0])), before, after, paths)
        bad += b
        for k in ev:
            ev[k] += e[k]
        sims += w
    if int(orc.tree(0)["N"][0]) != 1 + sims:
        bad.append(f"root N {int(orc.tree(0)['N'][0])}, 1 + {sims} simulations")
    return bad, ev


def run_oracle_gomoku(stones, cap, seed):
    model = games.gomoku(BS)
    board = _board(stones, seed)
    empty = int((board == 0).sum())
    return _run_oracle(model, cap, seed, games.legal_masks(model, board, 1),
                       lambda tr, key: lambda path: empty - (len(path) - 1))


def run_oracle_sparse(cap, seed):
    """Sparse model: a node's count is hashed from its key, the chain of child keys along the
    path's actions from the root's key."""
    def k_of_tree(tr, root_key):
        def k_of(path):
            key = root_key
            for node in path[1:]:
                key = games.child_key(key, int(tr["action"][node]))
            return games.sparse_root_count(SPARSE, key)
        return k_of
    return _run_oracle(SPARSE, cap, seed, games.legal_masks(SPARSE, None, 1), k_of_tree)


def _toy_count(pacts):
    """Toy model of the restatement runs: 1-9 legal actions, hashed from the path's moves."""
    h = 0x51ED
    for a in pacts:
        h = games.splitmix64(h ^ (a + 1))
    return 1 + h % 9


def run_restatement(cap, seed, cap_variant=None, stones=None):
    """Gomoku (stones given) or the toy model on the numpy restatement."""
    if stones is not None:
        board = _board(stones, seed)
        root_empty = [a for a in range(BS * BS) if board.reshape(-1)[a] == 0]
        legal_of = lambda pacts: ref_np.board_legal(root_empty, pacts)  # noqa: E731
        A = BS * BS
    else:
        A = 64
        legal_of = lambda pacts: list(range(_toy_count(pacts)))  # noqa: E731
    t = ref_np.NpTree(cap, 1.4, 3.0, cap_variant=cap_variant)
    k_of = lambda path: len(legal_of([int(t.action[x]) for x in path[1:]]))  # noqa: E731
    bad, ev = [], dict.fromkeys(EVENTS, 0)
    for w, pol, val in _waves(seed, A):
        before = _snapshot(t.N, t.nchild, t.first, t.expanded, t.parent, t.num_nodes)
        paths, _ = ref_np.np_wave(t, w, 100, legal_of, pol, val)
        after = _snapshot(t.N, t.nchild, t.first, t.expanded, t.parent, t.num_nodes)
        b, e = check_wave(cap, k_of, before, after, paths)
        bad += b
        for k in ev:
            ev[k] += e[k]
    return bad, ev


def test_oracle_follows_capacity_rule():
    total = dict.fromkeys(EVENTS, 0)
    runs = [("gomoku", stones, cap, 40 + i) for i, (stones, cap) in enumerate(SCENARIOS)]
    runs += [("sparse", None, cap, 90 + i) for i, cap in enumerate(SPARSE_CAPS)]
    for kind, stones, cap, seed in runs:
        if kind == "gomoku":
            bad, ev = run_oracle_gomoku(stones, cap, seed)
        else:
            bad, ev = run_oracle_sparse(cap, seed)
        assert not bad, (kind, stones, cap, bad[:5])
        for k in total:
            total[k] += ev[k]
    # the scenarios exercise the rule: many refusals, and leaves that fit after one
    assert total["refused"] >= 1000, total
    assert total["fit_after_refusal"] >= 40, total


def test_restatement_follows_capacity_rule():
    for i, (stones, cap) in enumerate(SCENARIOS[::3]):
        bad, _ = run_restatement(cap, 40 + 3 * i, stones=stones)
        assert not bad, (stones, cap, bad[:5])
    for i, cap in enumerate(SPARSE_CAPS[::4]):
        bad, _ = run_restatement(cap, 90 + 4 * i)
        assert not bad, (cap, bad[:5])


@pytest.mark.parametrize("variant", ref_np.CAP_VARIANTS)
def test_planted_capacity_misreadings_fail(variant):
    failures = sum(bool(run_restatement(cap, 90 + i, cap_variant=variant)[0])
                   for i, cap in enumerate(SPARSE_CAPS))
    assert failures >= len(SPARSE_CAPS) // 4, (variant, failures)


def test_capacity_zero_room_never_partially_fills():
    """At one free node below capacity, a leaf of several children is refused whole."""
    t = ref_np.NpTree(4, 1.4, 3.0)
    assert t.expand(0, [0, 1], [0.5, 0.5])          # nodes 1, 2
    assert not t.expand(1, [2, 3], [0.5, 0.5])       # 3 + 2 > 4: refused, nothing written
    assert t.num_nodes == 3 and t.nchild[1] == 0 and not t.expanded[1]
    assert t.expand(2, [4], [1.0])                   # a later leaf of one child still fits
    assert t.num_nodes == 4 and t.first[2] == 2 and t.nchild[2] == 1
