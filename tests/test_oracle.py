"""CPU checks that pin the C oracle: known answers, error bounds, closed forms, an independent
numpy-float32 restatement (bit-equal trees), and brute force of the grouped selection."""
import math

import numpy as np
import pytest

from oracle import ref_np
from oracle.oracle import Oracle, load
from omoknuni_quantum_amd.synthetic import games

GOLDEN = 0x9E3779B97F4A7C15
M64 = (1 << 64) - 1


def test_splitmix64_published_sequence():
    # Vigna's splitmix64.c with state 0: the first three outputs
    expect = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    lib = load()
    for i, e in enumerate(expect):
        assert lib.orc_splitmix64((GOLDEN * i) & M64) == e
        assert games.splitmix64((GOLDEN * i) & M64) == e


def test_exp_cw_error_bound():
    lib = load()
    xs = np.concatenate([np.linspace(-86.9, 0.0, 20001), -np.logspace(-8, 1.9, 2000), [0.0]])
    for x in xs.astype(np.float32):
        got = lib.orc_exp_cw(float(x))
        ref = math.exp(float(x))
        assert abs(got - ref) <= 4e-7 * ref, (x, got, ref)
    assert lib.orc_exp_cw(-100.0) == 0.0
    assert lib.orc_exp_cw(0.0) == 1.0


def test_key_normal_moments_and_support():
    lib = load()
    z = np.array([lib.orc_key_normal(games.splitmix64(k), a) for k in range(400) for a in range(50)])
    assert abs(z.mean()) < 0.03 and abs(z.var() - 1.0) < 0.05
    assert z.min() >= -6.0 and z.max() <= 6.0
    # values are multiples of 2^-16 (integer construction)
    assert np.all(np.round(z * 65536) == z * 65536)


def test_key_value_exact_grid():
    lib = load()
    v = np.array([lib.orc_key_value(games.splitmix64(k)) for k in range(5000)], dtype=np.float64)
    assert v.min() >= -1.0 and v.max() < 1.0
    assert np.all(np.round((v + 1.0) * 2 ** 23) == (v + 1.0) * 2 ** 23)
    assert abs(v.mean()) < 0.05


def test_sum64_definition():
    lib = load()
    rng = np.random.default_rng(1)
    for n in (1, 3, 63, 64, 65, 200, 362):
        ints = rng.integers(0, 1000, n).astype(np.float32)  # exact sums
        assert lib.orc_sum64(ints.ctypes.data, n) == float(ints.sum())
        x = rng.random(n).astype(np.float32)
        assert lib.orc_sum64(x.ctypes.data, n) == float(ref_np.sum64(x))
        xd = rng.random(n)
        assert lib.orc_sum64d(xd.ctypes.data, n) == ref_np.sum64d(xd)


def test_ucb_closed_form():
    """Two visited children, parent visits 4 (incl. virtual loss): Q + c*P*sqrt(Np)/(1+N) with
    Q = W/(N + VL) (cython_tree_optimized.pyx:456-458)."""
    t = ref_np.NpTree(8, 1.4, 3.0)
    t.expand(0, [0, 1], [0.6, 0.4])
    t.N[1], t.W[1] = 2, 1.0
    t.N[2], t.W[2] = 1, -0.5
    sa = 1.0 / 5 + 1.4 * 0.6 * 2.0 / 3
    sb = -0.5 / 4 + 1.4 * 0.4 * 2.0 / 2
    assert sa > sb
    assert t.best_child(0, 4) == 1
    t.W[1] = -2.0  # now B wins
    assert -2.0 / 5 + 1.4 * 0.6 * 2.0 / 3 < sb
    assert t.best_child(0, 4) == 2
    # first unvisited child wins regardless of scores
    t.N[2] = 0
    assert t.best_child(0, 4) == 2


def test_backup_signs_closed_form():
    """Path root -> child -> grandchild, value 0.8 (test_mcts_phases_detailed.py:578-616):
    leaf +0.8, parent -0.8, root +0.8; N += 1 after the virtual loss is reverted."""
    for root_positive in (False, True):
        t = ref_np.NpTree(8, 1.4, 3.0)
        t.expand(0, [0], [1.0])
        t.expand(1, [0], [1.0])
        t.N[:3] = [0, 0, 0]
        for x in (0, 1, 2):
            t.N[x] += 3
        t.backup([0, 1, 2], 0.8, root_positive)
        assert list(t.N[:3]) == [1, 1, 1]
        assert np.allclose(t.W[:3], [0.8, -0.8, 0.8])
    t = ref_np.NpTree(8, 1.4, 3.0)
    t.N[:2] = [3, 3]
    t.backup([0, 1], 0.5, False)
    assert np.allclose(t.W[:2], [-0.5, 0.5])
    t.backup([0, 1], 0.5, True)
    assert np.allclose(t.W[:2], [0.0, 0.0])


def _run_pair(policy, root_positive, eps, seed, vl=3.0, W=8, sims=160, bs=5):
    model = games.gomoku(bs)
    A = model.num_actions
    rng = np.random.default_rng(seed)
    board = np.zeros((1, bs, bs), np.int8)
    board.reshape(1, -1)[0, rng.permutation(A)[:3]] = [1, 2, 1]
    legal_mask = games.legal_masks(model, board, 1)
    root_empty = [a for a in range(A) if board.reshape(-1)[a] == 0]
    noise = None
    if eps > 0:
        noise = np.zeros((1, A))
        noise[0, :len(root_empty)] = rng.dirichlet([0.3] * len(root_empty))
    cap = 4000
    orc = Oracle(model, 1, cap, max(W, 1), 100)
    orc.set_params(1.4, vl, 1 if policy == "reference_pw" else 0, 1 if root_positive else 0, 1.0, eps)
    orc.set_roots(games.root_keys(seed, 1), legal_mask, noise)
    orc.reset_tree(0)
    npt = ref_np.NpTree(cap, 1.4, vl)
    legal_of = lambda pacts: ref_np.board_legal(root_empty, pacts)
    waves = [1] + [W] * (sims // W)
    for wi, w in enumerate(waves):
        pol = rng.random((max(W, 1), A)).astype(np.float32) + np.float32(0.01)
        val = (rng.random(max(W, 1)) * 2 - 1).astype(np.float32)
        if wi % 5 == 3:  # ties: identical priors and values
            pol[:] = np.float32(0.5)
            val[:] = np.float32(0.25)
        orc.wave(0, w, replay_policy=pol, replay_values=val)
        ref_np.np_wave(npt, w, 100, legal_of, pol, val, policy,
                       None if noise is None else noise[0], eps, root_positive)
        tr = orc.tree(0)
        n = tr["num_nodes"]
        assert n == npt.num_nodes, (wi, n, npt.num_nodes)
        for k in ("N", "parent", "first", "nchild", "action"):
            assert np.array_equal(tr[k], getattr(npt, k)[:n]), (wi, k)
        for k in ("W", "P"):
            assert np.array_equal(tr[k].view(np.int32), getattr(npt, k)[:n].view(np.int32)), (wi, k)
        assert np.array_equal(tr["children"], npt.children[:n - 1])
    return npt


@pytest.mark.parametrize("policy", ["full", "reference_pw"])
@pytest.mark.parametrize("root_positive", [False, True])
@pytest.mark.parametrize("eps", [0.0, 0.25])
def test_oracle_matches_numpy_restatement(policy, root_positive, eps):
    npt = _run_pair(policy, root_positive, eps, seed=11)
    assert npt.N[0] == 2 + 160


@pytest.mark.parametrize("vl", [0.0, 1.0, 3.0])
def test_oracle_matches_numpy_small_waves(vl):
    _run_pair("full", False, 0.0, seed=5, vl=vl, W=3, sims=60, bs=4)


@pytest.mark.parametrize("seed", range(6))
def test_grouped_selection_equals_sequential(seed):
    """The device's grouped rank-VL schedule reproduces sequential select_path exactly."""
    rng = np.random.default_rng(100 + seed)
    bs = 4
    A = bs * bs
    root_empty = list(range(A))
    legal_of = lambda pacts: ref_np.board_legal(root_empty, pacts)
    vl = [3.0, 1.0, 0.0][seed % 3]
    t = ref_np.NpTree(3000, 1.4, vl)
    waves = [1] + [int(rng.integers(2, 9)) for _ in range(12)]
    for w in waves:
        pol = rng.random((w, A)).astype(np.float32)
        if seed % 2:
            pol[:] = 1.0  # equal priors: many exact ties
        val = np.round(rng.random(w) * 4 - 2).astype(np.float32) / 4
        W = int(rng.integers(2, 12))
        import copy
        a, b = copy.deepcopy(t), copy.deepcopy(t)
        seq = [a.select_path(100) for _ in range(W)]
        grp = b.grouped_select(W, 100) if hasattr(b, "grouped_select") else ref_np.grouped_select(b, W, 100)
        assert seq == grp
        assert np.array_equal(a.N, b.N)
        ref_np.np_wave(t, w, 100, legal_of, pol, val)


@pytest.mark.parametrize("seed", range(6))
def test_overlap_selection_equals_sequential(seed):
    """The level overlap (root chain, then each root child's chain continued block by block
    with the virtual loss kept in N) reproduces sequential select_path exactly."""
    import copy
    rng = np.random.default_rng(300 + seed)
    bs = 4
    A = bs * bs
    root_empty = list(range(A))
    legal_of = lambda pacts: ref_np.board_legal(root_empty, pacts)
    vl = [3.0, 1.0, 2.0][seed % 3]
    t = ref_np.NpTree(4000, 1.4, vl)
    for it in range(14):
        w = 1 if it == 0 else int(rng.integers(2, 9))
        pol = rng.random((w, A)).astype(np.float32)
        if seed % 2:
            pol[:] = 1.0  # equal priors: many exact ties
        val = np.round(rng.random(w) * 4 - 2).astype(np.float32) / 4
        W = int(rng.integers(2, 14))
        for block in (1, 2, 3, 5):
            for max_depth in (100, 2, 3):
                a, b = copy.deepcopy(t), copy.deepcopy(t)
                seq = [a.select_path(max_depth) for _ in range(W)]
                ovl = ref_np.overlap_select(b, W, max_depth, block)
                assert seq == ovl, (it, block, max_depth)
                assert np.array_equal(a.N, b.N), (it, block, max_depth)
        ref_np.np_wave(t, w, 100, legal_of, pol, val)


def _runahead_check(seed):
    """Run-ahead schedules against sequential select_path on one seeded search; returns how
    often each planted misreading differed."""
    import copy
    rng = np.random.default_rng(500 + seed)
    bs = 3  # (9 actions: rows fill up, so that picks depend on the parent count)
    A = bs * bs
    root_empty = list(range(A))
    legal_of = lambda pacts: ref_np.board_legal(root_empty, pacts)
    vl = [3.0, 1.0, 2.0][seed % 3]
    t = ref_np.NpTree(4000, 1.4, vl)
    caught = {v: 0 for v in ref_np.RUNAHEAD_VARIANTS}
    compared = 0
    for it in range(30):
        w = 1 if it == 0 else int(rng.integers(2, 9))
        pol = rng.random((w, A)).astype(np.float32)
        if seed % 2:
            pol[:] = 1.0  # equal priors: many exact ties
        val = np.round(rng.random(w) * 4 - 2).astype(np.float32) / 4
        W = int(rng.integers(2, 16))
        if t.expanded[0] and t.nchild[0] > 0:
            f, k = int(t.first[0]), int(t.nchild[0])
            kids = [int(t.children[f + i]) for i in range(k)]
            for max_depth in (100, 3):
                for trial in range(4):
                    chosen = rng.choice(kids, size=min(len(kids), int(rng.integers(1, 5))),
                                        replace=False)
                    budgets = {int(c): int(rng.integers(1, W + 3)) for c in chosen}
                    done = {c: int(rng.integers(0, M + 1)) for c, M in budgets.items()}
                    a, b = copy.deepcopy(t), copy.deepcopy(t)
                    seq = [a.select_path(max_depth) for _ in range(W)]
                    ra = ref_np.runahead_select(b, W, max_depth, budgets, done)
                    assert seq == ra, (it, max_depth, budgets, done)
                    assert np.array_equal(a.N, b.N), (it, max_depth)
                    compared += 1
                    for v in ref_np.RUNAHEAD_VARIANTS:
                        c = copy.deepcopy(t)
                        bad = ref_np.runahead_select(c, W, max_depth, budgets, done, variant=v)
                        caught[v] += int(bad != seq)
        ref_np.np_wave(t, w, 100, legal_of, pol, val)
    assert compared >= 40
    return caught


@pytest.mark.parametrize("seed", range(6))
def test_runahead_selection_equals_sequential(seed):
    """Level-1 chains run ahead of the root chain from the wave's start state, replayed whole
    or in part and continued (run-ahead budgets and ranks done drawn at random, from none of a
    group's ranks to more than all), reproduce sequential select_path exactly; continuing
    without the recorded picks' virtual loss does not."""
    assert _runahead_check(seed)["resume_without_counts"] > 0


def test_runahead_planted_parent_count():
    """Continuing a recorded chain with the parent count of rank 0 instead of the rank reached
    differs from sequential select_path (over the seeded searches of the test above)."""
    assert sum(_runahead_check(seed)["resume_parent_count_restarted"] for seed in (0, 2, 4)) > 0


def test_search_invariants_all_workload_models():
    from omoknuni_quantum_amd.synthetic.workloads import get
    for name, kw in [("C1", {"num_simulations": 256}), ("C3", {"num_trees": 1, "num_simulations": 2048}),
                     ("C4", {"num_trees": 1, "num_simulations": 4096, "capacity": 200_000})]:
        wl = get(name).scaled(**kw)
        orc = Oracle(wl.model, 1, wl.capacity, wl.wave_size, wl.max_depth)
        orc.set_params(wl.c_puct, wl.virtual_loss, 0, 0, wl.logit_scale, wl.dirichlet_epsilon)
        orc.set_roots(*wl.root_inputs())
        orc.search(wl.num_simulations, wl.wave_size)
        tr = orc.tree(0)
        f, k = tr["first"][0], tr["nchild"][0]
        kids = tr["children"][f:f + k]
        assert tr["N"][0] == 2 + wl.num_simulations          # root: init 1, root expansion, sims
        assert tr["N"][kids].sum() == wl.num_simulations     # every simulation passes a child
        assert np.array_equal(tr["children"], np.arange(1, tr["num_nodes"], dtype=np.int32))
        assert np.all(tr["parent"][1:] >= 0) and np.all(tr["parent"][1:] < np.arange(1, tr["num_nodes"]))
        # each expanded node's priors sum to ~1 over its children (full expansion)
        for p in np.flatnonzero(tr["nchild"] > 0)[:50]:
            s = tr["P"][tr["first"][p] + 1:tr["first"][p] + 1 + tr["nchild"][p]].sum()
            assert abs(s - 1.0) < 1e-4, (name, p, s)
        pol = orc.root_policy(0)
        assert abs(pol.sum() - 1.0) < 1e-12
