"""The numpy restatements of the reference module's selection, noise, backup and subtree
operators (oracle/ref_np.py: parallel_select_with_virtual_loss, fused_ucb_with_noise,
batched_ucb_selection_dense, parallel_bfs_subtree, extract_subtree_edges), pinned by known
answers worked out by hand; each case is built so that one planted misreading (the *_VARIANTS
of ref_np) changes its answer, and every misreading fails one.  The Dirichlet rows of
batched_dirichlet_noise are restated with the C oracle's gamma variates and pinned by their
moments."""
import ctypes
import math

import numpy as np
import pytest

from oracle import ref_np
from oracle.oracle import load

F = np.float32


# ---- parallel_select_with_virtual_loss -------------------------------------------------------
def _psvl_case():
    """Nine parents, one per case (W / N / VL of a child, P 0 unless the case needs it):
    node 0  root: child 1 (q 0.9, action 5), child 2 (q 0.3); the simulation's mask forbids 5,
            which a root ignores -> 1                                   (mask_at_root -> 2)
    node 3  N 3: child 4 unvisited, P 0.5 -> 0.5 * sqrt(3 + 1) = 1.0 against child 5's q 0.9
            -> 4                                                        (sqrt(3): 0.87 -> 5)
    node 6  N 0, VL 3: child 7 unvisited, P 0.5 -> 0.5 * sqrt(0 + 1) = 0.5 against child 8's
            q 0.9 -> 8                                          (parent_with_vl: 1.0 -> 7)
    node 9  child 10: N 1, VL 1, W -0.5, value -0.5 + 1 * (-1) over n = 2: q -0.75; child 11:
            q -0.5 -> 11                                   (value_without_vl: -0.25 -> 10)
    node 12 row [13 (q 0.3), -1, 14 (q 0.9)]: the -1 is skipped -> 14 (row_ends_at_neg -> 13)
    node 15 two simulations: child 16 q 0.9, child 17 q 0.85; both see the same counts -> 16,
            16 (vl_between_sims: 16's q falls to (0.9 - 1) / 2 -> 17 for the second)
    node 18 non-root: child 19 (q 0.9, action 3) forbidden by the mask -> 20 (q 0.3)
    parent -1 and parent 99 (past the table) -> -1."""
    nn = 21
    children = np.full((nn, 4), -1, np.int32)
    rows = {0: [1, 2], 3: [4, 5], 6: [7, 8], 9: [10, 11], 12: [13, -1, 14], 15: [16, 17],
            18: [19, 20]}
    for p, r in rows.items():
        children[p, :len(r)] = r
    N = np.zeros(nn, np.int32)
    W = np.zeros(nn, F)
    P = np.zeros(nn, F)
    VL = np.zeros(nn, np.int32)
    acts = np.zeros(nn, np.int32)
    N[[0, 3, 6, 9, 12, 15, 18]] = [4, 3, 0, 5, 5, 5, 5]
    VL[6] = 3
    for c, n, w in ((1, 1, 0.9), (2, 1, 0.3), (5, 1, 0.9), (8, 1, 0.9), (10, 1, -0.5),
                    (11, 1, -0.5), (13, 1, 0.3), (14, 1, 0.9), (16, 1, 0.9), (17, 1, 0.85),
                    (19, 1, 0.9), (20, 1, 0.3)):
        N[c], W[c] = n, w
    VL[10] = 1
    P[[4, 7]] = 0.5
    acts[1], acts[2], acts[19], acts[20] = 5, 6, 3, 4
    parents = np.array([0, 3, 6, 9, 12, 15, 15, 18, -1, 99], np.int32)
    masks = np.ones((len(parents), 8), bool)
    masks[0, 5] = False
    masks[7, 3] = False
    return parents, children, N, VL, W, P, acts, masks


PSVL_EXPECT = [1, 4, 8, 11, 14, 16, 16, 20, -1, -1]


def test_psvl_known_answer():
    parents, children, N, VL, W, P, acts, masks = _psvl_case()
    sel, vl = ref_np.parallel_select_with_virtual_loss(parents, children, N, VL, W, P, acts, 1.0,
                                                       -1.0, masks)
    assert sel.tolist() == PSVL_EXPECT
    want = VL.copy()
    for c in PSVL_EXPECT:
        if c >= 0:
            want[c] += 1
    assert vl.tolist() == want.tolist()  # +1 per selection, after all of them
    # without the masks the non-root case takes its best child
    sel, _ = ref_np.parallel_select_with_virtual_loss(parents, children, N, VL, W, P, acts, 1.0,
                                                      -1.0, None)
    assert sel[7] == 19


@pytest.mark.parametrize("variant", ref_np.PSVL_VARIANTS)
def test_psvl_misreadings_fail(variant):
    parents, children, N, VL, W, P, acts, masks = _psvl_case()
    sel, _ = ref_np.parallel_select_with_virtual_loss(parents, children, N, VL, W, P, acts, 1.0,
                                                      -1.0, masks, variant=variant)
    assert sel.tolist() != PSVL_EXPECT, variant


def test_psvl_per_simulation_priors():
    """Per-simulation priors [sims, nodes]: two simulations at node 3 with P(4) = 0.5 and 0.4
    score child 4 at 1.0 and 0.8 against child 5's 0.9."""
    parents, children, N, VL, W, P, acts, masks = _psvl_case()
    pp = np.zeros((2, len(N)), F)
    pp[0, 4], pp[1, 4] = 0.5, 0.4
    sel, _ = ref_np.parallel_select_with_virtual_loss(np.array([3, 3], np.int32), children, N,
                                                      VL, W, pp, acts, 1.0, -1.0)
    assert sel.tolist() == [4, 5]


# ---- fused_ucb_with_noise ----------------------------------------------------------------------
def _ucbn_case():
    q = np.array([0.5, 0.4, 0.0], F)
    n = np.array([1, 0, 3], np.int32)
    p = np.array([0.2, 0.4, 0.8], F)
    noise = np.array([[1, 0, 0], [0, 0, 1]], F)
    return q, n, p, noise


def test_ucbn_known_answer():
    """sqrt 2, c 1, eps 0.5.  Simulation 0: priors 0.6 0.2 0.4, ucb 0.5 + 0.6 = 1.1, 0.4 + 0.4,
    0 + 0.2 -> 0.  Simulation 1: priors 0.1 0.2 0.9, ucb 0.6, 0.8, 0.45 -> 1 (the unvisited
    child keeps its q: with q = 0 it would score 0.4 -> 0; without the noise simulation 0's
    priors give 0.7, 1.2, 0.4 -> 1)."""
    q, n, p, noise = _ucbn_case()
    assert ref_np.fused_ucb_with_noise(q, n, p, noise, 2.0, 1.0, 0.5).tolist() == [0, 1]
    # nothing above -1e10: position 0
    low = np.full(3, -1e11, F)
    assert ref_np.fused_ucb_with_noise(low, n, p, noise, 2.0, 1.0, 0.5).tolist() == [0, 0]


@pytest.mark.parametrize("variant", ref_np.UCBN_VARIANTS)
def test_ucbn_misreadings_fail(variant):
    q, n, p, noise = _ucbn_case()
    low = np.full(3, -1e11, F)
    got = (ref_np.fused_ucb_with_noise(q, n, p, noise, 2.0, 1.0, 0.5, variant).tolist(),
           ref_np.fused_ucb_with_noise(low, n, p, noise, 2.0, 1.0, 0.5, variant).tolist())
    assert got != ([0, 1], [0, 0]), variant


# ---- batched_ucb_selection_dense -------------------------------------------------------------
def _ucbd_case():
    bc = np.array([[2, 0, 1], [1, 5, -1], [0, 1, 2], [0, 1, 2]], np.int32)
    bp = np.array([[0.5, 0.25, 0.25], [0.5, 0.5, 0.5], [0.0, 0.5, 0.0], [1, 1, 1]], F)
    valid = np.array([[1, 1, 1], [1, 1, 1], [1, 1, 0], [0, 0, 0]], bool)
    pv = np.array([3, 0, 3, 9], np.int32)
    cn = np.array([1, 0, 2], np.int32)
    cv = np.array([0.9, 0.7, 0.1], F)
    return bc, bp, pv, cn, cv, valid


UCBD_EXPECT = [0, 1, 1, -1]


def test_ucbd_known_answer():
    """Item 0, sqrt(3 + 1) = 2: child 2 0.1 + 0.5*2/3 = 0.433, child 0 0.9 + 0.25*2/2 = 1.15,
    child 1 (unvisited: value 0) 0.25*2/1 = 0.5 -> child 0 (slot 1).  Item 1: child 1 0.5, child
    5 past the children, -1 -> child 1.  Item 2: child 0 0.9, child 1 0.5*2 = 1.0 (sqrt(3)
    would give 0.87) -> child 1.  Item 3: no valid slot -> -1."""
    assert ref_np.batched_ucb_selection_dense(*_ucbd_case(), 1.0).tolist() == UCBD_EXPECT


@pytest.mark.parametrize("variant", ref_np.UCBD_VARIANTS)
def test_ucbd_misreadings_fail(variant):
    got = ref_np.batched_ucb_selection_dense(*_ucbd_case(), 1.0, variant=variant).tolist()
    assert got != UCBD_EXPECT, variant


# ---- parallel_bfs_subtree / extract_subtree_edges --------------------------------------------
def _csr(rows):
    ptr, col = [0], []
    for r in rows:
        col += r
        ptr.append(len(col))
    return np.array(ptr, np.int32), np.array(col, np.int32)


G_TREE = [[1, 2, 3], [4, 5], [], [6], [7], [], [], []]
G_DAG = [[3, 1, 3, 9], [2, 0], [], [2, 1, 4], []]  # repeats, a cycle, a child past max_nodes


def test_bfs_known_answers():
    ptr, col = _csr(G_TREE)
    ins, remap, n = ref_np.parallel_bfs_subtree(ptr, col, 0, 8)
    assert n == 8 and remap.tolist() == list(range(8))  # breadth-first = the ids here
    ins, remap, n = ref_np.parallel_bfs_subtree(ptr, col, 1, 8)
    assert n == 4 and remap.tolist() == [-1, 0, -1, -1, 1, 2, -1, 3]
    assert ins.tolist() == [False, True, False, False, True, True, False, True]
    # level 1 of the DAG from 0: 3, 1 (3 again and 9 skipped); level 2: 2 (from 3), 4 (from
    # 3); 1 and 0 are in already
    ptr, col = _csr(G_DAG)
    ins, remap, n = ref_np.parallel_bfs_subtree(ptr, col, 0, 5)
    assert n == 5 and remap.tolist() == [0, 2, 3, 1, 4]
    # from 1: 2, 0 then 3 (0's row; 1 is in, 9 skipped), then 4 (from 3)
    ins, remap, n = ref_np.parallel_bfs_subtree(ptr, col, 1, 5)
    assert remap.tolist() == [2, 0, 1, 3, 4]


@pytest.mark.parametrize("variant", ref_np.BFS_VARIANTS)
def test_bfs_misreadings_fail(variant):
    got = []
    for rows, root, n in ((G_TREE, 0, 8), (G_DAG, 0, 5), (G_DAG, 1, 5)):
        ptr, col = _csr(rows)
        got.append(ref_np.parallel_bfs_subtree(ptr, col, root, n, variant)[1].tolist())
    assert got != [list(range(8)), [0, 2, 3, 1, 4], [2, 0, 1, 3, 4]], variant


def _edge_case():
    ptr, col = _csr(G_DAG)
    act = np.arange(10, 10 + len(col)).astype(np.int16)
    ins = np.array([1, 1, 1, 1, 0], bool)  # node 4 left out
    remap = np.array([0, 2, 3, 1, -1], np.int32)
    return ptr, col, act, ins, remap


EDGE_EXPECT = ([0, 0, 0, 2, 2, 1, 1], [1, 2, 1, 3, 0, 3, 2], [10, 11, 12, 14, 15, 16, 17])


def test_edges_known_answer():
    """Node 0 (new 0): edges to 3, 1, 3 (9 is past the nodes); node 1 (new 2): to 2, 0; node 3
    (new 1): to 2, 1 (4 is outside the subtree).  Old node order, row order."""
    p, c, a = ref_np.extract_subtree_edges(*_edge_case())
    assert (p.tolist(), c.tolist(), a.tolist()) == EDGE_EXPECT
    ptr, col, act, ins, remap = _edge_case()
    p, c, a = ref_np.extract_subtree_edges(ptr, col, None, ins, remap)
    assert a.tolist() == [0] * 7


@pytest.mark.parametrize("variant", ref_np.EDGE_VARIANTS)
def test_edges_misreadings_fail(variant):
    p, c, a = ref_np.extract_subtree_edges(*_edge_case(), variant=variant)
    assert (p.tolist(), c.tolist(), a.tolist()) != EDGE_EXPECT, variant


def test_bfs_and_edges_rebuild_the_subtree():
    """On random trees the edges of the BFS subtree rebuild it: every kept node but the root
    has exactly one incoming edge, from its parent's new index, and new indices grow with
    depth."""
    rng = np.random.default_rng(5)
    for trial in range(20):
        n = int(rng.integers(2, 200))
        parent = [-1] + [int(rng.integers(0, i)) for i in range(1, n)]
        rows = [[] for _ in range(n)]
        for i in range(1, n):
            rows[parent[i]].append(i)
        ptr, col = _csr(rows)
        root = int(rng.integers(0, n))
        ins, remap, k = ref_np.parallel_bfs_subtree(ptr, col, root, n)
        p, c, _ = ref_np.extract_subtree_edges(ptr, col, None, ins, remap)
        assert len(c) == k - 1 and sorted(c.tolist()) == list(range(1, k))
        old = {int(remap[i]): i for i in range(n) if ins[i]}
        for pp, cc in zip(p, c):
            assert parent[old[int(cc)]] == old[int(pp)]
            assert pp < cc


# ---- batched_dirichlet_noise (host restatement with the C oracle's gammas) -------------------
def dirichlet_rows(num_sims, num_actions, alpha, seed, counter):
    """The rows omq_batched_dirichlet_noise computes: gamma variates of the stream keyed by
    (seed, counter, row, entry), their canonical float64 sum, quotients rounded to float32."""
    lib = load()
    out = np.zeros((num_sims, num_actions), F)
    for r in range(num_sims):
        g = np.array([lib.orc_gamma(alpha, seed, counter, r, i) for i in range(num_actions)])
        S = lib.orc_sum64d(g.ctypes.data_as(ctypes.c_void_p), num_actions)
        out[r] = (g / S).astype(F) if S > 0 else 0.0
    return out


def test_dirichlet_rows_moments():
    """Dirichlet(alpha, K): mean 1/K, variance (K - 1) / (K^2 (K alpha + 1)), rows summing to
    1 (to float32 rounding)."""
    K = 10
    for alpha in (0.3, 1.5):
        rows = dirichlet_rows(3000, K, alpha, 77, 3).astype(np.float64)
        assert np.all(rows >= 0) and np.allclose(rows.sum(1), 1.0, atol=5e-6)
        var = (K - 1) / (K * K * (K * alpha + 1))
        assert abs(rows.mean() - 1 / K) < 4 * math.sqrt(var / rows.size) + 1e-9
        assert abs(rows.var() / var - 1) < 0.08, (alpha, rows.var(), var)
    a = dirichlet_rows(4, K, 0.3, 77, 3)
    assert not np.array_equal(a, dirichlet_rows(4, K, 0.3, 77, 4))  # the counter changes them
