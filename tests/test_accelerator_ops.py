"""The numpy restatements of the reference accelerator's operators (oracle/ref_np.py:
find_expansion_nodes, batched_ucb_selection, fused_select_expand,
fused_select_expand_optimized, batched_add_children), pinned by known answers worked out by
hand, with the mistakes each answer is chosen to catch; the C-ABI argument checks; and the
accelerator class refusing a non-HIP device."""
import ctypes

import numpy as np
import pytest

from omoknuni_quantum_amd import _lib
from oracle import ref_np

F = np.float32


# ---- find_expansion_nodes ------------------------------------------------------------------
def test_find_expansion_known_answer():
    children = np.array([[1, 2, -1], [-1, -1, -1], [3, -1, -1], [-1, -1, -1], [-1, 2, -1]],
                        np.int32)
    visits = np.array([5, 0, 2, 0, 0], np.int32)
    cur = np.array([1, 3, 0, 4, 1, 7, -1, 3], np.int32)
    valid = np.array([1, 1, 1, 1, 1, 1, 1, 0], bool)
    # path 0: node 1 (no child, unvisited); 1: node 3; 2: node 0 has children; 3: node 4 has a
    # child after a negative entry (the whole row counts); 4: node 1 again (listed twice);
    # 5: node 7 is past the table; 6: -1; 7: not a valid path
    assert ref_np.find_expansion_nodes(cur, valid, 8, children, visits).tolist() == [1, 3, 1]
    assert ref_np.find_expansion_nodes(cur, valid, 2, children, visits).tolist() == [1, 3]
    visits[3] = 1  # a visited node without children is not listed
    assert ref_np.find_expansion_nodes(cur, valid, 8, children, visits).tolist() == [1, 1]


# ---- batched_ucb_selection -----------------------------------------------------------------
def _ucb_case():
    q = np.array([0.5, 0.9, 0.25, -2.0, 0.0, -0.5], F)
    visits = np.array([3, 0, 3, 1, 0, 0], np.int32)
    col = np.array([0, 1, 2, 3, -1, 5], np.int32)
    priors = np.array([0.25, 0.125, 0.5, 0.5, 0.5, 0.25], F)
    pv = np.array([15, 7, 0, 9, 3], np.int32)
    row_ptr = np.array([0, 3, 3, 5, 4, 6], np.int32)
    return q, visits, pv, priors, row_ptr, col


def test_batched_ucb_known_answer():
    q, visits, pv, priors, row_ptr, col = _ucb_case()
    sel, sc = ref_np.batched_ucb_selection(q, visits, pv, priors, row_ptr, col, 1.0)
    # row 0, sqrt(15 + 1) = 4: 0.5 + 0.25*4/4 = 0.75; 0 + 0.125*4/1 = 0.5 (unvisited: q not
    # used); 0.25 + 0.5*4/4 = 0.75 -> the first of the tie.  Row 1 is empty.  Row 2, sqrt(1):
    # -2 + 0.5/2 = -1.75, then an edge with child -1 is skipped.  Row 3 decreases (5 -> 4).
    # Row 4: the skipped edge keeps its position, child 5 (unvisited) 0.25*2/1 = 0.5 at 1.
    assert sel.tolist() == [0, -1, 0, 0, 1]
    assert sc.tolist() == [0.75, 0.0, -1.75, 0.0, 0.5]
    # c = 2: 1.0, 1.0, 1.25.  sqrt(N) in place of sqrt(N + 1) would give 1.218...
    sel, sc = ref_np.batched_ucb_selection(q, visits, pv, priors, row_ptr, col, 2.0)
    assert sel[0] == 2 and sc[0] == F(1.25)


def test_batched_ucb_nothing_above_threshold():
    q, visits, pv, priors, row_ptr, col = _ucb_case()
    q[3] = F(-1e11)
    sel, sc = ref_np.batched_ucb_selection(q, visits, pv, priors, row_ptr, col, 1.0)
    assert sel[2] == 0 and sc[2] == F(-1e10)
    row_ptr2 = row_ptr.copy()
    row_ptr2[0] = -1  # a negative start
    sel, sc = ref_np.batched_ucb_selection(q, visits, pv, priors, row_ptr2, col, 1.0)
    assert sel[0] == 0 and sc[0] == 0


def test_batched_ucb_agrees_with_fused_ucb():
    """With parent_visits = N - 1 both operators score sqrt(N) the same way; their selections
    agree wherever some score is above -1e10 (fused_ucb_selection is pinned on its own)."""
    rng = np.random.default_rng(3)
    rows = [list(range(40 + 9 * i, 40 + 9 * i + int(rng.integers(1, 9)))) for i in range(40)]
    starts = np.array([r[0] - 40 for r in rows], np.int32)
    nn = 40 + 9 * 40
    # per-node arrays for the fused operator; per-child arrays for the batched one
    visits = rng.integers(0, 5, nn).astype(np.int32)
    visits[:40] = rng.integers(1, 50, 40)
    q = np.round(rng.random(nn) * 8 - 4).astype(F) / 8
    flat = [c for r in rows for c in r]
    edge_of = {c: i for i, c in enumerate(flat)}
    pri_node = np.round(rng.random(nn) * 8).astype(F) / 8
    row_ptr = np.zeros(41, np.int32)
    for i, r in enumerate(rows):
        row_ptr[i + 1] = row_ptr[i] + len(r)
    col = np.arange(len(flat), dtype=np.int32)  # child ids of the batched form = edge ids
    qc = q[flat]
    vc = visits[flat]
    pc = pri_node[flat]
    sel, _ = ref_np.batched_ucb_selection(qc, vc, visits[:40] - 1, pc, row_ptr, col, 1.3)
    children = np.array(flat, np.int32)
    st = np.array([edge_of[r[0]] for r in rows], np.int32)
    en = np.array([edge_of[r[-1]] + 1 for r in rows], np.int32)
    want = ref_np.fused_ucb_selection(np.arange(40), st, en, children, q, visits, pc, 1.3)
    assert np.array_equal(sel, want)
    assert len(set(starts.tolist())) == 40


# ---- fused_select_expand -------------------------------------------------------------------
def _descent_tree():
    children = np.array([[1, 2, 3], [4, -1, 5], [-1, -1, -1], [-1, -1, -1], [-1, -1, -1],
                         [-1, -1, -1]], np.int32)
    visits = np.array([10, 4, 0, 3, 0, 9], np.int32)
    prior = np.array([0, 0.5, 0.25, 0.25, 0.5, 0.5], F)
    expanded = np.array([1, 1, 0, 0, 0, 1], bool)
    return children, visits, prior, expanded


def test_fused_select_expand_known_answers():
    children, visits, prior, expanded = _descent_tree()
    q = np.array([0, 0.5, 0.0, 0.25, 0.0, 100.0], F)
    roots = np.array([0], np.int32)
    # child 2 is unvisited: +inf, first such child
    p, L, e, need = ref_np.fused_select_expand(roots, children, visits, q, prior, expanded, 8,
                                               1.0)
    assert p[0].tolist() == [0, 2, -1, -1, -1, -1, -1, -1] and (L[0], e[0], need[0]) == (
        2, 2, True)
    # all visited, sqrt(10) = 3.162: 0.5 + 0.5*3.162/5 = 0.816; 0 + 0.25*3.162/2 = 0.395;
    # 0.25 + 0.25*3.162/4 = 0.448 -> child 1.  Node 1's row ends at -1: child 4 (0 +
    # 0.5*2/2 = 0.5) and not child 5 (q = 100) behind the -1.  Node 4 is not expanded.
    visits[2] = visits[4] = 1
    p, L, e, need = ref_np.fused_select_expand(roots, children, visits, q, prior, expanded, 8,
                                               1.0)
    assert p[0, :4].tolist() == [0, 1, 4, -1] and (L[0], e[0], need[0]) == (3, 4, True)
    # the depth limit: max_depth 2 stops at depth 1 with no expansion reported
    p, L, e, need = ref_np.fused_select_expand(roots, children, visits, q, prior, expanded, 2,
                                               1.0)
    assert p[0].tolist() == [0, 1] and (L[0], e[0], need[0]) == (0, 0, False)
    # a root that is not expanded
    expanded[0] = False
    p, L, e, need = ref_np.fused_select_expand(roots, children, visits, q, prior, expanded, 4,
                                               1.0)
    assert p[0].tolist() == [0, -1, -1, -1] and (L[0], e[0], need[0]) == (1, 0, True)


def test_fused_select_expand_no_child_above_minus_inf():
    children, visits, prior, expanded = _descent_tree()
    visits[:] = 1
    q = np.array([0, -np.inf, np.nan, -np.inf, 0, 0], F)
    p, L, e, need = ref_np.fused_select_expand(np.array([0], np.int32), children, visits, q,
                                               prior, expanded, 4, 1.0)
    assert (L[0], e[0], need[0]) == (1, 0, True)


# ---- fused_select_expand_optimized ---------------------------------------------------------
def test_fused_select_expand_optimized_known_answers():
    children, visits, prior, _ = _descent_tree()
    visits = np.array([10, 4, 1, 3, 0, 9], np.int32)
    W = np.array([0, 2.0, 0.0, 0.75, 0, 900], F)
    p, L, u = ref_np.fused_select_expand_optimized(np.array([0, 4], np.int32), children, visits,
                                                   W, prior, 8, 1.0)
    # root: sqrt(11) = 3.3166: 2/4 + 0.5*3.3166/5 = 0.8317; 0 + 0.25*3.3166/2 = 0.4146;
    # 0.75/3 + 0.25*3.3166/4 = 0.4573 -> child 1; node 1 (4 visits): child 4 only (0 +
    # 0.5*sqrt(5)/1); node 4 has no visits: the path ends there.  Root 4 has no visits.
    assert p[0, :4].tolist() == [0, 1, 4, -1] and L.tolist() == [3, 1]
    s11 = np.sqrt(11.0)
    want = [0.5 + 0.5 * s11 / 5, 0.25 * s11 / 2, 0.25 + 0.25 * s11 / 4]
    assert np.allclose(u[0], want, rtol=0, atol=1e-6)
    assert u[1].tolist() == [0, 0, 0] and p[1].tolist() == [4] + [-1] * 7


def test_fused_select_expand_optimized_depth_cap():
    """A chain of visited nodes: the descent stops at depth 32 (path of 33 nodes) however deep
    max_depth allows, and at max_depth - 1 below that."""
    n = 40
    children = np.full((n, 2), -1, np.int32)
    children[:-1, 0] = np.arange(1, n)
    visits = np.full(n, 3, np.int32)
    W = np.zeros(n, F)
    pri = np.full(n, 0.5, F)
    p, L, _ = ref_np.fused_select_expand_optimized(np.array([0], np.int32), children, visits, W,
                                                   pri, 50, 1.0)
    assert L[0] == 33 and p[0, :33].tolist() == list(range(33)) and p[0, 33] == -1
    p, L, _ = ref_np.fused_select_expand_optimized(np.array([0], np.int32), children, visits, W,
                                                   pri, 10, 1.0)
    assert L[0] == 10 and p[0].tolist() == list(range(10))


def test_rsqrt_of_rcp_is_sqrt_to_rounding():
    for pv in [1, 2, 3, 10, 99, 1000, 12345, 2**20]:
        got = float(ref_np._rsqrt_of_rcp(pv))
        assert abs(got - np.sqrt(pv + 1.0)) <= 2 * np.spacing(F(got)), pv


# ---- batched_add_children ------------------------------------------------------------------
def _empty_tree(max_nodes, max_children, max_edges, nc=0, ec=0):
    return dict(node_counter=np.array([nc], np.int32), edge_counter=np.array([ec], np.int32),
                children=np.full(max_nodes * max_children, -1, np.int32),
                parent_indices_out=np.full(max_nodes, -7, np.int32),
                parent_actions_out=np.full(max_nodes, -7, np.int32),
                node_priors_out=np.full(max_nodes, -7, F),
                visit_counts_out=np.full(max_nodes, 9, np.int32),
                value_sums_out=np.full(max_nodes, 9, F),
                col_indices=np.full(max_edges, -7, np.int32),
                edge_actions=np.full(max_edges, -7, np.int32),
                edge_priors=np.full(max_edges, -7, F))


def test_batched_add_children_known_answer():
    tr = _empty_tree(10, 3, 10, nc=2, ec=4)
    parents = np.array([0, 11, 1, 5, 2, 3], np.int32)
    nchild = np.array([2, 3, 0, 3, 2, 5], np.int32)
    acts = np.arange(18, dtype=np.int32) + 100
    pri = (np.arange(18) / 32).astype(F)
    out = ref_np.batched_add_children(parents, acts, pri, nchild, tr, 10, 3, 10)
    # item 0: nodes 2,3, edges 4,5; item 1: parent 11 >= max_nodes; item 2: no children;
    # item 3: nodes 4..6, edges 6..8; item 4: nodes 7,8 fit but edges 9,10 do not (counters
    # still advance); item 5: 5 children from node 9 do not fit.
    assert out.reshape(6, 3).tolist() == [[2, 3, -1], [-1] * 3, [-1] * 3, [4, 5, 6], [-1] * 3,
                                          [-1] * 3]
    assert (tr["node_counter"][0], tr["edge_counter"][0]) == (2 + 2 + 3 + 2 + 5, 4 + 12)
    assert tr["children"][:3].tolist() == [2, 3, -1] and tr["children"][15:18].tolist() == [
        4, 5, 6]
    assert tr["children"][6:9].tolist() == [-1] * 3  # item 4 wrote nothing
    assert tr["parent_indices_out"].tolist() == [-7, -7, 0, 0, 5, 5, 5, -7, -7, -7]
    assert tr["parent_actions_out"][2:7].tolist() == [100, 101, 109, 110, 111]
    assert tr["node_priors_out"][2:7].tolist() == [0, 1 / 32, 9 / 32, 10 / 32, 11 / 32]
    assert tr["visit_counts_out"].tolist() == [9, 9, 0, 0, 0, 0, 0, 9, 9, 9]
    assert tr["value_sums_out"].tolist() == [9, 9, 0, 0, 0, 0, 0, 9, 9, 9]
    assert tr["col_indices"].tolist() == [-7] * 4 + [2, 3, 4, 5, 6, -7]
    assert tr["edge_actions"][4:9].tolist() == [100, 101, 109, 110, 111]
    assert tr["edge_priors"][4:9].tolist() == [0, 1 / 32, 9 / 32, 10 / 32, 11 / 32]


def test_batched_add_children_more_than_max_children():
    tr = _empty_tree(20, 3, 20)
    out = ref_np.batched_add_children(np.array([1], np.int32), np.arange(3, dtype=np.int32),
                                      np.zeros(3, F), np.array([5], np.int32), tr, 20, 3, 20)
    # 5 nodes and 5 edges taken, 3 written
    assert out.tolist() == [0, 1, 2] and tr["node_counter"][0] == 5
    assert tr["edge_counter"][0] == 5 and tr["parent_indices_out"][3] == -7


# ---- C ABI ---------------------------------------------------------------------------------
def test_abi_argument_checks():
    lib = _lib.load()
    E = _lib.OMQ_E_ARG
    assert lib.omq_find_expansion_nodes(None, None, -1, None, 3, None, 4, None, 8, None) == E
    assert lib.omq_find_expansion_nodes(None, None, 4, None, 3, None, 4, None, None, None) == E
    assert lib.omq_find_expansion_nodes(8, 8, 4, None, 3, 8, 4, 8, 8, None) == E
    assert "null" in lib.omq_last_error().decode()
    assert lib.omq_batched_ucb_selection(None, None, 0, None, None, None, None, 0, 1.0, None,
                                         None, None) == 0
    assert lib.omq_batched_ucb_selection(8, 8, 4, 8, 8, 8, None, 2, 1.0, 8, None, None) == E
    assert lib.omq_fused_select_expand(8, 1, 8, 4, 3, 8, 8, 8, 8, 0, 1.0, 8, 8, 8, 8,
                                       None) == E
    assert "max_depth" in lib.omq_last_error().decode()
    assert lib.omq_fused_select_expand(None, 0, None, 0, 0, None, None, None, None, 1, 1.0,
                                       None, None, None, None, None) == 0
    assert lib.omq_fused_select_expand_optimized(8, 1, 8, 4, 3, 8, 8, 8, 4, 1.0, None, 8, 8,
                                                 None) == E
    args = [8, 2, 8, 8, 8, 8, 8, 8, 8, 8, 8, 8, 8, 8, 8, 8, 10, 0, 10, 8, None]
    assert lib.omq_batched_add_children(*args) == E  # max_children 0
    args[17] = 3
    args[13] = None  # col_indices
    assert lib.omq_batched_add_children(*args) == E
    assert "null" in lib.omq_last_error().decode()


def test_accelerator_refuses_cpu():
    from omoknuni_quantum_amd.mcts_gpu_accelerator import MCTSGPUAccelerator

    with pytest.raises(RuntimeError, match="not a HIP device"):
        MCTSGPUAccelerator("cpu")


def test_accelerator_symbols_exported():
    lib = ctypes.CDLL(_lib.load()._name)
    for name in ("omq_find_expansion_nodes", "omq_batched_ucb_selection",
                 "omq_fused_select_expand", "omq_fused_select_expand_optimized",
                 "omq_batched_add_children"):
        assert hasattr(lib, name), name
