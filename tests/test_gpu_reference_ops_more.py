"""The reference module's selection, noise, backup and subtree operators on the GPU (through
torch_ops, the accelerator class and the C ABI) against the numpy restatements and the C
oracle, bit for bit: random dense tables with negative and out-of-range entries, coarse values
(exact ties), per-simulation priors and legal masks; Dirichlet rows against the oracle's gamma
stream; random trees and graphs with repeated children and cycles, with levels beyond one
1024-thread chunk."""
import numpy as np
import pytest
import torch

from omoknuni_quantum_amd import torch_ops
from omoknuni_quantum_amd.mcts_gpu_accelerator import get_mcts_gpu_accelerator
from oracle import ref_np

from test_reference_ops_more import (EDGE_EXPECT, PSVL_EXPECT, UCBD_EXPECT, _csr, _edge_case,
                                     _psvl_case, _ucbd_case, dirichlet_rows)

pytestmark = pytest.mark.gpu
F = np.float32


def _t(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def _np(x):
    torch.cuda.synchronize()
    return x.cpu().numpy()


# ---- parallel_select_with_virtual_loss -------------------------------------------------------
def test_psvl_known_answer_on_gpu(device):
    parents, children, N, VL, W, P, acts, masks = _psvl_case()
    vl = _t(VL, device)
    sel = torch_ops.parallel_select_with_virtual_loss(
        _t(parents, device), _t(children, device), _t(N, device), vl, _t(W, device),
        _t(P, device), None, _t(masks, device), _t(acts, device), 1.0, -1.0, 0.0, True)
    assert _np(sel).tolist() == PSVL_EXPECT
    _, vl_want = ref_np.parallel_select_with_virtual_loss(parents, children, N, VL, W, P, acts,
                                                          1.0, -1.0, masks)
    assert _np(vl).tolist() == vl_want.tolist()


@pytest.mark.parametrize("seed,mc,per_sim,masked", [(0, 8, False, False), (1, 64, False, True),
                                                    (2, 65, True, False), (3, 300, True, True),
                                                    (4, 1000, True, True)])
def test_psvl_random(device, seed, mc, per_sim, masked):
    rng = np.random.default_rng(40 + seed)
    nn, S, A = 1500, 2100, 50
    ch = rng.integers(-2, nn + 3, (nn, mc)).astype(np.int32)  # negatives and ids past the nodes
    N = rng.integers(0, 6, nn).astype(np.int32)
    VL = rng.integers(0, 3, nn).astype(np.int32)
    W = (np.round(rng.random(nn) * 16 - 8) / 8).astype(F)
    acts = rng.integers(-1, A + 2, nn).astype(np.int32)
    parents = rng.integers(-2, nn + 2, S).astype(np.int32)
    parents[:50] = 0  # the root, which ignores the masks
    if per_sim:
        P = (np.round(rng.random((S, nn - 7)) * 8) / 8).astype(F)  # children past it skipped
    else:
        P = (np.round(rng.random(nn) * 8) / 8).astype(F)
    masks = rng.random((S, A)) < 0.7 if masked else None
    exp, vl_exp = ref_np.parallel_select_with_virtual_loss(parents, ch, N, VL, W, P, acts, 1.4,
                                                           1.0, masks)
    vl = _t(VL, device)
    got = torch_ops.parallel_select_with_virtual_loss(
        _t(parents, device), _t(ch, device), _t(N, device), vl, _t(W, device), _t(P, device),
        None, _t(masks, device) if masked else None, _t(acts, device), 1.4, 1.0, 0.0, masked)
    assert np.array_equal(_np(got), exp)
    assert np.array_equal(_np(vl), vl_exp)


def test_psvl_accelerator_method(device):
    """MCTSGPUAccelerator.parallel_select_with_virtual_loss (mcts_gpu_accelerator.py:289-297):
    nine arguments, no masks."""
    parents, children, N, VL, W, P, acts, masks = _psvl_case()
    acc = get_mcts_gpu_accelerator(device)
    got = acc.parallel_select_with_virtual_loss(
        _t(parents, device), _t(children, device), _t(N, device), _t(VL, device),
        _t(W, device), _t(P, device), _t(acts, device), 1.0, -1.0)
    exp, _ = ref_np.parallel_select_with_virtual_loss(parents, children, N, VL, W, P, acts, 1.0,
                                                      -1.0, None)
    assert np.array_equal(_np(got), exp)


# ---- fused_ucb_with_noise ----------------------------------------------------------------------
@pytest.mark.parametrize("C", [1, 64, 65, 362, 4672])
def test_fused_ucb_with_noise_random(device, C):
    rng = np.random.default_rng(C)
    S = 700
    q = (np.round(rng.random(C) * 8 - 4) / 8).astype(F)
    n = rng.integers(0, 5, C).astype(np.int32)
    p = (np.round(rng.random(C) * 8) / 8).astype(F)
    noise = (np.round(rng.random((S, C)) * 4) / 4).astype(F)
    noise[:3] = 0.0  # identical rows: exact ties settle on the lowest position
    exp = ref_np.fused_ucb_with_noise(q, n, p, noise, 3.0, 1.4, 0.25)
    got = torch_ops.fused_ucb_with_noise(_t(q, device), _t(n, device), _t(p, device),
                                         _t(noise, device), 3.0, 1.4, 0.25)
    assert np.array_equal(_np(got), exp)
    acc = get_mcts_gpu_accelerator(device)
    got2 = acc.fused_ucb_with_noise(_t(q, device), _t(n, device), _t(p, device),
                                    _t(noise, device), 3.0, 1.4, 0.25)
    assert np.array_equal(_np(got2), exp)
    low = np.full(C, -1e11, F)  # nothing above -1e10: position 0
    got3 = torch_ops.fused_ucb_with_noise(_t(low, device), _t(n, device), _t(p, device),
                                          _t(noise, device), 3.0, 1.4, 0.25)
    assert not _np(got3).any()


# ---- batched_ucb_selection_dense -------------------------------------------------------------
def test_ucb_dense_known_answer_on_gpu(device):
    args = [_t(a, device) for a in _ucbd_case()]
    assert _np(torch_ops.batched_ucb_selection_dense(*args, 1.0)).tolist() == UCBD_EXPECT


@pytest.mark.parametrize("M", [3, 64, 65, 200, 1000])
def test_ucb_dense_random(device, M):
    rng = np.random.default_rng(100 + M)
    B, NV = 1300, 400
    bc = rng.integers(-2, NV + 3, (B, M)).astype(np.int32)
    bp = (np.round(rng.random((B, M)) * 8) / 8).astype(F)
    valid = rng.random((B, M)) < 0.8
    pv = rng.integers(0, 30, B).astype(np.int32)
    cn = rng.integers(0, 4, NV).astype(np.int32)
    cv = (np.round(rng.random(NV) * 8 - 4) / 8).astype(F)
    exp = ref_np.batched_ucb_selection_dense(bc, bp, pv, cn, cv, valid, 1.4)
    got = torch_ops.batched_ucb_selection_dense(_t(bc, device), _t(bp, device), _t(pv, device),
                                                _t(cn, device), _t(cv, device),
                                                _t(valid, device), 1.4)
    assert np.array_equal(_np(got), exp)


# ---- batched_dirichlet_noise -------------------------------------------------------------------
@pytest.mark.parametrize("S,A,alpha", [(5, 362, 0.03), (40, 225, 0.3), (3, 1, 1.5),
                                       (7, 70, 2.5), (2, 4672, 0.3)])
def test_dirichlet_rows_match_oracle(device, S, A, alpha):
    torch_ops.set_noise_seed(1234)
    got = torch_ops.batched_dirichlet_noise(S, A, alpha, 0.25, device)
    got2 = torch_ops.batched_dirichlet_noise(S, A, alpha, 0.25, device)  # counter 1
    assert np.array_equal(_np(got), dirichlet_rows(S, A, alpha, 1234, 0))
    assert np.array_equal(_np(got2), dirichlet_rows(S, A, alpha, 1234, 1))
    acc = get_mcts_gpu_accelerator(device)
    got3 = acc.batched_dirichlet_noise(S, A, alpha, 0.25, device)  # counter 2
    assert np.array_equal(_np(got3), dirichlet_rows(S, A, alpha, 1234, 2))


# ---- optimized_backup_scatter -------------------------------------------------------------------
def test_optimized_backup_scatter_equals_vectorized_backup(device):
    rng = np.random.default_rng(9)
    B, D, nn = 300, 7, 80
    paths = rng.integers(-1, nn + 2, (B, D)).astype(np.int32)
    plen = rng.integers(0, D + 2, B).astype(np.int32)
    vals = (rng.integers(-4, 5, B) / 4).astype(F)  # exact sums in any order
    # expected: per path, d < min(len, D), node in range: N += 1, W += v (-1)^(len-1-d)
    n_exp = np.zeros(nn, np.int32)
    w_exp = np.zeros(nn, np.float64)
    for b in range(B):
        L = int(plen[b])
        for d in range(min(L, D)):
            x = int(paths[b, d])
            if 0 <= x < nn:
                n_exp[x] += 1
                w_exp[x] += vals[b] * (-1) ** (L - 1 - d)
    n1, w1 = torch.zeros(nn, dtype=torch.int32, device=device), torch.zeros(nn, device=device)
    torch_ops.optimized_backup_scatter(_t(paths, device), _t(plen, device), _t(vals, device),
                                       n1, w1)
    acc = get_mcts_gpu_accelerator(device)
    n2, w2 = torch.zeros_like(n1), torch.zeros_like(w1)
    acc.optimized_backup_scatter(_t(paths, device), _t(plen, device), _t(vals, device), n2, w2)
    n3, w3 = torch.zeros_like(n1), torch.zeros_like(w1)
    torch_ops.vectorized_backup(_t(paths, device), _t(plen, device), _t(vals, device), n3, w3)
    assert np.array_equal(_np(n1), n_exp) and np.array_equal(_np(w1), w_exp.astype(F))
    assert torch.equal(n1, n2) and torch.equal(w1, w2)
    assert torch.equal(n1, n3) and torch.equal(w1, w3)


# ---- parallel_bfs_subtree / extract_subtree_edges --------------------------------------------
def _check_subtree(device, rows, root, n, actions=True):
    ptr, col = _csr(rows)
    ins_e, remap_e, k_e = ref_np.parallel_bfs_subtree(ptr, col, root, n)
    ins, remap, cnt = torch_ops.parallel_bfs_subtree(_t(ptr, device), _t(col, device), root, n)
    assert int(_np(cnt)[0]) == k_e
    assert np.array_equal(_np(ins), ins_e) and np.array_equal(_np(remap), remap_e)
    act = np.arange(len(col)).astype(np.int16) if actions else None
    pe, ce, ae = ref_np.extract_subtree_edges(ptr, col, act, ins_e, remap_e)
    p, c, a = torch_ops.extract_subtree_edges(_t(ptr, device), _t(col, device),
                                              _t(act, device) if actions else None, ins, remap,
                                              max(len(col), 1))
    assert np.array_equal(_np(p), pe) and np.array_equal(_np(c), ce)
    assert np.array_equal(_np(a), ae)


def test_subtree_known_answers_on_gpu(device):
    from test_reference_ops_more import G_DAG, G_TREE
    _check_subtree(device, G_TREE, 0, 8)
    _check_subtree(device, G_TREE, 1, 8, actions=False)
    _check_subtree(device, G_DAG, 0, 5)
    _check_subtree(device, G_DAG, 1, 5)
    ptr, col, act, ins, remap = _edge_case()
    p, c, a = torch_ops.extract_subtree_edges(_t(ptr, device), _t(col, device), _t(act, device),
                                              _t(ins, device), _t(remap, device), 20)
    assert (_np(p).tolist(), _np(c).tolist(), _np(a).tolist()) == EDGE_EXPECT
    with pytest.raises(RuntimeError, match="max_edges"):
        torch_ops.extract_subtree_edges(_t(ptr, device), _t(col, device), _t(act, device),
                                        _t(ins, device), _t(remap, device), 6)


@pytest.mark.parametrize("seed", range(4))
def test_subtree_random_trees(device, seed):
    """Random trees (levels beyond one 1024-thread chunk in the wide ones) and the subtree of
    a random node."""
    rng = np.random.default_rng(60 + seed)
    n = [3000, 20000, 60000, 5][seed]
    fan = [2, 40, 300, 3][seed]
    parent = [-1] + [max(0, i - 1 - int(rng.integers(0, fan))) for i in range(1, n)]
    rows = [[] for _ in range(n)]
    for i in range(1, n):
        rows[parent[i]].append(i)
    for r in rows:
        rng.shuffle(r)
    for root in (0, int(rng.integers(0, n))):
        _check_subtree(device, rows, root, n)


@pytest.mark.parametrize("seed", range(3))
def test_subtree_random_graphs(device, seed):
    """Graphs with repeated children, cycles and ids past max_nodes: the first occurrence in
    breadth-first order numbers a node."""
    rng = np.random.default_rng(80 + seed)
    n = [50, 3000, 20000][seed]
    rows = [list(rng.integers(0, n + 3, int(rng.integers(0, 6)))) for _ in range(n)]
    rows = [[int(c) for c in r] for r in rows]
    _check_subtree(device, rows, int(rng.integers(0, n)), n)
