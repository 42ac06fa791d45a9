"""The reference's fused UCB selection operator on the GPU (omq_fused_ucb_selection through
torch.ops.omq) against the numpy restatement, position for position."""
import numpy as np
import pytest
import torch

from omoknuni_quantum_amd import torch_ops  # noqa: F401  (registers torch.ops.omq)
from oracle.ref_np import fused_ucb_selection

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", range(3))
def test_fused_ucb_matches_restatement(device, seed):
    rng = np.random.default_rng(10 + seed)
    n_par = 300
    sizes = rng.integers(0, 400, n_par)          # rows of 0 to 399 children (some empty)
    sizes[:5] = [0, 1, 64, 65, 300]
    starts = np.zeros(n_par, np.int32)
    ends = np.zeros(n_par, np.int32)
    children = []
    nxt = n_par
    for p, k in enumerate(sizes):
        starts[p] = len(children)
        children.extend(range(nxt, nxt + k))
        nxt += k
        ends[p] = len(children)
    children = np.array(children, np.int32)
    nn = nxt
    visits = rng.integers(0, 6, nn).astype(np.int32)   # many unvisited children
    visits[:20] = 0                                    # parents without visits
    q = np.round(rng.random(nn) * 8 - 4).astype(np.float32) / 8   # coarse values: exact ties
    priors = np.round(rng.random(len(children)) * 8).astype(np.float32) / 8
    nodes = rng.permutation(n_par).astype(np.int32)
    exp = fused_ucb_selection(nodes, starts, ends, children, q, visits, priors, 1.4)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    got = torch.ops.omq.fused_ucb_selection(t(nodes), t(starts), t(ends), t(children), t(q),
                                            t(visits), t(priors), 1.4)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), exp)
    # the reference's own operator name (torch_custom_ops.py:108), where AsyncWaveSearch looks
    got2 = torch.ops.mcts.fused_ucb_selection(t(nodes), t(starts), t(ends), t(children), t(q),
                                              t(visits), t(priors), 1.4)
    torch.cuda.synchronize()
    assert np.array_equal(got2.cpu().numpy(), exp)


def test_warp_vectorized_backup_equals_vectorized_backup(device):
    rng = np.random.default_rng(5)
    B, D, nn = 64, 6, 50
    paths = rng.integers(-1, nn, (B, D)).astype(np.int32)
    plen = rng.integers(0, D + 1, B).astype(np.int32)
    vals = (rng.integers(-4, 5, B) / 4).astype(np.float32)  # exact sums in any order
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    n1, w1 = torch.zeros(nn, dtype=torch.int32, device=device), torch.zeros(nn, device=device)
    n2, w2 = n1.clone(), w1.clone()
    torch.ops.omq.vectorized_backup(t(paths), t(plen), t(vals), n1, w1)
    torch.ops.omq.warp_vectorized_backup(t(paths), t(plen), t(vals), n2, w2)
    n3, w3 = torch.zeros_like(n1), torch.zeros_like(w1)
    n4, w4 = torch.zeros_like(n1), torch.zeros_like(w1)
    torch.ops.mcts.vectorized_backup(t(paths), t(plen), t(vals), n3, w3)
    torch.ops.mcts.warp_vectorized_backup(t(paths), t(plen), t(vals), n4, w4)
    torch.cuda.synchronize()
    assert torch.equal(n1, n2) and torch.equal(w1, w2)
    assert torch.equal(n1, n3) and torch.equal(w1, w3)
    assert torch.equal(n1, n4) and torch.equal(w1, w4)
