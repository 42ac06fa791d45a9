"""A whole search recorded as a HIP graph: every replay builds the same trees as the eager
search, with eager work and synchronisation between the replays."""
import numpy as np
import pytest
import torch

from oracle.parity import make_pair
from omoknuni_quantum_amd.synthetic.workloads import get

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["C1", "C4"])
def test_graph_replays_match_eager_search(device, name):
    wl = get(name).scaled(num_trees=min(get(name).num_trees, 4), num_simulations=512,
                          capacity=150_000)
    eng, orc, ev = make_pair(wl, device=device)
    eng.search(wl.num_simulations, wl.wave_size, ev)
    torch.cuda.synchronize()
    want = [eng.host_tree(t) for t in range(eng.T)]
    g = eng.capture_search(wl.num_simulations, wl.wave_size, ev)
    for rep in range(3):
        eng.N.fill_(7)      # eager work between replays: scribble over the trees
        eng.W.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for t in range(eng.T):
            got = eng.host_tree(t)
            assert got["num_nodes"] == want[t]["num_nodes"], (rep, t)
            for k in ("N", "parent", "first", "nchild", "action"):
                assert np.array_equal(got[k], want[t][k]), (rep, t, k)
            for k in ("W", "P"):
                assert np.array_equal(got[k].view(np.int32), want[t][k].view(np.int32)), (rep, t, k)
    # and the eager search still equals the oracle's
    orc.search(wl.num_simulations, wl.wave_size)
    for t in range(eng.T):
        o = orc.tree(t)
        assert np.array_equal(want[t]["N"], o["N"]) and want[t]["num_nodes"] == o["num_nodes"]
