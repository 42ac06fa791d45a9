"""omq_shift_root_noalloc (the library's own workspace, no allocation) against omq_shift_root
(a caller workspace), through the C ABI: two calls in a row on one GPU, the second on a
smaller forest, each bit-equal to the entry point with a workspace on an identical forest."""
import ctypes

import numpy as np
import pytest
import torch

from omoknuni_quantum_amd import _lib
from omoknuni_quantum_amd.core.engine import SearchParams, WaveEngine
from omoknuni_quantum_amd.synthetic.evaluator import SyntheticEvaluator
from omoknuni_quantum_amd.synthetic.workloads import get

pytestmark = pytest.mark.gpu

FIELDS = ("N", "W", "P", "parent", "first", "nchild", "action")


def _searched_pair(wl, device):
    """Two engines holding the same searched forest (the search is deterministic)."""
    out = []
    for _ in range(2):
        p = SearchParams(c_puct=wl.c_puct, virtual_loss=wl.virtual_loss, max_depth=wl.max_depth,
                         dirichlet_epsilon=wl.dirichlet_epsilon)
        eng = WaveEngine(wl.model, wl.num_trees, wl.capacity, wl.wave_size, wl.max_depth,
                         device, p)
        eng.set_roots(*wl.root_inputs())
        eng.search(wl.num_simulations, wl.wave_size, SyntheticEvaluator(wl.logit_scale))
        out.append(eng)
    torch.cuda.synchronize()
    return out


def _most_visited_children(eng):
    roots = []
    for t in range(eng.T):
        tr = eng.host_tree(t)
        f, k = int(tr["first"][0]), int(tr["nchild"][0])
        kids = np.arange(f + 1, f + 1 + k)
        roots.append(int(kids[np.argmax(tr["N"][kids])]) if k > 0 else -1)
    return np.array(roots, np.int32)


def _compare(a, b, ctx):
    for t in range(a.T):
        ta, tb = a.host_tree(t), b.host_tree(t)
        assert ta["num_nodes"] == tb["num_nodes"], ctx
        for k in FIELDS:
            x, y = ta[k], tb[k]
            if x.dtype == np.float32:
                x, y = x.view(np.int32), y.view(np.int32)
            assert np.array_equal(x, y), (ctx, t, k)


def _noalloc(eng, roots):
    d = torch.from_numpy(roots).to(eng.device)
    lib = _lib.load()
    _lib.check(lib.omq_shift_root_noalloc(eng.forest_ref, d.data_ptr(), eng.stream_handle()),
               "omq_shift_root_noalloc")
    torch.cuda.synchronize()


@pytest.mark.parametrize("order", ["large_then_small"])
def test_noalloc_shift_matches_workspace_entry(device, order):
    big = get("C2").scaled(num_trees=3, num_simulations=1024, capacity=200_000, name="big")
    small = get("C4").scaled(num_trees=2, num_simulations=2048, wave_size=512,
                             capacity=60_000, name="small")
    assert big.num_trees * big.capacity > small.num_trees * small.capacity
    for wl in (big, small):
        print(f"[no-alloc] {wl.name}: T={wl.num_trees} capacity={wl.capacity}", flush=True)
        a, b = _searched_pair(wl, device)
        _compare(a, b, f"{wl.name} before")
        roots = _most_visited_children(a)
        a.shift_roots(roots)           # omq_shift_root, caller workspace
        _noalloc(b, roots)             # omq_shift_root_noalloc, the library's workspace
        _compare(a, b, f"{wl.name} after")
        assert int(b.num_nodes.sum().item()) < wl.num_trees * wl.capacity
        # the reused trees search on identically
        ev = SyntheticEvaluator(wl.logit_scale)
        a.run_wave(wl.wave_size, ev)
        b.run_wave(wl.wave_size, ev)
        torch.cuda.synchronize()
        _compare(a, b, f"{wl.name} continued")


def test_noalloc_shift_over_limit_leaves_forest_unchanged(device):
    """A searched forest beyond the library's workspace (2 trees x 600k nodes > 1,048,576):
    OMQ_E_LIMIT, and nothing is launched, so every tree stays as it was."""
    wl = get("C4").scaled(num_trees=2, num_simulations=512, wave_size=256, capacity=600_000,
                          name="over-limit")
    assert wl.num_trees * wl.capacity * _lib.OMQ_SHIFT_WORKSPACE_PER_NODE > \
        _lib.OMQ_NOALLOC_SHIFT_INTS
    print(f"[no-alloc] {wl.name}: T={wl.num_trees} capacity={wl.capacity}", flush=True)
    a, b = _searched_pair(wl, device)
    roots = torch.from_numpy(_most_visited_children(b)).to(b.device)
    lib = _lib.load()
    rc = lib.omq_shift_root_noalloc(b.forest_ref, roots.data_ptr(), b.stream_handle())
    assert rc == _lib.OMQ_E_LIMIT
    assert "omq_shift_root_noalloc" in lib.omq_last_error().decode()
    torch.cuda.synchronize()
    _compare(a, b, "over-limit, refused")
