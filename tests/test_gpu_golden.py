"""The HIP path against the committed golden fixtures (tests/golden/), through the C ABI:
crafted selection rows and small whole searches with replayed evaluator rows."""
import os

import numpy as np
import pytest
import torch

from omoknuni_quantum_amd import _lib
from omoknuni_quantum_amd.core.engine import SearchParams, WaveEngine
from omoknuni_quantum_amd.synthetic import games
from oracle import golden

pytestmark = pytest.mark.gpu

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _rows():
    with np.load(os.path.join(HERE, "select_rows.npz")) as z:
        return golden.unpack_crafted(z)


def _put(t: torch.Tensor, values, dtype) -> None:
    v = torch.from_numpy(np.ascontiguousarray(values, dtype=dtype))
    t[:v.numel()].copy_(v)


def test_select_rows(device):
    """Every simulation's pick and the visit counts after one wave at a crafted root equal the
    fixture: ties, one-ulp differences, late unvisited children, exact-only rows, NaN values,
    VL 0/1/2.5, and every chain width (1..8 slots per lane) under the kernel of its game model."""
    fails = []
    for i, c in enumerate(_rows()):
        k, m = c["k"], c["m"]
        print(f"case {i}: {c['kind']} model {c['model']} k={k} m={m}", flush=True)
        model = golden.model_from_name(c["model"])
        eng = WaveEngine(model, 1, k + 1, m, 100, device,
                         SearchParams(c_puct=c["c"], virtual_loss=c["vl"]))
        eng.reset()
        _put(eng.N, np.concatenate([[c["N0"]], c["N"]]), np.int32)
        _put(eng.W, np.concatenate([[0.0], c["W"]]), np.float32)
        _put(eng.P, np.concatenate([[1.0], c["P"]]), np.float32)
        _put(eng.parent, [-1] + [0] * k, np.int32)
        _put(eng.first, [0] + [-1] * k, np.int32)
        _put(eng.nchild, [k] + [0] * k, np.int32)
        _put(eng.action, [-1] + list(range(k)), np.int32)
        _put(eng.num_nodes, [k + 1], np.int32)
        eng.select(m)
        torch.cuda.synchronize()
        plen = eng.path_len[:m].cpu().numpy()
        paths = eng.paths.view(m, eng.MD)[:, :2].cpu().numpy()
        picks = np.where(plen > 1, paths[:, 1] - 1, -1)
        n_after = eng.N[:k + 1].cpu().numpy()
        if not np.array_equal(picks, c["picks"]):
            j = int(np.flatnonzero(picks != c["picks"])[0])
            fails.append(f"case {i} ({c['kind']}, k={k}, m={m}): simulation {j} picked "
                         f"{picks[j]}, fixture {c['picks'][j]}")
        elif not np.array_equal(n_after, c["N_after"]):
            fails.append(f"case {i} ({c['kind']}): visit counts after the wave differ")
    assert not fails, "\n".join(fails)


class _Replay:
    """Evaluator that writes the fixture's rows for the unique leaves of each wave."""

    device_native = True

    def __init__(self, policy, values):
        self.policy, self.values, self.wave = policy, values, 0

    def evaluate_wave(self, eng) -> None:
        rows = torch.from_numpy(self.policy[self.wave]).to(eng.device)
        eng.policy.view(-1, eng.A)[:rows.shape[0]].copy_(rows)
        eng.values[:rows.shape[0]].copy_(torch.from_numpy(self.values[self.wave]).to(eng.device))
        self.wave += 1


@pytest.mark.parametrize("case", golden.SEARCH_CASES, ids=lambda c: c["name"])
def test_search_trees(device, case):
    inp = golden.search_inputs(case)
    params = SearchParams(c_puct=golden.C_PUCT, virtual_loss=case["vl"],
                          expand_policy=(_lib.OMQ_EXPAND_REFERENCE_PW
                                         if case["policy"] == "reference_pw"
                                         else _lib.OMQ_EXPAND_FULL),
                          sign_mode=case["sign"], dirichlet_epsilon=case["eps"])
    eng = WaveEngine(inp["model"], 1, golden.CAPACITY, case["W"], 100, device, params)
    eng.set_roots(inp["keys"], inp["legal"], inp["noise"])
    eng.reset()
    ev = _Replay(inp["policy"], inp["values"])
    plens, pflat = [], []
    for w in inp["waves"]:
        eng.run_wave(w, ev)
        pl = eng.path_len[:w].cpu().numpy()
        pa = eng.paths.view(case["W"], eng.MD)[:w].cpu().numpy()
        for s in range(w):
            plens.append(int(pl[s]))
            pflat.extend(pa[s, :pl[s]].tolist())
    eng.check_status()
    with np.load(os.path.join(HERE, "search_trees.npz")) as z:
        g = lambda key: z[f"{case['name']}/{key}"]  # noqa: E731
        assert np.array_equal(np.array(plens, np.int32), g("path_len"))
        assert np.array_equal(np.array(pflat, np.int32), g("paths"))
        tr = eng.host_tree(0)
        assert tr["num_nodes"] == len(g("N"))
        for key in ("N", "parent", "first", "nchild", "action"):
            assert np.array_equal(tr[key], g(key)), key
        for key in ("W", "P"):
            assert np.array_equal(tr[key].view(np.int32), g(key).view(np.int32)), key


def test_reference_pw_rule(device):
    """The device expansion follows the closed form of the reference's progressive widening
    over the grid of root visit counts and legal-set sizes (oracle/golden.py pw_root_count),
    for the root row and for the row of the root's first child."""
    fails = []
    for n0 in golden.PW_GRID_N0:
        for L in golden.PW_GRID_L:
            seed = 1000 + L
            model, board, legal, acts, pol = golden.pw_inputs(L, seed)
            eng = WaveEngine(model, 1, 128, 1, 100, device,
                             SearchParams(c_puct=1.4, virtual_loss=3.0,
                                          expand_policy=_lib.OMQ_EXPAND_REFERENCE_PW))
            eng.set_roots(games.root_keys(seed, 1), legal)
            eng.reset()
            _put(eng.N, [n0], np.int32)
            ev = _Replay(np.stack([pol[None], pol[None]]), np.zeros((2, 1), np.float32))
            eng.run_wave(1, ev)
            tr = eng.host_tree(0)
            f0, k0 = int(tr["first"][0]), int(tr["nchild"][0])
            root = [int(a) for a in tr["action"][f0 + 1:f0 + 1 + k0]]
            want = golden.pw_expected(acts, pol, n0)
            if root != want:
                fails.append(f"N0={n0} L={L}: root row {root}, rule {want}")
                continue
            eng.run_wave(1, ev)
            tr = eng.host_tree(0)
            c0 = f0 + 1
            f, k = int(tr["first"][c0]), int(tr["nchild"][c0])
            child = [int(a) for a in tr["action"][f + 1:f + 1 + k]] if k > 0 else []
            rest = [a for a in acts if a != root[0]]
            want_c = golden.pw_expected(rest, pol, None) if rest else []
            if child != want_c:
                fails.append(f"N0={n0} L={L}: first child's row {child}, rule {want_c}")
    assert not fails, "\n".join(fails[:10])
