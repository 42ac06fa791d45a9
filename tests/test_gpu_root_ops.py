"""Per-move root operations on the GPU against the oracle: root policies, move selection
with a temperature, and root Dirichlet noise, bit for bit; a search with device noise."""
import numpy as np
import pytest
import torch

from omoknuni_quantum_amd import _lib
from omoknuni_quantum_amd.core.engine import SearchParams, WaveEngine
from omoknuni_quantum_amd.synthetic import games
from omoknuni_quantum_amd.synthetic.workloads import get
from oracle.oracle import Oracle, load
from oracle.parity import compare_wave, make_pair

pytestmark = pytest.mark.gpu


def test_policy_and_sampling_match_oracle(device):
    wl = get("C2").scaled(num_trees=8, num_simulations=512, wave_size=128, capacity=150_000)
    eng, orc, ev = make_pair(wl, device=device)
    eng.search(wl.num_simulations, wl.wave_size, ev)
    orc.search(wl.num_simulations, wl.wave_size)
    pol = eng.root_policies()
    lib = load()
    for t in range(wl.num_trees):
        assert np.array_equal(pol[t], orc.root_policy(t))
    for temperature in (0.0, 0.25, 1.0, 2.0):
        for counter in range(5):
            acts = eng.sample_actions(temperature, 1234, counter)
            for t in range(wl.num_trees):
                row = np.ascontiguousarray(pol[t])
                want = lib.orc_sample_action(row.ctypes.data, eng.A, temperature, 1234, counter, t)
                assert acts[t] == want, (temperature, counter, t)
                assert pol[t, acts[t]] > 0


def test_policy_corner_cases(device):
    """No children: uniform over the action space; children without visits: uniform over them."""
    model = games.gomoku(5)
    eng = WaveEngine(model, 2, 64, 4, 16, device, SearchParams())
    eng.reset()
    k = 6
    eng.first[64] = 0
    eng.nchild[64] = k
    eng.action[65:65 + k] = torch.tensor([3, 7, 8, 11, 20, 24], dtype=torch.int32)
    eng.N[65:65 + k] = 0
    eng.num_nodes[1] = 1 + k
    pol = eng.root_policies()
    assert np.all(pol[0] == 1.0 / 25)
    want = np.zeros(25)
    want[[3, 7, 8, 11, 20, 24]] = 1.0 / k
    assert np.array_equal(pol[1], want)


@pytest.mark.parametrize("name,alpha", [("C2", 0.3), ("C3", 0.03), ("C4", 1.5)])
def test_device_dirichlet_matches_oracle(device, name, alpha):
    wl = get(name).scaled(num_trees=6, capacity=1000)
    eng, orc, _ = make_pair(wl, device=device)
    eng.device_root_noise(alpha, 77, 2)
    got = eng.noise.view(eng.T, eng.A).cpu().numpy()
    for t in range(eng.T):
        want = orc.root_dirichlet(t, alpha, 77, 2)
        assert np.array_equal(got[t], want), (name, t)


def test_search_with_device_noise_matches_oracle(device):
    wl = get("C3").scaled(num_trees=3, num_simulations=2048, capacity=400_000)
    eng, orc, ev = make_pair(wl, device=device)
    eng.device_root_noise(wl.dirichlet_alpha, 5, 1)
    noise = eng.noise.view(eng.T, eng.A).cpu().numpy().copy()
    keys, legal, _ = wl.root_inputs()
    orc.set_roots(keys, legal, noise)
    eng.reset()
    for t in range(eng.T):
        orc.reset_tree(t)
    for i, w in enumerate([1] + [1024] * 2):
        eng.run_wave(w, ev)
        for t in range(eng.T):
            orc.wave(t, w)
        torch.cuda.synchronize()
        compare_wave(eng, orc, w, f"device noise wave {i}")


@pytest.mark.parametrize("kind,bs", [("gomoku", 22), ("go", 21)])
def test_root_ops_wide_boards(device, kind, bs):
    """Policies, move sampling and root noise on boards of 442-484 actions."""
    model = games.gomoku(bs) if kind == "gomoku" else games.go(bs)
    wl = get("C2" if kind == "gomoku" else "C3").scaled(
        model=model, num_trees=4, num_simulations=768, wave_size=256, max_stones=bs * bs // 4,
        capacity=1 + 4 * 256 * model.num_actions)
    eng, orc, ev = make_pair(wl, device=device)
    eng.search(wl.num_simulations, wl.wave_size, ev)
    orc.search(wl.num_simulations, wl.wave_size)
    pol = eng.root_policies()
    lib = load()
    for t in range(wl.num_trees):
        assert np.array_equal(pol[t], orc.root_policy(t))
    for temperature in (0.0, 1.0):
        for counter in range(3):
            acts = eng.sample_actions(temperature, 99, counter)
            for t in range(wl.num_trees):
                row = np.ascontiguousarray(pol[t])
                want = lib.orc_sample_action(row.ctypes.data, eng.A, temperature, 99, counter, t)
                assert acts[t] == want, (temperature, counter, t)
    eng.device_root_noise(0.03, 31, 4)
    got = eng.noise.view(eng.T, eng.A).cpu().numpy()
    for t in range(eng.T):
        assert np.array_equal(got[t], orc.root_dirichlet(t, 0.03, 31, 4)), t
