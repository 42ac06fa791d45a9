"""Wave parity with the oracle over randomly drawn small workloads (seeded): game model, board
size, tree count, wave size (across the select-records limit and the one-slot and wide
kernels), capacity (from cramped to ample), virtual loss, c_puct, noise, expansion policy and
depth limit.  Each case runs a whole search and compares every node after every wave."""
import numpy as np
import pytest

from omoknuni_quantum_amd.synthetic import games
from omoknuni_quantum_amd.synthetic.workloads import get
from oracle.parity import run_parity

pytestmark = pytest.mark.gpu

N_CASES = 48


def _case(i: int):
    rng = np.random.default_rng(9100 + i)
    kind = ["gomoku", "go", "sparse"][i % 3]
    if kind == "gomoku":
        bs = int(rng.integers(5, 16))
        model, base = games.gomoku(bs), "C2"
        extra = {"max_stones": int(rng.integers(0, bs * bs // 3))}
    elif kind == "go":
        bs = int(rng.choice([5, 9, 13, 19]))
        model, base = games.go(bs), "C3"
        extra = {"max_stones": int(rng.integers(0, bs * bs // 3))}
    else:
        lo = int(rng.integers(1, 30))
        model, base = games.chess_sparse(int(rng.choice([64, 512, 4672])), lo,
                                         lo + int(rng.integers(0, 30))), "C4"
        extra = {}
    W = int(rng.choice([1, 7, 16, 64, 200, 512, 513, 1024]))
    waves = int(rng.integers(2, 5))
    T = int(rng.integers(1, 5))
    cap_full = 1 + W * waves * max(1, model.num_actions if kind != "sparse" else lo + 30)
    capacity = int(cap_full if rng.random() < 0.6 else max(64, cap_full // int(rng.integers(3, 40))))
    kw = dict(model=model, num_trees=T, num_simulations=1 + W * waves, wave_size=W,
              capacity=capacity, virtual_loss=float(rng.choice([1.0, 2.0, 3.0])),
              c_puct=float(rng.choice([0.5, 1.0, 1.4, 2.5])),
              logit_scale=float(rng.choice([0.0, 1.0, 2.0, 6.0])),
              max_depth=int(rng.choice([2, 3, 100])),
              expand_policy="reference_pw" if rng.random() < 0.25 else "full",
              seed=int(rng.integers(1, 1 << 30)), **extra)
    if rng.random() < 0.3:
        kw.update(dirichlet_alpha=0.3, dirichlet_epsilon=0.25)
    return get(base).scaled(name=f"random-{i}-{kind}", **kw)


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_workload_parity(device, i):
    wl = _case(i)
    print(f"[random parity] {wl.name}: A={wl.model.num_actions} T={wl.num_trees} "
          f"W={wl.wave_size} sims={wl.num_simulations} cap={wl.capacity} "
          f"vl={wl.virtual_loss} c={wl.c_puct} depth={wl.max_depth} {wl.expand_policy} "
          f"eps={wl.dirichlet_epsilon}", flush=True)
    assert run_parity(wl, device=device) >= 2


N_RULE_CASES = 24


def _rule_case(i: int):
    """Board workloads with a rule on: the Gomoku terminal check (freestyle or renju) on dense
    boards, or the Go rules (ko, ko + suicide)."""
    rng = np.random.default_rng(9700 + i)
    W = int(rng.choice([1, 16, 64, 256, 513, 1024]))
    waves = int(rng.integers(2, 5))
    T = int(rng.integers(1, 4))
    if i % 2 == 0:
        bs = int(rng.integers(5, 16))
        wl = get("C2").scaled(name=f"random-rule-{i}-gomoku{bs}", model=games.gomoku(bs),
                              max_stones=int(rng.integers(bs * bs // 4, bs * bs // 2)),
                              num_trees=T, num_simulations=1 + W * waves, wave_size=W,
                              capacity=1 + W * waves * bs * bs,
                              seed=int(rng.integers(1, 1 << 30)))
        return wl, {"rule": int(rng.integers(0, 2))}
    bs = int(rng.choice([5, 7, 9, 13]))
    wl = get("C3").scaled(name=f"random-rule-{i}-go{bs}", model=games.go(bs),
                          max_stones=int(rng.integers(0, bs * bs // 2)), num_trees=T,
                          num_simulations=1 + W * waves, wave_size=W,
                          capacity=1 + W * waves * (bs * bs + 1),
                          seed=int(rng.integers(1, 1 << 30)))
    return wl, {"go_flags": int(rng.choice([1, 3]))}


@pytest.mark.parametrize("i", range(N_RULE_CASES))
def test_random_rules_parity(device, i):
    wl, kw = _rule_case(i)
    print(f"[random rules parity] {wl.name}: T={wl.num_trees} W={wl.wave_size} "
          f"sims={wl.num_simulations} {kw}", flush=True)
    assert run_parity(wl, device=device, **kw) >= 2
