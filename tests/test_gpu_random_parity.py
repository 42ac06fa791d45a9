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


def _case(i: int, seed: int = 9100, gomoku_sizes=range(5, 16), go_sizes=(5, 9, 13, 19),
          kinds=("gomoku", "go", "sparse")):
    rng = np.random.default_rng(seed + i)
    kind = kinds[i % len(kinds)]
    if kind == "gomoku":
        bs = int(rng.choice(list(gomoku_sizes)))
        model, base = games.gomoku(bs), "C2"
        extra = {"max_stones": int(rng.integers(0, bs * bs // 3))}
    elif kind == "go":
        bs = int(rng.choice(list(go_sizes)))
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


# Boards of 257-320 and 385-512 actions: the select kernels of five and eight slots per lane,
# which keep single-member groups with the chain groups (a level's group ordering once
# overwrote the next level's groups that its first-unvisited pass had formed there), and, above
# 384 actions, the expansion that reads the policy row from memory instead of staging it.
WIDE_BOARDS = [
    ("gomoku", 17, 256, {}), ("go", 17, 600, {"go_flags": 1}),
    ("gomoku", 20, 256, {}), ("gomoku", 21, 600, {}), ("gomoku", 22, 256, {"rule": 1}),
    ("go", 20, 600, {}), ("go", 21, 256, {"go_flags": 3}), ("go", 22, 1024, {"go_flags": 1}),
]


@pytest.mark.parametrize("i", range(len(WIDE_BOARDS)))
def test_wide_board_parity(device, i):
    kind, bs, W, kw = WIDE_BOARDS[i]
    rng = np.random.default_rng(9900 + i)
    model = games.gomoku(bs) if kind == "gomoku" else games.go(bs)
    waves = 3
    lo = bs * bs // 4 if "rule" in kw else 0
    wl = get("C2" if kind == "gomoku" else "C3").scaled(
        name=f"wide-{kind}{bs}", model=model, num_trees=2,
        max_stones=int(rng.integers(lo, bs * bs // 3)), num_simulations=1 + W * waves,
        wave_size=W, capacity=1 + W * waves * model.num_actions,
        seed=int(rng.integers(1, 1 << 30)))
    print(f"[wide board parity] {wl.name}: A={model.num_actions} W={W} {kw}", flush=True)
    assert run_parity(wl, device=device, **kw) >= 2


N_WIDE_CASES = 16


@pytest.mark.parametrize("i", range(N_WIDE_CASES))
def test_random_wide_board_parity(device, i):
    """The random knobs of test_random_workload_parity on boards of 257-512 actions (select
    kernels of five, six and eight slots per lane)."""
    wl = _case(i, seed=9300, gomoku_sizes=(17, 18, 20, 21, 22), go_sizes=(17, 18, 20, 21, 22),
               kinds=("gomoku", "go"))
    print(f"[random wide parity] {wl.name}: A={wl.model.num_actions} T={wl.num_trees} "
          f"W={wl.wave_size} sims={wl.num_simulations} cap={wl.capacity} "
          f"vl={wl.virtual_loss} c={wl.c_puct} depth={wl.max_depth} {wl.expand_policy} "
          f"eps={wl.dirichlet_epsilon}", flush=True)
    assert run_parity(wl, device=device) >= 2


N_EDGE_CASES = 24


def _edge_case(i: int):
    """Knobs at the edges of what the library accepts: virtual loss 0 (every rank of a chain
    takes the first rank's child), fractional (the count grows by its integer part, Q's
    denominator by the whole), or large; c_puct 0 (pure Q); depth limits of 1 (every path ends
    at the root) and 2; every select kernel width."""
    rng = np.random.default_rng(9500 + i)
    kind = ["gomoku", "go", "sparse"][i % 3]
    if kind == "gomoku":
        bs = int(rng.choice([5, 9, 15, 17, 19, 22]))
        model, base = games.gomoku(bs), "C2"
        extra = {"max_stones": int(rng.integers(0, bs * bs // 3))}
    elif kind == "go":
        bs = int(rng.choice([5, 13, 17, 19, 21]))
        model, base = games.go(bs), "C3"
        extra = {"max_stones": int(rng.integers(0, bs * bs // 3))}
    else:
        lo = int(rng.integers(1, 40))
        model, base = games.chess_sparse(int(rng.choice([64, 4672])), lo,
                                         lo + int(rng.integers(0, 25))), "C4"
        extra = {}
    W = int(rng.choice([1, 16, 64, 256, 600, 1024]))
    waves = int(rng.integers(2, 5))
    width = model.num_actions if kind != "sparse" else lo + 25
    return get(base).scaled(
        name=f"edge-{i}-{kind}", model=model, num_trees=int(rng.integers(1, 4)),
        num_simulations=1 + W * waves, wave_size=W, capacity=1 + W * waves * width,
        virtual_loss=float(rng.choice([0.0, 0.5, 1.5, 2.5, 7.0])),
        c_puct=float(rng.choice([0.0, 0.25, 1.0, 3.0])),
        max_depth=int(rng.choice([1, 2, 5, 100])),
        expand_policy="reference_pw" if rng.random() < 0.25 else "full",
        seed=int(rng.integers(1, 1 << 30)), **extra)


@pytest.mark.parametrize("i", range(N_EDGE_CASES))
def test_edge_knob_parity(device, i):
    wl = _edge_case(i)
    print(f"[edge parity] {wl.name}: A={wl.model.num_actions} T={wl.num_trees} "
          f"W={wl.wave_size} sims={wl.num_simulations} vl={wl.virtual_loss} c={wl.c_puct} "
          f"depth={wl.max_depth} {wl.expand_policy}", flush=True)
    assert run_parity(wl, device=device) >= 2


N_MODE_CASES = 18


@pytest.mark.parametrize("i", range(N_MODE_CASES))
def test_random_modes_parity(device, i):
    """The random workloads with the other accumulation modes, over every select kernel width:
    atomic virtual loss (one atomic per arrival), atomic W (float atomics, compared within
    1e-5) and the root-positive sign, one or two of them at a time."""
    wl = _case(i, seed=9600, gomoku_sizes=(5, 9, 15, 17, 20, 22), go_sizes=(5, 13, 17, 19, 21))
    rng = np.random.default_rng(9650 + i)
    kw = [dict(vl_atomic=True), dict(w_mode=1), dict(sign_mode=1),
          dict(vl_atomic=True, w_mode=1), dict(vl_atomic=True, sign_mode=1),
          dict(w_mode=1, sign_mode=1)][int(rng.integers(0, 6))]
    print(f"[random modes parity] {wl.name}: A={wl.model.num_actions} T={wl.num_trees} "
          f"W={wl.wave_size} sims={wl.num_simulations} {kw}", flush=True)
    assert run_parity(wl, device=device, **kw) >= 2


@pytest.mark.parametrize("lo,hi,W,depth", [(1, 1, 4, 128), (1, 2, 16, 128), (1, 2, 64, 60),
                                           (1, 3, 1, 128)])
def test_deep_paths_parity(device, lo, hi, W, depth):
    """Narrow sparse rows (one to three children), so that paths grow by about a node a wave
    and reach the depth limit: up to OMQ_MAX_DEPTH (128) nodes on a path."""
    waves = 150 if W <= 4 else 40
    wl = get("C4").scaled(name=f"deep-{lo}-{hi}-W{W}", model=games.chess_sparse(64, lo, hi),
                          num_trees=2, num_simulations=1 + W * waves, wave_size=W,
                          capacity=1 + W * waves * hi, max_depth=depth, seed=4242 + W)
    print(f"[deep parity] {wl.name}: depth limit {depth}, {waves} waves", flush=True)
    assert run_parity(wl, device=device, check_every=10) >= 2


@pytest.mark.parametrize("base,model,T,W", [("C2", games.gomoku(9), 300, 16),
                                            ("C3", games.go(19), 130, 64),
                                            ("C4", games.chess_sparse(4672, 20, 45), 257, 33)])
def test_many_trees_parity(device, base, model, T, W):
    """Forests of more trees than the device has CUs (select: one workgroup per tree; the
    expansion's and backup's grids remapped over the XCDs)."""
    width = model.max_legal if model.kind == "sparse" else model.num_actions
    wl = get(base).scaled(name=f"many-{base}-T{T}", model=model, num_trees=T,
                          num_simulations=1 + 3 * W, wave_size=W,
                          capacity=1 + 3 * W * width, max_stones=5)
    print(f"[many trees parity] {wl.name}: A={model.num_actions} W={W}", flush=True)
    assert run_parity(wl, device=device) >= 2


N_RULE_KNOB_CASES = 16


@pytest.mark.parametrize("i", range(N_RULE_KNOB_CASES))
def test_random_rules_with_knobs_parity(device, i):
    """The rules with the other knobs drawn too: the widening rule, root noise, virtual loss,
    c_puct, cramped capacities and depth limits, on boards of 5x5 to 22x22."""
    rng = np.random.default_rng(9800 + i)
    W = int(rng.choice([1, 16, 64, 256, 600, 1024]))
    waves = int(rng.integers(2, 5))
    gomoku = i % 2 == 0
    bs = int(rng.choice([5, 9, 15, 17, 20, 22] if gomoku else [5, 7, 13, 17, 19, 21]))
    model = games.gomoku(bs) if gomoku else games.go(bs)
    cap_full = 1 + W * waves * model.num_actions
    wl = get("C2" if gomoku else "C3").scaled(
        name=f"rule-knobs-{i}-{model.kind}{bs}", model=model, num_trees=int(rng.integers(1, 4)),
        max_stones=int(rng.integers(bs * bs // 5, bs * bs // 2)),
        num_simulations=1 + W * waves, wave_size=W,
        capacity=int(cap_full if rng.random() < 0.6 else max(64, cap_full // 8)),
        virtual_loss=float(rng.choice([0.5, 1.0, 3.0])), c_puct=float(rng.choice([0.5, 1.4, 3.0])),
        max_depth=int(rng.choice([3, 100])),
        expand_policy="reference_pw" if rng.random() < 0.5 else "full",
        dirichlet_alpha=0.3, dirichlet_epsilon=0.25 if rng.random() < 0.5 else 0.0,
        seed=int(rng.integers(1, 1 << 30)))
    kw = {"rule": int(rng.integers(0, 2))} if gomoku else {"go_flags": int(rng.choice([1, 3]))}
    print(f"[rules+knobs parity] {wl.name}: T={wl.num_trees} W={W} cap={wl.capacity} "
          f"vl={wl.virtual_loss} {wl.expand_policy} eps={wl.dirichlet_epsilon} {kw}", flush=True)
    assert run_parity(wl, device=device, **kw) >= 2


def test_parity_on_a_side_stream(device):
    """Every launch and copy of a search goes to the caller's current stream: a search run
    under another stream (default priority) follows the oracle too."""
    import torch

    wl = get("C3").scaled(name="side-stream", num_trees=3, num_simulations=1 + 3 * 600,
                          wave_size=600, capacity=1 + 3 * 600 * 362)
    s = torch.cuda.Stream(device=device)
    with torch.cuda.stream(s):
        assert run_parity(wl, device=device) >= 2


def test_interleaved_engines_parity(device):
    """Three engines of different models (select kernels of eight, six and one slot; board and
    sparse expansion) in one process, their waves interleaved, each against its own oracle."""
    import torch

    from oracle.parity import compare_wave, make_pair

    wls = [get("C2").scaled(name="mix-gomoku20", model=games.gomoku(20), num_trees=2,
                            num_simulations=1 + 3 * 256, wave_size=256,
                            capacity=1 + 3 * 256 * 400, max_stones=40),
           get("C3").scaled(name="mix-go19", num_trees=2, num_simulations=1 + 3 * 600,
                            wave_size=600, capacity=1 + 3 * 600 * 362),
           get("C4").scaled(name="mix-sparse", num_trees=2, num_simulations=1 + 3 * 1024,
                            wave_size=1024, capacity=1 + 3 * 1024 * 45)]
    pairs = [make_pair(wl, device=device) for wl in wls]
    for eng, orc, _ in pairs:
        eng.reset()
        for t in range(eng.T):
            orc.reset_tree(t)
    for i in range(4):
        for wl, (eng, orc, ev) in zip(wls, pairs):
            W = 1 if i == 0 else wl.wave_size
            eng.run_wave(W, ev)
            for t in range(eng.T):
                orc.wave(t, W)
        torch.cuda.synchronize()
        for wl, (eng, orc, _) in zip(wls, pairs):
            compare_wave(eng, orc, 1 if i == 0 else wl.wave_size, f"{wl.name} wave {i}")
