"""Parity of the HIP tree operations with the CPU oracle, wave by wave (bit-exact paths,
visit counts, CSR rows, priors and ordered-mode W)."""
import pytest

from omoknuni_quantum_amd.synthetic import games
from omoknuni_quantum_amd.synthetic.workloads import get
from oracle.parity import run_parity

CASES = {
    # C1 at its full size, both expansion policies
    "C1-full": ("C1", {}),
    "C1-reference_pw": ("C1", {"expand_policy": "reference_pw"}),
    # reduced tree counts / simulations of C2-C4 (the full sizes run in the bench tests)
    "C2-small": ("C2", {"num_trees": 4, "num_simulations": 768, "wave_size": 256,
                        "capacity": 200_000}),
    "C3-small": ("C3", {"num_trees": 2, "num_simulations": 2048, "wave_size": 1024,
                        "capacity": 500_000}),
    "C3-capacity": ("C3", {"num_trees": 2, "num_simulations": 3072, "wave_size": 1024,
                           "capacity": 60_000}),
    "C4-small": ("C4", {"num_trees": 2, "num_simulations": 4096, "wave_size": 2048,
                        "capacity": 200_000}),
    # the root chain overlapped with the level-1 chains (kernels of rows up to 192 children):
    # a last block of 8 picks, level-1 leaves forced by the depth limit, and a small board
    "overlap-ragged": ("C4", {"num_trees": 3, "num_simulations": 600, "wave_size": 200,
                              "capacity": 100_000}),
    "overlap-depth2": ("C4", {"num_trees": 2, "num_simulations": 900, "wave_size": 300,
                              "capacity": 100_000, "max_depth": 2}),
    "overlap-board7": ("C2", {"model": games.gomoku(7), "max_stones": 10, "num_trees": 3,
                              "num_simulations": 768, "wave_size": 384, "capacity": 100_000}),
    "overlap-knobs": ("C4", {"num_trees": 2, "num_simulations": 1536, "wave_size": 512,
                             "capacity": 100_000, "virtual_loss": 2.5, "c_puct": 0.5,
                             "expand_policy": "reference_pw", "dirichlet_alpha": 0.3,
                             "dirichlet_epsilon": 0.25}),
    # uniform priors (logit scale 0): close and equal scores, so that many steps have several
    # candidates and go to the exact comparison, in the 4-slot and the 1-slot kernels
    "uniform-priors-C2": ("C2", {"num_trees": 3, "num_simulations": 768, "wave_size": 256,
                                 "capacity": 100_000, "logit_scale": 0.0}),
    "uniform-priors-C4": ("C4", {"num_trees": 2, "num_simulations": 2048, "wave_size": 1024,
                                 "capacity": 100_000, "logit_scale": 0.0}),
    # a negative c_puct: every step is compared exactly (no fast path)
    "negative-cpuct": ("C2", {"num_trees": 2, "num_simulations": 512, "wave_size": 256,
                              "capacity": 100_000, "c_puct": -0.5}),
    # full simulation counts and capacities of C3 and C4 on two trees: contender windows deep
    # into a search, the 6-slot kernel on a deep tree, C3's capacity-full rule (tens of
    # thousands of refused expansions per tree) and C4's 2048-simulation waves
    "C3-fullcount": ("C3", {"num_trees": 2}),
    "C4-fullcount": ("C4", {"num_trees": 2}),
    # C2 at its full simulation count and capacity on two trees (1600 simulations, waves of 256)
    "C2-fullcount": ("C2", {"num_trees": 2}),
    # peaked priors on Go rows: one root child takes most of a wave, so that level-1 groups
    # outgrow the chains run ahead for them (replayed in part and continued, or run anew)
    "runahead-peaked": ("C3", {"num_trees": 4, "num_simulations": 3072, "wave_size": 1024,
                               "capacity": 500_000, "logit_scale": 10.0}),
    "runahead-depth3": ("C3", {"num_trees": 2, "num_simulations": 2048, "wave_size": 512,
                               "capacity": 500_000, "max_depth": 3}),
    # the largest wave (OMQ_MAX_WAVE): no run-ahead chains and no level overlap (their LDS
    # records hold waves of at most 2048 simulations), in the 6-, 4- and 1-slot kernels
    "maxwave-C3": ("C3", {"num_trees": 1, "num_simulations": 8192, "wave_size": 4096,
                          "capacity": 1_000_000}),
    "maxwave-C2": ("C2", {"num_trees": 2, "num_simulations": 8192, "wave_size": 4096,
                          "capacity": 400_000}),
    "maxwave-C4": ("C4", {"num_trees": 1, "num_simulations": 8192, "wave_size": 4096,
                          "capacity": 400_000}),
    # the widest and the five-slot select kernels at the largest wave
    "maxwave-gomoku22": ("C2", {"num_trees": 1, "num_simulations": 8192, "wave_size": 4096,
                                "capacity": 1_000_000, "model": games.gomoku(22),
                                "max_stones": 60}),
    "maxwave-go17": ("C3", {"num_trees": 1, "num_simulations": 8192, "wave_size": 4096,
                            "capacity": 1_000_000, "model": games.go(17)}),
    # tiny capacities: the capacity-full rule at every fill level (first fit in first-occurrence
    # order, refused leaves backed up), with 1-10 children per leaf or counts falling by depth
    "capacity-sparse-60": ("C4", {"model": games.chess_sparse(64, 1, 10), "num_trees": 16,
                                  "num_simulations": 192, "wave_size": 16, "capacity": 60}),
    "capacity-sparse-150": ("C4", {"model": games.chess_sparse(64, 1, 10), "num_trees": 16,
                                   "num_simulations": 192, "wave_size": 16, "capacity": 150}),
    "capacity-gomoku5": ("C2", {"model": games.gomoku(5), "max_stones": 17, "num_trees": 16,
                                "num_simulations": 192, "wave_size": 16, "capacity": 55}),
}
# compared after every wave, except the full-count cases (every third wave and the last)
CHECK_EVERY = {"C3-fullcount": 3, "C4-fullcount": 3, "C2-fullcount": 2}


@pytest.mark.gpu
@pytest.mark.parametrize("case", list(CASES))
def test_wave_parity(case, device):
    name, kw = CASES[case]
    wl = get(name).scaled(name=case, **kw)
    print(f"[parity] {case}: T={wl.num_trees} sims={wl.num_simulations} W={wl.wave_size}",
          flush=True)
    n = run_parity(wl, check_every=CHECK_EVERY.get(case, 1), device=device)
    assert n >= 2


@pytest.mark.gpu
def test_follower_wait_running_out(device):
    """A follower whose bounded wait runs out (spin limit 0, set from the host) sets
    OMQ_STATUS_STALL; the kernel exits normally, every path stays inside its tree, and the
    engine searches on after a reset."""
    import numpy as np
    import torch

    from omoknuni_quantum_amd import _lib
    from oracle.parity import make_pair

    lib = _lib.load()
    wl = get("C4").scaled(name="stall", num_trees=2, num_simulations=600, wave_size=200,
                          capacity=100_000)
    eng, orc, ev = make_pair(wl, device=device)
    eng.reset()
    eng.run_wave(1, ev)
    eng.run_wave(wl.wave_size, ev)  # an expanded first level, so that the overlap runs
    try:
        _lib.check(lib.omq_select_options(0), "omq_select_options")
        eng.select(wl.wave_size)
        torch.cuda.synchronize()
    finally:
        _lib.check(lib.omq_select_options(_lib.OMQ_SPIN_LIMIT_DEFAULT), "omq_select_options")
    assert int(eng.status[0].item()) & _lib.OMQ_STATUS_STALL
    with pytest.raises(_lib.OmqError):
        eng.check_status()
    T, MW = eng.T, eng.MW
    plen = eng.path_len.view(T, MW)[:, :wl.wave_size].cpu().numpy()
    leaves = eng.leaves.view(T, MW)[:, :wl.wave_size].cpu().numpy()
    nn = eng.num_nodes.cpu().numpy()
    assert np.all((plen >= 1) & (plen <= 2))  # the held-up members end at their level-1 node
    assert np.all((leaves >= 0) & (leaves < nn[:, None]))
    # a reset clears the status; the same engine then searches without error
    eng.reset()
    eng.check_status()
    eng.search(wl.num_simulations, wl.wave_size, ev)
    eng.check_status()
    # and a fresh pair follows the oracle bit for bit
    assert run_parity(wl, check_every=2, device=device) >= 2
