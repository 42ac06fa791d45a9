"""Go rules on the GPU (omq_go_rules through the C ABI) against the oracle: legal masks of every
unique leaf, terminal codes, legal counts and whole trees after every wave, on C3-shaped
searches (Go 19x19 + pass, random root positions, a ko point in every other tree, a root pass in
every third) and on small dense boards where full boards and closed points are common."""
import numpy as np
import pytest
import torch

from omoknuni_quantum_amd import _lib
from omoknuni_quantum_amd.synthetic import games
from omoknuni_quantum_amd.synthetic.workloads import get
from oracle.parity import compare_wave, make_pair, run_parity

pytestmark = pytest.mark.gpu

KO_SUICIDE = _lib.OMQ_GO_KO | _lib.OMQ_GO_SUICIDE


@pytest.mark.parametrize("flags", [_lib.OMQ_GO_KO, KO_SUICIDE])
def test_c3_shaped_parity(device, flags):
    wl = get("C3").scaled(name=f"C3-go-rules-{flags}", num_trees=8, num_simulations=3072,
                          wave_size=1024, capacity=400_000)
    stats = {}
    print(f"go rules C3-shaped flags={flags}", flush=True)
    assert run_parity(wl, device=device, stats=stats, go_flags=flags) >= 4
    assert stats["terminal"] > 0


def test_c3_full_count(device):
    """C3's own sizes (32 trees x 10,000 simulations, waves of 1024) with both rules on,
    compared every fourth wave and at the end."""
    wl = get("C3")
    stats = {}
    print("go rules C3 full count", flush=True)
    assert run_parity(wl, check_every=4, device=device, stats=stats, go_flags=KO_SUICIDE) >= 3
    assert stats["terminal"] > 0


def test_dense_small_boards(device):
    """5x5 boards with 12-20 stones: full boards, closed points and pass-pass endings."""
    wl = get("C3").scaled(name="go5-dense", model=games.go(5), max_stones=20, num_trees=8,
                          num_simulations=1024, wave_size=64, capacity=60_000)
    stats = {}
    assert run_parity(wl, device=device, stats=stats, go_flags=KO_SUICIDE) >= 10
    assert stats["terminal"] > 50


def _path_moves(eng, t, s, A):
    L = int(eng.path_len.view(eng.T, eng.MW)[t, s])
    path = eng.paths.view(eng.T, eng.MW, eng.MD)[t, s, :L].cpu().numpy()
    acts = eng.action.view(eng.T, -1)[t].cpu().numpy()
    return [int(acts[x]) for x in path[1:]]


def test_umask_matches_oracle(device):
    """The legal mask of every unique leaf, bit for bit, against the oracle's legal list of
    the leaf's position (9x9, both rules, ko points and root passes)."""
    wl = get("C3").scaled(name="go9-umask", model=games.go(9), max_stones=30, num_trees=4,
                          num_simulations=512, wave_size=64, capacity=40_000)
    eng, orc, ev = make_pair(wl, device=device, go_flags=KO_SUICIDE)
    A, LW = wl.model.num_actions, wl.model.legal_words
    eng.reset()
    for t in range(wl.num_trees):
        orc.reset_tree(t)
    checked = 0
    for i, W in enumerate([1] + [64] * 8):
        eng.run_wave(W, ev)
        for t in range(wl.num_trees):
            orc.wave(t, W)
        torch.cuda.synchronize()
        compare_wave(eng, orc, W, f"umask wave {i}")
        umask = eng.umask.view(eng.T, eng.MW, LW).cpu().numpy().view(np.uint32)
        ucount = eng.ucount.cpu().numpy()
        ufirst = eng.ufirst.view(eng.T, eng.MW).cpu().numpy()
        for t in range(wl.num_trees):
            for u in range(int(ucount[t])):
                moves = _path_moves(eng, t, int(ufirst[t, u]), A)
                want, _ = orc.go_leaf_rules(t, moves)
                bits = np.unpackbits(umask[t, u].view(np.uint8), bitorder="little")[:A]
                got = np.flatnonzero(bits).tolist()
                assert got == want, (i, t, u, moves)
                checked += 1
    assert checked > 500
