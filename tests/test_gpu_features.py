"""Feature planes on the GPU (omq_leaf_features through the C ABI) against the numpy
restatement of the reference's planes (oracle/ref_np.py), slot by slot, bit for bit, on every
wave of a search, in both dtypes, both layouts and both plane counts."""
import numpy as np
import pytest
import torch

from omoknuni_quantum_amd.core.engine import SearchParams, WaveEngine
from omoknuni_quantum_amd.synthetic import games
from omoknuni_quantum_amd.synthetic.evaluator import SyntheticEvaluator
from omoknuni_quantum_amd.synthetic.workloads import get
from oracle.ref_np import leaf_position, nn_features

pytestmark = pytest.mark.gpu


def _expected(eng, boards, planes, root_player=None, root_moves=None):
    """float32 [T*MW, planes, bs, bs] from the engine's wave arrays and the numpy planes."""
    T, MW, MD, cap = eng.T, eng.MW, eng.MD, eng.cap
    bs = eng.model.board_size
    ucount = eng.ucount.cpu().numpy()
    ufirst = eng.ufirst.cpu().numpy().reshape(T, MW)
    plen = eng.path_len.cpu().numpy().reshape(T, MW)
    paths = eng.paths.cpu().numpy().reshape(T, MW, MD)
    action = eng.action.cpu().numpy().reshape(T, cap)
    out = np.zeros((T * MW, planes, bs, bs), np.float32)
    for t in range(T):
        for u in range(int(ucount[t])):
            s = int(ufirst[t, u])
            nodes = paths[t, s, :plen[t, s]]
            acts = [int(action[t, n]) for n in nodes[1:]]
            b, player, count = leaf_position(
                boards[t], acts, None if root_player is None else root_player[t],
                None if root_moves is None else root_moves[t])
            out[t * MW + u] = nn_features(b, player, count, planes)
    return out, ucount


class _CheckingEvaluator:
    """Checks the feature planes of every wave before the synthetic evaluator runs."""

    def __init__(self, eng, boards, root_player=None, root_moves=None):
        self.inner = SyntheticEvaluator(1.0)
        self.boards = boards
        self.dev_boards = torch.from_numpy(boards.reshape(-1).copy()).to(eng.device)
        self.rp = root_player
        self.rm = root_moves
        self.dev_rp = None if root_player is None else torch.from_numpy(
            np.asarray(root_player, np.int32)).to(eng.device)
        self.dev_rm = None if root_moves is None else torch.from_numpy(
            np.asarray(root_moves, np.int32)).to(eng.device)
        self.waves = 0
        self.leaves = 0

    def evaluate_wave(self, eng):
        n = eng.T * eng.MW * eng.A
        for planes in (18, 19):
            exp, ucount = _expected(eng, self.boards, planes, self.rp, self.rm)
            exp_bf = torch.from_numpy(exp).to(torch.bfloat16).view(torch.int16).numpy()
            for dtype in (torch.float32, torch.bfloat16):
                for nhwc in (False, True):
                    out = torch.full((n * planes,), float("nan"), dtype=dtype, device=eng.device)
                    eng.leaf_features(out, self.dev_boards, planes, self.dev_rp, self.dev_rm, nhwc)
                    got = out.view(eng.T * eng.MW, eng.model.board_size, eng.model.board_size,
                                   planes).permute(0, 3, 1, 2) if nhwc else out.view(
                        eng.T * eng.MW, planes, eng.model.board_size, eng.model.board_size)
                    got = got.contiguous().cpu()
                    ctx = (self.waves, planes, dtype, nhwc)
                    if dtype == torch.float32:
                        assert np.array_equal(got.numpy().view(np.int32), exp.view(np.int32)), ctx
                    else:
                        assert np.array_equal(got.view(torch.int16).numpy(), exp_bf), ctx
        self.waves += 1
        self.leaves += int(ucount.sum())
        self.inner.evaluate_wave(eng)


@pytest.mark.parametrize("explicit", [False, True])
def test_features_match_reference_planes(device, explicit):
    wl = get("C2").scaled(num_trees=3, num_simulations=96, wave_size=32, capacity=30_000)
    keys, legal, _ = wl.root_inputs()
    boards = wl.boards()
    eng = WaveEngine(wl.model, wl.num_trees, wl.capacity, wl.wave_size, wl.max_depth, device,
                     SearchParams(c_puct=wl.c_puct, virtual_loss=wl.virtual_loss))
    eng.set_roots(keys, legal)
    rp = rm = None
    if explicit:
        rp = np.array([2, 1, 2], np.int32)
        rm = np.array([0, 17, 300], np.int32)
    ev = _CheckingEvaluator(eng, boards, rp, rm)
    eng.search(wl.num_simulations, wl.wave_size, ev)
    torch.cuda.synchronize()
    assert ev.waves == 1 + 96 // 32
    assert ev.leaves > 3 * 64  # root waves plus wide later waves


def test_features_small_board_deep_paths(device):
    # 7x7 with a full-ish root: long paths, the move count plane past 100
    model = games.gomoku(7)
    T, W = 2, 16
    boards = games.random_boards(T, 7, 30, 5)
    keys = games.root_keys(5, T)
    legal = games.legal_masks(model, boards, T)
    eng = WaveEngine(model, T, 20_000, W, 100, device, SearchParams(c_puct=1.4, virtual_loss=3.0))
    eng.set_roots(keys, legal)
    ev = _CheckingEvaluator(eng, boards, None, np.array([95, 120], np.int32))
    eng.search(160, W, ev)
    torch.cuda.synchronize()
    assert ev.waves == 11


@pytest.mark.parametrize("bs", [5, 11, 19, 22])
def test_features_board_sizes(device, bs):
    # boards from 5x5 to 22x22 (484 cells, the widest board the library takes), a third full
    model = games.gomoku(bs)
    T, W = 2, 64
    boards = games.random_boards(T, bs, bs * bs // 3, 11 + bs)
    keys = games.root_keys(11 + bs, T)
    legal = games.legal_masks(model, boards, T)
    eng = WaveEngine(model, T, 1 + 4 * W * bs * bs, W, 100, device,
                     SearchParams(c_puct=1.4, virtual_loss=3.0))
    eng.set_roots(keys, legal)
    ev = _CheckingEvaluator(eng, boards)
    eng.search(3 * W, W, ev)
    torch.cuda.synchronize()
    assert ev.waves == 4
