"""The MCTS / MCTSConfig API over the HIP library, checked against the oracle."""
import numpy as np
import pytest
import torch

from omoknuni_quantum_amd.core.mcts import MCTS
from omoknuni_quantum_amd.core.mcts_config import GameType, MCTSConfig
from omoknuni_quantum_amd.synthetic import games
from omoknuni_quantum_amd.synthetic.evaluator import SyntheticEvaluator
from oracle.oracle import Oracle
from oracle.ref_np import leaf_position, nn_features

pytestmark = pytest.mark.gpu


def _config(**kw):
    base = dict(num_simulations=256, c_puct=1.4, virtual_loss=3.0, max_wave_size=32,
                dirichlet_epsilon=0.0, max_tree_nodes=100_000, seed=7, board_size=15,
                game_type=GameType.GOMOKU, device="cuda")
    base.update(kw)
    return MCTSConfig(**base)


def _board(seed=1, stones=20):
    return games.random_boards(1, 15, stones, seed, min_stones=stones)[0]


def _oracle_for(cfg, boards, noise=None):
    model = MCTS._game_model(cfg)
    T = boards.shape[0] if boards is not None else cfg.num_trees
    orc = Oracle(model, T, cfg.max_tree_nodes, cfg.max_wave_size, cfg.max_depth)
    orc.set_params(cfg.c_puct, cfg.virtual_loss, 0 if cfg.expansion_policy == "full" else 1,
                   0 if cfg.backup_sign == "leaf_positive" else 1, 1.0, cfg.dirichlet_epsilon)
    orc.set_roots(games.root_keys(cfg.seed, T), games.legal_masks(model, boards, T), noise)
    if model.kind == "gomoku" and cfg.gomoku_rules != "off":
        b = boards if boards is not None else np.zeros((T, cfg.board_size, cfg.board_size), np.int8)
        orc.set_gomoku_rules(b, 1 if cfg.gomoku_rules == "renju" else 0)
    return orc


def _assert_tree_equal(mcts, orc, t=0):
    g = mcts.engine.host_tree(t)
    o = orc.tree(t)
    assert g["num_nodes"] == o["num_nodes"]
    for k in ("N", "parent", "first", "nchild", "action"):
        assert np.array_equal(g[k], o[k]), k
    for k in ("W", "P"):
        assert np.array_equal(g[k].view(np.int32), o[k].view(np.int32)), k


def test_search_matches_oracle(device):
    cfg = _config()
    board = _board()
    m = MCTS(cfg, SyntheticEvaluator())
    pol = m.search(board)
    orc = _oracle_for(cfg, board[None])
    orc.search(256, 32)
    assert pol.shape == (225,)
    assert np.array_equal(pol, orc.root_policy(0))
    _assert_tree_equal(m, orc)
    assert abs(pol.sum() - 1.0) < 1e-12
    assert np.all(pol[board.reshape(-1) != 0] == 0)  # occupied cells never visited


def test_second_search_continues_tree(device):
    cfg = _config(num_simulations=64)
    board = _board()
    m = MCTS(cfg, SyntheticEvaluator())
    m.search(board)
    m.search(board)
    assert int(m.engine.N[0].item()) == 2 + 128
    m.search(_board(seed=2))  # a different root resets the tree
    assert int(m.engine.N[0].item()) == 2 + 64


def test_zero_simulations_and_shape_check(device):
    # num_simulations=0 runs the configured count (mcts.py:940 `num_simulations or
    # config.num_simulations`); a configured count of 0 gives the uniform policy
    board = _board()
    m = MCTS(_config(num_simulations=64), SyntheticEvaluator())
    pol = m.search(board, num_simulations=0)
    assert int(m.engine.N[0].item()) == 2 + 64
    orc = _oracle_for(_config(num_simulations=64), board[None])
    orc.search(64, 32)
    assert np.array_equal(pol, orc.root_policy(0))
    m0 = MCTS(_config(num_simulations=0), SyntheticEvaluator())
    assert np.allclose(m0.search(board), 1.0 / 225)
    with pytest.raises(ValueError):
        m.search(np.zeros((9, 9), np.int8))


def test_select_action_update_root_root_value(device):
    m = MCTS(_config(), SyntheticEvaluator())
    board = _board()
    pol = m.search(board)
    assert m.select_action(board, temperature=0, policy=pol) == int(np.argmax(pol))
    a = m.select_action(board, temperature=1.0, policy=pol)
    assert pol[a] > 0
    n, w = int(m.engine.N[0].item()), float(m.engine.W[0].item())
    assert m.get_root_value() == pytest.approx(w / n)
    with pytest.raises(ValueError):
        m.update_root(-1)
    with pytest.raises(ValueError):
        m.update_root(225)
    nb = board.copy()
    nb.reshape(-1)[a] = 1
    m.update_root(a, nb)
    assert int(m.engine.num_nodes[0].item()) == 1
    stats = m.get_statistics()
    assert stats["total_searches"] == 1 and stats["total_simulations"] == 256
    with MCTS(_config(), SyntheticEvaluator()) as m2:
        m2.search(board, num_simulations=32)


def test_search_batch_matches_oracle(device):
    cfg = _config(num_trees=4, num_simulations=128, max_wave_size=64)
    boards = games.random_boards(4, 15, 40, seed=9)
    m = MCTS(cfg, SyntheticEvaluator())
    pol = m.search_batch(boards)
    orc = _oracle_for(cfg, boards)
    orc.search(128, 64)
    for t in range(4):
        assert np.array_equal(pol[t], orc.root_policy(t))
        _assert_tree_equal(m, orc, t)
    with pytest.raises(ValueError):
        m.search(boards[0])


def test_root_dirichlet_noise_matches_oracle(device):
    cfg = _config(dirichlet_epsilon=0.25, dirichlet_alpha=0.03, num_simulations=96)
    board = _board()
    m = MCTS(cfg, SyntheticEvaluator())
    pol = m.search(board)
    model = MCTS._game_model(cfg)
    legal = games.legal_masks(model, board[None], 1)
    noise = games.dirichlet_noise(model, games.legal_counts(model, legal), 0.03, cfg.seed + 7919)
    orc = _oracle_for(cfg, board[None], noise)
    orc.search(96, 32)
    assert np.array_equal(pol, orc.root_policy(0))
    _assert_tree_equal(m, orc)


def test_reference_pw_and_root_positive_via_api(device):
    cfg = _config(expansion_policy="reference_pw", backup_sign="root_positive",
                  num_simulations=200)
    board = _board()
    m = MCTS(cfg, SyntheticEvaluator())
    pol = m.search(board)
    orc = _oracle_for(cfg, board[None])
    orc.search(200, 32)
    assert np.array_equal(pol, orc.root_policy(0))
    _assert_tree_equal(m, orc)
    assert int(m.engine.nchild[0].item()) == 8  # MAX_CHILDREN at the root


class _RecordingEvaluator:
    """A reference-protocol evaluator: features -> (policy, value) from a fixed random conv,
    recording its outputs for replay into the oracle."""

    def __init__(self, seed=0):
        g = torch.Generator().manual_seed(seed)
        self.w = (torch.randn(19, generator=g) * 0.5)
        self.calls = []
        self.feats = []

    def evaluate_batch(self, feats):
        self.feats.append(feats.cpu().numpy().copy())
        x = feats.float()
        w = self.w.to(x.device)[None, :, None, None]
        logits = (x * w).sum(dim=1).reshape(x.shape[0], -1) * 3
        pol = torch.softmax(logits, dim=1)
        val = torch.tanh(x[:, 0].mean(dim=(1, 2)) - x[:, 1].mean(dim=(1, 2)) + logits.mean(1))
        self.calls.append((pol.cpu().numpy().copy(), val.cpu().numpy().copy()))
        return pol, val


def test_feature_evaluator_replay_parity(device):
    cfg = _config(num_simulations=160)
    board = _board(stones=30)
    ev = _RecordingEvaluator()
    m = MCTS(cfg, ev)
    pol = m.search(board)
    assert len(ev.calls) == 1 + 160 // 32
    # reference 'basic' planes; the root wave's one leaf is the root position itself, and
    # every call holds exactly the wave's unique leaves
    assert ev.feats[0].shape == (1, 19, 15, 15)
    b, player, count = leaf_position(board, [])
    assert np.array_equal(ev.feats[0][0], nn_features(b, player, count, 19))
    assert all(1 <= f.shape[0] <= 32 for f in ev.feats[1:])
    orc = _oracle_for(cfg, board[None])
    orc.reset_tree(0)
    sizes = [1] + [32] * 5
    for (p, v), W in zip(ev.calls, sizes):
        assert p.shape[0] == v.shape[0] <= W
        rp = np.zeros((W, 225), np.float32)
        rv = np.zeros(W, np.float32)
        rp[:p.shape[0]], rv[:v.shape[0]] = p, v
        orc.wave(0, W, replay_policy=rp, replay_values=rv)
    assert np.array_equal(pol, orc.root_policy(0))
    _assert_tree_equal(m, orc)


class _StubState:
    """A game-state object with the reference's interface (the C++ game state's Python
    surface): get_basic_tensor_representation (18 planes), get_tensor_representation (3
    planes: the mover's stones, the opponent's, the colour to play), get_current_player,
    get_move_history."""

    def __init__(self, board, player, history):
        self.board, self.player, self.history = np.asarray(board, np.int8), player, history

    def get_tensor_representation(self):
        b = self.board
        return np.stack([(b == self.player), (b == 3 - self.player),
                         np.full(b.shape, self.player == 1)]).astype(np.float32)

    def get_basic_tensor_representation(self):
        t = np.zeros((18,) + self.board.shape, np.float32)
        t[0] = self.board != 0
        t[1] = self.player == 1
        return t

    def get_current_player(self):
        return self.player

    def get_move_history(self):
        return list(self.history)


def test_state_object_roots_match_oracle(device):
    """search() takes the reference's game-state objects (mcts.py:1520-1600): the board comes
    from the 3-channel form mapped by the player to move, who plays the first path move."""
    cfg = _config(num_simulations=512)
    board = _board(stones=21)  # odd stone count: parity would give player 2 ...
    state = _StubState(board, 1, history=list(range(21)))  # ... the state says player 1
    m = MCTS(cfg, SyntheticEvaluator())
    pol = m.search(state)
    orc = _oracle_for(cfg, board[None])
    orc.set_gomoku_rules(board[None], 0, root_player=np.array([1], np.int32))
    orc.search(512, 32)
    assert np.array_equal(pol, orc.root_policy(0))
    _assert_tree_equal(m, orc)
    # a game interface's state_to_numpy is used when there is one
    class _Iface:
        calls = 0

        def state_to_numpy(self, s, representation_type=None):
            _Iface.calls += 1
            if representation_type == "minimal":
                return s.get_tensor_representation()
            return s.get_basic_tensor_representation()

    m2 = MCTS(cfg, SyntheticEvaluator(), game_interface=_Iface())
    pol2 = m2.search(state)
    assert _Iface.calls == 2 and np.array_equal(pol2, pol)
    # the same root twice continues the tree; update_root with a state object keeps the
    # played child's subtree, and the state's player moves next
    m.search(state)
    assert int(m.engine.N[0].item()) == 2 + 1024
    nb = board.copy()
    a = int(np.argmax(pol))
    nb.reshape(-1)[a] = 1
    tr = m.engine.host_tree(0)
    kids = np.arange(tr["first"][0] + 1, tr["first"][0] + 1 + tr["nchild"][0])
    n_child = int(tr["N"][kids[tr["action"][kids] == a][0]])
    m.update_root(a, _StubState(nb, 2, history=list(range(22))))
    assert m.stats["tree_reuse_count"] == 1
    assert int(m.engine.N[0].item()) == n_child
    assert list(m._root_players_host) == [2] and list(m._root_moves_host) == [22]


def test_feature_evaluator_batch_replay_parity(device):
    """search_batch with a reference-protocol evaluator: each call holds the unique leaves of
    tree 0, then tree 1, ...; replayed into the oracle tree by tree, the trees are bit-equal."""
    cfg = _config(num_trees=3, num_simulations=96, max_wave_size=32)
    boards = games.random_boards(3, 15, 30, seed=4)
    ev = _RecordingEvaluator(seed=3)
    m = MCTS(cfg, ev)
    pol = m.search_batch(boards)
    orc = _oracle_for(cfg, boards)
    sizes = [1] + [32] * 3
    assert len(ev.calls) == len(sizes)
    for t in range(3):
        orc.reset_tree(t)
    for (p, v), W in zip(ev.calls, sizes):
        off = 0
        for t in range(3):
            rp = np.zeros((W, 225), np.float32)
            rv = np.zeros(W, np.float32)
            n = min(W, p.shape[0] - off)
            rp[:n], rv[:n] = p[off:off + n], v[off:off + n]
            orc.wave(t, W, replay_policy=rp, replay_values=rv)
            off += int(orc.last_wave(t, W)["ucount"])
        assert off == p.shape[0]
    for t in range(3):
        assert np.array_equal(pol[t], orc.root_policy(t))
        _assert_tree_equal(m, orc, t)


class _GoStubState(_StubState):
    """A Go state: also get_ko_point (GoState::getKoPoint)."""

    def __init__(self, board, player, history, ko):
        super().__init__(board, player, history)
        self.ko = ko

    def get_ko_point(self):
        return self.ko


@pytest.mark.parametrize("rules", ["ko", "ko_suicide"])
def test_go_rules_via_api(device, rules):
    """MCTSConfig(go_rules=...) on a Go game-state root whose history ends in a pass and that
    has a ko point: the tree equals the oracle's with the same root passes and ko point; the
    ko point is never a child, and a pass reply to the root's pass is a terminal leaf (visited,
    never expanded)."""
    bs = 9
    cfg = _config(game_type=GameType.GO, board_size=bs, num_simulations=1024, max_wave_size=64,
                  go_rules=rules)
    board = games.random_boards(1, bs, 24, 5, min_stones=24)[0]
    pass_action = bs * bs
    ko = int(np.flatnonzero(board.reshape(-1) == 0)[3])
    state = _GoStubState(board, 1, history=[0] * 23 + [pass_action], ko=ko)
    m = MCTS(cfg, SyntheticEvaluator())
    pol = m.search(state)
    flags = 1 if rules == "ko" else 3
    orc = _oracle_for(cfg, board[None])
    orc.set_go_rules(board[None], flags, root_player=[1], root_passes=[1], root_ko=[ko])
    # the root's legal set under the rules is what the host hands the oracle too
    orc.set_roots(games.root_keys(cfg.seed, 1), m._root_legal_host, None)
    orc.search(1024, 64)
    assert np.array_equal(pol, orc.root_policy(0))
    _assert_tree_equal(m, orc)
    tr = m.engine.host_tree(0)
    n = tr["num_nodes"]
    assert ko not in tr["action"][1:n].tolist()
    kids = np.arange(tr["first"][0] + 1, tr["first"][0] + 1 + tr["nchild"][0])
    p = kids[tr["action"][kids] == pass_action]
    assert p.size == 1 and tr["N"][p[0]] > 0 and tr["nchild"][p[0]] == 0


def test_search_graph_replay_matches_eager(device):
    """use_cuda_graphs: the first search of a launch signature runs eagerly and is recorded,
    later ones replay the recording.  The same sequence of searches (new roots, each searched
    twice so that the second continues the tree) with recording on and off gives the same
    policies and trees, bit for bit."""
    boards = [_board(seed=s) for s in (1, 2, 3, 1)]
    runs = {}
    for graphs in (False, True):
        m = MCTS(_config(num_simulations=96, use_cuda_graphs=graphs), SyntheticEvaluator())
        out = []
        for b in boards:
            for _ in range(2):
                out.append(m.search(b))
                t = m.engine.host_tree(0)
                out.append((t["num_nodes"], t["N"].copy(), t["W"].view(np.int32).copy(),
                            t["P"].view(np.int32).copy(), t["first"].copy(), t["action"].copy()))
        # a fresh root and a continued tree: two recordings, replayed by the later searches
        assert len(m._graphs) == (2 if graphs else 0)
        runs[graphs] = out
    for i, (a, b) in enumerate(zip(runs[False], runs[True])):
        if isinstance(a, np.ndarray):
            assert np.array_equal(a, b), i
        else:
            assert a[0] == b[0], i
            for x, y in zip(a[1:], b[1:]):
                assert np.array_equal(x, y), i


@pytest.mark.parametrize("game,bs,wave", [("gomoku", 20, 64), ("go", 21, 256), ("gomoku", 9, 16)])
def test_search_board_sizes_match_oracle(device, game, bs, wave):
    """MCTS.search on boards of other sizes (81-484 actions) and wave sizes."""
    gt = GameType.GOMOKU if game == "gomoku" else GameType.GO
    cfg = _config(board_size=bs, game_type=gt, max_wave_size=wave, num_simulations=4 * wave,
                  max_tree_nodes=1 + 5 * wave * (bs * bs + 1))
    board = games.random_boards(1, bs, bs * bs // 5, 3 + bs)[0]
    m = MCTS(cfg, SyntheticEvaluator())
    pol = m.search(board)
    orc = _oracle_for(cfg, board[None])
    orc.search(4 * wave, wave)
    A = bs * bs + (1 if game == "go" else 0)
    assert pol.shape == (A,)
    assert np.array_equal(pol, orc.root_policy(0))
    _assert_tree_equal(m, orc)
