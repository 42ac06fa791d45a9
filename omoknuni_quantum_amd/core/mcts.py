"""MCTS: the search API of the reference over the HIP tree operations.

Drop-in for python/mcts/core/mcts.py:43-2216 of cosmosapjw-quantum/omoknuni_quantum, GPU tree
backend: ``MCTS(config, evaluator, game_interface=None, single_gpu_mode=False)`` with
``search``, ``select_action``, ``update_root``, ``get_root_value``, ``clear``/``reset_tree``,
``get_statistics``, ``warmup``, ``shutdown`` and the context-manager protocol, plus
``search_batch`` for ``config.num_trees`` independent trees searched together.

A search follows mcts.py:923-1063: the root is expanded first if it has no children (a
one-simulation wave on the lone root; its value is backed up, mcts.py:1659-1691), then waves
of min(max_wave_size, remaining) simulations run until num_simulations are done, and the
policy is the root children's visit distribution (mcts.py:1069-1137).  Every wave runs on the
device: selection with virtual loss, leaf evaluation, expansion, backup.

Evaluators: a device-native evaluator (``evaluate_wave(engine)``, e.g. SyntheticEvaluator) is
called with the wave engine; any other evaluator is called as in the reference,
``evaluate_batch(features) -> (policies [B, A], values [B])``, on feature planes of the wave's
unique leaves built on the device (core/features.py).
"""
from __future__ import annotations

import logging
import time
from collections import defaultdict
from typing import Any, Dict, Optional

import numpy as np
import torch

from .. import _lib
from ..synthetic import games
from .engine import SearchParams, WaveEngine
from .mcts_config import GameType, MCTSConfig

logger = logging.getLogger(__name__)


def _input_planes(evaluator) -> int:
    """Feature planes a reference-protocol evaluator takes: the 19 of the reference's 'basic'
    representation (cpu_game_states.py:452-494, ResNetConfig.input_channels = 19 in
    neural_networks/resnet_model.py:21), or 18 when the evaluator or its network says
    input_channels = 18."""
    for obj in (evaluator, getattr(evaluator, "model", None), getattr(evaluator, "network", None)):
        ch = getattr(obj, "input_channels", None)
        if ch is not None:
            if int(ch) not in (18, 19):
                raise ValueError(f"evaluator input_channels {ch}: feature planes are 18 or 19")
            return int(ch)
    return 19


class _BatchEvaluatorAdapter:
    """Runs a reference-protocol evaluator on the device-built features of the wave's unique
    leaves and writes its outputs into the engine's policy/value rows.  As in the reference
    driver (optimized_wave_search.py:312-365), the evaluator sees one row per leaf to evaluate:
    the unique leaves of tree 0, then of tree 1, and so on (no padding slots)."""

    def __init__(self, evaluator, builder):
        self.evaluator = evaluator
        self.builder = builder

    def evaluate_wave(self, engine) -> None:
        feats = self.builder.build()
        counts = engine.ucount.cpu()  # the leaf counts decide the batch (one small copy)
        MW = engine.MW
        if engine.T == 1:
            idx = None
            feats = feats[:int(counts[0])]
        else:
            idx = torch.cat([torch.arange(int(c), dtype=torch.int64) + t * MW
                             for t, c in enumerate(counts.tolist())]).to(engine.device)
            feats = feats.index_select(0, idx)
        if feats.shape[0] == 0:
            return
        pol, val = self.evaluator.evaluate_batch(feats)
        pol = torch.as_tensor(pol, device=engine.device, dtype=torch.float32).reshape(-1, engine.A)
        val = torch.as_tensor(val, device=engine.device, dtype=torch.float32).reshape(-1)
        if pol.shape[0] != feats.shape[0] or val.shape[0] != feats.shape[0]:
            raise ValueError(f"evaluate_batch returned {pol.shape[0]} policies and "
                             f"{val.shape[0]} values for {feats.shape[0]} positions")
        rows = engine.policy.view(-1, engine.A)
        if idx is None:
            rows[:pol.shape[0]].copy_(pol)
            engine.values[:val.shape[0]].copy_(val)
        else:
            rows.index_copy_(0, idx, pol)
            engine.values.index_copy_(0, idx, val)


class MCTS:
    """High-level MCTS over the HIP wave tree operations (GPU tree backend)."""

    def __init__(self, config: MCTSConfig, evaluator: Any, game_interface: Optional[Any] = None,
                 single_gpu_mode: bool = False):
        self.config = config
        self.evaluator = evaluator
        self.game_interface = game_interface
        self.single_gpu_mode = single_gpu_mode
        if config.backend != "gpu":
            raise NotImplementedError(
                f"backend '{config.backend}': this library implements the tree operations on the "
                "GPU (backend='gpu'); the reference's Cython CPU tree is not part of it")
        if game_interface is not None:
            gt = getattr(game_interface, "game_type", None)
            if gt is not None:
                name = getattr(gt, "name", str(gt)).upper()
                if name in GameType.__members__:
                    config.game_type = GameType[name]
            if getattr(game_interface, "board_size", None):
                config.board_size = int(game_interface.board_size)
        self.device = torch.device(config.device if config.device != "cuda" else "cuda:0")
        self.model = self._game_model(config)
        self.action_size = config.action_space_size()
        self.wave = config.effective_wave_size()
        if self.wave > _lib.OMQ_MAX_WAVE:
            raise ValueError(f"max_wave_size {self.wave} exceeds the library limit "
                             f"{_lib.OMQ_MAX_WAVE}")
        self.params = SearchParams(
            c_puct=float(config.c_puct), virtual_loss=config.effective_virtual_loss(),
            max_depth=int(config.max_depth),
            expand_policy=(_lib.OMQ_EXPAND_FULL if config.expansion_policy == "full"
                           else _lib.OMQ_EXPAND_REFERENCE_PW),
            sign_mode=(_lib.OMQ_SIGN_LEAF_POSITIVE if config.backup_sign == "leaf_positive"
                       else _lib.OMQ_SIGN_ROOT_POSITIVE),
            w_mode=(_lib.OMQ_WACC_ORDERED if config.w_accum == "ordered" else _lib.OMQ_WACC_ATOMIC),
            vl_atomic=bool(config.vl_atomic), dirichlet_epsilon=float(config.dirichlet_epsilon))
        self.engine = WaveEngine(self.model, config.num_trees, int(config.max_tree_nodes),
                                 self.wave, int(config.max_depth), self.device, self.params)
        self._roots_key: Optional[bytes] = None
        self._boards: Optional[torch.Tensor] = None
        self._eval = None
        self._graphs: dict = {}  # recorded searches by launch signature (use_cuda_graphs)
        self._search_count = 0
        self.last_selected_action = None
        self._initialize_statistics()

    # ---- setup ---------------------------------------------------------------------------
    @staticmethod
    def _game_model(config: MCTSConfig) -> games.GameModel:
        if config.game_type == GameType.GOMOKU:
            return games.gomoku(config.board_size)
        if config.game_type == GameType.GO:
            return games.go(config.board_size)
        lo, hi = config.sparse_legal
        return games.chess_sparse(config.action_space_size(), int(lo), int(hi))

    def _initialize_statistics(self):
        # mcts.py:783-796
        self.stats = {
            "total_searches": 0, "total_simulations": 0, "total_time": 0.0,
            "avg_sims_per_second": 0.0, "peak_sims_per_second": 0.0,
            "last_search_sims_per_second": 0.0, "tree_reuse_count": 0, "tree_reuse_nodes": 0,
        }
        self.stats_internal = defaultdict(float)

    @staticmethod
    def _is_state_object(state) -> bool:
        return hasattr(state, "get_basic_tensor_representation")

    def _state_to_numpy(self, state, representation_type: Optional[str] = None) -> np.ndarray:
        """GameInterface.state_to_numpy (python/mcts/core/game_interface.py:276-306): the game
        interface's when it has one, else the state's own representation methods, which is
        what the reference's interface calls ('basic' by default, 'minimal' for the
        3-channel form)."""
        gi = self.game_interface
        if gi is not None and hasattr(gi, "state_to_numpy"):
            if representation_type is None:
                return np.asarray(gi.state_to_numpy(state))
            return np.asarray(gi.state_to_numpy(state, representation_type=representation_type))
        if representation_type == "minimal":
            return np.asarray(state.get_tensor_representation())
        return np.asarray(state.get_basic_tensor_representation())

    def _board_of_state(self, state):
        """Board, player to move and move count of a game-state object, as
        MCTS._initialize_root reads them (python/mcts/core/mcts.py:1520-1600): a 3-channel
        observation holds player 1's and player 2's stones in channels 0 and 1; otherwise the
        3-channel 'minimal' form holds the mover's and the opponent's stones, mapped to
        colours by state.get_current_player().  The move count is the length of the state's
        move history."""
        bs = self.config.board_size
        obs = self._state_to_numpy(state)
        board = np.zeros((bs, bs), np.int8)
        player = int(state.get_current_player())
        if obs.shape[0] == 3:
            board[np.asarray(obs[0])[:bs, :bs] > 0.5] = 1
            board[np.asarray(obs[1])[:bs, :bs] > 0.5] = 2
        else:
            obs3 = self._state_to_numpy(state, "minimal")
            if obs3.shape[0] < 2:
                raise ValueError(f"state representation with {obs3.shape[0]} channels")
            board[np.asarray(obs3[0])[:bs, :bs] > 0.5] = player
            board[np.asarray(obs3[1])[:bs, :bs] > 0.5] = 3 - player
        if obs.shape[-2:] != (bs, bs):
            raise ValueError(f"Invalid state shape: {obs.shape}, expected board {(bs, bs)}")
        hist = state.get_move_history() if hasattr(state, "get_move_history") else None
        moves = int(np.count_nonzero(board)) if hist is None else len(hist)
        return board, player, moves

    def _root_states(self, states):
        """Root positions of the trees: (boards int8 [T, bs, bs], players, move counts), where
        players and move counts are None for ndarray boards (then player 1 moves when the
        stone count is even, and the move count is the stone count, as mcts.py:1503-1508).
        states: one [bs, bs] board per tree as an array, or game-state objects (one, or a
        sequence of one per tree) as the reference's callers pass them."""
        if states is None or not self.model.is_board:
            return None, None, None
        objs = None
        if self._is_state_object(states):
            objs = [states]
        elif isinstance(states, (list, tuple)) and states and all(
                self._is_state_object(s) for s in states):
            objs = list(states)
        self._root_go_host = None
        if objs is not None:
            conv = [self._board_of_state(s) for s in objs]
            boards = np.stack([c[0] for c in conv]).astype(np.int8)
            if self.model.kind == "go":
                self._root_go_host = self._go_state_info(objs)
            return (boards, np.array([c[1] for c in conv], np.int32),
                    np.array([c[2] for c in conv], np.int32))
        bs = self.config.board_size
        arr = np.asarray(states)
        if arr.shape[-2:] != (bs, bs):
            raise ValueError(f"Invalid state shape: {arr.shape}, expected {(bs, bs)}")
        return arr.reshape(-1, bs, bs).astype(np.int8), None, None

    def _go_state_info(self, objs):
        """(trailing passes, ko point) of Go state objects: the passes that end the state's
        move history, and get_ko_point() where the state has it (GoState::getKoPoint,
        include/games/go/go_state.h:192), else -1."""
        pass_action = self.action_size - 1
        passes, ko = [], []
        for st in objs:
            hist = list(st.get_move_history()) if hasattr(st, "get_move_history") else []
            n = 0
            while n < len(hist) and int(hist[-1 - n]) == pass_action:
                n += 1
            passes.append(n)
            ko.append(int(st.get_ko_point()) if hasattr(st, "get_ko_point") else -1)
        return np.array(passes, np.int32), np.array(ko, np.int32)

    def _go_flags(self) -> Optional[int]:
        if self.model.kind != "go" or self.config.go_rules == "off":
            return None
        flags = _lib.OMQ_GO_KO
        if self.config.go_rules == "ko_suicide":
            flags |= _lib.OMQ_GO_SUICIDE
        return flags

    def _states_array(self, states) -> Optional[np.ndarray]:
        return self._root_states(states)[0]

    @staticmethod
    def _roots_key_of(boards, players=None, moves=None) -> bytes:
        if boards is None:
            return b""
        key = np.ascontiguousarray(boards, np.int8).tobytes()
        for extra in (players, moves):
            key += b"|" + (b"" if extra is None else np.asarray(extra, np.int32).tobytes())
        return key

    def _go_key(self) -> bytes:
        info = getattr(self, "_root_go_host", None)
        if info is None or self._go_flags() is None:
            return b""
        return b"|go" + info[0].tobytes() + info[1].tobytes()

    def _set_roots(self, boards: Optional[np.ndarray], players=None, moves=None) -> None:
        T = self.engine.T
        if boards is not None and boards.shape[0] != T:
            raise ValueError(f"{boards.shape[0]} states given for {T} trees")
        key = self._roots_key_of(boards, players, moves) + self._go_key()
        if key == self._roots_key and self._eval is not None:
            return
        keys = games.root_keys(self.config.seed, T)
        legal = games.legal_masks(self.model, boards, T)
        self._install_roots(keys, legal, boards, players, moves)
        self.engine.reset()

    def _root_noise(self, keys: np.ndarray, legal: np.ndarray) -> Optional[np.ndarray]:
        if self.config.dirichlet_epsilon <= 0 or self.config.root_noise_source == "device":
            return None
        if self.model.is_board:
            counts = games.legal_counts(self.model, legal)
        else:
            counts = np.array([games.sparse_root_count(self.model, int(k)) for k in keys])
        return games.dirichlet_noise(self.model, counts, float(self.config.dirichlet_alpha),
                                     self.config.seed + 7919 * (self._search_count + 1))

    def _install_roots(self, keys: np.ndarray, legal: np.ndarray,
                       boards: Optional[np.ndarray], players=None, moves=None) -> None:
        """Root inputs of every tree on the device (keys, legal masks, noise, Gomoku boards,
        the player to move and move count of game-state roots) and the evaluator built on
        them; the tree arrays are left as they are."""
        T = self.engine.T
        go_flags = self._go_flags()
        if go_flags is not None:
            if boards is None:
                boards = np.zeros((T, self.config.board_size, self.config.board_size), np.int8)
            info = getattr(self, "_root_go_host", None)
            self._root_go_host = info if info is not None else (
                np.zeros(T, np.int32), np.full(T, -1, np.int32))
            legal = self._go_root_legal(boards, go_flags)
        self._root_keys_host = np.asarray(keys, dtype=np.uint64).copy()
        self._root_legal_host = np.asarray(legal, dtype=np.uint32).copy()
        self._root_boards_host = None if boards is None else np.asarray(boards, np.int8).copy()
        self._root_players_host = None if players is None else np.asarray(players, np.int32).copy()
        self._root_moves_host = None if moves is None else np.asarray(moves, np.int32).copy()
        self.engine.set_roots(keys, legal, self._root_noise(keys, legal))
        if self.config.dirichlet_epsilon > 0 and self.config.root_noise_source == "device":
            self.engine.device_root_noise(float(self.config.dirichlet_alpha), self.config.seed,
                                          self._search_count + 1)
        rule = self._gomoku_rule()
        if rule is not None:
            b = boards if boards is not None else np.zeros(
                (T, self.config.board_size, self.config.board_size), np.int8)
            self.engine.set_gomoku_rules(b, rule, root_player=players)
        if go_flags is not None:
            passes, ko = self._root_go_host
            self.engine.set_go_rules(boards, go_flags, root_player=players, root_passes=passes,
                                     root_ko=ko)
        self._roots_key = self._roots_key_of(boards, players, moves) + self._go_key()
        self._boards = None if boards is None else torch.from_numpy(
            np.ascontiguousarray(boards, np.int8)).to(self.device)
        self._eval = self._make_evaluator()

    def _go_root_legal(self, boards: np.ndarray, flags: int) -> np.ndarray:
        """Root legal masks under the Go rules: the empty points and the pass, without the
        root's ko point (OMQ_GO_KO) and the points with no empty orthogonal neighbour
        (OMQ_GO_SUICIDE), so that the root's Dirichlet noise has one entry per legal move."""
        T = boards.shape[0]
        legal = games.legal_masks(self.model, boards, T)
        ko = self._root_go_host[1]
        empty = boards == 0
        closed = np.zeros_like(empty)
        if flags & _lib.OMQ_GO_SUICIDE:
            pad = np.zeros((T, boards.shape[1] + 2, boards.shape[2] + 2), bool)
            pad[:, 1:-1, 1:-1] = empty
            open_nb = pad[:, :-2, 1:-1] | pad[:, 2:, 1:-1] | pad[:, 1:-1, :-2] | pad[:, 1:-1, 2:]
            closed = empty & ~open_nb
        for t in range(T):
            drop = np.flatnonzero(closed[t].reshape(-1)).tolist()
            if flags & _lib.OMQ_GO_KO and 0 <= int(ko[t]) < empty[t].size:
                drop.append(int(ko[t]))
            for a in drop:
                legal[t, a // 32] &= np.uint32(~(1 << (a % 32)) & 0xFFFFFFFF)
        return legal

    def _gomoku_rule(self) -> Optional[int]:
        """Terminal rule of Gomoku leaves: the config's, renju when the game interface says
        use_renju (fast_terminal_check.py:34-40 reads it there); None for other games."""
        if self.model.kind != "gomoku" or self.config.gomoku_rules == "off":
            return None
        if self.config.gomoku_rules == "renju" or getattr(self.game_interface, "use_renju", False):
            return _lib.OMQ_RULE_RENJU
        return _lib.OMQ_RULE_FREESTYLE

    def _make_evaluator(self):
        if getattr(self.evaluator, "device_native", False) or hasattr(self.evaluator, "evaluate_wave"):
            return self.evaluator
        if not hasattr(self.evaluator, "evaluate_batch"):
            raise TypeError("evaluator must provide evaluate_wave(engine) or evaluate_batch(states)")
        if not self.model.is_board:
            raise NotImplementedError("feature-plane evaluators need a board game model")
        from .features import LeafFeatureBuilder
        planes = _input_planes(self.evaluator)
        boards = self._boards
        if boards is None:
            boards = torch.zeros((self.engine.T, self.config.board_size, self.config.board_size),
                                 dtype=torch.int8, device=self.device)
        return _BatchEvaluatorAdapter(self.evaluator, LeafFeatureBuilder(
            self.engine, boards, planes, root_player=self._root_players_host,
            root_moves=self._root_moves_host))

    # ---- search --------------------------------------------------------------------------
    def search(self, state: Any, num_simulations: Optional[int] = None) -> np.ndarray:
        """Run the search from `state`; returns the root visit distribution [action_size]."""
        if self.engine.T != 1:
            raise ValueError("search() drives one tree; use search_batch() with num_trees > 1")
        if state is None or self._is_state_object(state):
            return self.search_batch(state, num_simulations)[0]
        arr = np.asarray(state)
        bs = self.config.board_size
        if self.model.is_board and arr.shape != (bs, bs):  # mcts.py:935-938
            raise ValueError(f"Invalid state shape: {arr.shape}, expected {(bs, bs)}")
        return self.search_batch(arr[None], num_simulations)[0]

    def search_batch(self, states: Any, num_simulations: Optional[int] = None) -> np.ndarray:
        """Search num_trees independent trees together; returns [num_trees, action_size].
        states: [num_trees, bs, bs] boards, or game-state objects (one per tree)."""
        boards, players, moves = self._root_states(states)
        # mcts.py:940: 0 or None runs the configured count
        num_sims = int(num_simulations or self.config.num_simulations)
        start = time.perf_counter()
        if not self.config.enable_subtree_reuse:
            self._roots_key = None
        self._set_roots(boards, players, moves)
        self.engine.clear_status()
        if num_sims == 0:  # mcts.py:1022-1030 (a configured count of 0)
            return np.full((self.engine.T, self.action_size), 1.0 / self.action_size)
        eng = self.engine
        fresh = int(eng.nchild[0].item()) == 0 and int(eng.num_nodes[0].item()) == 1
        key = self._graph_key(num_sims, fresh)
        if key is not None:
            self._graph_waves(key, num_sims, fresh)
        else:
            self._waves(num_sims, fresh, check_first=True)
        eng.check_status()
        policy = eng.root_policies()
        elapsed = time.perf_counter() - start
        self._search_count += 1
        self._update_statistics(num_sims * eng.T, elapsed)
        return policy

    def _waves(self, num_sims: int, fresh: bool, check_first: bool = False) -> None:
        """The search's waves: the root expansion of a lone root (its own backup), then waves
        of min(wave, remaining) simulations."""
        eng = self.engine
        if fresh:
            eng.run_wave(1, self._eval)
        done = 0
        while done < num_sims:
            w = min(self.wave, num_sims - done)
            eng.run_wave(w, self._eval)
            done += w
            if check_first and done == w:
                eng.check_status()  # (a device error stops the search after its first wave)

    def _graph_key(self, num_sims: int, fresh: bool):
        """Launch signature of this search's waves when they can be recorded as a HIP graph
        (config.use_cuda_graphs, as the reference's flag of that name, mcts_config.py:96, and
        an evaluator that launches device work only and says so with graph_key()); None
        otherwise."""
        gk = getattr(self._eval, "graph_key", None)
        if not self.config.use_cuda_graphs or gk is None or self.device.type != "cuda":
            return None
        return (num_sims, self.wave, fresh, self.engine.launch_signature(), gk())

    def _graph_waves(self, key, num_sims: int, fresh: bool) -> None:
        """The waves as one graph launch.  The first search of a signature runs eagerly (on a
        side stream, which also sets every kernel attribute) and is then recorded; later ones
        replay the recording, which reads the roots and trees from the same buffers."""
        g = self._graphs.get(key)
        if g is not None:
            g.replay()
            return
        cur = torch.cuda.current_stream(self.device)
        side = torch.cuda.Stream(self.device)
        side.wait_stream(cur)
        with torch.cuda.stream(side):
            self._waves(num_sims, fresh, check_first=True)
        cur.wait_stream(side)
        torch.cuda.synchronize(self.device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._waves(num_sims, fresh)
        if len(self._graphs) >= 8:
            self._graphs.pop(next(iter(self._graphs)))
        self._graphs[key] = g

    def _update_statistics(self, num_simulations: int, elapsed_time: float):
        # mcts.py:1442-1456
        self.stats["total_searches"] += 1
        self.stats["total_simulations"] += num_simulations
        self.stats["total_time"] += elapsed_time
        sps = num_simulations / elapsed_time if elapsed_time > 0 else 0
        self.stats["last_search_sims_per_second"] = sps
        self.stats["peak_sims_per_second"] = max(self.stats["peak_sims_per_second"], sps)
        tt = self.stats["total_time"]
        self.stats["avg_sims_per_second"] = self.stats["total_simulations"] / tt if tt > 0 else 0

    # ---- actions and root ----------------------------------------------------------------
    def select_action(self, state: Any, temperature: float = 1.0,
                      policy: Optional[np.ndarray] = None) -> int:
        """mcts.py:1167-1203: temperature 0 takes the first maximum; otherwise samples
        policy^(1/T)."""
        if policy is None:
            policy = self.search(state)
        if temperature == 0:
            action = 0 if policy.max() == 0 else int(np.argmax(policy))
        else:
            p = np.power(policy, 1.0 / temperature)
            p /= p.sum()
            action = int(np.random.choice(len(policy), p=p))
        self.last_selected_action = action
        return action

    def select_actions(self, temperature: float = 1.0, seed: Optional[int] = None) -> np.ndarray:
        """One move per tree from the current root policies, on the device
        (omq_sample_actions): temperature 0 takes the first maximum, as select_action does;
        otherwise each tree draws from p^(1/temperature) with a counter-based stream keyed by
        the seed and a per-call counter (in place of numpy's global generator)."""
        self._sample_count = getattr(self, "_sample_count", 0) + 1
        return self.engine.sample_actions(temperature,
                                          self.config.seed if seed is None else seed,
                                          self._sample_count)

    def update_root(self, action: int, new_state: Any = None) -> None:
        """mcts.py:1205-1245.  Validates the action, then reuses the subtree of the root's
        child for `action` when enable_subtree_reuse is set and that child has at least
        subtree_reuse_min_visits visits (default 10; tree_operations.py:53-133).  Otherwise
        the tree is reset (_efficient_tree_reset) and the new state, if given, becomes the
        root."""
        if self.engine.T != 1:
            raise ValueError("update_root() drives one tree; use update_roots() with num_trees > 1")
        if new_state is not None and not self._is_state_object(new_state):
            new_state = np.asarray(new_state)[None]
        self.update_roots([action], new_state)

    def update_roots(self, actions, new_states: Any = None) -> bool:
        """update_root for every tree at once (actions[t] played in tree t).  Returns whether
        the subtrees were reused (all trees or none)."""
        actions = [int(a) for a in np.asarray(actions).reshape(-1)]
        if len(actions) != self.engine.T:
            raise ValueError(f"{len(actions)} actions for {self.engine.T} trees")
        for a in actions:
            if a < 0 or a >= self.action_size:
                raise ValueError(f"Invalid action {a}. Must be in range [0, {self.action_size})")
        boards, players, moves = self._root_states(new_states)
        if self.config.enable_subtree_reuse and self._roots_key is not None:
            kept = self._reuse_subtrees(actions, boards, players, moves)
            if kept is not None:
                self.stats["tree_reuse_count"] += 1
                self.stats["tree_reuse_nodes"] += kept
                return True
        self._roots_key = None
        self.engine.reset()
        if boards is not None:
            self._set_roots(boards, players, moves)
        return False

    def _reuse_subtrees(self, actions, boards: Optional[np.ndarray], players=None,
                        moves=None) -> Optional[int]:
        """Shift every tree's root to its child for actions[t] (CSRTree.shift_root on the
        device).  None, with nothing changed, when some tree lacks that child or the child has
        fewer than subtree_reuse_min_visits visits."""
        eng = self.engine
        T, cap = eng.T, eng.cap
        min_visits = int(self.config.extra.get("subtree_reuse_min_visits", 10))
        roots = torch.arange(T, device=eng.device, dtype=torch.int64) * cap
        first = eng.first[roots].cpu().numpy()
        k = eng.nchild[roots].cpu().numpy()
        new_roots = np.full(T, -1, np.int32)
        for t, a in enumerate(actions):
            if k[t] <= 0:
                return None
            lo = t * cap + int(first[t]) + 1
            acts = eng.action[lo:lo + int(k[t])].cpu().numpy()
            hit = np.flatnonzero(acts == a)
            if hit.size == 0:
                return None
            node = int(first[t]) + 1 + int(hit[0])
            if int(eng.N[t * cap + node].item()) < min_visits:
                return None
            new_roots[t] = node
        eng.shift_roots(new_roots)
        keys = np.array([games.child_key(int(key), a)
                         for key, a in zip(self._root_keys_host, actions)], np.uint64)
        legal = self._root_legal_host.copy()
        if self.model.is_board:
            pass_action = self.action_size - 1 if self.model.kind == "go" else -1
            for t, a in enumerate(actions):
                if a != pass_action:  # Go's pass stays legal
                    legal[t, a // 32] &= np.uint32(~(1 << (a % 32)) & 0xFFFFFFFF)
            if boards is None:
                prev = self._root_boards_host
                if prev is None:
                    bs = self.config.board_size
                    prev = np.zeros((T, bs, bs), np.int8)
                boards = prev.copy()
                pp, pm = self._root_players_host, self._root_moves_host
                for t, a in enumerate(actions):
                    flat = boards[t].reshape(-1)
                    mover = (int(pp[t]) if pp is not None
                             else (1 if int((boards[t] != 0).sum()) % 2 == 0 else 2))
                    if a < flat.size:  # Go's pass occupies no cell
                        flat[a] = mover
                # a game-state root keeps its own player and move count: the opponent moves next
                players = None if pp is None else (3 - pp).astype(np.int32)
                moves = None if pm is None else (pm + 1).astype(np.int32)
                # Go: a pass adds to the root's trailing passes, a stone ends them; no capture
                # is modelled, so no new ko point arises
                info = getattr(self, "_root_go_host", None)
                if self.model.kind == "go" and info is not None:
                    pass_action = self.action_size - 1
                    self._root_go_host = (
                        np.array([int(info[0][t]) + 1 if a == pass_action else 0
                                  for t, a in enumerate(actions)], np.int32),
                        np.full(T, -1, np.int32))
        self._install_roots(keys, legal, boards, players, moves)
        return int(eng.num_nodes.sum().item())

    def update_with_move(self, move: int) -> None:
        self.update_root(move, None)

    def get_root_value(self) -> float:
        """Q of the root, W/N (mcts.py:1139-1165, GPU tree branch)."""
        n = int(self.engine.N[0].item())
        return float(self.engine.W[0].item()) / n if n > 0 else 0.0

    def clear(self) -> None:
        self._roots_key = None
        self.engine.reset()

    def reset_tree(self) -> None:
        self.clear()

    def get_statistics(self) -> Dict[str, Any]:
        st = dict(self.stats)
        n = int(self.engine.num_nodes[0].item())
        st.update({"num_nodes": n, "root_visits": int(self.engine.N[0].item()),
                   "root_children": int(self.engine.nchild[0].item())})
        st.update({f"op_{k}": v for k, v in self.engine.host_stats().items()})
        st.update(self.stats_internal)
        return st

    def warmup(self, state: Any = None, num_simulations: int = 100) -> None:
        if state is None and self.model.is_board:
            state = np.zeros((self.config.board_size, self.config.board_size), dtype=np.int8)
        if self.engine.T == 1:
            self.search(state, num_simulations)
        else:
            self.search_batch(None if state is None else np.repeat(np.asarray(state)[None],
                                                                   self.engine.T, 0),
                              num_simulations)
        self.clear()

    def shutdown(self) -> None:
        self.clear()

    def __enter__(self):
        return self

    def __exit__(self, exc_type, exc_val, exc_tb):
        self.shutdown()
        return False
