"""Device-resident forest of CSR trees and the per-wave driver over the HIP library.

All tree arrays and wave buffers are torch tensors on one HIP device, allocated once at
capacity (no growth inside a search).  Every operation is launched through the C ABI of
libomq_tree_ops.so on torch's current stream of that device; nothing synchronises inside a
wave.  The wave loop follows the reference driver (python/mcts/core/mcts.py:1020-1063,
python/mcts/cpu/optimized_wave_search.py:153-177): select -> evaluate unique leaves ->
expand -> backup.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from .. import _lib
from ..synthetic.games import GameModel


@dataclass
class SearchParams:
    c_puct: float = 1.414
    virtual_loss: float = 3.0
    max_depth: int = 100
    expand_policy: int = _lib.OMQ_EXPAND_FULL
    sign_mode: int = _lib.OMQ_SIGN_LEAF_POSITIVE
    w_mode: int = _lib.OMQ_WACC_ORDERED
    vl_atomic: bool = False
    dirichlet_epsilon: float = 0.0


def _u64_to_i64(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint64).view(np.int64)


class WaveEngine:
    """T independent trees of one game model, sharing wave buffers of max_wave simulations."""

    def __init__(self, model: GameModel, num_trees: int, capacity: int, max_wave: int,
                 max_depth: int = 100, device: str | torch.device = "cuda",
                 params: SearchParams | None = None):
        self.lib = _lib.load()
        if not torch.cuda.is_available():
            raise RuntimeError("WaveEngine needs a HIP device (torch.cuda.is_available() is False)")
        if max_wave > _lib.OMQ_MAX_WAVE or max_depth > _lib.OMQ_MAX_DEPTH:
            raise ValueError(f"max_wave {max_wave} / max_depth {max_depth} beyond the library "
                             f"limits {_lib.OMQ_MAX_WAVE} / {_lib.OMQ_MAX_DEPTH}")
        self.model = model
        self.T = int(num_trees)
        self.cap = int(capacity)
        self.MW = int(max_wave)
        self.MD = int(max_depth)
        self.A = model.num_actions
        self.device = torch.device(device)
        self.params = params or SearchParams()
        dev = self.device
        T, cap, MW, MD, A = self.T, self.cap, self.MW, self.MD, self.A
        i32, f32, i64 = torch.int32, torch.float32, torch.int64

        def z(n, dt):
            return torch.zeros(n, dtype=dt, device=dev)

        # tree arrays
        self.N = z(T * cap, i32)
        self.W = z(T * cap, f32)
        self.P = z(T * cap, f32)
        self.parent = z(T * cap, i32)
        self.first = z(T * cap, i32)
        self.nchild = z(T * cap, i32)
        self.action = z(T * cap, i32)
        self.num_nodes = z(T, i32)
        self.root_keys = z(T, i64)
        self.root_legal = z(T * model.legal_words, i32)
        # wave buffers
        self.paths = z(T * MW * MD, i32)
        self.path_len = z(T * MW, i32)
        self.leaves = z(T * MW, i32)
        self.sim_uid = z(T * MW, i32)
        self.uleaf = z(T * MW, i32)
        self.ufirst = z(T * MW, i32)
        self.ucount = z(T, i32)
        self.glog = z(T * MW * MD * 4, i32)
        self.gcount = z(T, i32)
        self.gmembers = z(T * MD * MW, torch.int16)
        self.ukey = z(T * MW, i64)
        self.ulegal = z(T * MW, i32)
        self.uedge = z(T * MW, i32)
        self.unew = z(T * MW, i32)
        self.policy = z(T * MW * A, f32)
        self.values = z(T * MW, f32)
        self.sim_value = z(T * MW, f32)
        self.stats = z(T * _lib.OMQ_NSTATS, i64)
        self.status = z(4, i32)
        self.sel_scratch = z(_lib.sel_scratch_ints(T, MW), i32)
        self.noise = z(T * A, torch.float64)
        self.has_noise = False
        # Gomoku rules (terminal leaves are not expanded), off until set_gomoku_rules
        self.uterm = z(T * MW, i32)
        self.rule: int | None = None
        self.root_boards: torch.Tensor | None = None
        self.root_player: torch.Tensor | None = None
        # Go rules (legal masks per unique leaf, terminal leaves), off until set_go_rules
        self.go_flags: int | None = None
        self.umask: torch.Tensor | None = None
        self.root_passes: torch.Tensor | None = None
        self.root_ko: torch.Tensor | None = None
        self._shift_ws: torch.Tensor | None = None  # subtree-reuse workspace, made on first use
        self._policy: torch.Tensor | None = None    # root policies [T, A] float64

        f = _lib.OmqForest()
        f.num_trees, f.capacity, f.num_actions, f.game = T, cap, A, model.code
        f.legal_words = model.legal_words
        f.min_legal, f.max_legal = model.min_legal, model.max_legal
        for name, t in (("visit_counts", self.N), ("value_sums", self.W), ("priors", self.P),
                        ("parents", self.parent), ("first_child", self.first),
                        ("num_children", self.nchild), ("actions", self.action),
                        ("num_nodes", self.num_nodes), ("root_keys", self.root_keys),
                        ("root_legal", self.root_legal)):
            setattr(f, name, t.data_ptr())
        w = _lib.OmqWave()
        w.max_wave, w.max_depth = MW, MD
        for name in ("paths", "path_len", "leaves", "sim_uid", "uleaf", "ufirst", "ucount",
                     "glog", "gcount", "gmembers", "ukey", "ulegal", "uedge", "unew", "policy",
                     "values", "sim_value", "stats", "status", "sel_scratch"):
            setattr(w, name, getattr(self, name).data_ptr())
        self.forest = f
        self.wave = w
        self.forest_ref = ctypes.byref(self.forest)
        self.wave_ref = ctypes.byref(self.wave)

    # ---- plumbing ---------------------------------------------------------------------
    def stream_handle(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def set_roots(self, keys: np.ndarray, legal: np.ndarray | None = None,
                  noise: np.ndarray | None = None) -> None:
        """Root keys uint64[T], root legal masks uint32[T, legal_words], noise float64[T, A]."""
        self.root_keys.copy_(torch.from_numpy(_u64_to_i64(keys)))
        if legal is not None:
            lw = np.ascontiguousarray(legal, dtype=np.uint32).reshape(-1).view(np.int32)
            self.root_legal.copy_(torch.from_numpy(lw.copy()))
        self.has_noise = noise is not None
        if noise is not None:
            self.noise.copy_(torch.from_numpy(np.ascontiguousarray(noise, dtype=np.float64).reshape(-1)))

    def set_gomoku_rules(self, boards, rule: int = _lib.OMQ_RULE_FREESTYLE,
                         root_player=None) -> None:
        """Turn on the Gomoku terminal check of every wave's leaves.  boards: int8 [T, bs, bs]
        root positions (0 empty, 1/2 stones); root_player: [T] player of the first path move
        (default: 1 for an even stone count, else 2).  boards=None turns the check off."""
        if boards is None:
            self.rule, self.root_boards, self.root_player = None, None, None
            return
        if self.model.kind != "gomoku":
            raise ValueError("the Gomoku terminal rule needs a gomoku game model")
        b = torch.as_tensor(np.ascontiguousarray(boards, dtype=np.int8)).reshape(-1)
        if b.numel() != self.T * self.A:
            raise ValueError(f"boards hold {b.numel()} cells, expected {self.T} x {self.A}")
        self.root_boards = self._reuse(self.root_boards, b)
        rp = None
        if root_player is not None:
            rp = torch.as_tensor(np.ascontiguousarray(root_player, dtype=np.int32)).reshape(-1)
            if rp.numel() != self.T:
                raise ValueError("one root player per tree")
        self.root_player = None if rp is None else self._reuse(self.root_player, rp)
        self.rule = int(rule)

    def _reuse(self, cur: torch.Tensor | None, x: torch.Tensor) -> torch.Tensor:
        """x on the device, in cur's storage when cur has its size and type: root inputs keep
        their addresses from one position to the next, so that a recorded search (whose
        kernels hold those addresses) stays valid."""
        if cur is not None and cur.numel() == x.numel() and cur.dtype == x.dtype:
            cur.copy_(x)
            return cur
        return x.to(self.device)

    def set_go_rules(self, boards, flags: int = _lib.OMQ_GO_KO, root_player=None,
                     root_passes=None, root_ko=None) -> None:
        """Turn on the Go rules of every wave's leaves (omq_go_rules): legal moves from the leaf
        position (the root's ko point excluded in the whole tree with OMQ_GO_KO, points without
        an empty neighbour with OMQ_GO_SUICIDE), leaves after two consecutive passes or without
        an empty point terminal.  boards: int8 [T, bs, bs] root positions; root_player,
        root_passes (the root's trailing passes) and root_ko (a point or -1): optional [T].
        boards=None turns them off."""
        if boards is None:
            self.go_flags = None
            self.root_passes = self.root_ko = None
            self.wave.umask = None
            if self.rule is None:
                self.root_boards = self.root_player = None
            return
        if self.model.kind != "go":
            raise ValueError("the Go rules need a go game model")
        cells = self.A - 1
        b = torch.as_tensor(np.ascontiguousarray(boards, dtype=np.int8)).reshape(-1)
        if b.numel() != self.T * cells:
            raise ValueError(f"boards hold {b.numel()} points, expected {self.T} x {cells}")

        def per_tree(cur, x, name):
            if x is None:
                return None
            v = torch.as_tensor(np.ascontiguousarray(x, dtype=np.int32)).reshape(-1)
            if v.numel() != self.T:
                raise ValueError(f"one {name} per tree")
            return self._reuse(cur, v)

        self.root_boards = self._reuse(self.root_boards, b)
        self.root_player = per_tree(self.root_player, root_player, "root player")
        self.root_passes = per_tree(self.root_passes, root_passes, "root pass count")
        self.root_ko = per_tree(self.root_ko, root_ko, "ko point")
        if self.umask is None:
            self.umask = torch.zeros(self.T * self.MW * self.model.legal_words,
                                     dtype=torch.int32, device=self.device)
        self.wave.umask = self.umask.data_ptr()
        self.go_flags = int(flags)

    def _check(self, rc: int, what: str) -> None:
        _lib.check(rc, what)

    # ---- operations -------------------------------------------------------------------
    def reset(self) -> None:
        """Every tree back to a lone root; the device status flags are cleared too."""
        self._check(self.lib.omq_forest_reset(self.forest_ref, self.stream_handle()),
                    "omq_forest_reset")
        self.clear_status()

    def clear_status(self) -> None:
        """Zero the device status flags (the library sets bits and never clears them)."""
        self.status.zero_()

    def select(self, wave_size: int) -> None:
        p = self.params
        self._check(self.lib.omq_select(self.forest_ref, self.wave_ref, wave_size, p.c_puct,
                                        p.virtual_loss, p.max_depth, int(p.vl_atomic),
                                        self.stream_handle()), "omq_select")

    def needs_leaf_info(self, wave_size: int) -> bool:
        """Whether a wave of wave_size simulations needs leaf_info before its evaluation: its
        leaves' keys and legal counts are not formed by select, or a rule is on."""
        return (wave_size > _lib.OMQ_SELECT_RECORDS_MAX_WAVE or self.rule is not None
                or self.go_flags is not None)

    def leaf_info(self, wave_size: int) -> None:
        """The unique leaves' keys and legal counts, where select did not form them (waves of
        more than OMQ_SELECT_RECORDS_MAX_WAVE simulations), then the rule checks (the Gomoku
        terminal check: terminal leaves get no legal action, so they are not expanded; the Go
        rules' legal masks)."""
        if wave_size > _lib.OMQ_SELECT_RECORDS_MAX_WAVE:
            self._check(self.lib.omq_leaf_info(self.forest_ref, self.wave_ref,
                                               self.stream_handle()), "omq_leaf_info")
        if self.rule is not None:
            self.leaf_info_terminal_only()
        if self.go_flags is not None:
            ptr = lambda x: None if x is None else x.data_ptr()  # noqa: E731
            self._check(self.lib.omq_go_rules(
                self.forest_ref, self.wave_ref, self.root_boards.data_ptr(), ptr(self.root_player),
                ptr(self.root_passes), ptr(self.root_ko), self.go_flags, self.uterm.data_ptr(),
                self.stream_handle()), "omq_go_rules")

    def leaf_info_terminal_only(self) -> None:
        """The Gomoku terminal check alone, over the unique leaves already looked up."""
        if self.rule is not None:
            self._check(self.lib.omq_gomoku_terminal(
                self.forest_ref, self.wave_ref, self.root_boards.data_ptr(),
                None if self.root_player is None else self.root_player.data_ptr(), self.rule,
                self.uterm.data_ptr(), self.stream_handle()), "omq_gomoku_terminal")

    def leaf_features(self, out: torch.Tensor, boards: torch.Tensor, planes: int = 18,
                      root_player: torch.Tensor | None = None,
                      root_moves: torch.Tensor | None = None, nhwc: bool = False) -> None:
        """Feature planes of every wave slot (omq_leaf_features) into out: float32 or bfloat16,
        T*max_wave*planes*A values on the engine's device; boards: int8 [T*A] root positions;
        root_player / root_moves: optional int32 [T]."""
        if out.dtype == torch.float32:
            dt = _lib.OMQ_DTYPE_F32
        elif out.dtype == torch.bfloat16:
            dt = _lib.OMQ_DTYPE_BF16
        else:
            raise ValueError(f"feature planes are float32 or bfloat16, not {out.dtype}")
        if out.numel() != self.T * self.MW * planes * self.A or not out.is_contiguous():
            raise ValueError("out must be a contiguous buffer of T*max_wave*planes*A values")
        for name, x, n, dty in (("boards", boards, self.T * self.A, torch.int8),
                                ("root_player", root_player, self.T, torch.int32),
                                ("root_moves", root_moves, self.T, torch.int32)):
            if x is not None and (x.dtype != dty or x.numel() != n or not x.is_contiguous()
                                  or x.device != out.device):
                raise ValueError(f"{name} must be contiguous {dty} [{n}] on {out.device}")
        self._check(self.lib.omq_leaf_features(
            self.forest_ref, self.wave_ref, boards.data_ptr(),
            None if root_player is None else root_player.data_ptr(),
            None if root_moves is None else root_moves.data_ptr(), planes, dt,
            _lib.OMQ_LAYOUT_NHWC if nhwc else _lib.OMQ_LAYOUT_NCHW, out.data_ptr(),
            self.stream_handle()), "omq_leaf_features")

    def expand(self, wave_size: int) -> None:
        p = self.params
        noise = self.noise.data_ptr() if (self.has_noise and p.dirichlet_epsilon > 0) else None
        self._check(self.lib.omq_expand(self.forest_ref, self.wave_ref, wave_size,
                                        p.virtual_loss, p.expand_policy, noise,
                                        p.dirichlet_epsilon, self.stream_handle()), "omq_expand")

    def backup(self, wave_size: int) -> None:
        p = self.params
        self._check(self.lib.omq_backup(self.forest_ref, self.wave_ref, wave_size, p.virtual_loss,
                                        p.sign_mode, p.w_mode, self.stream_handle()),
                    "omq_backup")

    def expand_backup(self, wave_size: int) -> None:
        """expand then backup (omq_expand_backup: their kernels side by side where the two
        cannot interfere, else one after the other)."""
        p = self.params
        noise = self.noise.data_ptr() if (self.has_noise and p.dirichlet_epsilon > 0) else None
        self._check(self.lib.omq_expand_backup(self.forest_ref, self.wave_ref, wave_size,
                                               p.virtual_loss, p.expand_policy, noise,
                                               p.dirichlet_epsilon, p.sign_mode, p.w_mode,
                                               self.stream_handle()), "omq_expand_backup")

    def shift_roots(self, new_roots) -> None:
        """Subtree reuse (CSRTree.shift_root): node new_roots[t] of tree t becomes its root
        and keeps its subtree, renumbered breadth-first; -1 (or 0) leaves a tree unchanged.
        Root keys, legal masks and boards are the caller's to update."""
        nr = np.ascontiguousarray(new_roots, dtype=np.int32).reshape(-1)
        if nr.size != self.T:
            raise ValueError(f"{nr.size} new roots for {self.T} trees")
        need = _lib.OMQ_SHIFT_WORKSPACE_PER_NODE * self.T * self.cap
        if self._shift_ws is None or self._shift_ws.numel() < need:
            self._shift_ws = torch.empty(need, dtype=torch.int32, device=self.device)
        d = torch.from_numpy(nr).to(self.device)
        self._check(self.lib.omq_shift_root(self.forest_ref, d.data_ptr(),
                                            self._shift_ws.data_ptr(), self._shift_ws.numel(),
                                            self.stream_handle()), "omq_shift_root")

    def _tree_of(self, tree_of, n: int):
        if tree_of is None:
            return None
        t = torch.as_tensor(tree_of, dtype=torch.int32, device=self.device).reshape(-1)
        if t.numel() != n:
            raise ValueError(f"tree_of has {t.numel()} entries for {n} rows")
        return t.contiguous()

    def apply_virtual_loss(self, nodes, tree_of=None, amount: int | None = None) -> None:
        """N[tree_of[i], nodes[i]] += amount (default: the virtual loss) for every listed
        node (csr_tree.py:759-763, mcts_kernels.cu batch_apply_virtual_loss)."""
        delta = int(self.params.virtual_loss) if amount is None else int(amount)
        self._virtual_loss(nodes, tree_of, delta)

    def remove_virtual_loss(self, nodes, tree_of=None, amount: int | None = None) -> None:
        delta = int(self.params.virtual_loss) if amount is None else int(amount)
        self._virtual_loss(nodes, tree_of, -delta)

    def _virtual_loss(self, nodes, tree_of, delta: int) -> None:
        n = torch.as_tensor(nodes, dtype=torch.int32, device=self.device).reshape(-1).contiguous()
        t = self._tree_of(tree_of, n.numel())
        self._check(self.lib.omq_virtual_loss(self.forest_ref, n.data_ptr(),
                                              None if t is None else t.data_ptr(), n.numel(),
                                              delta, self.stream_handle()), "omq_virtual_loss")

    def backup_paths(self, paths, path_lengths, values, tree_of=None) -> None:
        """Reference vectorized_backup over an explicit [B, D] path matrix (root first, -1
        padded): N[x] += 1 and W[x] += signed value along each path, float atomics
        (torch_custom_ops.py:27-55, mcts_kernels.cu vectorized_backup)."""
        p = torch.as_tensor(paths, dtype=torch.int32, device=self.device)
        if p.dim() != 2:
            raise ValueError("paths must be [batch, max_depth]")
        B, D = p.shape
        p = p.contiguous()
        L = torch.as_tensor(path_lengths, dtype=torch.int32, device=self.device).reshape(-1).contiguous()
        v = torch.as_tensor(values, dtype=torch.float32, device=self.device).reshape(-1).contiguous()
        if L.numel() != B or v.numel() != B:
            raise ValueError("path_lengths and values need one entry per path")
        t = self._tree_of(tree_of, B)
        self._check(self.lib.omq_paths_backup(self.forest_ref, p.data_ptr(), L.data_ptr(),
                                              None if t is None else t.data_ptr(), v.data_ptr(),
                                              B, D, self.params.sign_mode, self.stream_handle()),
                    "omq_paths_backup")

    def run_wave(self, wave_size: int, evaluator, timer=None) -> None:
        """One wave in every tree: select, leaf info, evaluate, then expand and backup in one
        call (omq_expand_backup).  With a PhaseTimer, every phase is bracketed by events on the
        launch stream (expand and backup are one phase, "expand_backup")."""
        mark = timer.mark if timer is not None else (lambda _p: None)
        mark("select")
        self.select(wave_size)
        if self.needs_leaf_info(wave_size):
            mark("leaf_info")
            self.leaf_info(wave_size)
        mark("eval")
        evaluator.evaluate_wave(self)
        mark("expand_backup")
        self.expand_backup(wave_size)
        mark(None)

    def launch_signature(self) -> tuple:
        """Everything on the host side that a wave's launches take as arguments besides the
        wave size: search parameters, noise on or off, the addresses of the rule inputs and
        the library's process-wide spin limit (omq_select_options).  Two searches with the
        same signature and wave sizes launch the same kernels with the same arguments (the
        tree, wave and root buffers keep their addresses)."""
        ptr = lambda x: 0 if x is None else x.data_ptr()  # noqa: E731
        p = self.params
        return (p.c_puct, p.virtual_loss, p.max_depth, p.expand_policy, p.sign_mode, p.w_mode,
                p.vl_atomic, p.dirichlet_epsilon, self.has_noise, self.rule, self.go_flags,
                ptr(self.root_boards), ptr(self.root_player), ptr(self.root_passes),
                ptr(self.root_ko), int(self.wave.umask or 0),
                int(self.lib.omq_select_spin_limit()))

    def search(self, num_simulations: int, wave_size: int, evaluator, timer=None) -> None:
        """MCTS.search on every tree: reset, root expansion (one-simulation wave on the lone
        root; mcts.py:1659-1691), then waves of min(wave_size, remaining) simulations."""
        if wave_size > self.MW:
            raise ValueError(f"wave_size {wave_size} > max_wave {self.MW}")
        self.reset()
        self.run_wave(1, evaluator, timer)
        done = 0
        while done < num_simulations:
            w = min(wave_size, num_simulations - done)
            self.run_wave(w, evaluator, timer)
            done += w

    def capture_search(self, num_simulations: int, wave_size: int, evaluator):
        """Record one whole search (reset, root expansion, every wave) as a HIP graph; each
        g.replay() then runs it again with one launch from the host.  The evaluator must be
        device-native and free of host synchronisation (the synthetic evaluator is).  The
        search is run once eagerly first, on the capture's side stream, so that every kernel
        attribute is set before recording."""
        import torch

        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            self.search(num_simulations, wave_size, evaluator)
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.search(num_simulations, wave_size, evaluator)
        torch.cuda.synchronize(self.device)
        return g

    # ---- results ----------------------------------------------------------------------
    def check_status(self) -> None:
        st = int(self.status[0].item())
        if st & _lib.OMQ_STATUS_STALL:
            raise _lib.OmqError("omq_select: a bounded wait ran out; the selection is incomplete")
        if st & _lib.OMQ_STATUS_ROWLIMIT:
            raise _lib.OmqError(f"a node has more than {_lib.OMQ_MAX_ROW} legal actions; "
                                "its expansion was refused by the library")
        if st & _lib.OMQ_STATUS_COUNTLIMIT:
            raise _lib.OmqError("a root's visit count plus the wave's virtual loss reached 2^24; "
                                "the selection's float visit counts are exact only below it")

    def root_policies(self, device: bool = False):
        """pi[t, a] = N(child_a) / sum N over the root's children (mcts.py:1069-1137): uniform
        over the children's actions when they have no visits, uniform over the action space
        for a root without children.  float64 [T, A], as numpy (or the device tensor)."""
        if self._policy is None:
            self._policy = torch.empty((self.T, self.A), dtype=torch.float64, device=self.device)
        self._check(self.lib.omq_root_policy(self.forest_ref, self._policy.data_ptr(),
                                             self.stream_handle()), "omq_root_policy")
        return self._policy if device else self._policy.cpu().numpy()

    def sample_actions(self, temperature: float, seed: int, counter: int) -> np.ndarray:
        """One move per tree from the root policies (MCTS.select_action): the first maximum at
        temperature 0, else a draw from p^(1/T) keyed by (seed, counter, tree)."""
        pol = self.root_policies(device=True)
        out = torch.empty(self.T, dtype=torch.int32, device=self.device)
        self._check(self.lib.omq_sample_actions(self.forest_ref, pol.data_ptr(), float(temperature),
                                                int(seed) & (2**64 - 1), int(counter) & (2**64 - 1),
                                                out.data_ptr(), self.stream_handle()),
                    "omq_sample_actions")
        return out.cpu().numpy()

    def device_root_noise(self, alpha: float, seed: int, counter: int) -> None:
        """Root Dirichlet noise drawn on the device into the noise rows that omq_expand mixes at
        root expansion (entry i of row t: i-th legal root action)."""
        self._check(self.lib.omq_root_dirichlet(self.forest_ref, float(alpha),
                                                int(seed) & (2**64 - 1), int(counter) & (2**64 - 1),
                                                self.noise.data_ptr(), self.stream_handle()),
                    "omq_root_dirichlet")
        self.has_noise = True

    def host_tree(self, t: int) -> dict:
        """Copy of tree t's used prefix (tests and debugging)."""
        n = int(self.num_nodes[t].item())
        b = t * self.cap
        out = {}
        for name in ("N", "W", "P", "parent", "first", "nchild", "action"):
            out[name] = getattr(self, name)[b:b + n].cpu().numpy()
        out["num_nodes"] = n
        return out

    def host_stats(self) -> dict:
        st = self.stats.view(self.T, _lib.OMQ_NSTATS).sum(dim=0).cpu().numpy()
        return {name: int(st[i]) for i, name in enumerate(_lib.STAT_NAMES)}
