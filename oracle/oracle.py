"""ctypes wrapper of the C oracle (oracle/tree_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker; never by the product package.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(_HERE, "tree_oracle.c")
LIB = os.path.join(_HERE, "liborc.so")
CFLAGS = ["-O3", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-shared",
          "-Wall", "-Wextra"]

GAME_CODES = {"gomoku": 0, "go": 1, "sparse": 2}


def build(out: str = LIB) -> str:
    tmp = out + ".tmp"
    cmd = ["gcc", *CFLAGS, "-o", tmp, SRC, "-lm", "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, out)
    return out


_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB) or os.path.getmtime(LIB) < os.path.getmtime(SRC):
        build()
    lib = ctypes.CDLL(LIB)
    P = ctypes.c_void_p
    i, fl, d = ctypes.c_int, ctypes.c_float, ctypes.c_double
    u64 = ctypes.c_uint64
    sig = {
        "orc_create": (P, [i, i, i, i, i, i, i, i]),
        "orc_destroy": (None, [P]),
        "orc_set_params": (None, [P, fl, fl, i, i, fl, d]),
        "orc_set_roots": (None, [P, P, P, P]),
        "orc_reset_tree": (None, [P, i]),
        "orc_best_child": (i, [P, i, i]),
        "orc_wave_select": (None, [P, i, i, i]),
        "orc_wave_evaluate": (None, [P, i]),
        "orc_wave_expand": (None, [P, i, i]),
        "orc_wave_backup": (None, [P, i, i]),
        "orc_wave": (None, [P, i, i, i, P, P]),
        "orc_search_tree": (None, [P, i, i, i, i]),
        "orc_search": (i, [P, i, i, i, i]),
        "orc_splitmix64": (u64, [u64]),
        "orc_child_key": (u64, [u64, i]),
        "orc_key_value": (fl, [u64]),
        "orc_key_normal": (fl, [u64, i]),
        "orc_exp_cw": (fl, [fl]),
        "orc_sum64": (fl, [P, i]),
        "orc_sum64d": (d, [P, i]),
        "orc_set_gomoku_rules": (None, [P, i, i, P, P]),
        "orc_gomoku_terminal": (i, [P, i, i]),
        "orc_set_go_rules": (None, [P, i, i, P, P, P, P]),
        "orc_go_leaf_rules": (i, [P, i, P, i, P, P]),
        "orc_shift_root": (i, [P, i, i]),
        "orc_exp_d": (d, [d]),
        "orc_log_d": (d, [d]),
        "orc_gamma": (d, [d, u64, u64, i, i]),
        "orc_root_dirichlet": (None, [P, i, d, u64, u64, P]),
        "orc_sample_action": (i, [P, i, d, u64, u64, i]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    for name in ("N", "W", "P", "parent", "first", "nchild", "action", "expanded", "children",
                 "child_actions", "num_nodes", "num_edges", "paths", "path_len", "leaves",
                 "sim_uid", "uleaf", "ufirst", "ucount", "ukey", "ulegal", "uexpanded", "policy",
                 "values", "uterm"):
        fn = getattr(lib, "orc_" + name)
        fn.restype = P
        fn.argtypes = [P]
    _lib = lib
    return lib


_DT = {"N": np.int32, "W": np.float32, "P": np.float32, "parent": np.int32, "first": np.int32,
       "nchild": np.int32, "action": np.int32, "expanded": np.uint8, "children": np.int32,
       "child_actions": np.int32, "num_nodes": np.int32, "num_edges": np.int32,
       "paths": np.int32, "path_len": np.int32, "leaves": np.int32, "sim_uid": np.int32,
       "uleaf": np.int32, "ufirst": np.int32, "ucount": np.int32, "ukey": np.uint64,
       "ulegal": np.int32, "uexpanded": np.int32, "policy": np.float32, "values": np.float32,
       "uterm": np.int32}


class Oracle:
    """T trees of one game model on the CPU (sequential reference semantics)."""

    def __init__(self, model, num_trees: int, capacity: int, max_wave: int, max_depth: int = 100):
        self.lib = load()
        self.model = model
        self.T, self.cap, self.MW, self.MD = num_trees, capacity, max_wave, max_depth
        self.A = model.num_actions
        self.f = self.lib.orc_create(num_trees, capacity, model.num_actions,
                                     GAME_CODES[model.kind], model.min_legal, model.max_legal,
                                     max_wave, max_depth)
        if not self.f:
            raise MemoryError("orc_create failed")

    def __del__(self):
        if getattr(self, "f", None):
            self.lib.orc_destroy(self.f)
            self.f = None

    def set_params(self, c_puct=1.414, virtual_loss=3.0, expand_policy=0, sign_mode=0,
                   logit_scale=1.0, dirichlet_epsilon=0.0):
        self.lib.orc_set_params(self.f, c_puct, virtual_loss, expand_policy, sign_mode,
                                logit_scale, dirichlet_epsilon)

    def set_roots(self, keys, legal=None, noise=None):
        self._keys = np.ascontiguousarray(keys, dtype=np.uint64)
        self._legal = None if legal is None else np.ascontiguousarray(legal, dtype=np.uint32)
        self._noise = None if noise is None else np.ascontiguousarray(noise, dtype=np.float64)
        self.lib.orc_set_roots(self.f, self._keys.ctypes.data,
                               None if self._legal is None else self._legal.ctypes.data,
                               None if self._noise is None else self._noise.ctypes.data)

    def array(self, name: str, count: int, offset: int = 0) -> np.ndarray:
        ptr = getattr(self.lib, "orc_" + name)(self.f)
        dt = np.dtype(_DT[name])
        buf = (ctypes.c_char * ((offset + count) * dt.itemsize)).from_address(ptr)
        return np.frombuffer(buf, dtype=dt, count=count, offset=offset * dt.itemsize).copy()

    def set_gomoku_rules(self, boards, rule: int = 0, root_player=None) -> None:
        """Gomoku terminal checks on the leaves (boards: int8 [T, bs, bs] root positions);
        boards=None switches them off."""
        if boards is None:
            self.lib.orc_set_gomoku_rules(self.f, 0, 0, None, None)
            return
        self._boards = np.ascontiguousarray(boards, dtype=np.int8).reshape(self.T, self.A)
        self._rp = None if root_player is None else np.ascontiguousarray(root_player, np.int32)
        self.lib.orc_set_gomoku_rules(self.f, 1, rule, self._boards.ctypes.data,
                                      None if self._rp is None else self._rp.ctypes.data)

    def set_go_rules(self, boards, flags: int = 1, root_player=None, root_passes=None,
                     root_ko=None) -> None:
        """Go rules on the leaves (boards: int8 [T, bs, bs] root positions; flags 1 ko,
        2 suicide; per-tree root player, trailing passes and ko point); boards=None switches
        them off."""
        if boards is None:
            self.lib.orc_set_go_rules(self.f, 0, 0, None, None, None, None)
            return
        self._go = [np.ascontiguousarray(boards, dtype=np.int8).reshape(self.T, self.A - 1)]
        for x in (root_player, root_passes, root_ko):
            self._go.append(None if x is None else np.ascontiguousarray(x, np.int32).reshape(-1))
        ptr = lambda x: None if x is None else x.ctypes.data  # noqa: E731
        self.lib.orc_set_go_rules(self.f, 1, int(flags), *[ptr(x) for x in self._go])

    def go_leaf_rules(self, t: int, moves):
        """(legal list, terminal code) of tree t's position after the moves, Go rules on."""
        acts = np.ascontiguousarray(moves, dtype=np.int32)
        out = np.zeros(self.A + 1, np.int32)
        term = ctypes.c_int(0)
        n = self.lib.orc_go_leaf_rules(self.f, t, acts.ctypes.data if acts.size else None,
                                       int(acts.size), out.ctypes.data, ctypes.byref(term))
        return out[:n].tolist(), term.value

    def shift_root(self, t: int, node: int) -> int:
        """Subtree reuse on tree t (CSRTree.shift_root); returns the kept node count (0 when
        the tree is unchanged)."""
        return int(self.lib.orc_shift_root(self.f, t, node))

    def write(self, name: str, values, offset: int = 0) -> None:
        """Overwrite entries [offset, offset + len(values)) of an oracle array (crafted states
        for the known-answer tests)."""
        dt = np.dtype(_DT[name])
        v = np.ascontiguousarray(values, dtype=dt)
        ptr = getattr(self.lib, "orc_" + name)(self.f)
        ctypes.memmove(ptr + offset * dt.itemsize, v.ctypes.data, v.nbytes)

    def num_nodes(self, t: int) -> int:
        return int(self.array("num_nodes", 1, t)[0])

    def tree(self, t: int) -> dict:
        n = self.num_nodes(t)
        b = t * self.cap
        out = {k: self.array(k, n, b) for k in ("N", "W", "P", "parent", "first", "nchild",
                                                  "action", "expanded")}
        out["children"] = self.array("children", max(n - 1, 0), b)
        out["child_actions"] = self.array("child_actions", max(n - 1, 0), b)
        out["num_nodes"] = n
        return out

    def reset_tree(self, t: int):
        self.lib.orc_reset_tree(self.f, t)

    def wave(self, t: int, W: int, max_depth: int | None = None, replay_policy=None,
             replay_values=None):
        md = max_depth or self.MD
        if replay_policy is not None:
            rp = np.ascontiguousarray(replay_policy, dtype=np.float32)
            rv = np.ascontiguousarray(replay_values, dtype=np.float32)
            self.lib.orc_wave(self.f, t, W, md, rp.ctypes.data, rv.ctypes.data)
        else:
            self.lib.orc_wave(self.f, t, W, md, None, None)

    def search(self, num_sims: int, wave: int, max_depth: int | None = None, nthreads: int = 1):
        rc = self.lib.orc_search(self.f, num_sims, wave, max_depth or self.MD, nthreads)
        if rc != 0:
            raise RuntimeError("orc_search failed")

    def last_wave(self, t: int, W: int) -> dict:
        wb = t * self.MW
        nu = int(self.array("ucount", 1, t)[0])
        plen = self.array("path_len", W, wb)
        paths = self.array("paths", W * self.MD, wb * self.MD).reshape(W, self.MD)
        return {
            "path_len": plen,
            "paths": [paths[s, :plen[s]].copy() for s in range(W)],
            "leaves": self.array("leaves", W, wb),
            "sim_uid": self.array("sim_uid", W, wb),
            "uleaf": self.array("uleaf", nu, wb),
            "ufirst": self.array("ufirst", nu, wb),
            "ukey": self.array("ukey", nu, wb),
            "ulegal": self.array("ulegal", nu, wb),
            "values": self.array("values", nu, wb),
            "uterm": self.array("uterm", nu, wb),
            "ucount": nu,
        }

    def root_policy(self, t: int) -> np.ndarray:
        """MCTS._extract_policy (mcts.py:1069-1137): visits / total over the root's children;
        uniform over the children's actions when they have no visits, uniform over the action
        space when the root has no children."""
        tr = self.tree(t)
        pol = np.zeros(self.A)
        f, k = tr["first"][0], tr["nchild"][0]
        if k <= 0:
            return np.full(self.A, 1.0 / self.A)
        kids = tr["children"][f:f + k]
        acts = tr["child_actions"][f:f + k]
        tot = int(tr["N"][kids].sum())
        if tot == 0:
            pol[acts] = 1.0 / k
            return pol
        pol[acts] = tr["N"][kids] / tot
        return pol

    def root_dirichlet(self, t: int, alpha: float, seed: int, counter: int) -> np.ndarray:
        row = np.zeros(self.A, np.float64)
        self.lib.orc_root_dirichlet(self.f, t, alpha, seed, counter, row.ctypes.data)
        return row
