"""Synthetic game models of the benchmark workloads (host side).

A game model decides the legal actions of a tree node:

* ``gomoku`` (15x15, 225 actions) and ``go`` (19x19 + pass = 362 actions): legal = cells empty
  on the root board minus the cells played on the path from the root; for Go the pass action
  (index 361) is always legal and occupies nothing.
* ``sparse`` (chess-shaped, 4672 action slots): each node has L ~ U{min_legal..max_legal}
  distinct legal actions drawn from its hash key (Floyd sampling, computed on the device).

Node keys: root key ``splitmix64(seed ^ t)`` for tree t; the child reached by action a has key
``splitmix64(key ^ (a+1) * 0x9E3779B97F4A7C15)``.  The device code derives keys, legal sets
and synthetic evaluator outputs from these keys; this module produces the inputs that live on
the host: root boards, root legal masks, root keys and root Dirichlet noise.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .. import _lib

MASK64 = (1 << 64) - 1
GOLDEN = 0x9E3779B97F4A7C15


def splitmix64(x: int) -> int:
    """SplitMix64 finaliser on a Python int (reference value for the device hash)."""
    z = (x + GOLDEN) & MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    return z ^ (z >> 31)


def child_key(key: int, action: int) -> int:
    """Key of the child reached from a node with key `key` by `action`."""
    return splitmix64((key ^ (((action + 1) * GOLDEN) & MASK64)) & MASK64)


def root_keys(seed: int, num_trees: int) -> np.ndarray:
    return np.array([splitmix64((seed ^ t) & MASK64) for t in range(num_trees)], dtype=np.uint64)


@dataclass(frozen=True)
class GameModel:
    kind: str  # "gomoku" | "go" | "sparse"
    num_actions: int
    board_size: int = 0
    min_legal: int = 0
    max_legal: int = 0

    @property
    def code(self) -> int:
        return {"gomoku": _lib.OMQ_GAME_BOARD, "go": _lib.OMQ_GAME_GO,
                "sparse": _lib.OMQ_GAME_SPARSE}[self.kind]

    @property
    def legal_words(self) -> int:
        return (self.num_actions + 31) // 32

    @property
    def cells(self) -> int:
        return self.board_size * self.board_size

    @property
    def is_board(self) -> bool:
        return self.kind in ("gomoku", "go")


def gomoku(board_size: int = 15) -> GameModel:
    return GameModel("gomoku", board_size * board_size, board_size)


def go(board_size: int = 19) -> GameModel:
    return GameModel("go", board_size * board_size + 1, board_size)


def chess_sparse(num_actions: int = 4672, min_legal: int = 20, max_legal: int = 45) -> GameModel:
    return GameModel("sparse", num_actions, 0, min_legal, max_legal)


def random_boards(num_trees: int, board_size: int, max_stones: int, seed: int,
                  min_stones: int = 0) -> np.ndarray:
    """Random positions: s ~ U{min_stones..max_stones} stones on uniformly random empty cells,
    colours 1 and 2 alternating (no capture or win checks).  int8 [T, bs, bs]."""
    rng = np.random.Generator(np.random.PCG64(seed))
    cells = board_size * board_size
    boards = np.zeros((num_trees, cells), dtype=np.int8)
    for t in range(num_trees):
        s = int(rng.integers(min_stones, max_stones + 1))
        pos = rng.permutation(cells)[:s]
        boards[t, pos] = np.where(np.arange(s) % 2 == 0, 1, 2).astype(np.int8)
    return boards.reshape(num_trees, board_size, board_size)


def legal_masks(model: GameModel, boards: np.ndarray | None, num_trees: int) -> np.ndarray:
    """uint32 [T, legal_words] root legal bitmasks (bit a of word a//32)."""
    words = np.zeros((num_trees, model.legal_words), dtype=np.uint32)
    if not model.is_board:
        return words
    if boards is None:
        boards = np.zeros((num_trees, model.board_size, model.board_size), dtype=np.int8)
    flat = boards.reshape(num_trees, -1)
    if flat.shape[1] != model.cells:
        raise ValueError(f"boards have {flat.shape[1]} cells, model expects {model.cells}")
    legal = np.zeros((num_trees, model.legal_words * 32), dtype=bool)
    legal[:, :model.cells] = flat == 0
    if model.kind == "go":
        legal[:, model.num_actions - 1] = True
    bits = legal.reshape(num_trees, model.legal_words, 32).astype(np.uint64)
    weights = (np.uint64(1) << np.arange(32, dtype=np.uint64))
    return (bits * weights).sum(axis=2).astype(np.uint32)


def legal_counts(model: GameModel, masks: np.ndarray) -> np.ndarray:
    return np.array([int(sum(bin(int(w)).count("1") for w in row)) for row in masks],
                    dtype=np.int64)


def dirichlet_noise(model: GameModel, counts: np.ndarray, alpha: float, seed: int) -> np.ndarray:
    """Root Dirichlet noise, float64 [T, num_actions]: entry i of row t is the noise of the
    i-th legal root action (ascending action order); numpy PCG64 seeded with seed + t."""
    T = len(counts)
    noise = np.zeros((T, model.num_actions), dtype=np.float64)
    for t in range(T):
        L = int(counts[t])
        if L > 0:
            g = np.random.Generator(np.random.PCG64(seed + t))
            noise[t, :L] = g.dirichlet([alpha] * L)
    return noise


def sparse_root_count(model: GameModel, key: int) -> int:
    """Legal count of a sparse-model node with the given key (same rule as the device)."""
    span = model.max_legal - model.min_legal + 1
    return model.min_legal + ((splitmix64(key ^ 0x165667B19E3779F9) >> 33) % span)
