"""The benchmark workloads C1-C5 as concrete synthetic inputs.

C1  Gomoku 15x15, 1 tree x 800 simulations, wave 32, empty board.
C2  Gomoku 15x15, 64 trees x 1600, wave 256, capacity 400k, 0-60 random stones per tree.
C3  Go 19x19 + pass (362), 32 trees x 10000, wave 1024, capacity 2M, logits N(0, 2^2),
    root Dirichlet alpha 0.03 eps 0.25, 0-112 random stones (250-362 legal root moves).
C4  chess-shaped: 4672 slots, 20-45 hashed legal actions per node, 16 trees x 20000,
    wave 2048, capacity 1M.
C5  C2's game model with a ResNet evaluator: 32 trees x 1600, eval batch 512 read as
    16 wave slots per tree x 32 trees.
Shared: c_puct 1.4, virtual loss 3, max depth 100, leaf-positive backup sign.
"""
from __future__ import annotations

from dataclasses import dataclass, replace

import numpy as np

from . import games
from .games import GameModel


@dataclass(frozen=True)
class Workload:
    name: str
    model: GameModel
    num_trees: int
    num_simulations: int
    wave_size: int
    capacity: int
    max_stones: int = 0
    logit_scale: float = 1.0
    dirichlet_alpha: float = 0.0
    dirichlet_epsilon: float = 0.0
    c_puct: float = 1.4
    virtual_loss: float = 3.0
    max_depth: int = 100
    expand_policy: str = "full"  # "full" | "reference_pw"
    seed: int = 20260101
    evaluator: str = "synthetic"  # "synthetic" | "resnet"

    def scaled(self, **kw) -> "Workload":
        return replace(self, **kw)

    # inputs ---------------------------------------------------------------------------
    def boards(self) -> np.ndarray | None:
        if not self.model.is_board:
            return None
        return games.random_boards(self.num_trees, self.model.board_size, self.max_stones,
                                   self.seed)

    def root_inputs(self):
        """(keys uint64[T], legal uint32[T, words], noise float64[T, A] or None)."""
        keys = games.root_keys(self.seed, self.num_trees)
        legal = games.legal_masks(self.model, self.boards(), self.num_trees)
        noise = None
        if self.dirichlet_epsilon > 0:
            if self.model.is_board:
                counts = games.legal_counts(self.model, legal)
            else:
                counts = np.array([games.sparse_root_count(self.model, int(k)) for k in keys])
            noise = games.dirichlet_noise(self.model, counts, self.dirichlet_alpha,
                                          self.seed + 7919)
        return keys, legal, noise


WORKLOADS = {
    "C1": Workload("C1", games.gomoku(15), 1, 800, 32, 100_000),
    "C2": Workload("C2", games.gomoku(15), 64, 1600, 256, 400_000, max_stones=60),
    "C3": Workload("C3", games.go(19), 32, 10_000, 1024, 2_000_000, max_stones=112,
                   logit_scale=2.0, dirichlet_alpha=0.03, dirichlet_epsilon=0.25),
    "C4": Workload("C4", games.chess_sparse(4672, 20, 45), 16, 20_000, 2048, 1_000_000),
    "C5": Workload("C5", games.gomoku(15), 32, 1600, 16, 400_000, max_stones=60,
                   evaluator="resnet"),
}


def get(name: str) -> Workload:
    return WORKLOADS[name]
