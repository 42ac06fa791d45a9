"""Synthetic workloads of the benchmark configurations: game models and evaluator."""
from .games import (GameModel, chess_sparse, dirichlet_noise, go, gomoku, legal_counts,
                    legal_masks, random_boards, root_keys, splitmix64)
from .evaluator import SyntheticEvaluator

__all__ = [
    "GameModel", "chess_sparse", "dirichlet_noise", "go", "gomoku", "legal_counts",
    "legal_masks", "random_boards", "root_keys", "splitmix64", "SyntheticEvaluator",
]
