"""Feature planes of a wave's unique leaves for a reference-protocol evaluator.

The HIP kernel behind omq_leaf_features builds the planes on the device. It rebuilds each
leaf's position from the root board and the moves on the leaf's path.

Planes follow the reference's 'basic' representation (python/mcts/cpu/cpu_game_states.py:
430-494), with 19 planes, or 18 without its all-ones plane:
  0     stones of the player to move
  1     stones of the opponent
  2-15  history (zero, as in the reference)
  16    colour to play (1 if player 1)
  17    move count / 100
  18    all ones (19 planes only)
The player to move at the root is 1 when the root board holds an even number of stones, and the
root's move count is its stone count (python/mcts/core/mcts.py:1503-1508), unless the root came
from a game-state object, whose own player and move-history length are used (mcts.py:1576-1600).
The moves along the path alternate colours from there.
"""
from __future__ import annotations

import torch

NUM_PLANES = 18


class LeafFeatureBuilder:
    """Owns the feature buffer of every wave slot: [T*max_wave, planes, bs, bs]."""

    def __init__(self, engine, boards: torch.Tensor, planes: int = NUM_PLANES,
                 dtype: torch.dtype = torch.float32, channels_last: bool = False,
                 root_player=None, root_moves=None):
        """boards: [T, bs, bs] root positions (0 empty, 1/2 stones); root_player / root_moves:
        optional [T] player to move and move count of each root (default: from the stone
        count)."""
        self.eng = engine
        self.bs = engine.model.board_size
        self.planes = planes
        self.channels_last = channels_last
        T, MW, bs = engine.T, engine.MW, self.bs
        self.boards = boards.to(engine.device, torch.int8).reshape(-1).contiguous()

        def per_tree(x):
            if x is None:
                return None
            v = torch.as_tensor(x, dtype=torch.int32).reshape(-1)
            if v.numel() != T:
                raise ValueError(f"{v.numel()} root values for {T} trees")
            return v.to(engine.device).contiguous()

        self.root_player = per_tree(root_player)
        self.root_moves = per_tree(root_moves)
        if channels_last:
            self.buf = torch.empty((T * MW, bs, bs, planes), dtype=dtype, device=engine.device)
            self.view = self.buf.permute(0, 3, 1, 2)  # NCHW shape, channels-last strides
        else:
            self.buf = torch.empty((T * MW, planes, bs, bs), dtype=dtype, device=engine.device)
            self.view = self.buf

    def build(self) -> torch.Tensor:
        """The planes of the current wave (a view of the builder's buffer).  Slots past a tree's
        unique-leaf count hold zeros."""
        self.eng.leaf_features(self.buf, self.boards, self.planes, root_player=self.root_player,
                               root_moves=self.root_moves, nhwc=self.channels_last)
        return self.view
