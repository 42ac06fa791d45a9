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
The player to move at the root is 1 when the root board holds an even number of stones. The
moves along the path alternate colours from there. The root's move count is its stone count
(python/mcts/core/mcts.py:1503-1508).
"""
from __future__ import annotations

import torch

NUM_PLANES = 18


class LeafFeatureBuilder:
    """Owns the feature buffer of every wave slot: [T*max_wave, planes, bs, bs]."""

    def __init__(self, engine, boards: torch.Tensor, planes: int = NUM_PLANES,
                 dtype: torch.dtype = torch.float32, channels_last: bool = False):
        """boards: [T, bs, bs] root positions (0 empty, 1/2 stones)."""
        self.eng = engine
        self.bs = engine.model.board_size
        self.planes = planes
        self.channels_last = channels_last
        T, MW, bs = engine.T, engine.MW, self.bs
        self.boards = boards.to(engine.device, torch.int8).reshape(-1).contiguous()
        if channels_last:
            self.buf = torch.empty((T * MW, bs, bs, planes), dtype=dtype, device=engine.device)
            self.view = self.buf.permute(0, 3, 1, 2)  # NCHW shape, channels-last strides
        else:
            self.buf = torch.empty((T * MW, planes, bs, bs), dtype=dtype, device=engine.device)
            self.view = self.buf

    def build(self) -> torch.Tensor:
        """The planes of the current wave (a view of the builder's buffer).  Slots past a tree's
        unique-leaf count hold zeros."""
        self.eng.leaf_features(self.buf, self.boards, self.planes, nhwc=self.channels_last)
        return self.view
