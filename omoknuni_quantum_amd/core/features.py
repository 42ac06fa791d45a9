"""Feature planes of the unique leaves of a wave, built on the device from the root board and
the path moves (glue between the tree operations and a reference-protocol evaluator).

Planes follow the reference's basic representation (python/mcts/cpu/cpu_game_states.py:
452-494) without its all-ones plane, 18 planes per position:
  0  stones of the player to move      1  stones of the opponent
  2-15 history (zero, as in the reference)
  16 colour to play (1 if player 1)    17 move count / 100
The player to move at the root is 1 when the root board holds an even number of stones;
moves along the path alternate colours from there.
"""
from __future__ import annotations

import torch

NUM_PLANES = 18


class LeafFeatureBuilder:
    def __init__(self, engine, boards: torch.Tensor):
        """boards: int8 [T, bs, bs] root positions (0 empty, 1/2 stones) on the engine device."""
        self.eng = engine
        T = engine.T
        self.bs = engine.model.board_size
        cells = self.bs * self.bs
        b = boards.to(engine.device).reshape(T, cells)
        stones = (b != 0).sum(dim=1)
        self.root_player = torch.where(stones % 2 == 0, 1, 2).to(torch.int64)  # [T]
        self.root_moves = stones.to(torch.float32)
        self.root_board = b.to(torch.int64)

    def build(self) -> torch.Tensor:
        """float32 [T*max_wave, 18, bs, bs]; rows past a tree's unique-leaf count are unused."""
        e = self.eng
        T, MW, MD, cap = e.T, e.MW, e.MD, e.cap
        cells = self.bs * self.bs
        dev = e.device
        first = e.ufirst.view(T, MW).to(torch.int64)                        # [T, MW]
        first = first.clamp_(0, MW - 1)
        plen = torch.gather(e.path_len.view(T, MW), 1, first).to(torch.int64)
        paths = e.paths.view(T, MW, MD)
        rows = torch.gather(paths, 1, first[:, :, None].expand(T, MW, MD)).to(torch.int64)
        d = torch.arange(MD, device=dev)
        onpath = (d[None, None, :] >= 1) & (d[None, None, :] < plen[:, :, None])
        nodes = torch.where(onpath, rows, 0) + (torch.arange(T, device=dev) * cap)[:, None, None]
        acts = e.action[nodes.reshape(-1)].view(T, MW, MD).to(torch.int64)
        mover = torch.where(((d - 1) % 2 == 0)[None, None, :],
                            self.root_player[:, None, None], 3 - self.root_player[:, None, None])
        board = self.root_board[:, None, :].expand(T, MW, cells).clone()
        valid = onpath & (acts >= 0) & (acts < cells)
        colour = torch.where(valid, mover, 0)
        _scatter_moves(board, acts, colour, valid)
        moves = (plen - 1).to(torch.float32)
        to_move = torch.where(moves.to(torch.int64) % 2 == 0, self.root_player[:, None],
                              3 - self.root_player[:, None])                   # [T, MW]
        feat = torch.zeros((T, MW, NUM_PLANES, cells), dtype=torch.float32, device=dev)
        feat[:, :, 0] = (board == to_move[:, :, None]).to(torch.float32)
        feat[:, :, 1] = (board == (3 - to_move)[:, :, None]).to(torch.float32)
        feat[:, :, 16] = (to_move == 1).to(torch.float32)[:, :, None]
        feat[:, :, 17] = ((self.root_moves[:, None] + moves) / 100.0)[:, :, None]
        return feat.view(T * MW, NUM_PLANES, self.bs, self.bs)


def _scatter_moves(board: torch.Tensor, acts: torch.Tensor, colour: torch.Tensor,
                   valid: torch.Tensor) -> None:
    """board[t, u, acts[t, u, d]] = colour[t, u, d] for valid entries (distinct cells)."""
    T, MW, cells = board.shape
    idx = torch.where(valid, acts, cells)  # invalid entries go to a spill column
    ext = torch.cat([board, torch.zeros((T, MW, 1), dtype=board.dtype, device=board.device)], 2)
    ext.scatter_(2, idx, torch.where(valid, colour, 0).to(board.dtype))
    board.copy_(ext[:, :, :cells])
