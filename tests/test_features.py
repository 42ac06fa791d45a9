"""The feature-plane restatement (oracle/ref_np.py: leaf_position, nn_features) pinned by
known positions and by what the reference's plane definitions fix.  These are the checks the
GPU feature kernel is compared against."""
import numpy as np
import pytest

from oracle.ref_np import leaf_position, nn_features


def test_known_position_three_moves():
    # empty board, moves 112 (player 1), 113 (player 2), 0 (player 1): player 2 to move
    b, player, count = leaf_position(np.zeros((15, 15), np.int8), [112, 113, 0])
    assert player == 2 and count == 3
    assert b[7, 7] == 1 and b[7, 8] == 2 and b[0, 0] == 1 and np.count_nonzero(b) == 3
    f = nn_features(b, player, count)
    assert f.shape == (19, 15, 15) and f.dtype == np.float32
    assert set(zip(*np.nonzero(f[0]))) == {(7, 8)}              # the mover's (player 2) stones
    assert set(zip(*np.nonzero(f[1]))) == {(7, 7), (0, 0)}      # the opponent's
    assert not f[2:16].any()
    assert not f[16].any()                                       # player 2 to move
    assert np.all(f[17] == np.float32(0.03)) and np.all(f[18] == 1.0)


def test_root_player_from_stone_parity():
    # mcts.py:1503-1508: player 1 moves when the stone count is even
    b0 = np.zeros((9, 9), np.int8)
    b0[4, 4] = 1
    b, player, count = leaf_position(b0, [])
    assert player == 2 and count == 1
    f = nn_features(b, player, count, planes=18)
    assert f.shape == (18, 9, 9)
    assert f[1, 4, 4] == 1.0 and f[0].sum() == 0 and not f[16].any()
    b, player, count = leaf_position(b0, [0])
    assert b[0, 0] == 2 and player == 1 and count == 2 and np.all(f[17] == np.float32(0.01))
    # explicit root player and move count override the board's
    b, player, count = leaf_position(b0, [0], root_player=1, root_moves=40)
    assert b[0, 0] == 1 and player == 2 and count == 41


@pytest.mark.parametrize("seed", range(4))
def test_planes_partition_the_board(seed):
    rng = np.random.default_rng(seed)
    bs = 15
    root = np.zeros(bs * bs, np.int8)
    occ = rng.choice(bs * bs, size=int(rng.integers(0, 60)), replace=False)
    root[occ] = rng.integers(1, 3, size=occ.size)
    free = np.flatnonzero(root == 0)
    path = rng.choice(free, size=int(rng.integers(0, 20)), replace=False)
    b, player, count = leaf_position(root.reshape(bs, bs), path)
    f = nn_features(b, player, count)
    # the two stone planes cover the occupied cells exactly, without overlap
    assert np.array_equal(f[0] + f[1], (b != 0).astype(np.float32))
    assert np.array_equal(f[0], (b == player).astype(np.float32))
    # stones on the path alternate from the root player, and the leaf's mover continues it
    rp = 1 if np.count_nonzero(root) % 2 == 0 else 2
    for j, a in enumerate(path):
        assert b.reshape(-1)[a] == (rp if j % 2 == 0 else 3 - rp)
    assert player == (rp if len(path) % 2 == 0 else 3 - rp)
    assert np.all(f[16] == (1.0 if player == 1 else 0.0))
    assert count == np.count_nonzero(root) + len(path)


def test_move_count_plane_rounding():
    # the reference divides an int16 count by 100.0 in double and stores float32; for every
    # int16 count this equals the correctly rounded float32 quotient
    m = np.arange(0, 32768, dtype=np.int16)
    ref = (m / 100.0).astype(np.float32)
    assert np.array_equal(ref, m.astype(np.float32) / np.float32(100.0))
    for c in (0, 1, 7, 99, 100, 225, 32767):
        f = nn_features(np.zeros((3, 3), np.int8), 1, c)
        assert f[17, 0, 0] == np.float32(c / 100.0)
