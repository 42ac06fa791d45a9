"""MCTSConfig keeps the reference's field names and defaults; the synthetic workloads have the
shapes BASELINE.json states."""
import numpy as np
import pytest

from omoknuni_quantum_amd.core.mcts_config import GameType, MCTSConfig, create_optimized_config
from omoknuni_quantum_amd.synthetic import games
from omoknuni_quantum_amd.synthetic.workloads import WORKLOADS, get

# python/mcts/core/mcts_config.py:34-155 defaults of the fields the tree path reads
REFERENCE_DEFAULTS = {
    "num_simulations": 10000, "c_puct": 1.414, "temperature": 1.0, "dirichlet_alpha": 0.3,
    "dirichlet_epsilon": 0.25, "max_depth": 100, "wave_size": None, "min_wave_size": 1024,
    "max_wave_size": 1024, "cpu_optimal_wave_size": 32, "device": "cuda", "backend": "gpu",
    "board_size": 15, "enable_virtual_loss": True, "virtual_loss": 1.0,
    "max_tree_nodes": 2000000, "initial_tree_nodes": 100000, "max_children_per_node": 50,
    "progressive_widening_constant": 10.0, "progressive_widening_exponent": 0.5,
    "csr_max_actions": 225, "enable_subtree_reuse": True, "use_cuda_graphs": True,
}


def test_reference_defaults():
    c = MCTSConfig()
    for k, v in REFERENCE_DEFAULTS.items():
        assert getattr(c, k) == v, k
    assert c.game_type == GameType.GOMOKU


def test_reference_only_fields_accepted():
    c = MCTSConfig(enable_quantum=False, use_mixed_precision=False, num_cuda_streams=8,
                   gomoku_win_boost=100.0)
    assert c.extra["num_cuda_streams"] == 8
    assert c.to_dict()["gomoku_win_boost"] == 100.0
    c2 = create_optimized_config(num_simulations=50, device="cpu")
    assert c2.num_simulations == 50 and c2.extra["enable_quantum"] is False


def test_validation():
    with pytest.raises(ValueError):
        MCTSConfig(backend="tpu")
    with pytest.raises(TypeError):
        MCTSConfig(not_a_field=1)
    with pytest.raises(ValueError):
        MCTSConfig(expansion_policy="greedy")
    assert MCTSConfig(game_type="go", board_size=19).action_space_size() == 362
    assert MCTSConfig(game_type=GameType.CHESS).action_space_size() == 4672
    assert MCTSConfig(backend="cpu").effective_wave_size() == 32
    assert MCTSConfig(max_wave_size=256).effective_wave_size() == 256
    assert MCTSConfig(enable_virtual_loss=False, virtual_loss=3.0).effective_virtual_loss() == 0.0


def test_workload_shapes():
    assert [WORKLOADS[n].num_trees for n in ("C1", "C2", "C3", "C4", "C5")] == [1, 64, 32, 16, 32]
    assert WORKLOADS["C2"].capacity == 400_000 and WORKLOADS["C3"].capacity == 2_000_000
    assert WORKLOADS["C3"].model.num_actions == 362 and WORKLOADS["C4"].model.num_actions == 4672
    keys, legal, noise = get("C3").root_inputs()
    counts = games.legal_counts(get("C3").model, legal)
    assert counts.min() >= 250 and counts.max() <= 362
    assert noise is not None and np.allclose(noise.sum(axis=1), 1.0)
    for t in range(len(counts)):
        assert np.all(noise[t, counts[t]:] == 0)
    keys2, legal2, _ = get("C2").root_inputs()
    c2 = games.legal_counts(get("C2").model, legal2)
    assert c2.min() >= 225 - 60 and c2.max() <= 225
    assert len(set(keys2.tolist())) == 64


def test_boards_alternate_colours():
    b = games.random_boards(8, 15, 60, seed=3)
    for t in range(8):
        ones, twos = int((b[t] == 1).sum()), int((b[t] == 2).sum())
        assert ones - twos in (0, 1)


def test_go_pass_always_legal():
    m = games.go(19)
    b = np.ones((1, 19, 19), np.int8)
    legal = games.legal_masks(m, b, 1)
    assert games.legal_counts(m, legal)[0] == 1
    assert (int(legal[0, 361 // 32]) >> (361 % 32)) & 1
