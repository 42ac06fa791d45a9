"""MCTSConfig: search configuration with the field names and defaults of the reference.

Mirrors python/mcts/core/mcts_config.py:16-284 of cosmosapjw-quantum/omoknuni_quantum for
every field the tree-operation path reads (a1 of the path: num_simulations, c_puct,
dirichlet_alpha/epsilon, max_depth, wave sizes, device/backend, virtual loss, tree capacity,
progressive widening, csr_max_actions).  Fields of the reference that configure subsystems
outside this path (quantum analysis, tactical boosts, hybrid backends, memory pools, ...)
are accepted and kept in ``extra`` so that existing callers construct the config unchanged;
they have no effect here.

New fields of this build:
  expansion_policy  'full' (every legal action becomes a child; the GPU reference's
                    add_children_vectorized, python/mcts/gpu/csr_tree.py:295-389) or
                    'reference_pw' (the CPU driver's progressive widening,
                    python/mcts/cpu/optimized_wave_search.py:394-415, with MAX_CHILDREN=8)
  backup_sign       'leaf_positive' (optimized_wave_search.py:472-483, the CUDA backup kernels)
                    or 'root_positive' (cython_tree_optimized.pyx:216-224)
  w_accum           'ordered' (deterministic, bit-identical to the sequential loop) or 'atomic'
  vl_atomic         apply virtual loss with one atomic per path entry
  num_trees         independent trees searched together (search_batch)
  seed              seeds root keys and root Dirichlet noise
  sparse_legal      (min, max) legal actions per node for the chess-shaped synthetic model
  gomoku_rules      'freestyle' (five or more win), 'renju' (an overline of player 1 does
                    not win) or 'off': the terminal check of Gomoku leaves, as the
                    reference's game states run it after every move
                    (python/mcts/utils/fast_terminal_check.py:132-232); terminal leaves are
                    not expanded
  go_rules          'off' (a Go leaf's legal moves are the root's minus the path's points),
                    'ko' or 'ko_suicide': the Go rules of the reference's GPU game states
                    (python/mcts/gpu/go_kernels.py:17-110, gpu_game_states.py:373-395):
                    legal moves from the leaf position without the root's ko point (and,
                    with 'ko_suicide', without points lacking an empty neighbour); two
                    consecutive passes or a board without an empty point end the game
  root_noise_source 'host' (numpy PCG64 Dirichlet, per tree seed + t) or 'device'
                    (omq_root_dirichlet: Marsaglia-Tsang gamma variates from a counter-based
                    SplitMix64 stream keyed by seed and search count)
"""
from __future__ import annotations

import dataclasses
from dataclasses import dataclass, field
from enum import IntEnum
from typing import Any, Dict, Optional


class GameType(IntEnum):
    """Game identifiers of the reference (python/mcts/gpu/gpu_game_states.py:33-37)."""
    CHESS = 0
    GO = 1
    GOMOKU = 2


# Reference MCTSConfig fields outside the tree-operation path: accepted, stored, unused.
REFERENCE_ONLY_FIELDS = frozenset("""
classical_only_mode enable_fast_ucb enable_multi_stream num_cuda_streams stream_memory_pool_size
wave_min_size wave_max_size wave_adaptive_sizing cpu_threads_per_worker wave_target_sims_per_second
wave_target_gpu_utilization wave_num_pipelines wave_async_expansion wave_prefetch_evaluations
wave_memory_pool_mb enable_quantum memory_pool_size_mb tree_growth_factor enable_dynamic_allocation
gc_threshold use_gpu_tree_reuse tree_memory_fraction buffer_memory_fraction max_tree_nodes_per_worker
use_mixed_precision use_tensor_cores enable_kernel_fusion gpu_memory_fraction
initial_capacity_factor enable_memory_pooling enable_pinned_memory enable_async_evaluation
enable_coalesced_access use_lazy_gpu_states initial_gpu_states_capacity gpu_states_growth_factor
use_parallel_mcts num_mcts_workers worker_batch_size initial_children_per_expansion
progressive_expansion_threshold initial_expansion_children csr_use_sparse_operations
use_blocked_csr_layout block_size batch_size inference_batch_size tree_batch_size
gpu_batch_timeout worker_batch_timeout max_coordination_batch_size training_batch_queue_size
target_sims_per_second cache_legal_moves cache_features use_zobrist_hashing
subtree_reuse_min_visits adaptive_tree_reuse tree_reuse_min_child_visits tree_reuse_visit_ratio
tree_reuse_absolute_threshold enable_efficient_tree_reuse tree_reuse_validation_level
disable_tree_reuse_for_hybrid enable_debug_logging enable_state_pool_debug profile_gpu_kernels
enable_tactical_boost tactical_boost_strength tactical_boost_decay gomoku_win_boost
gomoku_block_win_boost gomoku_open_four_boost gomoku_block_four_boost gomoku_threat_base_boost
gomoku_threat_multiplier gomoku_three_boost gomoku_block_three_boost gomoku_center_boost
gomoku_connection_boost chess_capture_good_base chess_capture_equal chess_capture_bad
chess_check_boost chess_check_capture_boost chess_promotion_boost chess_center_boost
chess_center_core_boost chess_development_boost chess_castling_boost go_capture_boost
go_escape_boost go_atari_boost go_save_boost go_territory_boost go_connection_boost
go_eye_boost go_corner_boost use_cython_hybrid use_genuine_hybrid use_fixed_hybrid
use_optimized_hybrid use_optimized_fixed_hybrid use_unified_memory use_cuda_streams
enable_work_stealing hybrid_cpu_batch_size hybrid_gpu_batch_size hybrid_load_balance_interval
hybrid_target_gpu_utilization hybrid_target_cpu_utilization hybrid_pipeline_depth
hybrid_num_buffers use_tensorrt
""".split())

_EXPANSION = ("full", "reference_pw")
_SIGNS = ("leaf_positive", "root_positive")
_WACC = ("ordered", "atomic")
_RULES = ("freestyle", "renju", "off")
_GO_RULES = ("off", "ko", "ko_suicide")


@dataclass
class _ConfigFields:
    # core parameters (mcts_config.py:34-39)
    num_simulations: int = 10000
    c_puct: float = 1.414
    temperature: float = 1.0
    dirichlet_alpha: float = 0.3
    dirichlet_epsilon: float = 0.25
    max_depth: int = 100
    # waves (mcts_config.py:51-59)
    wave_size: Optional[int] = None
    min_wave_size: int = 1024
    max_wave_size: int = 1024
    cpu_optimal_wave_size: int = 32
    # device (mcts_config.py:69-74)
    device: str = "cuda"
    backend: str = "gpu"
    game_type: Any = GameType.GOMOKU
    board_size: int = 15
    # virtual loss (mcts_config.py:80-81)
    enable_virtual_loss: bool = True
    virtual_loss: float = 1.0
    # tree capacity (mcts_config.py:86-87): max_tree_nodes is the per-tree capacity, allocated
    # once (the reference grows from initial_tree_nodes up to max_tree_nodes)
    max_tree_nodes: int = 2000000
    initial_tree_nodes: int = 100000
    use_cuda_graphs: bool = True
    # progressive widening (mcts_config.py:120-126)
    max_children_per_node: int = 50
    progressive_widening_constant: float = 10.0
    progressive_widening_exponent: float = 0.5
    csr_max_actions: int = 225
    # subtree reuse (mcts_config.py:155)
    enable_subtree_reuse: bool = True
    # this build
    expansion_policy: str = "full"
    backup_sign: str = "leaf_positive"
    w_accum: str = "ordered"
    vl_atomic: bool = False
    num_trees: int = 1
    seed: int = 0
    sparse_legal: tuple = (20, 45)
    gomoku_rules: str = "freestyle"
    go_rules: str = "off"
    root_noise_source: str = "host"
    extra: Dict[str, Any] = field(default_factory=dict)


class MCTSConfig(_ConfigFields):
    """Configuration of the MCTS search (reference field names and defaults)."""

    def __init__(self, **kwargs):
        known = {f.name for f in dataclasses.fields(_ConfigFields)}
        extra = dict(kwargs.pop("extra", {}) or {})
        for k in list(kwargs):
            if k not in known:
                if k not in REFERENCE_ONLY_FIELDS:
                    raise TypeError(f"MCTSConfig got an unexpected keyword argument '{k}'")
                extra[k] = kwargs.pop(k)
        super().__init__(**kwargs, extra=extra)
        self.__post_init__()

    def __post_init__(self):
        # mcts_config.py:269-279
        if self.backend not in ("gpu", "cpu", "hybrid"):
            raise ValueError(f"backend must be 'gpu', 'cpu', or 'hybrid', got '{self.backend}'")
        if isinstance(self.game_type, str):
            self.game_type = GameType[self.game_type.upper()]
        else:
            self.game_type = GameType(int(self.game_type))
        if self.board_size is None:
            self.board_size = {GameType.CHESS: 8, GameType.GO: 19, GameType.GOMOKU: 15}[self.game_type]
        if self.expansion_policy not in _EXPANSION:
            raise ValueError(f"expansion_policy must be one of {_EXPANSION}")
        if self.backup_sign not in _SIGNS:
            raise ValueError(f"backup_sign must be one of {_SIGNS}")
        if self.w_accum not in _WACC:
            raise ValueError(f"w_accum must be one of {_WACC}")
        if self.num_trees < 1:
            raise ValueError("num_trees must be >= 1")
        if self.gomoku_rules not in _RULES:
            raise ValueError(f"gomoku_rules must be one of {_RULES}")
        if self.go_rules not in _GO_RULES:
            raise ValueError(f"go_rules must be one of {_GO_RULES}")
        if self.root_noise_source not in ("host", "device"):
            raise ValueError("root_noise_source must be 'host' or 'device'")

    # effective values ---------------------------------------------------------------------
    def effective_wave_size(self) -> int:
        """Simulations per wave: max_wave_size (the wave loop, mcts.py:1040-1042); with
        backend='cpu' and no wave_size, cpu_optimal_wave_size (mcts.py:491-498)."""
        if self.backend == "cpu" and self.wave_size is None:
            return int(self.cpu_optimal_wave_size)
        return int(self.max_wave_size)

    def effective_virtual_loss(self) -> float:
        return float(self.virtual_loss) if self.enable_virtual_loss else 0.0

    def action_space_size(self) -> int:
        """Actions per node (mcts.py:1024-1030, 1080-1083): board^2, +1 pass for Go, 4672
        action slots for the chess-shaped model."""
        if self.game_type == GameType.GO:
            return self.board_size * self.board_size + 1
        if self.game_type == GameType.CHESS:
            return 4672
        return self.board_size * self.board_size

    def to_dict(self) -> Dict[str, Any]:
        d = {f.name: getattr(self, f.name) for f in dataclasses.fields(_ConfigFields)}
        extra = d.pop("extra")
        d.update(extra)
        return d


def create_optimized_config(game_type=GameType.GOMOKU, num_simulations: int = 10000,
                            device: str = "cuda", enable_quantum: bool = False, **kwargs):
    """mcts_config.py:287-312."""
    return MCTSConfig(game_type=game_type, num_simulations=num_simulations, device=device,
                      enable_quantum=enable_quantum, **kwargs)


def create_performance_config(wave_size: int = 3072, memory_pool_mb: int = 2048, **kwargs):
    """mcts_config.py:315-339."""
    return MCTSConfig(wave_size=wave_size, memory_pool_size_mb=memory_pool_mb,
                      classical_only_mode=True, enable_fast_ucb=True, use_mixed_precision=True,
                      use_cuda_graphs=True, use_tensor_cores=True, **kwargs)
