"""The reference's accelerator interface (python/mcts/gpu/mcts_gpu_accelerator.py:41-207,
252-336, 386-408) over this package's HIP operators.

``MCTSGPUAccelerator`` keeps the reference's method names and argument order: each method
forwards to the operator of torch_ops.py with the reference pybind function's signature.
There is no PyTorch fallback: the constructor raises unless the device is a HIP device and
libomq_tree_ops.so loads (``DISABLE_CUDA_KERNELS=1``, which selects the reference's fallback,
raises too).  ``get_mcts_gpu_accelerator`` keeps one instance per process, as the reference's
does (mcts_gpu_accelerator.py:386-400).
"""
from __future__ import annotations

import os

import torch

from . import _lib, torch_ops


class MCTSGPUAccelerator:
    """GPU operators of the reference's wave search, on this package's kernels."""

    def __init__(self, device: torch.device | str | None = None):
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        if os.environ.get("DISABLE_CUDA_KERNELS", "0") == "1":
            raise RuntimeError("MCTSGPUAccelerator: DISABLE_CUDA_KERNELS=1 selects the "
                               "reference's PyTorch fallback, which this package does not have")
        if self.device.type != "cuda":
            raise RuntimeError(f"MCTSGPUAccelerator: {self.device} is not a HIP device")
        _lib.load()  # raises when the library is missing
        self.stats = {"ucb_calls": 0, "backup_calls": 0, "expansion_calls": 0}

    # mcts_gpu_accelerator.py:81-83
    def batched_ucb_selection(self, q_values, visit_counts, parent_visits, priors, row_ptr,
                              col_indices, c_puct):
        self.stats["ucb_calls"] += 1
        return torch_ops.batched_ucb_selection(q_values, visit_counts, parent_visits, priors,
                                               row_ptr, col_indices, c_puct)

    # mcts_gpu_accelerator.py:85-89
    def vectorized_backup(self, paths, path_lengths, values, visit_counts, value_sums):
        self.stats["backup_calls"] += 1
        torch_ops.vectorized_backup(paths, path_lengths, values, visit_counts, value_sums)

    # mcts_gpu_accelerator.py:91-97 (keywords as ConsolidatedKernelInterface passes them,
    # mcts_gpu_accelerator.py:299-314)
    def fused_select_expand(self, roots, children, visit_counts, q_values, prior_probs,
                            is_expanded, max_depth, c_puct):
        return torch_ops.fused_select_expand(roots, children, visit_counts, q_values,
                                             prior_probs, is_expanded, max_depth, c_puct)

    # mcts_gpu_accelerator.py:99-109
    def fused_select_expand_optimized(self, root_nodes, children, visit_counts, value_sums,
                                      priors, max_depth, c_puct):
        return torch_ops.fused_select_expand_optimized(root_nodes, children, visit_counts,
                                                       value_sums, priors, max_depth, c_puct)

    # mcts_gpu_accelerator.py:112-116
    def find_expansion_nodes(self, current_nodes, children, visit_counts, valid_path_mask,
                             wave_size, max_children):
        self.stats["expansion_calls"] += 1
        return torch_ops.find_expansion_nodes(current_nodes, children, visit_counts,
                                              valid_path_mask, wave_size, max_children)

    # mcts_gpu_accelerator.py:119-207: 18 positional arguments, type-checked
    _ADD_CHILDREN_ARGS = ("parent_indices", "actions", "priors", "num_children", "node_counter",
                          "edge_counter", "children", "parent_indices_out",
                          "parent_actions_out", "node_priors_out", "visit_counts_out",
                          "value_sums_out", "col_indices", "edge_actions", "edge_priors")

    def batched_add_children(self, *args):
        if len(args) < 18:
            raise ValueError(f"batched_add_children requires 18 arguments, got {len(args)}. "
                             "Required: " + ", ".join(self._ADD_CHILDREN_ARGS) +
                             ", max_nodes, max_children, max_edges")
        for i, name in enumerate(self._ADD_CHILDREN_ARGS):
            if not isinstance(args[i], torch.Tensor):
                raise TypeError(f"Argument '{name}' (position {i}) must be a torch.Tensor, "
                                f"got {type(args[i]).__name__}")
        return torch_ops.batched_add_children(*args[:18])

    # the virtual-loss operators of ConsolidatedKernelInterface (mcts_gpu_accelerator.py:273-290)
    def batch_apply_virtual_loss(self, node_indices, virtual_loss_counts):
        torch_ops.batch_apply_virtual_loss(node_indices, virtual_loss_counts)

    def warp_aggregated_virtual_loss(self, node_indices, virtual_loss_counts):
        torch_ops.batch_apply_virtual_loss(node_indices, virtual_loss_counts)

    def batch_remove_virtual_loss(self, node_indices, virtual_loss_counts):
        torch_ops.batch_remove_virtual_loss(node_indices, virtual_loss_counts)

    # mcts_gpu_accelerator.py:289-297: the module's operator with no noise, no legal masks and
    # epsilon 0
    def parallel_select_with_virtual_loss(self, parent_nodes, children, visit_counts,
                                          virtual_loss_counts, value_sums, priors,
                                          child_actions, c_puct, virtual_loss_value):
        return torch_ops.parallel_select_with_virtual_loss(
            parent_nodes, children, visit_counts, virtual_loss_counts, value_sums, priors,
            None, None, child_actions, c_puct, virtual_loss_value, 0.0)

    # mcts_gpu_accelerator.py:323-330: pass-through to the module's operators
    def batched_dirichlet_noise(self, *args, **kwargs):
        return torch_ops.batched_dirichlet_noise(*args, **kwargs)

    def fused_ucb_with_noise(self, *args, **kwargs):
        return torch_ops.fused_ucb_with_noise(*args, **kwargs)

    def optimized_backup_scatter(self, *args, **kwargs):
        self.stats["backup_calls"] += 1
        return torch_ops.optimized_backup_scatter(*args, **kwargs)

    def get_stats(self) -> dict:
        return {"device": str(self.device), "interface_type": "HIPKernelInterface",
                "library": _lib.load()._name, **self.stats}

    def reset_stats(self) -> None:
        for k in self.stats:
            self.stats[k] = 0


_GLOBAL: MCTSGPUAccelerator | None = None


def get_mcts_gpu_accelerator(device: torch.device | str | None = None) -> MCTSGPUAccelerator:
    """One accelerator per process (a new one after a fork)."""
    global _GLOBAL
    pid = os.getpid()
    if _GLOBAL is None or getattr(_GLOBAL, "_process_id", None) != pid:
        _GLOBAL = MCTSGPUAccelerator(device)
        _GLOBAL._process_id = pid
    return _GLOBAL


def get_global_accelerator() -> MCTSGPUAccelerator:
    return get_mcts_gpu_accelerator()
