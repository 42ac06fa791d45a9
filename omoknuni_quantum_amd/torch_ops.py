"""torch.library operators over the C ABI, with the reference's operator signatures.

The reference registers ``mcts::vectorized_backup`` (python/mcts/gpu/torch_custom_ops.py:26-55)
and reaches ``batch_apply_virtual_loss`` / ``batch_remove_virtual_loss``
(python/mcts/gpu/mcts_kernels.cu:845-860,934-953) through its pybind11 module.  The same
operations are registered here in the ``omq`` namespace, mutating their tensor arguments in
place on the caller's current HIP stream; the three the reference registers itself are also
registered under its own names, ``mcts::vectorized_backup``, ``mcts::warp_vectorized_backup``
and ``mcts::fused_ucb_selection`` (torch_custom_ops.py:26,71,108), which is where
AsyncWaveSearch probes for them (python/mcts/core/async_wave_search.py:255-260):

    torch.ops.omq.vectorized_backup(paths, path_lengths, values, visit_counts, value_sums)
    torch.ops.omq.warp_vectorized_backup(paths, path_lengths, values, visit_counts, value_sums)
    torch.ops.omq.batch_apply_virtual_loss(node_indices, virtual_loss_counts)
    torch.ops.omq.batch_remove_virtual_loss(node_indices, virtual_loss_counts)
    torch.ops.omq.fused_ucb_selection(node_indices, children_start, children_end, children,
                                      q_values, visit_counts, priors, c_puct) -> int32 [batch]

``vectorized_backup`` follows the reference kernel (mcts_kernels.cu:121-158): for every path b
and d < min(path_lengths[b], max_depth), node x = paths[b, d] in [0, num_nodes) gets
visit_counts[x] += 1 and value_sums[x] += v * (-1)^(path_lengths[b]-1-d) (sign by distance
from the leaf); other entries are skipped.  ``warp_vectorized_backup`` is the same operation: the
reference's warp variant (mcts_kernels.cu:164-230) never leaves out a lane, so it adds the same
terms.  The virtual-loss operators add +1 / -1 per listed node (duplicates accumulate; indices
outside the array are skipped).  ``fused_ucb_selection`` follows the reference's operator
(torch_custom_ops.py:108-193, kernel mcts_kernels.cu:1466-1512): per parent, the row position
of the first maximum of q + c*P*sqrt(N_parent)/(1+n), with q = 0 for an unvisited child.

There is no CPU implementation: tensors must be on a HIP device, and a missing library raises.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib


def _check_device(name: str, *tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    if dev.type != "cuda":
        raise RuntimeError(f"omq::{name}: tensors must be on a HIP device (got {dev})")
    for t in tensors:
        if t.device != dev:
            raise RuntimeError(f"omq::{name}: all tensors must be on {dev}")
        if not t.is_contiguous():
            raise RuntimeError(f"omq::{name}: tensors must be contiguous")
    return dev


def _forest(counts: torch.Tensor, sums: torch.Tensor | None) -> _lib.OmqForest:
    f = _lib.OmqForest()
    f.num_trees = 1
    f.capacity = counts.numel()
    f.visit_counts = counts.data_ptr()
    if sums is not None:
        f.value_sums = sums.data_ptr()
    return f


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def vectorized_backup(paths: torch.Tensor, path_lengths: torch.Tensor, values: torch.Tensor,
                      visit_counts: torch.Tensor, value_sums: torch.Tensor) -> None:
    dev = _check_device("vectorized_backup", paths, path_lengths, values, visit_counts,
                        value_sums)
    if paths.dim() != 2 or paths.dtype != torch.int32 or path_lengths.dtype != torch.int32:
        raise RuntimeError("omq::vectorized_backup: paths int32 [B, D], path_lengths int32 [B]")
    if values.dtype != torch.float32 or visit_counts.dtype != torch.int32 or \
            value_sums.dtype != torch.float32:
        raise RuntimeError("omq::vectorized_backup: values/value_sums float32, visit_counts int32")
    B, D = paths.shape
    if path_lengths.numel() != B or values.numel() != B:
        raise RuntimeError("omq::vectorized_backup: one length and one value per path")
    if visit_counts.numel() != value_sums.numel():
        raise RuntimeError("omq::vectorized_backup: visit_counts and value_sums differ in size")
    if B == 0 or visit_counts.numel() == 0:
        return
    f = _forest(visit_counts, value_sums)
    lib = _lib.load()
    _lib.check(lib.omq_paths_backup(ctypes.byref(f), paths.data_ptr(), path_lengths.data_ptr(),
                                    None, values.data_ptr(), B, max(D, 1),
                                    _lib.OMQ_SIGN_LEAF_POSITIVE, _stream(dev)),
               "omq_paths_backup")


def _virtual_loss(name: str, node_indices: torch.Tensor, counts: torch.Tensor, delta: int):
    dev = _check_device(name, node_indices, counts)
    if node_indices.dtype != torch.int32 or counts.dtype != torch.int32:
        raise RuntimeError(f"omq::{name}: node_indices and virtual_loss_counts must be int32")
    n = node_indices.numel()
    if n == 0 or counts.numel() == 0:
        return
    f = _forest(counts, None)
    lib = _lib.load()
    _lib.check(lib.omq_virtual_loss(ctypes.byref(f), node_indices.data_ptr(), None, n, delta,
                                    _stream(dev)), "omq_virtual_loss")


def batch_apply_virtual_loss(node_indices: torch.Tensor,
                             virtual_loss_counts: torch.Tensor) -> None:
    _virtual_loss("batch_apply_virtual_loss", node_indices, virtual_loss_counts, 1)


def batch_remove_virtual_loss(node_indices: torch.Tensor,
                              virtual_loss_counts: torch.Tensor) -> None:
    _virtual_loss("batch_remove_virtual_loss", node_indices, virtual_loss_counts, -1)


def warp_vectorized_backup(paths: torch.Tensor, path_lengths: torch.Tensor, values: torch.Tensor,
                           visit_counts: torch.Tensor, value_sums: torch.Tensor) -> None:
    vectorized_backup(paths, path_lengths, values, visit_counts, value_sums)


def fused_ucb_selection(node_indices: torch.Tensor, children_start: torch.Tensor,
                        children_end: torch.Tensor, children: torch.Tensor,
                        q_values: torch.Tensor, visit_counts: torch.Tensor,
                        priors: torch.Tensor, c_puct: float) -> torch.Tensor:
    dev = _check_device("fused_ucb_selection", node_indices, children_start, children_end,
                        children, q_values, visit_counts, priors)
    for name, t, dt in (("node_indices", node_indices, torch.int32),
                        ("children_start", children_start, torch.int32),
                        ("children_end", children_end, torch.int32),
                        ("children", children, torch.int32),
                        ("q_values", q_values, torch.float32),
                        ("visit_counts", visit_counts, torch.int32),
                        ("priors", priors, torch.float32)):
        if t.dtype != dt:
            raise RuntimeError(f"omq::fused_ucb_selection: {name} must be {dt}, not {t.dtype}")
    selected = torch.empty(node_indices.numel(), dtype=torch.int32, device=dev)
    _lib.check(_lib.load().omq_fused_ucb_selection(
        node_indices.data_ptr(), node_indices.numel(), children_start.data_ptr(),
        children_end.data_ptr(), children.data_ptr(), q_values.data_ptr(),
        visit_counts.data_ptr(), priors.data_ptr(), float(c_puct), selected.data_ptr(),
        _stream(dev)), "omq_fused_ucb_selection")
    return selected


def _fused_ucb_fake(node_indices, children_start, children_end, children, q_values, visit_counts,
                    priors, c_puct):
    return torch.empty_like(node_indices, dtype=torch.int32)


def _no_output(*args) -> None:
    return None


# (name, implementation, mutated arguments, fake, namespaces)
_OPS = (
    ("vectorized_backup", vectorized_backup, ("visit_counts", "value_sums"), _no_output,
     ("omq", "mcts")),
    ("warp_vectorized_backup", warp_vectorized_backup, ("visit_counts", "value_sums"),
     _no_output, ("omq", "mcts")),
    ("fused_ucb_selection", fused_ucb_selection, (), _fused_ucb_fake, ("omq", "mcts")),
    ("batch_apply_virtual_loss", batch_apply_virtual_loss, ("virtual_loss_counts",), _no_output,
     ("omq",)),
    ("batch_remove_virtual_loss", batch_remove_virtual_loss, ("virtual_loss_counts",),
     _no_output, ("omq",)),
)

REGISTERED: dict = {}


def _register() -> None:
    """Registers every operator under its namespaces.  A name already taken in the ``mcts``
    namespace (the reference's own module imported first) is left to its owner."""
    for name, fn, mutates, fake, namespaces in _OPS:
        for ns in namespaces:
            qual = f"{ns}::{name}"
            if ns == "mcts" and hasattr(torch.ops, "mcts") and hasattr(torch.ops.mcts, name):
                continue
            op = torch.library.custom_op(qual, fn, mutates_args=mutates)
            op.register_fake(fake)
            REGISTERED[qual] = op


_register()
