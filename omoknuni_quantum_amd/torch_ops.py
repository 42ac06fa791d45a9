"""torch operators over the C ABI, with the reference's operator signatures.

The reference registers ``mcts::vectorized_backup`` (python/mcts/gpu/torch_custom_ops.py:26-55)
and reaches ``batch_apply_virtual_loss`` / ``batch_remove_virtual_loss``
(python/mcts/gpu/mcts_kernels.cu:845-860,934-953) through its pybind11 module.  The same
operations are torch operators in the ``omq`` namespace, registered from C++ by
libomq_torch_ops.so (csrc/torch_ops.cpp, loaded here), which checks the tensors and calls the C
ABI on the caller's current HIP stream, mutating its tensor arguments in place; the three the
reference registers itself are also registered under its own names,
``mcts::vectorized_backup``, ``mcts::warp_vectorized_backup`` and ``mcts::fused_ucb_selection``
(torch_custom_ops.py:26,71,108), which is where AsyncWaveSearch probes for them
(python/mcts/core/async_wave_search.py:255-260):

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

The reference accelerator's other operators (MCTSGPUAccelerator,
python/mcts/gpu/mcts_gpu_accelerator.py:81-207, over its pybind module
mcts_kernels.cu:2342-2366) are plain functions here with the same signatures:
``find_expansion_nodes``, ``batched_ucb_selection``, ``fused_select_expand``,
``fused_select_expand_optimized`` and ``batched_add_children``, and the rest of that module's
selection, noise, backup and subtree operators (mcts_kernels.cu:2342-2410):
``parallel_select_with_virtual_loss``, ``fused_ucb_with_noise``, ``batched_ucb_selection_dense``,
``batched_dirichlet_noise``, ``optimized_backup_scatter``, ``parallel_bfs_subtree`` and
``extract_subtree_edges``; mcts_gpu_accelerator.py of this package wraps them in the
reference's accelerator class.

There is no CPU implementation: tensors must be on a HIP device, and a missing library raises.
"""
from __future__ import annotations

import ctypes
import os

import torch

from . import _lib

TORCH_OPS_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libomq_torch_ops.so")


def _load_torch_ops() -> None:
    """Loads libomq_torch_ops.so (the omq:: operators), after the tree library it links."""
    if hasattr(torch.ops.omq, "vectorized_backup"):
        return
    if not os.path.exists(TORCH_OPS_PATH):
        raise _lib.LibraryNotBuilt(
            f"{TORCH_OPS_PATH} is missing: run __graft_entry__.build() (or python -m "
            "omoknuni_quantum_amd.build) to compile it")
    _lib.load()
    torch.ops.load_library(TORCH_OPS_PATH)


_load_torch_ops()


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
    torch.ops.omq.vectorized_backup(paths, path_lengths, values, visit_counts, value_sums)


def warp_vectorized_backup(paths: torch.Tensor, path_lengths: torch.Tensor, values: torch.Tensor,
                           visit_counts: torch.Tensor, value_sums: torch.Tensor) -> None:
    torch.ops.omq.warp_vectorized_backup(paths, path_lengths, values, visit_counts, value_sums)


def batch_apply_virtual_loss(node_indices: torch.Tensor,
                             virtual_loss_counts: torch.Tensor) -> None:
    torch.ops.omq.batch_apply_virtual_loss(node_indices, virtual_loss_counts)


def batch_remove_virtual_loss(node_indices: torch.Tensor,
                              virtual_loss_counts: torch.Tensor) -> None:
    torch.ops.omq.batch_remove_virtual_loss(node_indices, virtual_loss_counts)


def fused_ucb_selection(node_indices: torch.Tensor, children_start: torch.Tensor,
                        children_end: torch.Tensor, children: torch.Tensor,
                        q_values: torch.Tensor, visit_counts: torch.Tensor,
                        priors: torch.Tensor, c_puct: float) -> torch.Tensor:
    return torch.ops.omq.fused_ucb_selection(node_indices, children_start, children_end,
                                             children, q_values, visit_counts, priors,
                                             float(c_puct))


def _need(name: str, **tensors) -> None:
    """dtype checks: name=(tensor, dtype)."""
    for arg, (t, dt) in tensors.items():
        if t.dtype != dt:
            raise RuntimeError(f"omq::{name}: {arg} must be {dt}, not {t.dtype}")


# ---- the reference accelerator's operators -------------------------------------------------
# Plain functions with the signatures of the reference's pybind module
# (python/mcts/gpu/mcts_kernels.cu:2342-2366), as MCTSGPUAccelerator calls them.

def find_expansion_nodes(current_nodes: torch.Tensor, children: torch.Tensor,
                         visit_counts: torch.Tensor, valid_path_mask: torch.Tensor,
                         wave_size: int, max_children: int) -> torch.Tensor:
    """The nodes among current_nodes[:wave_size] (valid paths) whose children row holds no
    child and whose visit count is 0, in path order (find_expansion_nodes_cuda,
    mcts_kernels.cu:1329-1362).  Waits for the device to read the count, as the reference
    does."""
    dev = _check_device("find_expansion_nodes", current_nodes, children, visit_counts,
                        valid_path_mask)
    _need("find_expansion_nodes", current_nodes=(current_nodes, torch.int32),
          children=(children, torch.int32), visit_counts=(visit_counts, torch.int32),
          valid_path_mask=(valid_path_mask, torch.bool))
    wave_size, max_children = int(wave_size), int(max_children)
    if wave_size < 0 or max_children < 0:
        raise RuntimeError("omq::find_expansion_nodes: negative wave_size or max_children")
    if wave_size > current_nodes.numel() or wave_size > valid_path_mask.numel():
        raise RuntimeError(f"omq::find_expansion_nodes: wave_size {wave_size} exceeds the "
                           f"paths given ({current_nodes.numel()}, {valid_path_mask.numel()})")
    rows = children.numel() // max_children if max_children else visit_counts.numel()
    num_nodes = min(rows, visit_counts.numel())
    out = torch.empty(max(wave_size, 1), dtype=torch.int32, device=dev)
    count = torch.empty(1, dtype=torch.int32, device=dev)
    _lib.check(_lib.load().omq_find_expansion_nodes(
        current_nodes.data_ptr(), valid_path_mask.data_ptr(), wave_size, children.data_ptr(),
        max_children, visit_counts.data_ptr(), num_nodes, out.data_ptr(), count.data_ptr(),
        _stream(dev)), "omq_find_expansion_nodes")
    return out[:int(count.item())]


def batched_ucb_selection(q_values: torch.Tensor, visit_counts: torch.Tensor,
                          parent_visits: torch.Tensor, priors: torch.Tensor,
                          row_ptr: torch.Tensor, col_indices: torch.Tensor,
                          c_puct: float) -> torch.Tensor:
    """The row position of each CSR row's UCB maximum (batched_ucb_selection_cuda,
    mcts_kernels.cu:1412-1464); all -1 for an empty batch, no children, or arrays whose sizes
    disagree, as the reference returns."""
    dev = _check_device("batched_ucb_selection", q_values, visit_counts, parent_visits, priors,
                        row_ptr, col_indices)
    _need("batched_ucb_selection", q_values=(q_values, torch.float32),
          visit_counts=(visit_counts, torch.int32), parent_visits=(parent_visits, torch.int32),
          priors=(priors, torch.float32), row_ptr=(row_ptr, torch.int32),
          col_indices=(col_indices, torch.int32))
    batch, nc = parent_visits.numel(), q_values.numel()
    selected = torch.full((batch,), -1, dtype=torch.int32, device=dev)
    if batch == 0 or nc == 0 or visit_counts.numel() != nc or priors.numel() != nc or \
            col_indices.numel() != nc or row_ptr.numel() != batch + 1:
        return selected
    _lib.check(_lib.load().omq_batched_ucb_selection(
        q_values.data_ptr(), visit_counts.data_ptr(), nc, parent_visits.data_ptr(),
        priors.data_ptr(), row_ptr.data_ptr(), col_indices.data_ptr(), batch, float(c_puct),
        selected.data_ptr(), None, _stream(dev)), "omq_batched_ucb_selection")
    return selected


def _table(name: str, children: torch.Tensor) -> tuple[int, int]:
    if children.dim() != 2:
        raise RuntimeError(f"omq::{name}: children must be [num_nodes, max_children]")
    return int(children.shape[0]), int(children.shape[1])


def fused_select_expand(roots: torch.Tensor, children: torch.Tensor, visit_counts: torch.Tensor,
                        q_values: torch.Tensor, prior_probs: torch.Tensor,
                        is_expanded: torch.Tensor, max_depth: int, c_puct: float):
    """(paths [W, max_depth], path_lengths, expand_nodes, needs_expansion) of one descent per
    root (fused_select_expand_cuda, mcts_kernels.cu:2002-2045)."""
    name = "fused_select_expand"
    dev = _check_device(name, roots, children, visit_counts, q_values, prior_probs, is_expanded)
    _need(name, roots=(roots, torch.int32), children=(children, torch.int32),
          visit_counts=(visit_counts, torch.int32), q_values=(q_values, torch.float32),
          prior_probs=(prior_probs, torch.float32), is_expanded=(is_expanded, torch.bool))
    rows, mc = _table(name, children)
    num_nodes = min(rows, visit_counts.numel(), q_values.numel(), prior_probs.numel(),
                    is_expanded.numel())
    W, D = roots.numel(), int(max_depth)
    if D < 1:
        raise RuntimeError(f"omq::{name}: max_depth {D} < 1")
    paths = torch.empty((W, D), dtype=torch.int32, device=dev)
    plen = torch.empty(W, dtype=torch.int32, device=dev)
    expand = torch.empty(W, dtype=torch.int32, device=dev)
    needs = torch.empty(W, dtype=torch.bool, device=dev)
    _lib.check(_lib.load().omq_fused_select_expand(
        roots.data_ptr(), W, children.data_ptr(), num_nodes, mc, visit_counts.data_ptr(),
        q_values.data_ptr(), prior_probs.data_ptr(), is_expanded.data_ptr(), D, float(c_puct),
        paths.data_ptr(), plen.data_ptr(), expand.data_ptr(), needs.data_ptr(), _stream(dev)),
        "omq_fused_select_expand")
    return paths, plen, expand, needs


def fused_select_expand_optimized(root_nodes: torch.Tensor, children: torch.Tensor,
                                  visit_counts: torch.Tensor, value_sums: torch.Tensor,
                                  priors: torch.Tensor, max_depth: int, c_puct: float):
    """(paths [B, max_depth], path_lengths, ucb_scores [B, max_children]) of the reference's
    second descent (fused_select_expand_optimized_cuda, mcts_kernels.cu:2047-2083)."""
    name = "fused_select_expand_optimized"
    dev = _check_device(name, root_nodes, children, visit_counts, value_sums, priors)
    _need(name, root_nodes=(root_nodes, torch.int32), children=(children, torch.int32),
          visit_counts=(visit_counts, torch.int32), value_sums=(value_sums, torch.float32),
          priors=(priors, torch.float32))
    rows, mc = _table(name, children)
    num_nodes = min(rows, visit_counts.numel(), value_sums.numel(), priors.numel())
    B, D = root_nodes.numel(), int(max_depth)
    if D < 1:
        raise RuntimeError(f"omq::{name}: max_depth {D} < 1")
    paths = torch.empty((B, D), dtype=torch.int32, device=dev)
    plen = torch.empty(B, dtype=torch.int32, device=dev)
    ucb = torch.empty((B, mc), dtype=torch.float32, device=dev)
    _lib.check(_lib.load().omq_fused_select_expand_optimized(
        root_nodes.data_ptr(), B, children.data_ptr(), num_nodes, mc, visit_counts.data_ptr(),
        value_sums.data_ptr(), priors.data_ptr(), D, float(c_puct), ucb.data_ptr(),
        paths.data_ptr(), plen.data_ptr(), _stream(dev)), "omq_fused_select_expand_optimized")
    return paths, plen, ucb


def batched_add_children(parent_indices, actions, priors, num_children, node_counter,
                         edge_counter, children, parent_indices_out, parent_actions_out,
                         node_priors_out, visit_counts_out, value_sums_out, col_indices,
                         edge_actions, edge_priors, max_nodes, max_children,
                         max_edges) -> torch.Tensor:
    """Children appended for a batch of parents in batch order, updating the tree tensors in
    place (batched_add_children_cuda, mcts_kernels.cu:1679-1733); returns child_indices
    [batch * max_children], -1 where no child is written.  Array sizes are checked against
    max_nodes / max_children / max_edges (the reference writes past short arrays)."""
    name = "batched_add_children"
    ints = dict(parent_indices=parent_indices, actions=actions, num_children=num_children,
                node_counter=node_counter, edge_counter=edge_counter, children=children,
                parent_indices_out=parent_indices_out, parent_actions_out=parent_actions_out,
                visit_counts_out=visit_counts_out, col_indices=col_indices,
                edge_actions=edge_actions)
    floats = dict(priors=priors, node_priors_out=node_priors_out,
                  value_sums_out=value_sums_out, edge_priors=edge_priors)
    dev = _check_device(name, *ints.values(), *floats.values())
    _need(name, **{k: (v, torch.int32) for k, v in ints.items()},
          **{k: (v, torch.float32) for k, v in floats.items()})
    B, mn, mc, me = parent_indices.numel(), int(max_nodes), int(max_children), int(max_edges)
    if mn < 0 or me < 0 or mc < 1:
        raise RuntimeError(f"omq::{name}: max_nodes {mn}, max_edges {me} >= 0 and "
                           f"max_children {mc} >= 1")
    short = [k for k, t, n in (("actions", actions, B * mc), ("priors", priors, B * mc),
                               ("num_children", num_children, B),
                               ("node_counter", node_counter, 1),
                               ("edge_counter", edge_counter, 1),
                               ("children", children, mn * mc),
                               ("parent_indices_out", parent_indices_out, mn),
                               ("parent_actions_out", parent_actions_out, mn),
                               ("node_priors_out", node_priors_out, mn),
                               ("visit_counts_out", visit_counts_out, mn),
                               ("value_sums_out", value_sums_out, mn),
                               ("col_indices", col_indices, me),
                               ("edge_actions", edge_actions, me),
                               ("edge_priors", edge_priors, me)) if t.numel() < n]
    if short:
        raise RuntimeError(f"omq::{name}: arrays shorter than the sizes given: {short}")
    child_indices = torch.empty(B * mc, dtype=torch.int32, device=dev)  # every entry written
    if B == 0:
        return child_indices
    _lib.check(_lib.load().omq_batched_add_children(
        parent_indices.data_ptr(), B, actions.data_ptr(), priors.data_ptr(),
        num_children.data_ptr(), node_counter.data_ptr(), edge_counter.data_ptr(),
        children.data_ptr(), parent_indices_out.data_ptr(), parent_actions_out.data_ptr(),
        node_priors_out.data_ptr(), visit_counts_out.data_ptr(), value_sums_out.data_ptr(),
        col_indices.data_ptr(), edge_actions.data_ptr(), edge_priors.data_ptr(), mn, mc, me,
        child_indices.data_ptr(), _stream(dev)), "omq_batched_add_children")
    return child_indices


def parallel_select_with_virtual_loss(parent_nodes: torch.Tensor, children: torch.Tensor,
                                      visit_counts: torch.Tensor,
                                      virtual_loss_counts: torch.Tensor,
                                      value_sums: torch.Tensor, priors: torch.Tensor,
                                      dirichlet_noise=None, legal_masks=None,
                                      child_actions: torch.Tensor | None = None,
                                      c_puct: float = 1.0, virtual_loss_value: float = 1.0,
                                      dirichlet_epsilon: float = 0.0,
                                      apply_legal_mask: bool = False) -> torch.Tensor:
    """Per-simulation child selection with virtual-loss counts over the dense children table,
    then +1 virtual loss on every selected child (parallel_select_with_virtual_loss_enhanced_cuda,
    mcts_kernels.cu:1936-2000, bound at :2371-2384 with these argument names and defaults).
    priors is [num_nodes] or per simulation [num_sims, stride]; dirichlet_noise and
    dirichlet_epsilon are ignored, as in the reference (priors come pre-mixed); legal_masks
    [num_sims, actions] bool applies when apply_legal_mask is set (non-root parents only)."""
    name = "parallel_select_with_virtual_loss"
    if child_actions is None:
        raise RuntimeError(f"omq::{name}: child_actions is required")
    tensors = [parent_nodes, children, visit_counts, virtual_loss_counts, value_sums, priors,
               child_actions]
    use_mask = bool(apply_legal_mask) and legal_masks is not None
    if use_mask:
        tensors.append(legal_masks)
    dev = _check_device(name, *tensors)
    _need(name, parent_nodes=(parent_nodes, torch.int32), children=(children, torch.int32),
          visit_counts=(visit_counts, torch.int32),
          virtual_loss_counts=(virtual_loss_counts, torch.int32),
          value_sums=(value_sums, torch.float32), priors=(priors, torch.float32),
          child_actions=(child_actions, torch.int32))
    rows, mc = _table(name, children)
    num_nodes = min(visit_counts.numel(), virtual_loss_counts.numel(), value_sums.numel(),
                    child_actions.numel())
    S = parent_nodes.numel()
    if priors.dim() == 2:
        if priors.shape[0] < S:
            raise RuntimeError(f"omq::{name}: per-simulation priors hold {priors.shape[0]} rows "
                               f"for {S} simulations")
        pstride = int(priors.shape[1])
    else:
        num_nodes = min(num_nodes, priors.numel())
        pstride = 0
    A = 0
    if use_mask:
        _need(name, legal_masks=(legal_masks, torch.bool))
        if legal_masks.dim() != 2 or legal_masks.shape[0] < S:
            raise RuntimeError(f"omq::{name}: legal_masks must be [num_sims, actions]")
        A = int(legal_masks.shape[1])
    selected = torch.empty(S, dtype=torch.int32, device=dev)
    if S == 0:
        return selected
    _lib.check(_lib.load().omq_parallel_select_with_virtual_loss(
        parent_nodes.data_ptr(), S, children.data_ptr(), rows, mc, mc, visit_counts.data_ptr(),
        virtual_loss_counts.data_ptr(), value_sums.data_ptr(), num_nodes, priors.data_ptr(),
        pstride, legal_masks.data_ptr() if use_mask else None, A, child_actions.data_ptr(),
        float(c_puct), float(virtual_loss_value), selected.data_ptr(), _stream(dev)),
        "omq_parallel_select_with_virtual_loss")
    return selected


_NOISE_STREAM = {"seed": None, "counter": 0}


def set_noise_seed(seed: int) -> None:
    """Seed of batched_dirichlet_noise's draws (by default 64 bits from os.urandom, drawn at
    the first call, as the reference seeds its cuRAND states from the clock)."""
    _NOISE_STREAM["seed"] = int(seed) & ((1 << 64) - 1)
    _NOISE_STREAM["counter"] = 0


def batched_dirichlet_noise(num_sims: int, num_actions: int, alpha: float, epsilon: float,
                            device) -> torch.Tensor:
    """float32 [num_sims, num_actions] rows of Dirichlet(alpha) noise (batched_dirichlet_noise
    _cuda, mcts_kernels.cu:1735-1790; epsilon is unused there too).  Every call takes fresh
    draws: the stream's counter advances per call."""
    import os

    dev = torch.device(device)
    if dev.type != "cuda":
        raise RuntimeError(f"omq::batched_dirichlet_noise: {dev} is not a HIP device")
    num_sims, num_actions = int(num_sims), int(num_actions)
    if num_sims < 0 or num_actions < 0:
        raise RuntimeError("omq::batched_dirichlet_noise: negative size")
    if _NOISE_STREAM["seed"] is None:
        set_noise_seed(int.from_bytes(os.urandom(8), "little"))
    seed, counter = _NOISE_STREAM["seed"], _NOISE_STREAM["counter"]
    _NOISE_STREAM["counter"] = counter + 1
    noise = torch.zeros((num_sims, num_actions), dtype=torch.float32, device=dev)
    if num_sims * num_actions == 0:
        return noise
    _lib.check(_lib.load().omq_batched_dirichlet_noise(
        num_sims, num_actions, float(alpha), seed, counter, noise.data_ptr(),
        _stream(dev)), "omq_batched_dirichlet_noise")
    return noise


def fused_ucb_with_noise(q_values: torch.Tensor, visit_counts: torch.Tensor, priors: torch.Tensor,
                         dirichlet_noise: torch.Tensor, parent_visits_sqrt: float,
                         c_puct: float, epsilon: float) -> torch.Tensor:
    """int32 [num_sims]: per simulation, the position of the UCB maximum over the shared row
    with priors mixed with the simulation's noise row (fused_ucb_with_noise_cuda,
    mcts_kernels.cu:1791-1823)."""
    name = "fused_ucb_with_noise"
    dev = _check_device(name, q_values, visit_counts, priors, dirichlet_noise)
    _need(name, q_values=(q_values, torch.float32), visit_counts=(visit_counts, torch.int32),
          priors=(priors, torch.float32), dirichlet_noise=(dirichlet_noise, torch.float32))
    C = q_values.numel()
    if dirichlet_noise.dim() != 2 or dirichlet_noise.shape[1] != C or \
            visit_counts.numel() < C or priors.numel() < C:
        raise RuntimeError(f"omq::{name}: noise [num_sims, {C}] and {C} visit counts and priors "
                           "expected")
    S = int(dirichlet_noise.shape[0])
    selected = torch.zeros(S, dtype=torch.int32, device=dev)
    if S == 0:
        return selected
    _lib.check(_lib.load().omq_fused_ucb_with_noise(
        q_values.data_ptr(), visit_counts.data_ptr(), priors.data_ptr(), C,
        dirichlet_noise.data_ptr(), S, float(parent_visits_sqrt), float(c_puct), float(epsilon),
        selected.data_ptr(), _stream(dev)), "omq_fused_ucb_with_noise")
    return selected


def batched_ucb_selection_dense(batch_children: torch.Tensor, batch_priors: torch.Tensor,
                                parent_visits: torch.Tensor, child_visits: torch.Tensor,
                                child_values: torch.Tensor, valid_mask: torch.Tensor,
                                c_puct: float) -> torch.Tensor:
    """int32 [batch]: the child of each item's UCB maximum over its valid slots, -1 without
    one (batched_ucb_selection_dense_cuda, mcts_kernels.cu:1563-1598)."""
    name = "batched_ucb_selection_dense"
    dev = _check_device(name, batch_children, batch_priors, parent_visits, child_visits,
                        child_values, valid_mask)
    _need(name, batch_children=(batch_children, torch.int32),
          batch_priors=(batch_priors, torch.float32), parent_visits=(parent_visits, torch.int32),
          child_visits=(child_visits, torch.int32), child_values=(child_values, torch.float32),
          valid_mask=(valid_mask, torch.bool))
    if batch_children.dim() != 2:
        raise RuntimeError(f"omq::{name}: batch_children must be [batch, max_children]")
    B, M = int(batch_children.shape[0]), int(batch_children.shape[1])
    if batch_priors.shape != batch_children.shape or valid_mask.shape != batch_children.shape \
            or parent_visits.numel() < B:
        raise RuntimeError(f"omq::{name}: priors and valid_mask [batch, max_children] and one "
                           "parent count per item expected")
    nv = child_visits.numel()
    if child_values.numel() < nv:
        raise RuntimeError(f"omq::{name}: child_values shorter than child_visits")
    selected = torch.full((B,), -1, dtype=torch.int32, device=dev)
    if B == 0:
        return selected
    _lib.check(_lib.load().omq_batched_ucb_selection_dense(
        batch_children.data_ptr(), batch_priors.data_ptr(), parent_visits.data_ptr(),
        valid_mask.data_ptr(), B, M, child_visits.data_ptr(), child_values.data_ptr(), nv,
        float(c_puct), selected.data_ptr(), _stream(dev)), "omq_batched_ucb_selection_dense")
    return selected


def optimized_backup_scatter(paths: torch.Tensor, path_lengths: torch.Tensor,
                             values: torch.Tensor, visit_counts: torch.Tensor,
                             value_sums: torch.Tensor) -> None:
    """vectorized_backup under the reference's other name (optimized_backup_scatter_cuda,
    mcts_kernels.cu:1825-1870, runs vectorized_backup_kernel), through its own entry point."""
    name = "optimized_backup_scatter"
    dev = _check_device(name, paths, path_lengths, values, visit_counts, value_sums)
    _need(name, paths=(paths, torch.int32), path_lengths=(path_lengths, torch.int32),
          values=(values, torch.float32), visit_counts=(visit_counts, torch.int32),
          value_sums=(value_sums, torch.float32))
    if paths.dim() != 2:
        raise RuntimeError(f"omq::{name}: paths must be [batch, max_depth]")
    B, D = int(paths.shape[0]), int(paths.shape[1])
    if path_lengths.numel() != B or values.numel() != B:
        raise RuntimeError(f"omq::{name}: one length and one value per path")
    n = min(visit_counts.numel(), value_sums.numel())
    if B == 0 or n == 0 or D == 0:
        return
    _lib.check(_lib.load().omq_optimized_backup_scatter(
        paths.data_ptr(), path_lengths.data_ptr(), values.data_ptr(), B, D,
        visit_counts.data_ptr(), value_sums.data_ptr(), n, _stream(dev)),
        "omq_optimized_backup_scatter")


def parallel_bfs_subtree(row_ptr: torch.Tensor, col_indices: torch.Tensor, root_idx: int,
                         max_nodes: int):
    """(in_subtree bool [max_nodes], node_remap int32 [max_nodes], subtree_count int32 [1]) of
    the breadth-first subtree of root_idx (parallel_bfs_subtree_cuda, mcts_kernels.cu:
    2246-2287): new indices in FIFO breadth-first order, children in row order."""
    name = "parallel_bfs_subtree"
    dev = _check_device(name, row_ptr, col_indices)
    _need(name, row_ptr=(row_ptr, torch.int32), col_indices=(col_indices, torch.int32))
    max_nodes, root_idx = int(max_nodes), int(root_idx)
    if max_nodes <= 0 or not (0 <= root_idx < max_nodes):
        raise RuntimeError(f"omq::{name}: root_idx {root_idx} outside [0, max_nodes={max_nodes})")
    if row_ptr.numel() < max_nodes + 1:
        raise RuntimeError(f"omq::{name}: row_ptr holds {row_ptr.numel()} offsets, "
                           f"{max_nodes} nodes need {max_nodes + 1}")
    in_subtree = torch.empty(max_nodes, dtype=torch.bool, device=dev)
    remap = torch.empty(max_nodes, dtype=torch.int32, device=dev)
    count = torch.empty(1, dtype=torch.int32, device=dev)
    ws = torch.empty(_lib.bfs_workspace_ints(max_nodes), dtype=torch.int32, device=dev)
    _lib.check(_lib.load().omq_parallel_bfs_subtree(
        row_ptr.data_ptr(), col_indices.data_ptr(), col_indices.numel(), root_idx, max_nodes,
        in_subtree.data_ptr(), remap.data_ptr(), count.data_ptr(), ws.data_ptr(), ws.numel(),
        _stream(dev)), "omq_parallel_bfs_subtree")
    return in_subtree, remap, count


def extract_subtree_edges(row_ptr: torch.Tensor, col_indices: torch.Tensor, edge_actions,
                          in_subtree: torch.Tensor, node_remap: torch.Tensor, max_edges: int):
    """(edge_parents, edge_children, edge_actions int16) of the subtree's edges, remapped,
    nodes in ascending old index and edges in row order (extract_subtree_edges_cuda,
    mcts_kernels.cu:2289-2337).  Waits for the device to read the count, as the reference
    does; raises when the edges exceed max_edges (the reference writes past its arrays)."""
    name = "extract_subtree_edges"
    tensors = [row_ptr, col_indices, in_subtree, node_remap]
    if edge_actions is not None:
        tensors.append(edge_actions)
    dev = _check_device(name, *tensors)
    _need(name, row_ptr=(row_ptr, torch.int32), col_indices=(col_indices, torch.int32),
          in_subtree=(in_subtree, torch.bool), node_remap=(node_remap, torch.int32))
    if edge_actions is not None:
        _need(name, edge_actions=(edge_actions, torch.int16))
        if edge_actions.numel() < col_indices.numel():
            raise RuntimeError(f"omq::{name}: one action per edge expected")
    n = in_subtree.numel()
    if node_remap.numel() < n or row_ptr.numel() < n + 1:
        raise RuntimeError(f"omq::{name}: node_remap [{n}] and row_ptr [{n + 1}] expected")
    max_edges = int(max_edges)
    if max_edges < 0:
        raise RuntimeError(f"omq::{name}: max_edges {max_edges} < 0")
    parents = torch.zeros(max_edges, dtype=torch.int32, device=dev)
    children = torch.zeros(max_edges, dtype=torch.int32, device=dev)
    actions = torch.zeros(max_edges, dtype=torch.int16, device=dev)
    count = torch.zeros(1, dtype=torch.int32, device=dev)
    ws = torch.empty(_lib.edges_workspace_ints(n), dtype=torch.int32, device=dev)
    _lib.check(_lib.load().omq_extract_subtree_edges(
        row_ptr.data_ptr(), col_indices.data_ptr(),
        edge_actions.data_ptr() if edge_actions is not None else None, col_indices.numel(),
        in_subtree.data_ptr(), node_remap.data_ptr(), n, max_edges, parents.data_ptr(),
        children.data_ptr(), actions.data_ptr(), count.data_ptr(), ws.data_ptr(), ws.numel(),
        _stream(dev)), "omq_extract_subtree_edges")
    k = int(count.item())
    if k > max_edges:
        raise RuntimeError(f"omq::{name}: the subtree has {k} edges, max_edges is {max_edges}")
    return parents[:k], children[:k], actions[:k]


# the operators the reference registers under its own namespace (torch_custom_ops.py:26,71,108)
MCTS_ALIASES = ("vectorized_backup", "warp_vectorized_backup", "fused_ucb_selection")

REGISTERED: dict = {}


def _register() -> None:
    """Records the omq:: operators and registers the reference's names under mcts::.  A name
    already taken in the ``mcts`` namespace (the reference's own module imported first) is left
    to its owner."""
    for name in ("vectorized_backup", "warp_vectorized_backup", "fused_ucb_selection",
                 "batch_apply_virtual_loss", "batch_remove_virtual_loss"):
        REGISTERED[f"omq::{name}"] = getattr(torch.ops.omq, name)
    for name in MCTS_ALIASES:
        if not torch.ops.omq._mcts_aliased(name):
            if hasattr(torch.ops, "mcts") and hasattr(torch.ops.mcts, name):
                continue
            torch.ops.omq._alias_mcts(name)
        REGISTERED[f"mcts::{name}"] = getattr(torch.ops.mcts, name)


_register()
