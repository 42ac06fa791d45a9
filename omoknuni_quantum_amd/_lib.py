"""ctypes binding of libomq_tree_ops.so (the C ABI declared in include/omq_tree_ops.h).

The library is loaded from the package directory; there is no fallback.  A missing or
stale library raises ``LibraryNotBuilt`` so that no caller silently runs anything else.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_NAME = "libomq_tree_ops.so"
LIB_PATH = os.path.join(_HERE, LIB_NAME)

ABI_VERSION = 4

# constants of include/omq_tree_ops.h
OMQ_OK, OMQ_E_ARG, OMQ_E_LAUNCH, OMQ_E_LIMIT = 0, -1, -2, -3
OMQ_GAME_BOARD, OMQ_GAME_GO, OMQ_GAME_SPARSE = 0, 1, 2
OMQ_EXPAND_FULL, OMQ_EXPAND_REFERENCE_PW = 0, 1
OMQ_SIGN_LEAF_POSITIVE, OMQ_SIGN_ROOT_POSITIVE = 0, 1
OMQ_WACC_ORDERED, OMQ_WACC_ATOMIC = 0, 1
OMQ_MAX_WAVE, OMQ_MAX_ROW, OMQ_MAX_DEPTH, OMQ_MAX_ACTIONS = 4096, 512, 128, 8192
OMQ_SELECT_RECORDS_MAX_WAVE = 512
OMQ_NSTATS = 16
STAT_NAMES = [
    "internal", "rowsum", "pathnodes", "pathentries", "uleaves", "expanded", "newchild",
    "sims", "steps", "capfail", "uleafpath", "rootchain",
]
OMQ_STATUS_NOCHILD, OMQ_STATUS_ROWLIMIT, OMQ_STATUS_STALL, OMQ_STATUS_COUNTLIMIT = 1, 2, 4, 8
OMQ_RULE_FREESTYLE, OMQ_RULE_RENJU = 0, 1
OMQ_TERM_NONE, OMQ_TERM_WIN1, OMQ_TERM_WIN2, OMQ_TERM_DRAW, OMQ_TERM_END = 0, 1, 2, 3, 4
OMQ_GO_KO, OMQ_GO_SUICIDE = 1, 2
OMQ_SHIFT_WORKSPACE_PER_NODE = 8
OMQ_NOALLOC_SHIFT_INTS = 8 * 1024 * 1024
OMQ_DTYPE_F32, OMQ_DTYPE_BF16 = 0, 1
OMQ_LAYOUT_NCHW, OMQ_LAYOUT_NHWC = 0, 1

_p = ctypes.c_void_p
_i32 = ctypes.c_int32


class OmqForest(ctypes.Structure):
    _fields_ = [
        ("num_trees", _i32), ("capacity", _i32), ("num_actions", _i32), ("game", _i32),
        ("legal_words", _i32), ("min_legal", _i32), ("max_legal", _i32), ("reserved", _i32),
        ("visit_counts", _p), ("value_sums", _p), ("priors", _p), ("parents", _p),
        ("first_child", _p), ("num_children", _p), ("actions", _p), ("num_nodes", _p),
        ("root_keys", _p), ("root_legal", _p),
    ]


class OmqWave(ctypes.Structure):
    _fields_ = [
        ("max_wave", _i32), ("max_depth", _i32),
        ("paths", _p), ("path_len", _p), ("leaves", _p), ("sim_uid", _p), ("uleaf", _p),
        ("ufirst", _p), ("ucount", _p), ("glog", _p), ("gcount", _p), ("gmembers", _p),
        ("ukey", _p), ("ulegal", _p), ("uedge", _p), ("unew", _p), ("policy", _p),
        ("values", _p), ("sim_value", _p), ("stats", _p), ("status", _p), ("sel_scratch", _p),
        ("umask", _p),
    ]


def sel_scratch_ints(T: int, MW: int) -> int:
    """OMQ_SEL_SCRATCH_INTS of include/omq_tree_ops.h."""
    return 2 * T * MW


OMQ_SPIN_LIMIT_DEFAULT = 1 << 22


# exported symbols and their signatures (name -> (restype, argtypes))
_FP = ctypes.POINTER(OmqForest)
_WP = ctypes.POINTER(OmqWave)
SIGNATURES = {
    "omq_abi_version": (ctypes.c_int, []),
    "omq_last_error": (ctypes.c_char_p, []),
    "omq_forest_reset": (ctypes.c_int, [_FP, _p]),
    "omq_select": (ctypes.c_int, [_FP, _WP, _i32, ctypes.c_float, ctypes.c_float, _i32, _i32, _p]),
    "omq_leaf_info": (ctypes.c_int, [_FP, _WP, _p]),
    "omq_expand_backup": (ctypes.c_int, [_FP, _WP, _i32, ctypes.c_float, _i32, _p,
                                         ctypes.c_double, _i32, _i32, _p]),
    "omq_select_options": (ctypes.c_int, [_i32]),
    "omq_select_spin_limit": (ctypes.c_int32, []),
    "omq_wall_clock_khz": (ctypes.c_int, [_p]),
    "omq_synthetic_evaluate": (ctypes.c_int, [_FP, _WP, ctypes.c_float, _p]),
    "omq_expand": (ctypes.c_int, [_FP, _WP, _i32, ctypes.c_float, _i32, _p, ctypes.c_double, _p]),
    "omq_backup": (ctypes.c_int, [_FP, _WP, _i32, ctypes.c_float, _i32, _i32, _p]),
    "omq_paths_backup": (ctypes.c_int, [_FP, _p, _p, _p, _p, _i32, _i32, _i32, _p]),
    "omq_virtual_loss": (ctypes.c_int, [_FP, _p, _p, _i32, _i32, _p]),
    "omq_gomoku_terminal": (ctypes.c_int, [_FP, _WP, _p, _p, _i32, _p, _p]),
    "omq_go_rules": (ctypes.c_int, [_FP, _WP, _p, _p, _p, _p, _i32, _p, _p]),
    "omq_shift_root": (ctypes.c_int, [_FP, _p, _p, ctypes.c_int64, _p]),
    "omq_shift_root_noalloc": (ctypes.c_int, [_FP, _p, _p]),
    "omq_leaf_features": (ctypes.c_int, [_FP, _WP, _p, _p, _p, _i32, _i32, _i32, _p, _p]),
    "omq_fused_ucb_selection": (ctypes.c_int, [_p, _i32, _p, _p, _p, _p, _p, _p, ctypes.c_float,
                                               _p, _p]),
    "omq_find_expansion_nodes": (ctypes.c_int, [_p, _p, _i32, _p, _i32, _p, _i32, _p, _p, _p]),
    "omq_batched_ucb_selection": (ctypes.c_int, [_p, _p, _i32, _p, _p, _p, _p, _i32,
                                                 ctypes.c_float, _p, _p, _p]),
    "omq_fused_select_expand": (ctypes.c_int, [_p, _i32, _p, _i32, _i32, _p, _p, _p, _p, _i32,
                                               ctypes.c_float, _p, _p, _p, _p, _p]),
    "omq_fused_select_expand_optimized": (ctypes.c_int, [_p, _i32, _p, _i32, _i32, _p, _p, _p,
                                                         _i32, ctypes.c_float, _p, _p, _p, _p]),
    "omq_batched_add_children": (ctypes.c_int, [_p, _i32, _p, _p, _p, _p, _p, _p, _p, _p, _p,
                                                _p, _p, _p, _p, _p, _i32, _i32, _i32, _p, _p]),
    "omq_root_policy": (ctypes.c_int, [_FP, _p, _p]),
    "omq_sample_actions": (ctypes.c_int, [_FP, _p, ctypes.c_double, ctypes.c_uint64,
                                          ctypes.c_uint64, _p, _p]),
    "omq_root_dirichlet": (ctypes.c_int, [_FP, ctypes.c_double, ctypes.c_uint64,
                                          ctypes.c_uint64, _p, _p]),
    "omq_parallel_select_with_virtual_loss": (ctypes.c_int, [_p, _i32, _p, _i32, _i32, _i32, _p,
                                                             _p, _p, _i32, _p, _i32, _p, _i32, _p,
                                                             ctypes.c_float, ctypes.c_float, _p,
                                                             _p]),
    "omq_fused_ucb_with_noise": (ctypes.c_int, [_p, _p, _p, _i32, _p, _i32, ctypes.c_float,
                                                ctypes.c_float, ctypes.c_float, _p, _p]),
    "omq_batched_ucb_selection_dense": (ctypes.c_int, [_p, _p, _p, _p, _i32, _i32, _p, _p, _i32,
                                                       ctypes.c_float, _p, _p]),
    "omq_batched_dirichlet_noise": (ctypes.c_int, [_i32, _i32, ctypes.c_double, ctypes.c_uint64,
                                                   ctypes.c_uint64, _p, _p]),
    "omq_optimized_backup_scatter": (ctypes.c_int, [_p, _p, _p, _i32, _i32, _p, _p, _i32, _p]),
    "omq_parallel_bfs_subtree": (ctypes.c_int, [_p, _p, _i32, _i32, _i32, _p, _p, _p, _p,
                                                ctypes.c_int64, _p]),
    "omq_extract_subtree_edges": (ctypes.c_int, [_p, _p, _p, _i32, _p, _p, _i32, _i32, _p, _p,
                                                 _p, _p, _p, ctypes.c_int64, _p]),
}


def bfs_workspace_ints(max_nodes: int) -> int:
    """OMQ_BFS_WORKSPACE_INTS of include/omq_tree_ops.h."""
    return 3 * max_nodes + 1


def edges_workspace_ints(num_nodes: int) -> int:
    """OMQ_EDGES_WORKSPACE_INTS of include/omq_tree_ops.h."""
    return num_nodes + (num_nodes + 1023) // 1024 + 1


class LibraryNotBuilt(RuntimeError):
    pass


class OmqError(RuntimeError):
    pass


_lib = None
_lock = threading.Lock()


def load(path: str | None = None) -> ctypes.CDLL:
    """Load the HIP library once; raise LibraryNotBuilt when it is absent.  torch is imported
    first: the library then binds the HIP runtime torch has loaded, so that both share one
    runtime (loaded first, the library would bring the system's and torch its own, and the
    second runtime finds no device)."""
    global _lib
    import torch  # noqa: F401  (the HIP runtime the library shares)

    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or LIB_PATH
        if not os.path.exists(p):
            raise LibraryNotBuilt(
                f"{p} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
                " (hipcc --offload-arch=gfx950); there is no fallback implementation")
        lib = ctypes.CDLL(p)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.omq_abi_version() != ABI_VERSION:
            raise LibraryNotBuilt(f"{p} has ABI {lib.omq_abi_version()}, expected {ABI_VERSION}")
        if path is None:
            _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc != OMQ_OK:
        msg = load().omq_last_error()
        raise OmqError(f"{what} failed ({rc}): {msg.decode() if msg else ''}")
