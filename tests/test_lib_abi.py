"""The C-ABI library loads on a host without a GPU, exports every entry point that
include/omq_tree_ops.h declares, and rejects invalid arguments before touching a device."""
import ctypes
import os
import re

import pytest

from omoknuni_quantum_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "omq_tree_ops.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(omq_[a-z_]+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    names = declared_functions()
    for n in ("omq_select", "omq_expand", "omq_backup", "omq_forest_reset", "omq_leaf_info",
              "omq_synthetic_evaluate", "omq_paths_backup", "omq_virtual_loss",
              "omq_gomoku_terminal", "omq_leaf_features", "omq_last_error",
              "omq_abi_version"):
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, name
    assert lib.omq_abi_version() == _lib.ABI_VERSION


def test_struct_layout_matches_header():
    # two int32 per 8 bytes, then pointers: offsets the C compiler uses
    assert ctypes.sizeof(_lib.OmqForest) == 8 * 4 + 10 * 8
    assert _lib.OmqForest.visit_counts.offset == 32
    assert ctypes.sizeof(_lib.OmqWave) == 8 + 21 * 8
    assert _lib.OmqWave.paths.offset == 8


def _forest(**kw):
    f = _lib.OmqForest()
    f.num_trees, f.capacity, f.num_actions, f.game = 1, 16, 25, _lib.OMQ_GAME_BOARD
    f.legal_words = 1
    for name in ("visit_counts", "value_sums", "priors", "parents", "first_child",
                 "num_children", "actions", "num_nodes", "root_keys", "root_legal"):
        setattr(f, name, 8)  # never dereferenced: the calls below fail validation first
    for k, v in kw.items():
        setattr(f, k, v)
    return f


@pytest.mark.parametrize("bad,msg", [
    ({"num_trees": 0}, "must be positive"),
    ({"num_actions": 9000}, "num_actions"),
    ({"game": 7}, "unknown game model"),
    ({"legal_words": 3}, "legal_words"),
    ({"num_actions": 600, "legal_words": 19}, "row limit"),
    ({"game": _lib.OMQ_GAME_SPARSE, "min_legal": 10, "max_legal": 80}, "sparse legal range"),
    ({"visit_counts": None}, "null array"),
])
def test_invalid_forest_rejected(bad, msg):
    lib = _lib.load()
    f = _forest(**bad)
    rc = lib.omq_forest_reset(ctypes.byref(f), None)
    assert rc == _lib.OMQ_E_ARG or rc == _lib.OMQ_E_LIMIT
    assert msg in lib.omq_last_error().decode()
    with pytest.raises(_lib.OmqError):
        _lib.check(rc, "omq_forest_reset")


def test_invalid_wave_arguments_rejected():
    lib = _lib.load()
    f = _forest()
    w = _lib.OmqWave()
    w.max_wave, w.max_depth = 8, 16
    rc = lib.omq_select(ctypes.byref(f), ctypes.byref(w), 4, 1.4, 3.0, 16, 0, None)
    assert rc == _lib.OMQ_E_ARG and "null array" in lib.omq_last_error().decode()
    for name, _ in _lib.OmqWave._fields_[2:]:
        setattr(w, name, 8)
    assert lib.omq_select(ctypes.byref(f), ctypes.byref(w), 9, 1.4, 3.0, 16, 0, None) == _lib.OMQ_E_ARG
    assert "wave_size" in lib.omq_last_error().decode()
    assert lib.omq_select(ctypes.byref(f), ctypes.byref(w), 4, 1.4, -1.0, 16, 0, None) == _lib.OMQ_E_ARG
    assert lib.omq_select(ctypes.byref(f), ctypes.byref(w), 4, 1.4, 3.0, 17, 0, None) == _lib.OMQ_E_ARG
    w.max_wave = 5000
    assert lib.omq_select(ctypes.byref(f), ctypes.byref(w), 4, 1.4, 3.0, 16, 0, None) == _lib.OMQ_E_LIMIT
    w.max_wave = 8
    assert lib.omq_expand(ctypes.byref(f), ctypes.byref(w), 4, 3.0, 5, None, 0.0, None) == _lib.OMQ_E_ARG
    assert lib.omq_expand(ctypes.byref(f), ctypes.byref(w), 4, 3.0, 0, None, 2.0, None) == _lib.OMQ_E_ARG
    assert lib.omq_backup(ctypes.byref(f), ctypes.byref(w), 4, 3.0, 9, 0, None) == _lib.OMQ_E_ARG
    assert lib.omq_backup(ctypes.byref(f), ctypes.byref(w), 4, 3.0, 0, 9, None) == _lib.OMQ_E_ARG
    assert lib.omq_paths_backup(ctypes.byref(f), None, None, None, None, 0, 4, 0, None) == 0
    assert lib.omq_virtual_loss(ctypes.byref(f), None, None, -1, 3, None) == _lib.OMQ_E_ARG
    # gomoku terminal check: square board forests only, a board array, a known rule
    assert lib.omq_gomoku_terminal(ctypes.byref(f), ctypes.byref(w), None, None, 0, None,
                                   None) == _lib.OMQ_E_ARG
    assert "root_boards" in lib.omq_last_error().decode()
    assert lib.omq_gomoku_terminal(ctypes.byref(f), ctypes.byref(w), 8, None, 5, None,
                                   None) == _lib.OMQ_E_ARG
    assert "rule" in lib.omq_last_error().decode()
    g = _forest(num_actions=24)
    assert lib.omq_gomoku_terminal(ctypes.byref(g), ctypes.byref(w), 8, None, 0, None,
                                   None) == _lib.OMQ_E_ARG
    assert "square" in lib.omq_last_error().decode()
    g = _forest(game=_lib.OMQ_GAME_GO, num_actions=26)
    assert lib.omq_gomoku_terminal(ctypes.byref(g), ctypes.byref(w), 8, None, 0, None,
                                   None) == _lib.OMQ_E_ARG
    # feature planes: square board forests, boards and output, 18 or 19 planes, known formats
    assert lib.omq_leaf_features(ctypes.byref(f), ctypes.byref(w), None, None, None, 19, 0, 0,
                                 8, None) == _lib.OMQ_E_ARG
    assert "root_boards" in lib.omq_last_error().decode()
    assert lib.omq_leaf_features(ctypes.byref(f), ctypes.byref(w), 8, None, None, 17, 0, 0, 8,
                                 None) == _lib.OMQ_E_ARG
    assert "planes" in lib.omq_last_error().decode()
    assert lib.omq_leaf_features(ctypes.byref(f), ctypes.byref(w), 8, None, None, 18, 2, 0, 8,
                                 None) == _lib.OMQ_E_ARG
    assert "dtype" in lib.omq_last_error().decode()
    assert lib.omq_leaf_features(ctypes.byref(f), ctypes.byref(w), 8, None, None, 18, 1, 3, 8,
                                 None) == _lib.OMQ_E_ARG
    assert "layout" in lib.omq_last_error().decode()
    assert lib.omq_leaf_features(ctypes.byref(g), ctypes.byref(w), 8, None, None, 18, 0, 0, 8,
                                 None) == _lib.OMQ_E_ARG
    assert lib.omq_leaf_features(ctypes.byref(f), ctypes.byref(w), 8, None, None, 18, 0, 0, 12,
                                 None) == _lib.OMQ_E_ARG
    assert "aligned" in lib.omq_last_error().decode()


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(_lib.LibraryNotBuilt):
        _lib.load(str(tmp_path / "absent.so"))


def test_torch_ops_registered_and_refuse_host_tensors():
    import torch

    from omoknuni_quantum_amd import torch_ops  # noqa: F401

    for name in ("vectorized_backup", "batch_apply_virtual_loss", "batch_remove_virtual_loss"):
        assert hasattr(torch.ops.omq, name)
    p = torch.zeros((2, 3), dtype=torch.int32)
    with pytest.raises(RuntimeError, match="HIP device"):
        torch.ops.omq.vectorized_backup(p, torch.zeros(2, dtype=torch.int32), torch.zeros(2),
                                        torch.zeros(4, dtype=torch.int32), torch.zeros(4))
    with pytest.raises(RuntimeError, match="HIP device"):
        torch.ops.omq.batch_apply_virtual_loss(torch.zeros(2, dtype=torch.int32),
                                               torch.zeros(4, dtype=torch.int32))


def test_primitives_need_only_counts():
    """omq_paths_backup / omq_virtual_loss read only N (and W) of the forest."""
    lib = _lib.load()
    f = _lib.OmqForest()
    f.num_trees, f.capacity = 1, 10
    assert lib.omq_virtual_loss(ctypes.byref(f), None, None, 0, 1, None) == _lib.OMQ_E_ARG
    f.visit_counts = 8
    assert lib.omq_virtual_loss(ctypes.byref(f), None, None, 0, 1, None) == _lib.OMQ_OK
    assert lib.omq_paths_backup(ctypes.byref(f), None, None, None, None, 1, 4, 0, None) == _lib.OMQ_E_ARG
    assert "null" in lib.omq_last_error().decode()


def test_reference_operator_names_registered():
    """torch.ops.mcts carries the reference's three operators (torch_custom_ops.py:26,71,108),
    as AsyncWaveSearch probes for them (async_wave_search.py:255-260), beside torch.ops.omq."""
    import torch

    from omoknuni_quantum_amd import torch_ops

    for name in ("vectorized_backup", "warp_vectorized_backup", "fused_ucb_selection"):
        assert hasattr(torch.ops.mcts, name), name
        assert hasattr(torch.ops.omq, name), name
    assert {"omq::batch_apply_virtual_loss", "omq::batch_remove_virtual_loss"} <= set(
        torch_ops.REGISTERED)


def test_noalloc_shift_root_limit():
    """omq_shift_root_noalloc refuses forests beyond its own workspace, and a missing
    new_roots, before anything reaches the device."""
    lib = _lib.load()
    cap = _lib.OMQ_NOALLOC_SHIFT_INTS // _lib.OMQ_SHIFT_WORKSPACE_PER_NODE // 2 + 1
    f = _forest(num_trees=2, capacity=cap)
    assert lib.omq_shift_root_noalloc(ctypes.byref(f), 8, None) == _lib.OMQ_E_LIMIT
    msg = lib.omq_last_error().decode()
    assert "omq_shift_root_noalloc" in msg and str(_lib.OMQ_NOALLOC_SHIFT_INTS) in msg
    g = _forest(num_trees=2, capacity=cap - 1)
    assert lib.omq_shift_root_noalloc(ctypes.byref(g), None, None) == _lib.OMQ_E_ARG


def test_torch_ops_come_from_the_cpp_library():
    """The omq:: operators (and the reference's mcts:: names) are registered by the C++ library
    libomq_torch_ops.so with the reference's schemas; their Meta kernels give the shapes."""
    import torch

    from omoknuni_quantum_amd import torch_ops

    backup = ("(Tensor paths, Tensor path_lengths, Tensor values, Tensor(a!) visit_counts, "
              "Tensor(b!) value_sums) -> ()")
    for ns in ("omq", "mcts"):
        for name in ("vectorized_backup", "warp_vectorized_backup"):
            assert str(getattr(getattr(torch.ops, ns), name).default._schema) == \
                f"{ns}::{name}{backup}"
        assert f"{ns}::fused_ucb_selection" in torch_ops.REGISTERED
        assert torch.ops.omq._mcts_aliased("fused_ucb_selection")
    dump = torch._C._dispatch_dump("omq::vectorized_backup")
    assert "torch_ops.cpp" in dump
    m = torch.empty(5, dtype=torch.int32, device="meta")
    f = m.float()
    assert torch.ops.omq.fused_ucb_selection(m, m, m, m, f, m, f, 1.4).shape == (5,)


def test_mcts_name_taken_first_is_left_to_its_owner():
    """A module that registered mcts::vectorized_backup before this package keeps it."""
    import os
    import subprocess
    import sys

    code = (
        "import torch\n"
        "@torch.library.custom_op('mcts::vectorized_backup', mutates_args=('visit_counts', "
        "'value_sums'))\n"
        "def vb(paths: torch.Tensor, path_lengths: torch.Tensor, values: torch.Tensor, "
        "visit_counts: torch.Tensor, value_sums: torch.Tensor) -> None:\n"
        "    pass\n"
        "from omoknuni_quantum_amd import torch_ops\n"
        "assert 'mcts::vectorized_backup' not in torch_ops.REGISTERED\n"
        "assert not torch.ops.omq._mcts_aliased('vectorized_backup')\n"
        "assert 'mcts::fused_ucb_selection' in torch_ops.REGISTERED\n"
        "print('ok')\n")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", code], cwd=root, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout + r.stderr
