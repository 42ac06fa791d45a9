"""MI355X-native (gfx950) wave-MCTS tree operations behind the MCTS / MCTSConfig API.

The tree operations (PUCT selection with virtual loss, expansion into CSR arrays, backup)
run as hand-written HIP kernels in libomq_tree_ops.so, reached through its C ABI
(include/omq_tree_ops.h) with ctypes; torch provides device memory and streams.
"""
__version__ = "0.1.0"
