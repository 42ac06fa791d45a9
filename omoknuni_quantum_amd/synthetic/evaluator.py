"""Seeded synthetic evaluator (device side).

For every unique leaf of a wave: priors = softmax over the leaf's legal actions of
``logit_scale * z(key, a)``, z an Irwin-Hall(12) approximately standard-normal draw hashed from
the leaf key and the action; value = 2u - 1 with u a 24-bit hash fraction of the key.  The
kernel writes the priors into the policy rows at the legal action slots only (the expansion
gathers exactly those slots).  It stands in for ``Evaluator.evaluate_batch``
(python/mcts/core/evaluator.py:85-104 of the reference) in the benchmark workloads, and is
timed apart from the tree operations.
"""
from __future__ import annotations

from .. import _lib


class SyntheticEvaluator:
    """Device-native evaluator: evaluates the unique leaves held in a WaveEngine."""

    device_native = True

    def __init__(self, logit_scale: float = 1.0):
        self.logit_scale = float(logit_scale)
        self.stats = {"evaluations": 0, "batch_evaluations": 0}

    def graph_key(self) -> tuple:
        """evaluate_wave only launches a kernel whose one host argument is logit_scale, so a
        search with it can be recorded as a HIP graph (MCTS use_cuda_graphs)."""
        return ("synthetic", self.logit_scale)

    def evaluate_wave(self, engine) -> None:
        lib = _lib.load()
        _lib.check(lib.omq_synthetic_evaluate(engine.forest_ref, engine.wave_ref,
                                              self.logit_scale, engine.stream_handle()),
                   "omq_synthetic_evaluate")
        self.stats["batch_evaluations"] += 1

    def evaluate_batch(self, states, legal_masks=None, temperature: float = 1.0):
        raise NotImplementedError(
            "SyntheticEvaluator derives its outputs from tree-node keys on the device; it is "
            "driven through evaluate_wave by the MCTS engine, not through feature batches")
