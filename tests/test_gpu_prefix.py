"""The first-unvisited prefix of the select chains at the edges of its blocks: a crafted root
whose unvisited children (scattered among visited ones) number around a multiple of 64, with
waves that end inside the prefix, at its end and past it, under the kernels of 1, 4 and 6 slots
per lane (the last two start their chains after a partial prefix).  Every simulation's pick and
the visit counts after the wave must equal the C oracle's, which runs select_path one
simulation at a time."""
import numpy as np
import pytest
import torch

from omoknuni_quantum_amd.core.engine import SearchParams, WaveEngine
from oracle import golden

pytestmark = pytest.mark.gpu
F32 = np.float32


def _cases():
    rng = np.random.default_rng(77)
    out = []
    for model, k, unv in (("go:19", 362, (63, 64, 65, 127, 200)), ("gomoku:15", 225, (64, 65)),
                          ("sparse", 45, (10, 44))):
        for u in unv:
            for dm in (-1, 0, 37):
                m = u + dm
                Nc = rng.integers(1, 30, k).astype(np.int32)
                Nc[rng.choice(k, u, replace=False)] = 0
                Wc = (Nc * rng.uniform(-1, 1, k)).astype(F32)
                Pc = rng.dirichlet([0.3] * k).astype(F32)
                out.append({"kind": f"prefix u={u} m={m}", "model": model, "k": k, "m": m,
                            "c": 1.4, "vl": 3.0, "N0": int(Nc.sum()) + 1, "N": Nc, "W": Wc,
                            "P": Pc})
    return out


def _put(t: torch.Tensor, values, dtype) -> None:
    v = torch.from_numpy(np.ascontiguousarray(values, dtype=dtype))
    t[:v.numel()].copy_(v)


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"{c['model']}-{c['kind']}")
def test_prefix_block_edges(device, case):
    k, m = case["k"], case["m"]
    want_picks, want_n = golden.crafted_expected_oracle(case)
    model = golden.model_from_name(case["model"])
    eng = WaveEngine(model, 1, k + 1, m, 100, device,
                     SearchParams(c_puct=case["c"], virtual_loss=case["vl"]))
    eng.reset()
    _put(eng.N, np.concatenate([[case["N0"]], case["N"]]), np.int32)
    _put(eng.W, np.concatenate([[0.0], case["W"]]), np.float32)
    _put(eng.P, np.concatenate([[1.0], case["P"]]), np.float32)
    _put(eng.parent, [-1] + [0] * k, np.int32)
    _put(eng.first, [0] + [-1] * k, np.int32)
    _put(eng.nchild, [k] + [0] * k, np.int32)
    _put(eng.action, [-1] + list(range(k)), np.int32)
    _put(eng.num_nodes, [k + 1], np.int32)
    print(f"prefix case {case['model']} {case['kind']}", flush=True)
    eng.select(m)
    torch.cuda.synchronize()
    plen = eng.path_len[:m].cpu().numpy()
    paths = eng.paths.view(m, eng.MD)[:, :2].cpu().numpy()
    picks = np.where(plen > 1, paths[:, 1] - 1, -1)
    assert np.array_equal(picks, want_picks)
    assert np.array_equal(eng.N[:k + 1].cpu().numpy(), want_n)
    # the prefix takes the unvisited children first, in index order
    u = int((case["N"] == 0).sum())
    assert picks[:min(u, m)].tolist() == np.flatnonzero(case["N"] == 0)[:min(u, m)].tolist()
