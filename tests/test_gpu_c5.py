"""Workload C5: the tree operations driven by the bf16 ResNet evaluator, with the evaluator's
outputs replayed into the oracle (bit-exact trees)."""
import numpy as np
import pytest
import torch

from omoknuni_quantum_amd.core.engine import SearchParams, WaveEngine
from omoknuni_quantum_amd.synthetic.resnet_evaluator import ResNetEvaluator
from omoknuni_quantum_amd.synthetic.workloads import get
from oracle.oracle import Oracle


def _replay_parity(wl, device, num_blocks, channels):
    params = SearchParams(c_puct=wl.c_puct, virtual_loss=wl.virtual_loss, max_depth=wl.max_depth)
    eng = WaveEngine(wl.model, wl.num_trees, wl.capacity, wl.wave_size, wl.max_depth, device,
                     params)
    keys, legal, noise = wl.root_inputs()
    eng.set_roots(keys, legal, noise)
    boards = torch.from_numpy(wl.boards()).to(device)
    ev = ResNetEvaluator(eng, boards, num_blocks=num_blocks, channels=channels, record=True)
    eng.search(wl.num_simulations, wl.wave_size, ev)
    torch.cuda.synchronize()
    eng.check_status()
    sizes = [1] + [wl.wave_size] * (wl.num_simulations // wl.wave_size)
    assert len(ev.calls) == len(sizes)
    pol0 = ev.calls[1][0]
    assert np.allclose(pol0.sum(axis=2), 1.0, atol=1e-3)  # probabilities over all 225 slots
    orc = Oracle(wl.model, wl.num_trees, wl.capacity, wl.wave_size, wl.max_depth)
    orc.set_params(wl.c_puct, wl.virtual_loss, 0, 0, 1.0, 0.0)
    orc.set_roots(keys, legal, noise)
    for t in range(wl.num_trees):
        orc.reset_tree(t)
        for (pol, val), W in zip(ev.calls, sizes):
            orc.wave(t, W, replay_policy=pol[t], replay_values=val[t])
        g, o = eng.host_tree(t), orc.tree(t)
        assert g["num_nodes"] == o["num_nodes"]
        for k in ("N", "parent", "first", "nchild", "action"):
            assert np.array_equal(g[k], o[k]), (t, k)
        for k in ("W", "P"):
            assert np.array_equal(g[k].view(np.int32), o[k].view(np.int32)), (t, k)
        assert int(g["N"][0]) == 2 + wl.num_simulations


@pytest.mark.gpu
def test_c5_resnet_replay_parity(device):
    wl = get("C5").scaled(num_trees=4, num_simulations=96, capacity=50_000)
    _replay_parity(wl, device, num_blocks=2, channels=32)


@pytest.mark.gpu
def test_c5_full_network_fullcount_replay_parity(device):
    """C5's own network (10 blocks x 128 channels, bf16) on two trees at C5's full simulation
    count, wave and capacity (1600 simulations in waves of 16 slots per tree, 400k nodes)."""
    wl = get("C5").scaled(num_trees=2)
    assert wl.num_simulations == 1600 and wl.wave_size == 16 and wl.capacity == 400_000
    print(f"[c5] T={wl.num_trees} sims={wl.num_simulations} W={wl.wave_size}", flush=True)
    _replay_parity(wl, device, num_blocks=10, channels=128)


def test_resnet_architecture_shapes():
    from omoknuni_quantum_amd.synthetic.resnet_evaluator import AlphaZeroResNet

    net = AlphaZeroResNet(15, 225, num_blocks=10, channels=128).eval()
    n_params = sum(p.numel() for p in net.parameters())
    assert 3_100_000 < n_params < 3_300_000  # 20 convs of 3x3x128x128 (2.95 M) + heads
    with torch.no_grad():
        lp, v = net(torch.zeros(2, 18, 15, 15))
    assert lp.shape == (2, 225) and v.shape == (2,)
    assert torch.allclose(lp.exp().sum(1), torch.ones(2), atol=1e-5)


def test_batch_norm_folding_is_exact_in_float32():
    import copy

    from omoknuni_quantum_amd.synthetic.resnet_evaluator import AlphaZeroResNet, fold_batch_norm

    torch.manual_seed(0)
    net = AlphaZeroResNet(9, 81, num_blocks=2, channels=16).eval()
    for m in net.modules():  # non-trivial running statistics
        if isinstance(m, torch.nn.BatchNorm2d):
            m.running_mean.uniform_(-0.5, 0.5)
            m.running_var.uniform_(0.5, 2.0)
    x = torch.rand(4, 18, 9, 9)
    with torch.no_grad():
        lp, v = net(x)
        lp2, v2 = fold_batch_norm(copy.deepcopy(net))(x)
    assert not any(isinstance(m, torch.nn.BatchNorm2d) for m in fold_batch_norm(net).modules())
    assert torch.allclose(lp, lp2, atol=1e-5) and torch.allclose(v, v2, atol=1e-5)
