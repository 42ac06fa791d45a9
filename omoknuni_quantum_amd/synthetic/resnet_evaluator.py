"""Workload C5's evaluator: a randomly initialised AlphaZero ResNet in stock PyTorch-ROCm.

Architecture of the reference's ResNetModel (python/mcts/neural_networks/resnet_model.py:17-272):
an input 3x3 convolution + batch norm + ReLU, ``num_blocks`` residual blocks (two 3x3
convolutions with batch norm, identity skip, ReLU), a policy head (1x1 convolution to 2 planes,
batch norm, ReLU, FC to ``fc_hidden``, ReLU, FC to the action count, log-softmax) and a value
head (1x1 convolution to 1 plane, batch norm, ReLU, FC to ``fc_hidden``, ReLU, FC to 1, tanh).
It runs in eval mode in the inference form of the same network: every batch norm is folded
into the convolution before it (weights scaled by gamma/sqrt(var+eps), bias beta-mean*scale),
and weights and activations are bfloat16 in channels-last layout.  On one MI355X this takes
2.3 ms per 512-position forward pass, against 6.2 ms under bfloat16 autocast, which keeps
batch norm in float32 and converts activations around every layer.  The network is outside
the kernel target: it stands in for the evaluator so that end-to-end simulations/s and the
tree-operation share can be measured.

``ResNetEvaluator.evaluate_wave(engine)`` builds the 18 feature planes of every wave slot on the
device (omq_leaf_features, bfloat16, channels-last), runs one batched forward pass over all
trees' slots and writes the policy probabilities and values into the engine's rows.  With ``record=True`` it keeps a host
copy of every wave's outputs, so that the CPU oracle can replay the same evaluator outputs.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from ..core.features import NUM_PLANES, LeafFeatureBuilder


class _Residual(nn.Module):
    def __init__(self, ch: int):
        super().__init__()
        self.c1 = nn.Conv2d(ch, ch, 3, padding=1, bias=False)
        self.b1 = nn.BatchNorm2d(ch)
        self.c2 = nn.Conv2d(ch, ch, 3, padding=1, bias=False)
        self.b2 = nn.BatchNorm2d(ch)

    def forward(self, x):
        y = F.relu(self.b1(self.c1(x)))
        y = self.b2(self.c2(y))
        return F.relu(y + x)


class AlphaZeroResNet(nn.Module):
    def __init__(self, board_size: int = 15, num_actions: int = 225, num_blocks: int = 10,
                 channels: int = 128, in_planes: int = NUM_PLANES, fc_hidden: int = 256):
        super().__init__()
        cells = board_size * board_size
        self.stem = nn.Sequential(nn.Conv2d(in_planes, channels, 3, padding=1, bias=False),
                                  nn.BatchNorm2d(channels), nn.ReLU())
        self.blocks = nn.Sequential(*[_Residual(channels) for _ in range(num_blocks)])
        self.p_conv = nn.Sequential(nn.Conv2d(channels, 2, 1, bias=False), nn.BatchNorm2d(2),
                                    nn.ReLU())
        self.p_fc = nn.Sequential(nn.Linear(2 * cells, fc_hidden), nn.ReLU(),
                                  nn.Linear(fc_hidden, num_actions))
        self.v_conv = nn.Sequential(nn.Conv2d(channels, 1, 1, bias=False), nn.BatchNorm2d(1),
                                    nn.ReLU())
        self.v_fc = nn.Sequential(nn.Linear(cells, fc_hidden), nn.ReLU(),
                                  nn.Linear(fc_hidden, 1))
        for m in self.modules():
            if isinstance(m, nn.Conv2d):
                nn.init.kaiming_normal_(m.weight, mode="fan_in", nonlinearity="relu")
            elif isinstance(m, nn.BatchNorm2d):
                nn.init.normal_(m.weight, 1.0, 0.02)
                nn.init.zeros_(m.bias)
            elif isinstance(m, nn.Linear):
                nn.init.xavier_normal_(m.weight)
                nn.init.zeros_(m.bias)
        # small final policy layer: near-uniform priors from the untrained network
        nn.init.xavier_normal_(self.p_fc[2].weight, gain=0.1)

    def forward(self, x):
        h = self.blocks(self.stem(x))
        logp = F.log_softmax(self.p_fc(self.p_conv(h).flatten(1)).float(), dim=1)
        v = torch.tanh(self.v_fc(self.v_conv(h).flatten(1)).float()).squeeze(1)
        return logp, v


def fold_batch_norm(net: AlphaZeroResNet) -> AlphaZeroResNet:
    """Eval-mode batch norms folded into the preceding bias-free convolutions, in place:
    bn(conv(x)) = conv'(x) with W' = W*s and b' = beta - mean*s, s = gamma/sqrt(var + eps)."""
    def merge(conv: nn.Conv2d, bn: nn.BatchNorm2d) -> nn.Module:
        s = bn.weight.detach() / torch.sqrt(bn.running_var + bn.eps)
        folded = nn.Conv2d(conv.in_channels, conv.out_channels, conv.kernel_size,
                           padding=conv.padding, bias=True)
        with torch.no_grad():
            folded.weight.copy_(conv.weight * s[:, None, None, None])
            folded.bias.copy_(bn.bias.detach() - bn.running_mean * s)
        return folded

    net.stem = nn.Sequential(merge(net.stem[0], net.stem[1]), net.stem[2])
    for blk in net.blocks:
        blk.c1, blk.b1 = merge(blk.c1, blk.b1), nn.Identity()
        blk.c2, blk.b2 = merge(blk.c2, blk.b2), nn.Identity()
    net.p_conv = nn.Sequential(merge(net.p_conv[0], net.p_conv[1]), net.p_conv[2])
    net.v_conv = nn.Sequential(merge(net.v_conv[0], net.v_conv[1]), net.v_conv[2])
    return net


class ResNetEvaluator:
    """Device evaluator over the wave slots of a WaveEngine (board game models)."""

    device_native = True

    def __init__(self, engine, boards: torch.Tensor, num_blocks: int = 10, channels: int = 128,
                 seed: int = 0, record: bool = False, dtype: torch.dtype = torch.bfloat16):
        g = torch.Generator().manual_seed(seed)
        with torch.random.fork_rng(devices=[]):
            torch.manual_seed(int(torch.randint(0, 2**31 - 1, (1,), generator=g)))
            net = AlphaZeroResNet(engine.model.board_size, engine.A, num_blocks, channels)
        net = fold_batch_norm(net.eval())
        self.net = net.to(engine.device, dtype).to(memory_format=torch.channels_last)
        self.builder = LeafFeatureBuilder(engine, boards, NUM_PLANES, dtype=dtype,
                                          channels_last=True)
        self.dtype = dtype
        self.record = record
        self.calls = []  # [(policy [T, MW, A], values [T, MW])] on the host when recording

    @torch.no_grad()
    def evaluate_wave(self, engine) -> None:
        logp, v = self.net(self.builder.build())
        pol = torch.exp(logp)
        engine.policy.view(-1, engine.A).copy_(pol)
        engine.values.copy_(v)
        if self.record:
            self.calls.append((pol.view(engine.T, engine.MW, engine.A).cpu().numpy(),
                               v.view(engine.T, engine.MW).cpu().numpy()))
