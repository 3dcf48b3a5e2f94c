"""Pins the probe oracle (oracle/probes_ref.py) by brute force, in float64 on the CPU.

Each closed form is checked against an evaluation that does not use it: the moved logits (or the
moved stream, its RMS norm and the head) are formed explicitly, one forward per probe, and the
loss comes from torch.nn.functional.cross_entropy. A dropped target correction, a wrong sign of
the cross term in |x + s D|^2, a missing mask or a transposed C fails these.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from noise_amd.synthetic import probe_inputs
from oracle import probes_ref as P

F64 = torch.float64
EPS = float(np.finfo(np.float32).eps)


def readout_loss(x, weight, y, width):
    """Soft-capped readout CE of streams x [.., width] (train/val/run.py:238-242), float64."""
    logits = x * torch.rsqrt(x.square().sum(-1, keepdim=True) / width + EPS) @ weight.T
    logits = 15 * torch.tanh(logits / 15)
    return F.cross_entropy(logits, y.clamp(min=0), reduction='none') * (y >= 0)


def capped_ce(raw, y):
    return F.cross_entropy(15 * torch.tanh(raw / 15), y.clamp(min=0), reduction='none') * (y >= 0)


@pytest.mark.parametrize('sigma', [0.1, 0.5])
def test_coordinate_differences_brute_force(sigma):
    g = torch.Generator().manual_seed(3)
    n, V = 6, 96
    raw = torch.randn(n, V, generator=g, dtype=F64) * 12     # many logits in the cap's bend
    raw[0, :8] = torch.tensor([60., -60., 40., 0., 14.9, -30., 200., 1e-3], dtype=F64)
    y = torch.randint(0, V, (n,), generator=g)
    y[2] = -1
    y[3] = 0
    want = torch.empty(n, V, dtype=F64)
    for v in range(V):
        e = torch.zeros(V, dtype=F64)
        e[v] = sigma
        want[:, v] = (capped_ce(raw + e, y) - capped_ce(raw - e, y)) / (2 * sigma)
    got = P.coordinate_differences(raw.numpy(), y.numpy(), sigma)
    np.testing.assert_allclose(got, want.numpy(), rtol=1e-9, atol=1e-12)
    assert np.all(got[2] == 0)


@pytest.mark.parametrize('dirs', ['hadamard', 'gaussian'])
def test_cycle_derivatives_brute_force(dirs):
    width, V, n = 32, 80, 7
    d = probe_inputs(n, width, V, sigma=0.05, dirs=dirs, probes=24 if dirs == 'gaussian' else None,
                     seed=5, dtype=F64)
    d['y'][4] = -1
    x, W, D, y, s = d['x'], d['weight'], d['D'], d['y'], d['steps']
    clean = readout_loss(x, W, y, width)
    want = torch.stack([(readout_loss(x + s[:, None] * D[:, j], W, y, width) - clean) / s
                        for j in range(D.shape[1])], 1)
    got = P.cycle_derivatives(d['base'], d['C'], y, s, d['sq'], d['dots'], d['dir_sq'], width=width)
    np.testing.assert_allclose(got, want.numpy(), rtol=1e-8, atol=1e-10)
    assert np.all(got[4] == 0)


def test_row_derivatives_brute_force_and_cycle():
    width, V, n, K = 32, 64, 9, 5
    d = probe_inputs(n, width, V, sigma=0.02, seed=7, dtype=F64)
    g = torch.Generator().manual_seed(1)
    rows = torch.stack([torch.randperm(width, generator=g)[:K] for _ in range(n)])
    x, W, D, y, s = d['x'], d['weight'], d['D'], d['y'], d['steps']
    dots, dir_sq = d['dots'].gather(1, rows), d['dir_sq'][rows]
    got = P.row_derivatives(d['base'], d['C'], rows, y, s, d['sq'], dots, dir_sq, width=width)
    full = P.cycle_derivatives(d['base'], d['C'], y, s, d['sq'], d['dots'], d['dir_sq'], width=width)
    np.testing.assert_allclose(got, np.take_along_axis(full, rows.numpy(), 1), rtol=1e-12, atol=1e-14)
    clean = readout_loss(x, W, y, width)
    for i in range(n):
        for k in range(K):
            moved = readout_loss(x[i:i + 1] + s[i] * D[:, rows[i, k]], W, y[i:i + 1], width)
            assert abs(got[i, k] - float((moved - clean[i]) / s[i])) <= 1e-8 * (1 + abs(got[i, k]))


def test_cycle_derivatives_small_step_is_gradient():
    """As the step shrinks the forward difference tends to the directional derivative of the
    readout loss (autograd in float64); O(step) agreement rules out a wrong 1/step scaling."""
    width, V, n = 32, 64, 4
    d = probe_inputs(n, width, V, sigma=1e-6, seed=9, dtype=F64)
    x = d['x'].clone().requires_grad_(True)
    readout_loss(x, d['weight'], d['y'], width).sum().backward()
    want = (x.grad @ d['D']).numpy()
    got = P.cycle_derivatives(d['base'], d['C'], d['y'], d['steps'], d['sq'], d['dots'], d['dir_sq'],
                              width=width)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-6)
