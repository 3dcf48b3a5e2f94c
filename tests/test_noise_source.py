"""The perturbation source (train/val/eggroll.py:110-128) pinned to the reference's own draws.

tests/golden/golden_noise.npz holds what the reference's `Eggroll` drew on the CPU: the edges of
its 2^28-float N(0, 1) buffer, `offsets` of steps 1 and 2 for 4 pairs, and `noise` of pairs
(0, 3, 3) for six parameters. Generator draws have no closed form, so the fixture is the pin: the
oracle's restatement (oracle/es_ref.py) and the product's own `Eggroll.offsets` / `Eggroll.noise`
(run here on the CPU through a stand-in holding only what those methods read) must reproduce it
bit for bit. On the GPU the same calls draw from the device generator instead (distributional
parity only); tests/test_gpu_kernels.py checks the HIP gather against these methods there.
"""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from noise_amd.config import param_shapes
from noise_amd.eggroll import Eggroll
from oracle import es_ref

SIZE, SEED, PAIRS = 2 ** 28, 0, 4
DIRECTIONS = (0, 3, 3)


@pytest.fixture(scope='module')
def buffer():
    return es_ref.noise_buffer(SIZE, SEED)


@pytest.fixture(scope='module')
def shapes():
    return dict(param_shapes())


def _standin(buffer, shapes):
    params = {n: torch.empty(s, device='meta') for n, s in shapes.items()}
    return SimpleNamespace(device=torch.device('cpu'), seed=SEED, noise_size=SIZE, pairs=PAIRS, params=params,
                           buffer=buffer)


def _check_noise(nz, golden_noise):
    seen = 0
    for key, want in golden_noise.items():
        if not key.startswith('noise/'):
            continue
        _, name, part = key.split('/')
        v = nz[name]
        got = {'a': lambda: v[0], 'b': lambda: v[1], 'eps': lambda: v}[part]()
        assert np.array_equal(got.numpy(), want), key
        seen += 1
    assert seen == 11


def test_buffer_matches_reference(buffer, golden_noise):
    assert buffer.numel() == int(golden_noise['buffer_size'])
    assert np.array_equal(buffer[:64].numpy(), golden_noise['buffer_head'])
    assert np.array_equal(buffer[-64:].numpy(), golden_noise['buffer_tail'])


@pytest.mark.parametrize('step', [1, 2])
def test_oracle_offsets_match_reference(shapes, golden_noise, step):
    offs = es_ref.offsets(shapes, PAIRS, step, SEED, SIZE)
    assert np.array_equal(torch.stack(list(offs.values())).numpy(), golden_noise[f'step{step}/offsets'])


def test_oracle_noise_matches_reference(buffer, shapes, golden_noise):
    offs = es_ref.offsets(shapes, PAIRS, 1, SEED, SIZE)
    _check_noise(es_ref.noise(buffer, offs, shapes, torch.tensor(DIRECTIONS)), golden_noise)


@pytest.mark.parametrize('step', [1, 2])
def test_product_offsets_match_reference(buffer, shapes, golden_noise, step):
    offs = Eggroll.offsets(_standin(buffer, shapes), step)
    assert list(offs) == list(shapes)
    assert np.array_equal(torch.stack(list(offs.values())).numpy(), golden_noise[f'step{step}/offsets'])


def test_product_noise_matches_reference(buffer, shapes, golden_noise):
    es = _standin(buffer, shapes)
    _check_noise(Eggroll.noise(es, Eggroll.offsets(es, 1), torch.tensor(DIRECTIONS)), golden_noise)


def test_steps_and_ranges(shapes, golden_noise):
    """What the fixture itself fixes: steps draw different offsets, every slice fits the buffer."""
    o1, o2 = golden_noise['step1/offsets'], golden_noise['step2/offsets']
    assert not np.array_equal(o1, o2)
    widths = np.array([sum(s) for s in shapes.values()])[:, None]
    assert (o1 >= 0).all() and (o1 + widths <= SIZE).all() and (o2 + widths <= SIZE).all()
