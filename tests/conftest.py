import sys
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / 'tests' / 'golden'


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs a HIP device (MI355X) and the built libnoise_amd.so')


@pytest.fixture(scope='session')
def golden():
    with np.load(GOLDEN / 'golden.npz', allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope='session')
def golden_autocast():
    """The reference's population losses under bf16 autocast (tests/golden/make_golden.py --autocast)."""
    with np.load(GOLDEN / 'golden_autocast.npz', allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope='session')
def golden_scoring():
    """The reference's GPT.forward per-token losses in its GPU scoring arithmetic
    (tests/golden/make_golden.py --scoring)."""
    with np.load(GOLDEN / 'golden_scoring.npz', allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope='session')
def golden_noise():
    """The reference's perturbation source as drawn on the CPU (tests/golden/make_golden.py --noise)."""
    with np.load(GOLDEN / 'golden_noise.npz', allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope='session')
def golden_sensitive_small():
    """The reference's population losses on the sensitive weights at sigma = 1e-3, in float32 and
    under bf16 autocast (tests/golden/make_golden.py --sensitive-small)."""
    with np.load(GOLDEN / 'golden_sensitive_small.npz', allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope='session')
def golden_json():
    import json
    return json.loads((GOLDEN / 'golden.json').read_text())


@pytest.fixture(scope='session')
def init_params():
    from oracle.model_ref import init_params as ip
    return ip(0)


@pytest.fixture(scope='session')
def device():
    if not torch.cuda.is_available():
        pytest.skip('no HIP device')
    from noise_amd import _lib
    _lib.load()  # fails loudly if the library is missing
    return torch.device('cuda', 0)
