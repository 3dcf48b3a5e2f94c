"""MI355X-native population-perturbed forward pass of Noise (the EGGROLL path).

Public API (mirrors the reference's Python interface):
  population_loss(model, p, noise, sign, idx, targets) -> Tensor[m]   train/val/eggroll.py:66
  Eggroll(model, pairs, rank, world).step(x, y, optimizer, step)        train/val/eggroll.py:106-168
  GPT / GPTConfig / make_model                                          utils/model.py, eggroll.py:38
  AdamW                                                                 torch.optim.AdamW semantics
The compute runs in libnoise_amd.so (hand-written gfx950 HIP kernels, C ABI in include/noise_amd.h).
"""
from .config import GPTConfig, has_ve, param_shapes, window_sizes
from .eggroll import Eggroll
from .model import GPT, make_model
from .optim import AdamW
from .population import clean_loss, population_loss

__all__ = ['GPTConfig', 'GPT', 'make_model', 'population_loss', 'clean_loss', 'Eggroll', 'AdamW',
           'has_ve', 'param_shapes', 'window_sizes']
