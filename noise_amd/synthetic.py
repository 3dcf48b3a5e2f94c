"""Seeded synthetic inputs for the benchmark configurations (no dataset is available offline).

* token ids: Zipf(s) over the vocabulary, p(k) proportional to (k + 1)^-s, drawn with
  `torch.multinomial` from a seeded CPU generator;
* host-supplied perturbations: for every parameter, in `named_parameters()` order, one
  (a [pairs, out], b [pairs, in]) draw for a matrix or embedding and eps [pairs, L] for a mixing
  scalar vector, all N(0, 1) from one seeded CPU generator -- the shapes
  `Eggroll.noise` produces (train/val/eggroll.py:122-128);
* the antithetic member order of `Eggroll.step`: sign = [+sigma, -sigma] repeated and every
  pair's noise repeated twice (train/val/eggroll.py:138-142).
"""
import torch

from .config import GPTConfig, param_shapes


def zipf_tokens(n, vocab=4096, s=1.1, seed=0):
    """n token ids in [0, vocab) with p(k) proportional to (k+1)^-s."""
    g = torch.Generator().manual_seed(seed)
    weights = (torch.arange(vocab, dtype=torch.float64) + 1.0) ** (-s)
    return torch.multinomial(weights, n, replacement=True, generator=g).to(torch.int64)


def sequence(length, vocab=4096, s=1.1, seed=0):
    """(idx [length], targets [length]) from length + 1 Zipf draws, shifted by one."""
    tokens = zipf_tokens(length + 1, vocab, s, seed)
    return tokens[:-1].contiguous(), tokens[1:].contiguous()


def pair_noise(pairs, seed=0, cfg=GPTConfig(), dtype=torch.float32):
    """name -> (a [pairs, out], b [pairs, in]) or eps [pairs, L], N(0, 1), CPU."""
    g = torch.Generator().manual_seed(seed)
    out = {}
    for name, shape in param_shapes(cfg):
        if len(shape) == 2:
            a = torch.randn(pairs, shape[0], generator=g, dtype=dtype)
            b = torch.randn(pairs, shape[1], generator=g, dtype=dtype)
            out[name] = (a, b)
        else:
            out[name] = torch.randn(pairs, shape[0], generator=g, dtype=dtype)
    return out


def antithetic(noise, sigma):
    """Member-order noise and sign: member 2j is pair j at +sigma, member 2j+1 at -sigma."""
    member = {n: tuple(t.repeat_interleave(2, 0) for t in v) if isinstance(v, tuple)
              else v.repeat_interleave(2, 0) for n, v in noise.items()}
    first = next(iter(noise.values()))
    pairs = (first[0] if isinstance(first, tuple) else first).shape[0]
    sign = torch.tensor([sigma, -sigma], dtype=torch.float32).repeat(pairs)
    return member, sign
