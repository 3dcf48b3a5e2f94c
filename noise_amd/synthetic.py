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


def hadamard(d, dtype=torch.float32):
    """H_d by Sylvester's doubling H_2n = [[H_n, H_n], [H_n, -H_n]] from H_1 = [1]: d x d, +-1
    entries, rows mutually orthogonal. d must be a power of two."""
    if d < 1 or d & (d - 1):
        raise ValueError(f'hadamard: Sylvester doubling gives orders 1, 2, 4, ...; got {d}')
    H = torch.ones(1, 1, dtype=dtype)
    while H.shape[0] < d:
        H = torch.cat([torch.cat([H, H], 1), torch.cat([H, -H], 1)], 0)
    return H


def probe_inputs(n, width=512, vocab=4096, probes=None, sigma=0.005, seed=0, logit_scale=3.0,
                 x_rms=2.0, dirs='hadamard', masked=0.0, dtype=torch.float32):
    """Inputs of the readout probe (train/speedrun/run.py:250-263) for n tokens, CPU tensors.

    x [n, width] streams (N(0, x_rms^2)), weight [vocab, width] head (N(0, logit_scale^2 / width),
    so normalised logits are about N(0, logit_scale^2)), stream_dirs D [width, P]: a full cycle of
    sign-flipped Hadamard rows (dirs='hadamard', P = width) or Gaussian columns (dirs='gaussian').
    Derived exactly as the reference's caller does: base = x W^T, C = (W D)^T, steps = sigma *
    rms(x) clamped at 1e-6, sq = |x|^2, dots = x D, dir_sq = |D_j|^2. Targets are Zipf draws, a
    fraction `masked` of them set to -1. Products are formed in float64 and rounded to `dtype`.
    """
    g = torch.Generator().manual_seed(seed)
    f64 = torch.float64
    x = torch.randn(n, width, generator=g, dtype=f64) * x_rms
    weight = torch.randn(vocab, width, generator=g, dtype=f64) * (logit_scale / width ** 0.5)
    if dirs == 'hadamard':
        signs = torch.randint(0, 2, (width,), generator=g).to(f64) * 2 - 1
        D = (hadamard(width, f64) * signs).T
        if probes is not None:
            D = D[:, :probes]
    else:
        D = torch.randn(width, probes or width, generator=g, dtype=f64)
    y = zipf_tokens(n, vocab, seed=seed + 1)
    if masked:
        y[torch.rand(n, generator=g) < masked] = -1
    x, weight, D = x.to(dtype).to(f64), weight.to(dtype).to(f64), D.to(dtype).to(f64)
    out = dict(x=x, weight=weight, D=D, y=y,
               base=x @ weight.T, C=(weight @ D).T.contiguous(),
               steps=sigma * x.square().mean(-1).sqrt().clamp(min=1e-6),
               sq=x.square().sum(-1), dots=x @ D, dir_sq=D.square().sum(0))
    return {k: (v if k == 'y' else v.to(dtype)) for k, v in out.items()}
