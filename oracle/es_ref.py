"""CPU oracle of the EGGROLL update -- TEST INFRASTRUCTURE ONLY.

Only tests/, `__graft_entry__.smoke()` and bench.py's `cpu_baseline` leg may import this module.

Restates `Eggroll.step` after the population forward (train/val/eggroll.py:151-167):
* `fitness`      -- f_j = L[2j+1] - L[2j], divided by (unbiased std(f) + 1e-8), then
                    index_add into `pairs` slots at j % pairs (eggroll.py:151-154);
* `gradient`     -- g = -sum_j w_j a_j b_j^T / n for a matrix or embedding, -w . eps / n for a
                    mixing-scalar vector, n = len(f) (eggroll.py:155-166);
* `adamw_step`   -- torch.optim.AdamW's single-tensor update (decoupled weight decay, bias
                    corrections, eps outside the square root), the optimizer eggroll.py:205 builds;
* `centred_ranks`-- the optional rank-normalised fitness: ranks from a stable argsort, mapped to
                    rank / (n - 1) - 0.5 (a mode of this build, not of the reference).

and the perturbation source the update and the forward read (eggroll.py:110-128):
* `noise_buffer` -- the fixed N(0, 1) buffer, drawn once from a generator seeded with `seed`
                    (eggroll.py:113);
* `offsets`      -- per step, one generator seeded with 1,000,003 * seed + step, and per
                    parameter in named_parameters() order one randint(0, size - sum(shape)) draw of
                    `pairs` offsets (eggroll.py:116-120);
* `noise`        -- per parameter the rows buffer[offset + arange(sum(shape))] of the chosen pairs,
                    split into (a [n, out], b [n, in]) for a matrix or embedding, eps [n, L] for a
                    vector (eggroll.py:122-128).
These three are pinned by the reference's own draws on the CPU (tests/golden/golden_noise.npz).
"""
import torch


def noise_buffer(size, seed, device='cpu'):
    return torch.randn(size, device=device, generator=torch.Generator(device).manual_seed(seed))


def offsets(shapes, pairs, step, seed, size, device='cpu'):
    """name -> int64 [pairs] offsets of `step`; `shapes` in named_parameters() order."""
    g = torch.Generator(device).manual_seed(1_000_003 * seed + step)
    return {name: torch.randint(0, size - sum(shape), (pairs,), device=device, generator=g)
            for name, shape in shapes.items()}


def noise(buffer, offs, shapes, directions):
    """name -> (a, b) or eps for the pairs `directions` (an int64 tensor of pair indices)."""
    out = {}
    for name, shape in shapes.items():
        width = sum(shape)
        rows = buffer[offs[name][directions, None] + torch.arange(width, device=buffer.device)]
        out[name] = (rows[:, :shape[0]], rows[:, shape[0]:]) if len(shape) == 2 else rows
    return out


def fitness(losses, pairs):
    f = losses[1::2] - losses[0::2]
    f = f / (f.std() + 1e-8)
    return torch.zeros(pairs, dtype=f.dtype).index_add_(0, torch.arange(len(f)) % pairs, f), len(f)


def centred_ranks(f):
    n = f.numel()
    order = torch.argsort(f, stable=True)
    ranks = torch.empty(n, dtype=torch.int64)
    ranks[order] = torch.arange(n)
    return ranks.to(f.dtype) / max(n - 1, 1) - 0.5


def fitness_ranks(losses, pairs):
    """The rank-normalised variant of `fitness`: centred ranks of the same antithetic differences,
    index_add into the pair slots (the mode of this build named by config 4; the reference's own
    fitness is the z-score of eggroll.py:151-152). Returns (weight, ranked, n)."""
    f = losses[1::2] - losses[0::2]
    r = centred_ranks(f)
    return torch.zeros(pairs, dtype=f.dtype).index_add_(0, torch.arange(len(f)) % pairs, r), r, len(f)


def gradient(weight, pair_noise, n):
    """name -> gradient for the weights w [pairs] of the pair noise (a, b) / eps."""
    out = {}
    for name, v in pair_noise.items():
        if isinstance(v, tuple):
            a, b = (t.to(weight.dtype) for t in v)
            out[name] = -((weight[:, None] * a).t() @ b) / n
        else:
            out[name] = -(weight @ v.to(weight.dtype)) / n
    return out


def adamw_step(param, grad, exp_avg, exp_avg_sq, step, lr, betas=(0.9, 0.999), eps=1e-8,
               weight_decay=0.0):
    """One AdamW step in place; `step` counts from 1 for the first update."""
    beta1, beta2 = betas
    param.mul_(1 - lr * weight_decay)
    exp_avg.lerp_(grad, 1 - beta1)
    exp_avg_sq.mul_(beta2).addcmul_(grad, grad, value=1 - beta2)
    bias1 = 1 - beta1 ** step
    bias2 = 1 - beta2 ** step
    denom = (exp_avg_sq.sqrt() / bias2 ** 0.5).add_(eps)
    param.addcdiv_(exp_avg, denom, value=-lr / bias1)
    return param
