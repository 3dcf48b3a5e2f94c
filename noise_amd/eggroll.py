"""EGGROLL population step on libnoise_amd: the drop-in for train/val/eggroll.py:106-168.

`Eggroll(model, pairs, rank, world)` and `.step(x, y, optimizer, step) -> float` keep the
reference's interface and bookkeeping:

* one fixed N(0, 1) buffer of 2^28 floats drawn from a device generator seeded SEED
  (eggroll.py:114); a direction of a parameter is the contiguous slice of length out + in (or L)
  at an offset drawn per step from a generator seeded 1_000_003 * SEED + step, one randint per
  parameter in `named_parameters()` order (eggroll.py:117-120);
* members [rank * per_rank, (rank + 1) * per_rank) in chunks of 2 * CHUNK, member 2j / 2j+1 of a
  chunk being pair (start + 2j) % (2 pairs) // 2 at +sigma / -sigma (eggroll.py:137-146);
* all_gather of the losses across ranks (eggroll.py:147-150), then the fitness, the rank-1
  gradient rebuild and `optimizer.step()` (eggroll.py:151-167); returns the mean loss. The fitness
  is the reference's z-score of the antithetic differences; `fitness='ranks'` replaces it by their
  centred ranks (rank / (n - 1) - 0.5, stable ascending order).

What changes is where the work runs: the forward is the fused kernels of noise_amd.population
(pairs are passed once, each kernel maps member p to pair row p >> 1 instead of repeating the
noise), the fitness is one kernel, and the gradient kernel reads a_j and b_j straight out of the
noise buffer at the step's offsets instead of re-materialising them.
"""
import torch

from . import kernels as K
from .config import GPTConfig, param_shapes
from .kernels import NoiseRows
from .optim import AdamW
from .population import Engine, PreparedWeights

SEED = 0
SIGMA = 0.002
CHUNK = 256
NOISE = 2 ** 28


class Eggroll:
    def __init__(self, model, pairs, rank=0, world=1, sigma=SIGMA, chunk=CHUNK, noise_size=NOISE, seed=SEED,
                 fitness='zscore', head_split=False):
        if fitness not in ('zscore', 'ranks'):
            raise ValueError(f"fitness must be 'zscore' (the reference's) or 'ranks', not {fitness!r}")
        self.fitness = fitness
        self.model, self.pairs, self.rank, self.world = model, pairs, rank, world
        self.sigma, self.chunk, self.noise_size, self.seed = sigma, chunk, noise_size, seed
        self.device = next(model.parameters()).device
        self.params = dict(model.named_parameters())
        self.cfg = getattr(model, 'config', GPTConfig())
        self.shapes = dict(param_shapes(self.cfg))
        if list(self.params) != list(self.shapes):
            raise ValueError('model parameters do not follow the fixed GPT layout')
        self.buffer = torch.randn(noise_size, device=self.device,
                                  generator=torch.Generator(self.device).manual_seed(seed))
        self.weights = PreparedWeights(self.params, self.cfg, head_split)
        self.engine = Engine(self.device, self.cfg)
        self.grad_flat = torch.zeros(sum(torch.Size(s).numel() for s in self.shapes.values()),
                                     dtype=torch.float32, device=self.device)
        self.grads, off = {}, 0
        for name, shape in self.shapes.items():
            n = torch.Size(shape).numel()
            self.grads[name] = self.grad_flat[off:off + n].view(shape)
            off += n
        self.status = torch.zeros(1, dtype=torch.int32, device=self.device)
        self._grad_list = [self.grads[name] for name in self.shapes]
        self._layout = None    # column layout of the per-chunk noise gather

    def offsets(self, step):
        g = torch.Generator(self.device).manual_seed(1_000_003 * self.seed + step)
        return {name: torch.randint(0, self.noise_size - sum(p.shape), (self.pairs,), device=self.device,
                                    generator=g)
                for name, p in self.params.items()}

    def noise(self, offsets, directions):
        """name -> (a [n, out], b [n, in]) or eps [n, L]: views of one gathered [n, out + in] block."""
        out = {}
        for name, p in self.params.items():
            rows = self.buffer[offsets[name][directions, None] + torch.arange(sum(p.shape), device=self.device)]
            out[name] = rows.split(list(p.shape), dim=1) if p.dim() == 2 else rows
        return out

    def _pair_rows(self, table, directions):
        """name -> NoiseRows for the pairs `directions`: one gather (noise_pair_gather) of every
        parameter's [out + in] slice side by side (each block's first column a multiple of 4 floats,
        so every a and b view starts 16-byte aligned), instead of one gather per parameter.
        table: the int64 [params, pairs] stack of this step's offsets."""
        if self._layout is None:
            widths = [sum(s) for s in self.shapes.values()]
            padded = [-(-w // 4) * 4 for w in widths]
            starts = [sum(padded[:k]) for k in range(len(padded))]
            self._layout = (widths, starts, sum(padded))
        widths, starts, total = self._layout
        block = torch.empty(directions.numel(), total, dtype=torch.float32, device=self.device)
        K.pair_gather(self.buffer, table, directions, widths, starts, block)
        out = {}
        for (name, shape), st in zip(self.shapes.items(), starts):
            if len(shape) == 2:
                out[name] = NoiseRows(a=block[:, st:st + shape[0]], b=block[:, st + shape[0]:st + sum(shape)], shift=1)
            else:
                out[name] = NoiseRows(eps=block[:, st:st + shape[0]], shift=1)
        return out

    @torch.no_grad()
    def population_losses(self, x, y, offsets):
        """This rank's share of member losses [per_rank] (eggroll.py:133-146)."""
        pairs, chunk = self.pairs, self.chunk
        members = max(2 * pairs, 2 * len(x))
        per_seq, per_rank = members // len(x), members // self.world
        losses = torch.empty(per_rank, device=self.device)
        sign = torch.tensor([self.sigma, -self.sigma], device=self.device).repeat(chunk)
        T = x.shape[1]
        table = torch.stack([offsets[name] for name in self.shapes])  # [params, pairs]
        for start in range(self.rank * per_rank, (self.rank + 1) * per_rank, 2 * chunk):
            n = min(2 * chunk, (self.rank + 1) * per_rank - start)
            directions = torch.arange(start, start + n, 2, device=self.device) % (2 * pairs) // 2
            nz = self._pair_rows(table, directions)
            seq = start // per_seq
            lo = start - self.rank * per_rank
            self.engine.forward(self.weights, nz, sign[:n], x[seq].contiguous(), y[seq].contiguous(), T, n,
                                losses[lo:lo + n])
        return losses

    def gradient(self, weight, offsets, n):
        """grads[name] = -1/n sum_p weight[p] a_p^T b_p (or eps_p) for every parameter (eggroll.py:155-166):
        one launch over the tiles of every parameter (noise_es_gradient_params), on the current stream."""
        table = torch.stack([offsets[name] for name in self.shapes])  # [params, pairs]
        K.es_gradient_params(weight, self.buffer, table, list(self.shapes.values()), self._grad_list, -1.0 / n)

    @torch.no_grad()
    def step(self, x, y, optimizer, step):
        """Evaluate this rank's share of the population, gather the losses, rebuild the update."""
        pairs = self.pairs
        offsets = self.offsets(step)
        self.weights.refresh()
        losses = self.population_losses(x, y, offsets)
        if self.world > 1:
            gathered = [torch.empty_like(losses) for _ in range(self.world)]
            torch.distributed.all_gather(gathered, losses)
            losses = torch.cat(gathered)
        n = losses.numel() // 2
        weight = torch.empty(pairs, device=self.device)
        ranked = torch.empty(n, device=self.device) if self.fitness == 'ranks' else None
        K.fitness(losses, pairs, weight, self.status, self.fitness, ranked)
        self.gradient(weight, offsets, n)
        optimizer.zero_grad(set_to_none=True)
        for name, p in self.params.items():
            p.grad = self.grads[name]
        # One host sync per step: the status and the mean loss come back together (the reference
        # reads only the mean, eggroll.py:168). This package's AdamW is queued before that read and
        # skips its update on the device when the status is set; another optimizer steps after it.
        queued = isinstance(optimizer, AdamW)
        if queued:
            optimizer.step(unless=self.status)
        status, mean = torch.stack([self.status[0].to(torch.float32), losses.mean()]).tolist()
        if status != 0:
            if queued:
                optimizer.rewind()
            raise FloatingPointError('non-finite member loss in the population step')
        if not queued:
            optimizer.step()
        return mean
