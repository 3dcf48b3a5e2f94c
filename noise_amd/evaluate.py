"""Validation scoring on the HIP forward: the number a training run is judged by.

The score is the mean next-token cross-entropy of a state dict over every prediction of the
pinned validation split (the reference's utils/eval.py:33-53 over utils/prepare_data.py:19-47).
This module computes the same quantity with its own plan:

* `TokenSplit.open` reads a `torch.save`d int64 [rows, 2049] tensor with a safe loader and
  refuses (ValueError) a wrong shape or, for a file named in the digest table, a wrong sha256 of
  its int32 little-endian tokens -- the check utils/prepare_data.py:28-47 defines;
* `load_model` builds the fixed GPT from a strict state dict, its embedding tables rounded to
  bfloat16 as the reference stores them on a GPU (utils/model.py:171-175);
* `evaluate` gives each rank one contiguous block of rows, runs the unperturbed forward of the
  population kernels over many rows per launch sequence, keeps each row's summed loss on the
  device in float64, and reads one number back per rank; ranks combine their sums with one
  all_reduce. A non-finite score raises FloatingPointError.

Arithmetic: the forward keeps an fp32 residual stream with bf16 GEMM operands, and the head's
product takes the bf16 weight as the reference's autocast does (the fp32 soft cap and
log-sum-exp follow it). The reference scores in a bf16 stream under autocast; over 8192 tokens the
two differ by 2e-4 +- 1.7e-4 on perturbed weights and 3e-6 at initialisation, the per-token
scatter (sd 0.015) averaging out over the 1.1M validation predictions. A target of -1 scores 0,
as in GPT.forward's cross-entropy (ignore_index=-1, utils/model.py:206-209), and still counts in
the denominator, which is every prediction of the split (utils/eval.py:47-48).

    python -m noise_amd.evaluate CHECKPOINT [--data-dir DIR] [--rows-per-launch N]
"""
import argparse
import hashlib
import json
import math
import os
from dataclasses import dataclass
from pathlib import Path

import torch
from torch import distributed as dist

from .config import GPTConfig
from .model import GPT, IGNORE
from .population import clean_loss

ROW_TOKENS = 2049                 # 2048 predictions per row
VAL_ROWS = 544                    # 1,114,112 predictions
# sha256 over the int32 little-endian token bytes of each pinned split (utils/prepare_data.py:28-31)
EXPECTED = {
    'train.pt': '36ccb57eba6f5474b18acf99edd4a4793187260f7da7cc7053322cce59154bde',
    'val.pt': '5fdb9242ce8ab83e519ab5dd5cf8d64f4d8a99f6e74c137f4ca0f723da5f7437',
}
EMBEDDING_TABLES = ('transformer.wte.weight', 'value_embeds.')


def token_hash(tokens):
    """sha256 hex digest of the tokens as int32 little-endian bytes."""
    return hashlib.sha256(tokens.to(torch.int32).contiguous().numpy().tobytes()).hexdigest()


@dataclass
class TokenSplit:
    path: Path
    tokens: torch.Tensor          # int64 [rows, ROW_TOKENS], host memory

    @classmethod
    def open(cls, path, rows, digests=EXPECTED):
        path = Path(path)
        tokens = torch.load(path, map_location='cpu', weights_only=True)
        if not isinstance(tokens, torch.Tensor) or tokens.shape != (rows, ROW_TOKENS):
            raise ValueError(f'{path}: not a [{rows}, {ROW_TOKENS}] token tensor')
        digest = (digests or {}).get(path.name)
        if digest is not None and token_hash(tokens) != digest:
            raise ValueError(f'{path}: tokens differ from the pinned split (sha256 mismatch)')
        return cls(path, tokens.long())

    def shard(self, rank, world):
        """Rank `rank`'s contiguous block of rows (sizes differ by at most one)."""
        n = self.tokens.shape[0]
        lo, hi = n * rank // world, n * (rank + 1) // world
        return self.tokens[lo:hi]


def load_rows(path, rows, expected=EXPECTED):
    """int64 [rows, 2049] tokens of a verified split (ValueError otherwise)."""
    return TokenSplit.open(path, rows, expected).tokens


def load_model(state_dict, device):
    """The fixed GPT holding `state_dict` (strict: a missing, extra or reshaped tensor raises),
    embedding tables rounded to bfloat16, frozen."""
    model = GPT(GPTConfig(), device=device)
    model.load_state_dict(state_dict, strict=True)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.startswith(EMBEDDING_TABLES):
                p.copy_(p.bfloat16())
    return model.eval().requires_grad_(False)


def _topology():
    if dist.is_available() and dist.is_initialized():
        return dist.get_rank(), dist.get_world_size()
    return 0, 1


@torch.no_grad()
def row_loss_sums(model, tokens, rows_per_launch=16):
    """float64 [rows] on the model's device: each row's summed next-token loss."""
    params = dict(model.named_parameters())
    device = model.flat.device
    sums = torch.zeros(tokens.shape[0], dtype=torch.float64, device=device)
    for lo in range(0, tokens.shape[0], rows_per_launch):
        block = tokens[lo:lo + rows_per_launch].to(device, non_blocking=True)
        ce = clean_loss(params, block[:, :-1], block[:, 1:], model.config, batch_chunk=rows_per_launch,
                        ignore_index=IGNORE)
        sums[lo:lo + block.shape[0]] = ce.sum(1, dtype=torch.float64)
    return sums


@torch.no_grad()
def evaluate(state_dict, data_dir='data', batch_size=16, rows=VAL_ROWS, expected=EXPECTED):
    """Mean loss over every prediction of `data_dir`/val.pt; `batch_size` rows per forward."""
    rank, world = _topology()
    device = torch.device('cuda', torch.cuda.current_device())
    split = TokenSplit.open(Path(data_dir) / 'val.pt', rows, expected)
    model = load_model(state_dict, device)
    total = row_loss_sums(model, split.shard(rank, world), batch_size).sum().reshape(1)
    if world > 1:
        dist.all_reduce(total)
    score = total.item() / (rows * (ROW_TOKENS - 1))
    if not math.isfinite(score):
        raise FloatingPointError(f'validation loss is not finite ({score})')
    return score


def _cli(argv=None):
    ap = argparse.ArgumentParser(prog='python -m noise_amd.evaluate',
                                 description='Score a saved state dict on the pinned validation split.')
    ap.add_argument('checkpoint', type=Path)
    ap.add_argument('--data-dir', type=Path, default=Path('data'))
    ap.add_argument('--rows-per-launch', type=int, default=16)
    args = ap.parse_args(argv)
    launched = 'LOCAL_RANK' in os.environ and int(os.environ.get('WORLD_SIZE', '1')) > 1
    torch.cuda.set_device(int(os.environ.get('LOCAL_RANK', 0)))
    if launched:
        dist.init_process_group('nccl')
    try:
        weights = torch.load(args.checkpoint, map_location='cpu', weights_only=True)
        score = evaluate(weights, args.data_dir, args.rows_per_launch)
        if _topology()[0] == 0:
            print(json.dumps({'checkpoint': str(args.checkpoint), 'val_loss': score}), flush=True)
    finally:
        if launched:
            dist.destroy_process_group()


if __name__ == '__main__':
    _cli()
