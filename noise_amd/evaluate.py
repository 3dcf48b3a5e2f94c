"""The score of the reference's speedrun on the HIP forward: mean next-token cross-entropy of a state
dict on the fixed validation split (utils/eval.py:24-53, utils/prepare_data.py:19-47).

    python -m noise_amd.evaluate logs/val/final.pt [--data-dir data]

Same functions, arguments and errors as the reference: `load_model(state_dict, device)` (strict
state-dict load into the fixed architecture), `load_rows(path, rows)` (an int64 [rows, 2049] token
tensor whose int32 bytes must hash to the pinned digest), `evaluate(state_dict, data_dir,
batch_size)` (summed per-token loss over every prediction, rows split across ranks and
all-reduced under torch.distributed, FloatingPointError if the mean is not finite). The forward is
the unperturbed path of the population kernels (`noise_amd.GPT.forward` -> `clean_loss`).
"""
import argparse
import hashlib
import json
import os
from pathlib import Path

import torch
from torch import distributed as dist

from .config import GPTConfig
from .model import GPT

SEQ = 2049
VAL_ROWS = 544  # 1,114,112 prediction tokens
# sha256 of the int32 little-endian token bytes of the pinned splits (utils/prepare_data.py:28-31).
EXPECTED = {
    'train.pt': '36ccb57eba6f5474b18acf99edd4a4793187260f7da7cc7053322cce59154bde',
    'val.pt': '5fdb9242ce8ab83e519ab5dd5cf8d64f4d8a99f6e74c137f4ca0f723da5f7437',
}


def token_hash(rows):
    return hashlib.sha256(rows.to(torch.int32).contiguous().numpy().tobytes()).hexdigest()


def load_rows(path, rows, expected=EXPECTED):
    """int64 [rows, SEQ] tokens from a torch.save'd tensor; a wrong shape or (for a file named in
    `expected`) a wrong digest raises ValueError."""
    data = torch.load(path, map_location='cpu', weights_only=True)
    if not isinstance(data, torch.Tensor) or tuple(data.shape) != (rows, SEQ):
        raise ValueError(f'{path}: expected a [{rows}, {SEQ}] token tensor')
    want = (expected or {}).get(Path(path).name)
    if want is not None and token_hash(data) != want:
        raise ValueError(f'{path}: token hash mismatch; rerun utils/prepare_data.py')
    return data.long()


def load_model(state_dict, device):
    """The fixed architecture with these weights; a missing, extra or reshaped tensor is an error.
    The token and value embeddings are rounded to bfloat16, as the reference's GPU model stores
    them (utils/model.py:171-175: its load_state_dict copies into bfloat16 parameters)."""
    model = GPT(GPTConfig(), device=device)
    model.load_state_dict(state_dict, strict=True)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name == 'transformer.wte.weight' or name.startswith('value_embeds.'):
                p.copy_(p.bfloat16().float())
    return model.eval().requires_grad_(False)


@torch.no_grad()
def evaluate(state_dict, data_dir='data', batch_size=16, rows=VAL_ROWS, expected=EXPECTED):
    """Mean loss over every prediction of val.pt; under torch.distributed the rows are split
    across ranks and the (loss sum, count) pair is all-reduced."""
    rank, world = (dist.get_rank(), dist.get_world_size()) if dist.is_initialized() else (0, 1)
    device = torch.device('cuda', torch.cuda.current_device())
    model = load_model(state_dict, device)
    data = load_rows(Path(data_dir) / 'val.pt', rows, expected)[rank::world]
    total = torch.zeros(2, dtype=torch.float64, device=device)  # summed loss, predictions
    for batch in data.split(batch_size):
        batch = batch.to(device)
        loss = model(batch[:, :-1].contiguous(), batch[:, 1:].contiguous(), loss_reduction='sum')
        total[0] += loss.double()
        total[1] += batch[:, 1:].numel()
    if world > 1:
        dist.all_reduce(total)
    value = (total[0] / total[1]).item()
    if value != value:
        raise FloatingPointError('Non-finite validation loss')
    return value


def main():
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument('checkpoint', type=Path, help='A state dict saved by a training script.')
    parser.add_argument('--data-dir', type=Path, default=Path('data'))
    args = parser.parse_args()
    if 'RANK' in os.environ:
        torch.cuda.set_device(int(os.environ['LOCAL_RANK']))
        dist.init_process_group('nccl')
    else:
        torch.cuda.set_device(0)
    state_dict = torch.load(args.checkpoint, map_location='cpu', weights_only=True)
    value = evaluate(state_dict, args.data_dir)
    if not dist.is_initialized() or dist.get_rank() == 0:
        print(json.dumps(dict(checkpoint=str(args.checkpoint), val_loss=value)), flush=True)
    if dist.is_initialized():
        dist.destroy_process_group()


if __name__ == '__main__':
    main()
