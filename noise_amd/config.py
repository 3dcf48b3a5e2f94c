"""Dimensions and parameter layout of Noise's fixed 37.7M-parameter GPT.

Mirrors the reference's `GPTConfig` (utils/model.py:34-43), `has_ve` (utils/model.py:50-52),
`GPT._compute_window_sizes` (utils/model.py:185-191) and the order in which
`GPT.named_parameters()` yields the weights (utils/model.py:123-147: the root's own
`resid_lambdas`/`x0_lambdas` first, then `transformer.*`, `lm_head`, `value_embeds.*`).
That order fixes both the strict state-dict keys (utils/eval.py:24-31) and the order in which
`Eggroll.offsets` draws one offset vector per parameter (train/val/eggroll.py:117-120).
"""
from dataclasses import dataclass

import torch

# F.rms_norm(x, (d,)) with eps=None uses the float32 machine epsilon for the fp32 stream the
# population forward normalises (utils/model.py:46-47).
RMS_EPS = float(torch.finfo(torch.float32).eps)
SOFTCAP = 15.0          # utils/model.py:204
ROTARY_BASE = 10000     # utils/model.py:177
VE_GATE_CHANNELS = 32   # utils/model.py:75


@dataclass(frozen=True)
class GPTConfig:
    """utils/model.py:34-43."""
    sequence_len: int = 2048
    vocab_size: int = 4096
    n_layer: int = 8
    n_head: int = 8
    n_kv_head: int = 8
    n_embd: int = 512
    window_pattern: str = 'SSSL'

    @property
    def head_dim(self):
        return self.n_embd // self.n_head

    @property
    def padded_vocab(self):
        """utils/model.py:128 pads the vocabulary to a multiple of 64 (4096 stays 4096)."""
        return (self.vocab_size + 63) // 64 * 64

    @property
    def mlp_dim(self):
        return 4 * self.n_embd

    @property
    def rotary_seq_len(self):
        return self.sequence_len * 10  # utils/model.py:144


def has_ve(layer_idx, n_layer):
    """Value embeddings on every other block counting back from the last (utils/model.py:50-52)."""
    return layer_idx % 2 == (n_layer - 1) % 2


def window_sizes(cfg):
    """Left window per block: S = sequence_len // 2, L = sequence_len, last block always L
    (utils/model.py:185-191). A query at s sees keys s - w .. s (utils/model.py:17-21)."""
    pattern = cfg.window_pattern.upper()
    long_w, short_w = cfg.sequence_len, cfg.sequence_len // 2
    sizes = [long_w if pattern[i % len(pattern)] == 'L' else short_w for i in range(cfg.n_layer)]
    sizes[-1] = long_w
    return sizes


def param_shapes(cfg=GPTConfig()):
    """Ordered (name, shape) of every parameter, in `GPT.named_parameters()` order."""
    d, v, f, kv = cfg.n_embd, cfg.padded_vocab, cfg.mlp_dim, cfg.n_kv_head * cfg.head_dim
    out = [('resid_lambdas', (cfg.n_layer,)), ('x0_lambdas', (cfg.n_layer,)),
           ('transformer.wte.weight', (v, d))]
    for i in range(cfg.n_layer):
        pre = f'transformer.h.{i}.'
        out += [(pre + 'attn.c_q.weight', (cfg.n_head * cfg.head_dim, d)),
                (pre + 'attn.c_k.weight', (kv, d)),
                (pre + 'attn.c_v.weight', (kv, d)),
                (pre + 'attn.c_proj.weight', (d, d))]
        if has_ve(i, cfg.n_layer):
            out.append((pre + 'attn.ve_gate.weight', (cfg.n_kv_head, VE_GATE_CHANNELS)))
        out += [(pre + 'mlp.c_fc.weight', (f, d)), (pre + 'mlp.c_proj.weight', (d, f))]
    out.append(('lm_head.weight', (v, d)))
    for i in range(cfg.n_layer):
        if has_ve(i, cfg.n_layer):
            out.append((f'value_embeds.{i}.weight', (v, kv)))
    return out


def n_params(cfg=GPTConfig()):
    total = 0
    for _, shape in param_shapes(cfg):
        n = 1
        for s in shape:
            n *= s
        total += n
    return total


def noise_floats_per_pair(cfg=GPTConfig()):
    """Length of one direction: out + in for a matrix or embedding, L for a mixing-scalar vector
    (train/val/eggroll.py:119, 126)."""
    return sum(sum(shape) for _, shape in param_shapes(cfg))
