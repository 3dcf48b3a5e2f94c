"""The fixed 37.7M-parameter GPT of Noise, as the parameter container the kernels read.

Mirrors utils/model.py:61-147 module for module, so `state_dict()` has exactly the reference's
keys and shapes and round-trips through `load_state_dict(strict=True)` of the fixed module
(utils/eval.py:24-31). Two storage choices differ from nn.Module defaults:

* every parameter is a view into one flat fp32 buffer (`model.flat`), in `named_parameters()`
  order, so the optimizer's update is a single launch over 37.7M floats;
* embeddings stay fp32 on every device, as `make_model` leaves them for the ES update
  (train/val/eggroll.py:50-52).

`forward(idx, targets)` is the sigma = 0 scoring forward (utils/model.py:193-210) on the same
kernels as the population, returning the per-token losses reduced as `loss_reduction` says, or,
without targets, the capped logits.
"""
import torch
from torch import nn

from .config import GPTConfig, VE_GATE_CHANNELS, has_ve, param_shapes, window_sizes
from .population import clean_loss, rotary_tables

IGNORE = -1  # GPT.forward's ignore_index (utils/model.py:208)


class CausalSelfAttention(nn.Module):
    def __init__(self, cfg, layer_idx):
        super().__init__()
        d = cfg.n_embd
        self.c_q = nn.Linear(d, cfg.n_head * cfg.head_dim, bias=False)
        self.c_k = nn.Linear(d, cfg.n_kv_head * cfg.head_dim, bias=False)
        self.c_v = nn.Linear(d, cfg.n_kv_head * cfg.head_dim, bias=False)
        self.c_proj = nn.Linear(d, d, bias=False)
        self.ve_gate = (nn.Linear(VE_GATE_CHANNELS, cfg.n_kv_head, bias=False)
                        if has_ve(layer_idx, cfg.n_layer) else None)


class MLP(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.c_fc = nn.Linear(cfg.n_embd, cfg.mlp_dim, bias=False)
        self.c_proj = nn.Linear(cfg.mlp_dim, cfg.n_embd, bias=False)


class Block(nn.Module):
    def __init__(self, cfg, layer_idx):
        super().__init__()
        self.attn = CausalSelfAttention(cfg, layer_idx)
        self.mlp = MLP(cfg)


class GPT(nn.Module):
    def __init__(self, config=GPTConfig(), device='cpu'):
        super().__init__()
        self.config = config
        self.window_sizes = [(w, 0) for w in window_sizes(config)]
        v, d = config.padded_vocab, config.n_embd
        with torch.device('meta'):
            self.transformer = nn.ModuleDict({
                'wte': nn.Embedding(v, d),
                'h': nn.ModuleList([Block(config, i) for i in range(config.n_layer)]),
            })
            self.lm_head = nn.Linear(d, v, bias=False)
            self.resid_lambdas = nn.Parameter(torch.ones(config.n_layer))
            self.x0_lambdas = nn.Parameter(torch.zeros(config.n_layer))
            self.value_embeds = nn.ModuleDict({
                str(i): nn.Embedding(v, config.n_kv_head * config.head_dim)
                for i in range(config.n_layer) if has_ve(i, config.n_layer)})
        self._bind_flat(torch.device(device))
        cos, sin = rotary_tables(config.sequence_len, device, config)
        self.register_buffer('cos', cos, persistent=False)
        self.register_buffer('sin', sin, persistent=False)

    def _bind_flat(self, device):
        shapes = dict(param_shapes(self.config))
        names = [n for n, _ in self.named_parameters()]
        if names != list(shapes):
            raise AssertionError('parameter order differs from the fixed model layout')
        total = sum(torch.Size(s).numel() for s in shapes.values())
        self.flat = torch.zeros(total, dtype=torch.float32, device=device)
        views, off = {}, 0
        for name in names:
            n = torch.Size(shapes[name]).numel()
            views[name] = self.flat[off:off + n].view(shapes[name])
            off += n
        for mod_name, module in self.named_modules():
            for pname in [k for k, v in module._parameters.items() if v is not None]:
                full = f'{mod_name}.{pname}' if mod_name else pname
                module._parameters[pname] = nn.Parameter(views[full], requires_grad=False)

    @torch.no_grad()
    def init_weights(self):
        """utils/model.py:150-167: the same default-generator draws in the same order."""
        cfg = self.config
        torch.nn.init.normal_(self.transformer.wte.weight, mean=0.0, std=1.0)
        torch.nn.init.normal_(self.lm_head.weight, mean=0.0, std=0.001)
        s = 3 ** 0.5 * cfg.n_embd ** (-0.5)
        for block in self.transformer.h:
            torch.nn.init.uniform_(block.attn.c_q.weight, -s, s)
            torch.nn.init.uniform_(block.attn.c_k.weight, -s, s)
            torch.nn.init.uniform_(block.attn.c_v.weight, -s, s)
            torch.nn.init.zeros_(block.attn.c_proj.weight)
            torch.nn.init.uniform_(block.mlp.c_fc.weight, -s, s)
            torch.nn.init.zeros_(block.mlp.c_proj.weight)
        self.resid_lambdas.fill_(1.0)
        self.x0_lambdas.fill_(0.1)
        for ve in self.value_embeds.values():
            torch.nn.init.uniform_(ve.weight, -s, s)
        for block in self.transformer.h:
            if block.attn.ve_gate is not None:
                torch.nn.init.zeros_(block.attn.ve_gate.weight)

    def forward(self, idx, targets=None, loss_reduction='mean'):
        """utils/model.py:193-210. Without targets: the soft-capped logits [B, T, vocab] fp32.
        With targets: their cross-entropy with ignore_index=-1 (a -1 target scores 0 and, under
        'mean', is left out of the count), reduced as loss_reduction says."""
        if loss_reduction not in ('mean', 'sum', 'none'):
            raise ValueError(f'unknown loss_reduction {loss_reduction!r}')
        params = dict(self.named_parameters())
        B, T = idx.shape
        if targets is None:
            logits = torch.empty(B, T, self.config.padded_vocab, dtype=torch.float32, device=idx.device)
            clean_loss(params, idx, torch.full_like(idx, IGNORE), self.config, ignore_index=IGNORE, logits=logits)
            return logits[..., :self.config.vocab_size]
        ce = clean_loss(params, idx, targets, self.config, ignore_index=IGNORE)
        if loss_reduction == 'none':
            return ce.view(-1)
        if loss_reduction == 'sum':
            return ce.sum()
        return ce.sum() / (targets != IGNORE).sum()


def make_model(device, seed):
    """train/val/eggroll.py:38-53: seeded init, every c_proj re-drawn U(+-1.5 sqrt(3/fan_in)),
    embeddings fp32, no gradients."""
    torch.manual_seed(seed)
    model = GPT(GPTConfig(), device=device)
    model.init_weights()
    with torch.no_grad():
        for name, module in model.named_modules():
            if 'c_proj' in name and isinstance(module, torch.nn.Linear):
                scale = 1.5 * (3 / module.weight.shape[1]) ** 0.5
                torch.nn.init.uniform_(module.weight, -scale, scale)
    return model.requires_grad_(False)
