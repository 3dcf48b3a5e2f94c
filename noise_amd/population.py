"""The population-perturbed forward pass on libnoise_amd kernels.

`population_loss(model, p, noise, sign, idx, targets)` keeps the reference's signature and meaning
(train/val/eggroll.py:66-103): the mean cross-entropy [m] of m members, member j evaluating every
matrix and embedding at W + sign[j] a_j b_j^T and every mixing scalar at lambda + sign[j] eps_j, on
the one sequence idx -> targets. `noise` maps a matrix/embedding name to (a [m, out], b [m, in]) and
`resid_lambdas` / `x0_lambdas` to eps [m, L], exactly as `Eggroll.noise` builds it.

Per layer the engine runs (one launch each, all on the current stream):
  mix_norm      x = (lr + s er) x + (l0 + s e0) x0; h = bf16(norm x); u_q,k,v = h.b; VE gate
  qkv_rope_gemm [q|k|v] = h Wqkv^T + s u a^T, then in the epilogue
                q, k = bf16(norm(rot(.))); v = bf16(v + gate ve)
  attention     y = bf16(softmax_window(q k^T / 8) v); u_o = y.b_o per head
  mlp_fused     x += y Wo^T + s u_o a_o^T (the attention c_proj, in the prologue), then
                x += bf16(relu(h Wfc^T + s u_fc a_fc^T)^2) Wmp^T + s u_mp a_mp^T with
                h = bf16(norm x), u_fc = h.b_fc, u_mp = hid.b_mp: the hidden stays on chip;
                its epilogue runs the next layer's mix_norm on the finished rows
then the final norm + u_head (in the last MLP's epilogue), head_ce (bf16 head, soft-cap, CE) and
member_mean. Layer 0's mix_norm runs in the embedding launch.
"""
import math

import torch

from . import _lib
from . import kernels as K
from .config import GPTConfig, ROTARY_BASE, has_ve, param_shapes, window_sizes
from .kernels import NoiseRows

DEFAULT_CHUNK = 512  # members per batched forward (2 * CHUNK of train/val/eggroll.py:34)


def rotary_tables(length, device, cfg=GPTConfig()):
    """(cos, sin) [length, D/2] fp32 holding the bf16-rounded tables of GPT._precompute_rotary
    (utils/model.py:177-183), computed once on the host and uploaded."""
    d = cfg.head_dim
    inv_freq = 1.0 / ROTARY_BASE ** (torch.arange(0, d, 2, dtype=torch.float32) / d)
    t = torch.arange(cfg.rotary_seq_len, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    cos, sin = freqs.cos().bfloat16().float(), freqs.sin().bfloat16().float()
    return cos[:length].contiguous().to(device), sin[:length].contiguous().to(device)


class PreparedWeights:
    """The device-side weight set the kernels read: bf16 copies of every block matrix (q|k|v
    concatenated) and of the head, and the fp32 tables, gates and scalars.

    head_split: also keep the head's bf16 remainder lo = bf16(W - bf16(W)), so that head_ce
    forms h (hi + lo)^T, the fp32-weight product (twice the MFMA work). The default bf16 head is
    the product the reference's trainer runs under autocast (train/val/eggroll.py:144-145)."""

    def __init__(self, params, cfg=GPTConfig(), head_split=False):
        self.cfg = cfg
        self.params = params
        dev = params['transformer.wte.weight'].device
        d, f, L = cfg.n_embd, cfg.mlp_dim, cfg.n_layer
        bf = dict(dtype=torch.bfloat16, device=dev)
        self.qkv = [torch.empty(3 * d, d, **bf) for _ in range(L)]
        self.o = [torch.empty(d, d, **bf) for _ in range(L)]
        self.fc = [torch.empty(f, d, **bf) for _ in range(L)]
        self.mp = [torch.empty(d, f, **bf) for _ in range(L)]
        self.fc_packed = [torch.empty(K.MLP_PACKED_ELEMS, **bf) for _ in range(L)]
        self.mp_packed = [torch.empty(K.MLP_PACKED_ELEMS, **bf) for _ in range(L)]
        v = cfg.padded_vocab
        self.head_hi = torch.empty(v, d, **bf)
        self.head_lo = torch.empty(v, d, **bf) if head_split else None
        self.refresh()

    def refresh(self):
        """Re-derive the bf16 copies from the fp32 parameters (after every optimizer step)."""
        p, d = self.params, self.cfg.n_embd
        casts = []  # one launch for every plain copy
        for i in range(self.cfg.n_layer):
            pre = f'transformer.h.{i}.'
            for j, name in enumerate(('c_q', 'c_k', 'c_v')):
                casts.append((p[pre + f'attn.{name}.weight'].contiguous(), self.qkv[i][j * d:(j + 1) * d], None))
            casts.append((p[pre + 'attn.c_proj.weight'].contiguous(), self.o[i], None))
            casts.append((p[pre + 'mlp.c_fc.weight'].contiguous(), self.fc[i], None))
            casts.append((p[pre + 'mlp.c_proj.weight'].contiguous(), self.mp[i], None))
            K.mlp_pack(p[pre + 'mlp.c_fc.weight'].contiguous(), self.fc_packed[i],
                       p[pre + 'mlp.c_proj.weight'].contiguous(), self.mp_packed[i])
        casts.append((p['lm_head.weight'].contiguous(), self.head_hi, self.head_lo))
        for k in range(0, len(casts), 64):
            K.cast_bf16_many(casts[k:k + 64])

    def gate(self, i):
        return self.params[f'transformer.h.{i}.attn.ve_gate.weight']

    def table(self, name):
        return self.params[name]


class Workspace:
    """Activation buffers for `rows` member-token rows, reused across chunks and layers."""

    def __init__(self, rows, device, cfg=GPTConfig()):
        d, f = cfg.n_embd, cfg.mlp_dim
        f32 = dict(dtype=torch.float32, device=device)
        bf = dict(dtype=torch.bfloat16, device=device)
        self.rows = rows
        self.x = torch.empty(rows, d, **f32)
        self.x0 = torch.empty(rows, d, **f32)
        self.h = torch.empty(rows, d, **bf)
        self.u3 = torch.empty(rows, 3, **f32)
        self.u1 = torch.empty(rows, **f32)
        self.gate = torch.empty(rows, cfg.n_kv_head, **f32)
        self.qkv16 = torch.empty(rows, 3 * d, **bf)
        self.y = torch.empty(rows, d, **bf)
        self.uproj = torch.empty(rows, cfg.n_head, **f32)
        self.hid = None  # the unfused MLP's [rows, 2048] hidden, allocated only when used
        self.umlp = torch.empty(rows, f // 64, **f32)
        self.ce = torch.empty(rows, **f32)


class Engine:
    """Runs the forward for chunks of members; owns the workspace and rotary tables."""

    def __init__(self, device, cfg=GPTConfig()):
        self.device = torch.device(device)
        self.cfg = cfg
        self.ws = None
        self._rot = {}
        # When a list, every MLP launch is bracketed by timing events on the launch stream:
        # (before, after, rows) is appended per layer and chunk.
        self.probe = None
        # False runs the MLP as mix_norm + two lowrank_gemm launches through an HBM hidden
        # (kept to compare the two on the same inputs).
        self.fused_mlp = True
        # With the fused MLP: True runs the attention c_proj (+ its rank-1 term and the residual
        # add) in the MLP's prologue instead of as a GEMM launch of its own.
        self.fuse_attn_proj = True
        # True runs every mix_norm inside the launch before it (the embedding for the first layer,
        # the fused MLP for the later ones and the final norm) instead of as launches of their own.
        self.fuse_next_norm = True

    def _mark(self):
        if self.probe is None:
            return None
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        return ev

    def workspace(self, rows):
        if self.ws is None or self.ws.rows < rows:
            self.ws = None
            self.ws = Workspace(rows, self.device, self.cfg)
        return self.ws

    def rotary(self, T):
        if T not in self._rot:
            self._rot[T] = rotary_tables(T, self.device, self.cfg)
        return self._rot[T]

    def forward(self, W, nz, sign, idx, targets, T, members, losses_out=None, ce_out=None,
                idx_stride=0, ignore_index=-100, logits_out=None):
        """Per-member mean CE into losses_out [members] (and per-token CE into ce_out, the capped
        logits into logits_out [members * T, V] when given).

        nz: name -> NoiseRows for these members (None when sign is None). idx/targets: [T] shared
        (idx_stride 0) or [members, T] (idx_stride T). A target equal to ignore_index scores 0."""
        cfg = self.cfg
        M = members * T
        ws = self.workspace(M)
        x, x0, h, u3, u1 = ws.x[:M], ws.x0[:M], ws.h[:M], ws.u3[:M], ws.u1[:M]
        gate, qkv16, y = ws.gate[:M], ws.qkv16[:M], ws.y[:M]
        uproj, umlp, ce = ws.uproj[:M], ws.umlp[:M], ws.ce[:M]
        if not self.fused_mlp and (ws.hid is None or ws.hid.shape[0] < M):
            ws.hid = torch.empty(ws.rows, cfg.mlp_dim, dtype=torch.bfloat16, device=self.device)
        hid = None if self.fused_mlp else ws.hid[:M]
        cos, sin = self.rotary(T)
        pert = sign is not None
        g = (lambda name: nz[name]) if pert else (lambda name: None)
        shift = nz['transformer.wte.weight'].shift if pert else 0
        wins = window_sizes(cfg)
        P = W.params

        hd = g('lm_head.weight')

        def mixing(i):
            """Layer i's mix_norm (i == n_layer: the final norm with the head's dot)."""
            if i == cfg.n_layer:
                return K.mix_norm_args(x, h, T, sign, shift=shift, bs=(hd.b,) if pert else (), u=u1)
            pre = f'transformer.h.{i}.'
            ve = has_ve(i, cfg.n_layer)
            return K.mix_norm_args(
                x, h, T, sign, x0, P['resid_lambdas'][i], P['x0_lambdas'][i],
                g('resid_lambdas').eps[:, i] if pert else None, g('x0_lambdas').eps[:, i] if pert else None, shift,
                bs=tuple(g(pre + f'attn.{n}.weight').b for n in ('c_q', 'c_k', 'c_v')) if pert else (), u=u3,
                gate_w=W.gate(i) if ve else None, gate_nz=g(pre + 'attn.ve_gate.weight') if ve else None,
                gate=gate)

        # the first layer's mix_norm runs in the embedding launch, every later one (and the final
        # norm) in the epilogue of the MLP before it
        carried = self.fuse_next_norm
        K.embed_norm(P['transformer.wte.weight'], idx, T, members, sign, g('transformer.wte.weight'), x0,
                     None if carried else x, idx_stride, next_norm=mixing(0) if carried else None)
        for i in range(cfg.n_layer):
            pre = f'transformer.h.{i}.'
            q, k, v, o = (g(pre + f'attn.{n}.weight') for n in ('c_q', 'c_k', 'c_v', 'c_proj'))
            fc, mp = g(pre + 'mlp.c_fc.weight'), g(pre + 'mlp.c_proj.weight')
            ve = has_ve(i, cfg.n_layer)
            if not carried:
                K.run_mix_norm(mixing(i))
            r1 = K.rank1(sign, T, [q.a, k.a, v.a], [u3[:, 0], u3[:, 1], u3[:, 2]], 1, 3, shift) if pert else None
            K.qkv_rope_gemm(h, W.qkv[i], r1, qkv16, T, cos, sin, sign, gate if ve else None,
                            W.table(f'value_embeds.{i}.weight') if ve else None, idx,
                            g(f'value_embeds.{i}.weight') if ve else None, idx_stride)
            K.window_attention(qkv16, y, members, T, wins[i], o.b if pert else None, shift,
                               uproj if pert else None)
            fold = self.fused_mlp and self.fuse_attn_proj
            if not fold:
                r1 = K.rank1(sign, T, [o.a], [uproj], cfg.n_head, cfg.n_head, shift) if pert else None
                K.lowrank_gemm(y, W.o[i], r1, _lib.EPI_ADD_F32, x)
            ev = self._mark()
            carried = self.fused_mlp and self.fuse_next_norm
            if self.fused_mlp:
                K.mlp_fused(x, x, T, members, W.fc_packed[i], W.mp_packed[i], _lib.MLP_NORM | _lib.MLP_RESIDUAL,
                            sign, fc, mp, next_norm=mixing(i + 1) if carried else None,
                            attn=(y, W.o[i], uproj if pert else None, o) if fold else None)
            else:
                K.mix_norm(x, h, T, sign, shift=shift, bs=(fc.b,) if pert else (), u=u1)
                r1 = K.rank1(sign, T, [fc.a], [u1], 1, 1, shift) if pert else None
                K.lowrank_gemm(h, W.fc[i], r1, _lib.EPI_RELU2_BF16, hid, mp.b if pert else None,
                               umlp if pert else None)
                r1 = K.rank1(sign, T, [mp.a], [umlp], umlp.shape[1], umlp.shape[1], shift) if pert else None
                K.lowrank_gemm(hid, W.mp[i], r1, _lib.EPI_ADD_F32, x)
            if ev is not None:
                self.probe.append((ev, self._mark(), M))
        if not carried:
            K.run_mix_norm(mixing(cfg.n_layer))
        out_ce = ce if ce_out is None else ce_out
        K.head_ce(h, W.head_hi, W.head_lo, T, targets, out_ce, sign, hd, u1, idx_stride, ignore_index, logits_out)
        if losses_out is not None:
            K.member_mean(out_ce, members, T, losses_out)


def _noise_rows(noise, names, lo, hi, shift=0):
    """Slice member rows lo:hi of a reference-layout noise dict into NoiseRows."""
    out = {}
    for name in names:
        v = noise[name]
        if isinstance(v, tuple):
            a, b = v
            out[name] = NoiseRows(a=_f32rows(a[lo:hi]), b=_f32rows(b[lo:hi]), shift=shift)
        else:
            out[name] = NoiseRows(eps=_f32rows(v[lo:hi]), shift=shift)
    return out


def _f32rows(t):
    if (t.dtype != torch.float32 or t.stride(-1) != 1 or (t.dim() == 2 and t.stride(0) % 4)
            or t.data_ptr() % 16):
        t = t.to(torch.float32).contiguous()
    return t


_ENGINES = {}
_PREPARED = {}


def engine_for(device):
    key = str(torch.device(device))
    if key not in _ENGINES:
        _ENGINES[key] = Engine(device)
    return _ENGINES[key]


def population_loss(model, p, noise, sign, idx, targets, chunk=DEFAULT_CHUNK, head_split=False):
    """Mean cross-entropy [m] fp32 of m perturbed models on one sequence (train/val/eggroll.py:66).

    model: anything with a `config` (GPTConfig-compatible); p: parameters by name (device fp32);
    noise: name -> (a [m, out], b [m, in]) or eps [m, L]; sign [m]; idx, targets [T] int64.
    head_split: the head as the fp32-weight product (bf16 hi + lo halves) instead of the bf16
    product of the reference's autocast trainer (eggroll.py:144-145).
    """
    cfg = getattr(model, 'config', GPTConfig())
    cfg = GPTConfig(**{k: getattr(cfg, k) for k in GPTConfig.__dataclass_fields__})
    if cfg.n_embd != 512 or cfg.n_head != 8 or cfg.n_kv_head != 8:
        raise ValueError('the kernels are built for d_model 512 with 8 heads of 64')
    device = p['transformer.wte.weight'].device
    if device.type != 'cuda':
        raise ValueError('population_loss runs on the GPU; move the parameters to a HIP device')
    m, T = sign.shape[0], idx.shape[0]
    if targets.shape[0] != T:
        raise ValueError('idx and targets must have the same length')
    W = PreparedWeights(p, cfg, head_split)
    eng = engine_for(device)
    names = [n for n, _ in param_shapes(cfg)]
    idx = idx.to(device=device, dtype=torch.int64).contiguous()
    targets = targets.to(device=device, dtype=torch.int64).contiguous()
    sign = sign.to(device=device, dtype=torch.float32).contiguous()
    losses = torch.empty(m, dtype=torch.float32, device=device)
    for lo in range(0, m, chunk):
        hi = min(m, lo + chunk)
        nz = _noise_rows(noise, names, lo, hi)
        eng.forward(W, nz, sign[lo:hi], idx, targets, T, hi - lo, losses[lo:hi])
    return losses


def clean_loss(model_params, idx, targets, cfg=GPTConfig(), batch_chunk=64, ignore_index=-100, logits=None,
               head_split=False):
    """Per-token cross-entropy [B, T] of the unperturbed model on B sequences (utils/model.py:193-210):
    0 where the target is `ignore_index`; `logits` [B, T, V] fp32, when given, receives the capped
    logits. head_split: the fp32-weight head product instead of the bf16 one."""
    device = model_params['transformer.wte.weight'].device
    if device.type != 'cuda':
        raise ValueError('clean_loss runs on the GPU; move the parameters to a HIP device')
    B, T = idx.shape
    W = PreparedWeights(model_params, cfg, head_split)
    eng = engine_for(device)
    idx = idx.to(device=device, dtype=torch.int64).contiguous()
    targets = targets.to(device=device, dtype=torch.int64).contiguous()
    ce = torch.empty(B, T, dtype=torch.float32, device=device)
    for lo in range(0, B, batch_chunk):
        hi = min(B, lo + batch_chunk)
        eng.forward(W, None, None, idx[lo:hi], targets[lo:hi], T, hi - lo, None, ce[lo:hi].view(-1),
                    idx_stride=T, ignore_index=ignore_index,
                    logits_out=None if logits is None else logits[lo:hi].view((hi - lo) * T, -1))
    return ce
