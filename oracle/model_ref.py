"""CPU oracle of the population-perturbed forward pass -- TEST INFRASTRUCTURE ONLY.

Only tests/, `__graft_entry__.smoke()` and bench.py's `cpu_baseline` leg may import this module,
and only as the checker. The shipped path (noise_amd/) never calls it.

A restatement, in plain PyTorch on the CPU, of the reference's fixed model and its EGGROLL
population forward:

* `init_params`      -- make_model (train/val/eggroll.py:38-53) over GPT.init_weights
                        (utils/model.py:149-175): the same RNG calls in the same order;
* `rotary_tables`    -- GPT._precompute_rotary (utils/model.py:177-183), bf16-rounded tables;
* `rms_norm`         -- norm (utils/model.py:46-47), eps = float32 machine epsilon;
* `rotary`           -- apply_rotary_emb (utils/model.py:55-58);
* `window_attention` -- attention/window_mask (utils/model.py:17-31): softmax(q k^T / sqrt(D))
                        over keys with q >= k and q - k <= window, dense;
* `lowrank`          -- train/val/eggroll.py:56-58;  `lowrank_embed` -- eggroll.py:61-63;
* `forward`          -- population_loss (eggroll.py:66-103) and, with no noise, GPT.forward
                        (utils/model.py:193-210), returning per-token cross-entropy.

Precision policies:
  'fp32'  -- float32 throughout, as the reference runs eagerly on a CPU (pinned against
             tests/golden/golden.npz, written by the reference itself);
  'fp64'  -- float64 throughout (closed-form and derivative checks);
  'build' -- float64 arithmetic with bfloat16 rounding exactly where the HIP path rounds:
             GEMM inputs (normalised activations, attention inputs and output, relu^2 hidden)
             and the bf16 weight copies of every block matrix, plus the attention probabilities
             (bf16 under a constant softmax shift, `window_attention_shifted`), and the head
             weight (the bf16 product the reference's trainer runs under autocast,
             eggroll.py:144-145; `head_split=True` keeps it full precision, as the HIP path's
             hi + lo split does); the residual stream, norms, rank-1 terms, soft-cap and
             log-sum-exp stay full precision;
  'build32' -- the same cast points in float32 arithmetic. |build - build32| measures how far the
             bf16 cast points alone let two correct implementations drift on given inputs;
  'score16' -- (clean_loss only) the reference's GPU scoring arithmetic, a bf16 residual stream
             (`scoring_loss_bf16`), pinned against golden_scoring.npz: the reference's own
             GPT.forward with bf16 embedding tables under CPU bf16 autocast.

Pinning (tests/test_oracle.py): every function above against the reference's own outputs in
golden.npz; the whole forward against the reference's population_loss and GPT.forward goldens;
plus closed forms (materialised W + s a b^T, init loss ~ ln 4096, sign flip, fp64 JVP).
"""
import math

import torch
import torch.nn.functional as F

from noise_amd.config import (GPTConfig, RMS_EPS, ROTARY_BASE, SOFTCAP, VE_GATE_CHANNELS,
                              has_ve, param_shapes, window_sizes)

POLICIES = ('fp32', 'fp64', 'build', 'build32')


def _dtype(policy):
    if policy not in POLICIES:
        raise ValueError(f'unknown precision policy {policy!r}')
    return torch.float32 if policy in ('fp32', 'build32') else torch.float64


def _rb(x, policy):
    """Round to bfloat16 where the build's kernels store bf16 (identity for other policies)."""
    return x.to(torch.bfloat16).to(x.dtype) if policy in ('build', 'build32') else x


def init_params(seed=0, cfg=GPTConfig()):
    """Seeded fp32 weights, name -> tensor in named_parameters() order.

    Same sequence of default-generator draws as make_model (train/val/eggroll.py:40-49):
    wte ~ N(0,1), lm_head ~ N(0, 0.001^2), per block c_q/c_k/c_v/c_fc ~ U(+-sqrt(3/d)) with the
    two c_proj zeroed, lambdas 1.0 / 0.1, value embeddings ~ U(+-sqrt(3/d)), gates zero
    (utils/model.py:151-167), then every c_proj re-drawn U(+-1.5 sqrt(3/fan_in)) in module order
    (attn.c_proj, mlp.c_proj of block 0, then block 1, ...).
    """
    torch.manual_seed(seed)
    shapes = dict(param_shapes(cfg))
    p = {n: torch.empty(s, dtype=torch.float32) for n, s in shapes.items()}
    s = 3 ** 0.5 * cfg.n_embd ** (-0.5)
    p['transformer.wte.weight'].normal_(0.0, 1.0)
    p['lm_head.weight'].normal_(0.0, 0.001)
    for i in range(cfg.n_layer):
        pre = f'transformer.h.{i}.'
        p[pre + 'attn.c_q.weight'].uniform_(-s, s)
        p[pre + 'attn.c_k.weight'].uniform_(-s, s)
        p[pre + 'attn.c_v.weight'].uniform_(-s, s)
        p[pre + 'attn.c_proj.weight'].zero_()
        p[pre + 'mlp.c_fc.weight'].uniform_(-s, s)
        p[pre + 'mlp.c_proj.weight'].zero_()
    p['resid_lambdas'].fill_(1.0)
    p['x0_lambdas'].fill_(0.1)
    for i in range(cfg.n_layer):
        if has_ve(i, cfg.n_layer):
            p[f'value_embeds.{i}.weight'].uniform_(-s, s)
    for i in range(cfg.n_layer):
        if has_ve(i, cfg.n_layer):
            p[f'transformer.h.{i}.attn.ve_gate.weight'].zero_()
    for i in range(cfg.n_layer):
        for name in (f'transformer.h.{i}.attn.c_proj.weight', f'transformer.h.{i}.mlp.c_proj.weight'):
            scale = 1.5 * (3 / p[name].shape[1]) ** 0.5
            p[name].uniform_(-scale, scale)
    return {n: p[n] for n, _ in param_shapes(cfg)}


def rotary_tables(length, cfg=GPTConfig()):
    """(cos, sin) [length, D/2] as float32 holding the bfloat16-rounded table values."""
    d = cfg.head_dim
    inv_freq = 1.0 / ROTARY_BASE ** (torch.arange(0, d, 2, dtype=torch.float32) / d)
    t = torch.arange(cfg.rotary_seq_len, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    cos, sin = freqs.cos().bfloat16(), freqs.sin().bfloat16()
    return cos[:length].float(), sin[:length].float()


def rms_norm(x):
    return x * torch.rsqrt(x.square().mean(-1, keepdim=True) + RMS_EPS)


def rotary(x, cos, sin):
    """x [..., T, H, D] with cos/sin [T, D/2]: [x1 cos + x2 sin, -x1 sin + x2 cos]."""
    d = x.shape[-1] // 2
    x1, x2 = x[..., :d], x[..., d:]
    c, s = cos[:, None, :].to(x.dtype), sin[:, None, :].to(x.dtype)
    return torch.cat([x1 * c + x2 * s, x1 * -s + x2 * c], -1)


def window_attention(q, k, v, window):
    """q, k, v [..., T, H, D] -> [..., T, H, D]; key j visible to query i iff i >= j >= i - window."""
    t = q.shape[-3]
    i = torch.arange(t)[:, None]
    j = torch.arange(t)[None, :]
    allowed = (i >= j) & (i - j <= window)
    qh, kh, vh = (z.transpose(-3, -2) for z in (q, k, v))  # [..., H, T, D]
    scores = qh @ kh.transpose(-1, -2) / math.sqrt(q.shape[-1])
    scores = scores.masked_fill(~allowed, float('-inf'))
    return (torch.softmax(scores, -1) @ vh).transpose(-3, -2)


def window_attention_shifted(q, k, v, window, round_p=True):
    """The same attention with the build's probability rounding: the exponent (in log2 units,
    scale * log2 e) is shifted by the constant 64 * scale * log2 e -- the largest score unit-rms
    q and k reach -- instead of by the row maximum; the probabilities exp2(s - shift) are rounded
    to bf16 before they weight v, and the normaliser sums them unrounded. With the rounding
    removed (`round_p=False`) this is exactly softmax (shift invariance)."""
    t = q.shape[-3]
    i = torch.arange(t)[:, None]
    j = torch.arange(t)[None, :]
    allowed = (i >= j) & (i - j <= window)
    qh, kh, vh = (z.transpose(-3, -2) for z in (q, k, v))  # [..., H, T, D]
    scale = 1.0 / math.sqrt(q.shape[-1])
    sl2 = scale * math.log2(math.e)
    p = torch.exp2((qh @ kh.transpose(-1, -2)) * sl2 - 64.0 * sl2)
    p = p.masked_fill(~allowed, 0.0)
    pr = p.to(torch.bfloat16).to(p.dtype) if round_p else p
    out = (pr @ vh) / p.sum(-1, keepdim=True)
    return out.transpose(-3, -2)


def lowrank(x, weight, a, b, sign):
    """x [m, T, in] through (W + sign a b^T)^T: x W^T + sign (x b) a^T (eggroll.py:56-58)."""
    return x @ weight.t() + sign[:, None, None] * (x @ b.unsqueeze(-1)) * a[:, None, :]


def lowrank_embed(weight, a, b, idx, sign):
    """Rows idx of W [V, d] + sign a b^T, one (a [m, V], b [m, d]) per member (eggroll.py:61-63)."""
    return weight[idx].unsqueeze(0) + sign[:, None, None] * a[:, idx].unsqueeze(-1) * b[:, None, :]


def softcap_ce(logits, targets):
    """Per-token cross-entropy of 15 tanh(z / 15) (utils/model.py:203-209)."""
    z = SOFTCAP * torch.tanh(logits / SOFTCAP)
    return torch.logsumexp(z, -1) - z.gather(-1, targets.unsqueeze(-1)).squeeze(-1)


def forward(params, idx, targets, noise=None, sign=None, policy='fp32', cfg=GPTConfig(), capped_logits=False,
            head_split=False):
    """Per-token cross-entropy [m, T] of m perturbed models (or, with noise=None, of the clean
    model on the rows of idx [B, T]).

    With noise: idx/targets are one sequence [T] shared by all members; noise maps a matrix or
    embedding name to (a [m, out], b [m, in]) and a mixing-scalar name to eps [m, L]; sign [m]
    holds +-sigma (train/val/eggroll.py:66-103). Without noise: idx/targets [B, T]
    (utils/model.py:193-210).
    """
    dt = _dtype(policy)
    rb = lambda x: _rb(x, policy)
    p = {k: v.to(dt) for k, v in params.items()}
    heads, dim = cfg.n_head, cfg.head_dim
    if noise is None:
        batch, length = idx.shape
        m = batch
        nz = None
        s = torch.zeros(m, dtype=dt)
        tok = idx
    else:
        length = idx.shape[0]
        m = sign.shape[0]
        nz = {k: tuple(t.to(dt) for t in v) if isinstance(v, tuple) else v.to(dt) for k, v in noise.items()}
        s = sign.to(dt)
        tok = idx.expand(m, length)
    cos, sin = rotary_tables(length, cfg)
    s3 = s[:, None, None]

    def embed(name):
        w = p[name]
        rows = w[tok]                                       # [m, T, d] (exact integer gather)
        if nz is None:
            return rows
        a, b = nz[name]
        return rows + s3 * a.gather(1, tok).unsqueeze(-1) * b[:, None, :]

    def linear(name, x, round_weight=True):
        """Perturbed x W^T; x is already rounded where the build rounds its GEMM inputs."""
        w = rb(p[name]) if round_weight else p[name]
        y = x @ w.t()
        if nz is not None:
            a, b = nz[name]
            y = y + s3 * (x @ b.unsqueeze(-1)) * a[:, None, :]
        return y

    def scalar(name, i):
        v = p[name][i]
        if nz is None:
            return v
        return v + s3 * nz[name][:, i, None, None]

    x = x0 = rms_norm(embed('transformer.wte.weight'))
    for i in range(cfg.n_layer):
        pre = f'transformer.h.{i}.'
        x = scalar('resid_lambdas', i) * x + scalar('x0_lambdas', i) * x0
        h = rb(rms_norm(x))
        q = linear(pre + 'attn.c_q.weight', h).view(m, length, heads, dim)
        k = linear(pre + 'attn.c_k.weight', h).view(m, length, heads, dim)
        v = linear(pre + 'attn.c_v.weight', h).view(m, length, heads, dim)
        if has_ve(i, cfg.n_layer):
            ve = embed(f'value_embeds.{i}.weight').view(m, length, heads, dim)
            gate = 2 * torch.sigmoid(linear(pre + 'attn.ve_gate.weight', h[..., :VE_GATE_CHANNELS],
                                            round_weight=False))
            v = v + gate.unsqueeze(-1) * ve
        q = rb(rms_norm(rotary(q, cos, sin)))
        k = rb(rms_norm(rotary(k, cos, sin)))
        v = rb(v)
        attend = window_attention_shifted if policy in ('build', 'build32') else window_attention
        y = rb(attend(q, k, v, window_sizes(cfg)[i]).reshape(m, length, -1))
        x = x + linear(pre + 'attn.c_proj.weight', y)
        h2 = rb(rms_norm(x))
        hid = rb(F.relu(linear(pre + 'mlp.c_fc.weight', h2)).square())
        x = x + linear(pre + 'mlp.c_proj.weight', hid)
    hf = rb(rms_norm(x))
    logits = linear('lm_head.weight', hf, round_weight=not head_split)[..., :cfg.vocab_size]
    if capped_logits:  # GPT.forward without targets (utils/model.py:203-204, 210)
        return SOFTCAP * torch.tanh(logits / SOFTCAP)
    tgt = targets.expand(m, length) if noise is not None else targets
    return softcap_ce(logits, tgt)


def population_loss(params, noise, sign, idx, targets, policy='fp32', cfg=GPTConfig(), head_split=False):
    """Mean cross-entropy [m] of the m perturbed members (train/val/eggroll.py:66-103)."""
    return forward(params, idx, targets, noise, sign, policy, cfg, head_split=head_split).mean(-1)


def clean_loss(params, idx, targets, policy='fp32', cfg=GPTConfig(), head_split=False):
    """Per-token cross-entropy [B, T] of the unperturbed model (utils/model.py:193-210).
    policy 'score16' is the reference's GPU scoring arithmetic (`scoring_loss_bf16`)."""
    if policy == 'score16':
        return scoring_loss_bf16(params, idx, targets, cfg)
    return forward(params, idx, targets, None, None, policy, cfg, head_split=head_split)


def clean_logits(params, idx, policy='fp32', cfg=GPTConfig(), head_split=False):
    """Soft-capped logits [B, T, vocab] of the unperturbed model (GPT.forward without targets,
    utils/model.py:193-210)."""
    return forward(params, idx, None, None, None, policy, cfg, capped_logits=True, head_split=head_split)


def scoring_loss_bf16(params, idx, targets, cfg=GPTConfig()):
    """Per-token cross-entropy [B, T] in the arithmetic the reference scores with on a GPU
    (utils/eval.py:24-45): the token and value embedding tables stored in bfloat16
    (utils/model.py:171-175), the forward under bf16 autocast. There every nn.Linear takes bf16
    operands, accumulates in fp32 and returns bf16 (autocast's lower-precision list), and every
    other op -- rms_norm (on neither autocast list), the lambda mix, the residual adds, rotary,
    the gate, relu^2 -- runs in its bf16 input dtype, i.e. computes in fp32 and rounds its output
    to bf16. The 0-dim fp32 lambdas join a bf16 product as bf16 operands. Attention returns bf16
    (exact softmax here). The logits leave lm_head in bf16 and are widened before the fp32
    soft-cap and cross-entropy (utils/model.py:203-209). Each op below is one rounding r()."""
    r = lambda t: t.to(torch.bfloat16).float()
    p = {k: v.float() for k, v in params.items()}
    heads, dim = cfg.n_head, cfg.head_dim
    B, T = idx.shape
    cos, sin = rotary_tables(T, cfg)

    def lin(x, name):
        return r(x @ r(p[name]).t())

    def rot(x):
        d = x.shape[-1] // 2
        x1, x2 = x[..., :d], x[..., d:]
        c, s = cos[:, None, :], sin[:, None, :]
        return torch.cat([r(r(x1 * c) + r(x2 * s)), r(r(x1 * -s) + r(x2 * c))], -1)

    x = x0 = r(rms_norm(r(p['transformer.wte.weight'])[idx]))
    for i in range(cfg.n_layer):
        pre = f'transformer.h.{i}.'
        lr, l0 = r(p['resid_lambdas'][i]), r(p['x0_lambdas'][i])
        x = r(r(lr * x) + r(l0 * x0))
        h = r(rms_norm(x))
        q = lin(h, pre + 'attn.c_q.weight').view(B, T, heads, dim)
        k = lin(h, pre + 'attn.c_k.weight').view(B, T, heads, dim)
        v = lin(h, pre + 'attn.c_v.weight').view(B, T, heads, dim)
        if has_ve(i, cfg.n_layer):
            ve = r(p[f'value_embeds.{i}.weight'])[idx].view(B, T, heads, dim)
            gate = r(2 * r(torch.sigmoid(lin(h[..., :VE_GATE_CHANNELS], pre + 'attn.ve_gate.weight'))))
            v = r(v + r(gate.unsqueeze(-1) * ve))
        q, k = r(rms_norm(rot(q))), r(rms_norm(rot(k)))
        y = r(window_attention(q, k, v, window_sizes(cfg)[i])).reshape(B, T, -1)
        x = r(x + lin(y, pre + 'attn.c_proj.weight'))
        hid = r(torch.relu(lin(r(rms_norm(x)), pre + 'mlp.c_fc.weight')).square())
        x = r(x + lin(hid, pre + 'mlp.c_proj.weight'))
    logits = lin(r(rms_norm(x)), 'lm_head.weight')[..., :cfg.vocab_size]
    return softcap_ce(logits, targets)
