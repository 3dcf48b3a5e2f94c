"""Writes the golden vectors of tests/golden/ from the reference implementation itself.

Run once, in the build container only (the reference is not present on GPU machines):

    python tests/golden/make_golden.py /root/reference
    python tests/golden/make_golden.py /root/reference --autocast | --scoring | --noise | --sensitive-small

The reference has no tests, fixtures or known-answer vectors, so nothing else pins its
`population_loss` *as written* (train/val/eggroll.py:66-103), its seeded initialisation
(train/val/eggroll.py:38-53 over utils/model.py:149-175) or its flex-attention window semantics
(utils/model.py:17-31). This script imports those functions from the reference checkout, runs them
eagerly on the CPU in float32 on seeded synthetic inputs, and stores inputs and outputs as plain
arrays (`golden.npz`, loaded with allow_pickle=False) plus a JSON summary. Nothing of the
reference's source is stored.
"""
import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from noise_amd.synthetic import antithetic, pair_noise, sequence  # noqa: E402

CONFIG0 = dict(length=256, pairs=4, sigma=1e-3, token_seed=0, noise_seed=1)
SENSITIVE = dict(length=128, pairs=2, sigma=2e-2, token_seed=3, noise_seed=4, weight_seed=5)
# The sensitive weights at the configs' sigma: antithetic differences of order sigma, losses far
# from the chaotic regime of sigma = 0.02.
SENSITIVE_SMALL = dict(length=256, pairs=4, sigma=1e-3, token_seed=6, noise_seed=7, weight_seed=5)


def sensitive_weights(params, seed):
    """Init weights moved away from the init's degenerate points so that the loss depends on
    every upstream op: logits of order one, open value-embedding gates, varied mixing scalars."""
    g = torch.Generator().manual_seed(seed)
    p = {k: v.clone() for k, v in params.items()}
    p['lm_head.weight'] = torch.randn(p['lm_head.weight'].shape, generator=g) * 0.05
    for k in list(p):
        if k.endswith('ve_gate.weight'):
            p[k] = (torch.rand(p[k].shape, generator=g) - 0.5)
    p['resid_lambdas'] = 1.0 + 0.1 * torch.randn(p['resid_lambdas'].shape, generator=g)
    p['x0_lambdas'] = 0.1 + 0.05 * torch.randn(p['x0_lambdas'].shape, generator=g)
    return p


def main(ref_root):
    sys.path.insert(0, str(ref_root))
    from utils.model import GPT, GPTConfig, apply_rotary_emb, attention, norm
    from train.val.eggroll import lowrank, lowrank_embed, make_model, population_loss

    torch.set_grad_enabled(False)
    arrays, summary = {}, {}

    # Parameter order/shapes of the fixed module (strict state-dict keys, RNG order of offsets).
    with torch.device('meta'):
        meta = GPT(GPTConfig())
    summary['named_parameters'] = [[n, list(p.shape)] for n, p in meta.named_parameters()]
    summary['window_sizes'] = [w for w, _ in meta.window_sizes]

    model = make_model(torch.device('cpu'), 0)
    params = dict(model.named_parameters())
    summary['init'] = {n: dict(sum=float(p.double().sum()), sumsq=float(p.double().square().sum()),
                               head=[float(v) for v in p.flatten()[:4]])
                       for n, p in params.items()}
    for n in ('transformer.h.0.attn.c_q.weight', 'transformer.h.3.attn.c_proj.weight',
              'transformer.h.7.mlp.c_proj.weight', 'lm_head.weight', 'value_embeds.5.weight'):
        arrays['init/' + n] = p_np = params[n][:8, :16].numpy().copy()
        assert p_np.dtype == np.float32
    # bfloat16 rotary tables as raw bit patterns (uint16), first 2048 positions.
    arrays['cos_bits'] = model.cos[0, :2048, 0, :].contiguous().view(torch.int16).numpy().view(np.uint16)
    arrays['sin_bits'] = model.sin[0, :2048, 0, :].contiguous().view(torch.int16).numpy().view(np.uint16)

    # Config 0: population of 4 antithetic pairs on a 256-token Zipf sequence, seed-0 weights.
    idx, targets = sequence(CONFIG0['length'], seed=CONFIG0['token_seed'])
    noise, sign = antithetic(pair_noise(CONFIG0['pairs'], seed=CONFIG0['noise_seed']), CONFIG0['sigma'])
    arrays['config0/idx'], arrays['config0/targets'] = idx.numpy(), targets.numpy()
    arrays['config0/losses'] = population_loss(model, params, noise, sign, idx, targets).numpy()
    arrays['config0/clean'] = model(idx[None], targets[None], loss_reduction='none').numpy()

    # Sensitive variant: same forward, weights/sigma where every term moves the loss.
    sp = sensitive_weights(params, SENSITIVE['weight_seed'])
    idx, targets = sequence(SENSITIVE['length'], seed=SENSITIVE['token_seed'])
    noise, sign = antithetic(pair_noise(SENSITIVE['pairs'], seed=SENSITIVE['noise_seed']), SENSITIVE['sigma'])
    arrays['sensitive/idx'], arrays['sensitive/targets'] = idx.numpy(), targets.numpy()
    arrays['sensitive/losses'] = population_loss(model, sp, noise, sign, idx, targets).numpy()
    model.load_state_dict({k: v for k, v in sp.items()}, strict=True)
    arrays['sensitive/clean'] = model(idx[None], targets[None], loss_reduction='none').numpy()
    arrays['sensitive/logits'] = model(idx[None])[0, :2].numpy()

    # Per-function vectors on small seeded inputs.
    g = torch.Generator().manual_seed(11)
    x = torch.randn(2, 24, 3, 64, generator=g)
    cos = model.cos[:, :24]
    sin = model.sin[:, :24]
    arrays['fn/rotary_in'] = x.numpy()
    arrays['fn/rotary_out'] = apply_rotary_emb(x, cos, sin).numpy()
    y = torch.randn(5, 512, generator=g) * 3.0
    arrays['fn/norm_in'], arrays['fn/norm_out'] = y.numpy(), norm(y).numpy()
    for window, length in ((16, 96), (64, 96), (1024, 128)):
        q, k, v = (torch.randn(2, length, 2, 64, generator=g) for _ in range(3))
        tag = f'fn/attn_w{window}_t{length}'
        arrays[tag + '/q'], arrays[tag + '/k'], arrays[tag + '/v'] = q.numpy(), k.numpy(), v.numpy()
        arrays[tag + '/out'] = attention(q, k, v, window).numpy()
    m, t, din, dout = 4, 6, 32, 24
    xi = torch.randn(m, t, din, generator=g)
    w = torch.randn(dout, din, generator=g)
    a, b = torch.randn(m, dout, generator=g), torch.randn(m, din, generator=g)
    s = torch.tensor([0.5, -0.5, 0.25, -0.25])
    arrays.update({'fn/lowrank_x': xi.numpy(), 'fn/lowrank_w': w.numpy(), 'fn/lowrank_a': a.numpy(),
                   'fn/lowrank_b': b.numpy(), 'fn/lowrank_s': s.numpy(),
                   'fn/lowrank_out': lowrank(xi, w, a, b, s).numpy()})
    ew = torch.randn(10, 8, generator=g)
    ea, eb = torch.randn(m, 10, generator=g), torch.randn(m, 8, generator=g)
    eidx = torch.tensor([3, 0, 9, 3, 7])
    arrays.update({'fn/embed_w': ew.numpy(), 'fn/embed_a': ea.numpy(), 'fn/embed_b': eb.numpy(),
                   'fn/embed_idx': eidx.numpy(), 'fn/embed_s': s.numpy(),
                   'fn/embed_out': lowrank_embed(ew, ea, eb, eidx, s).numpy()})

    summary['config0'] = dict(CONFIG0, losses=[float(v) for v in arrays['config0/losses']])
    summary['sensitive'] = dict(SENSITIVE, losses=[float(v) for v in arrays['sensitive/losses']])
    summary['torch'] = torch.__version__
    np.savez_compressed(HERE / 'golden.npz', **arrays)
    (HERE / 'golden.json').write_text(json.dumps(summary, indent=1) + '\n')
    print(json.dumps({k: summary[k] for k in ('config0', 'sensitive', 'window_sizes')}, indent=1))


def autocast_losses(ref_root):
    """golden_autocast.npz: the reference's population_loss on the config-0 and sensitive inputs
    again, under torch.autocast('cpu', dtype=torch.bfloat16) -- the bf16 arithmetic its trainer
    runs the population forward in (train/val/eggroll.py:144-145 wraps the call in bf16 autocast,
    there on the GPU). The distance between these and the fp32 losses of golden.npz is the
    envelope of a correct bf16 evaluation of the reference's own forward."""
    sys.path.insert(0, str(ref_root))
    from train.val.eggroll import make_model, population_loss

    torch.set_grad_enabled(False)
    model = make_model(torch.device('cpu'), 0)
    params = dict(model.named_parameters())
    arrays = {}
    for tag, cfg, p in (('config0', CONFIG0, params),
                        ('sensitive', SENSITIVE, sensitive_weights(params, SENSITIVE['weight_seed']))):
        idx, targets = sequence(cfg['length'], seed=cfg['token_seed'])
        noise, sign = antithetic(pair_noise(cfg['pairs'], seed=cfg['noise_seed']), cfg['sigma'])
        with torch.autocast('cpu', dtype=torch.bfloat16):
            losses = population_loss(model, p, noise, sign, idx, targets)
        arrays[tag + '/losses_autocast'] = losses.float().numpy()
    np.savez_compressed(HERE / 'golden_autocast.npz', **arrays)
    print(json.dumps({k: [float(x) for x in v] for k, v in arrays.items()}, indent=1))


def scoring_losses(ref_root):
    """golden_scoring.npz: the reference's GPT.forward per-token losses on the config-0 and
    sensitive sequences with its GPU storage and arithmetic restated on the CPU -- token and
    value embeddings held in bfloat16 (utils/model.py:171-175 casts them when the model lives on
    a GPU) and the forward under bf16 autocast, as utils/eval.py:43-45 scores. This pins the
    oracle's 'score16' policy, the reference's scoring arithmetic."""
    sys.path.insert(0, str(ref_root))
    from train.val.eggroll import make_model

    torch.set_grad_enabled(False)
    arrays = {}
    for tag, cfg in (('config0', CONFIG0), ('sensitive', SENSITIVE)):
        model = make_model(torch.device('cpu'), 0)
        if tag == 'sensitive':
            p = sensitive_weights(dict(model.named_parameters()), SENSITIVE['weight_seed'])
            model.load_state_dict(p, strict=True)
        model.transformer.wte.to(dtype=torch.bfloat16)
        for ve in model.value_embeds.values():
            ve.to(dtype=torch.bfloat16)
        idx, targets = sequence(cfg['length'], seed=cfg['token_seed'])
        with torch.autocast('cpu', dtype=torch.bfloat16):
            ce = model(idx[None], targets[None], loss_reduction='none')
        arrays[tag + '/scoring_ce'] = ce.float().numpy()
    np.savez_compressed(HERE / 'golden_scoring.npz', **arrays)
    print(json.dumps({k: [float(v.mean()), float(v.min()), float(v.max())] for k, v in arrays.items()}))


def sensitive_small_sigma(ref_root):
    """golden_sensitive_small.npz: the reference's population_loss on the sensitive weights (O(1)
    logits, open gates) at sigma = 1e-3, once in float32 and once under bf16 autocast (the
    trainer's arithmetic, train/val/eggroll.py:144-145). Their distance is the envelope of a
    correct bf16 evaluation at the sigma the configs use."""
    sys.path.insert(0, str(ref_root))
    from train.val.eggroll import make_model, population_loss

    torch.set_grad_enabled(False)
    model = make_model(torch.device('cpu'), 0)
    c = SENSITIVE_SMALL
    p = sensitive_weights(dict(model.named_parameters()), c['weight_seed'])
    idx, targets = sequence(c['length'], seed=c['token_seed'])
    noise, sign = antithetic(pair_noise(c['pairs'], seed=c['noise_seed']), c['sigma'])
    arrays = {'idx': idx.numpy(), 'targets': targets.numpy(),
              'losses': population_loss(model, p, noise, sign, idx, targets).numpy()}
    with torch.autocast('cpu', dtype=torch.bfloat16):
        arrays['losses_autocast'] = population_loss(model, p, noise, sign, idx, targets).float().numpy()
    np.savez_compressed(HERE / 'golden_sensitive_small.npz', **arrays)
    print(json.dumps(dict(c, losses=[float(v) for v in arrays['losses']],
                          losses_autocast=[float(v) for v in arrays['losses_autocast']])))


NOISE_PAIRS = 4
NOISE_STEPS = (1, 2)
NOISE_DIRECTIONS = (0, 3, 3)
NOISE_PARAMS = ('resid_lambdas', 'transformer.wte.weight', 'transformer.h.0.attn.c_q.weight',
                'transformer.h.1.attn.ve_gate.weight', 'transformer.h.7.mlp.c_proj.weight', 'lm_head.weight')


def noise_source(ref_root):
    """golden_noise.npz: the reference's perturbation source as its own code draws it on the CPU
    (train/val/eggroll.py:110-128): the edges of the 2^28-float buffer, `Eggroll.offsets` of two
    steps for 4 pairs (one int64 row per parameter, named_parameters() order), and `Eggroll.noise`
    of pairs (0, 3, 3) for a few parameters. Generator draws have no closed form, so these pin the
    seeds, the draw order, the offset ranges and the slicing."""
    sys.path.insert(0, str(ref_root))
    from train.val.eggroll import Eggroll, make_model

    torch.set_grad_enabled(False)
    model = make_model(torch.device('cpu'), 0)
    es = Eggroll(model, NOISE_PAIRS)
    arrays = {'buffer_head': es.buffer[:64].numpy(), 'buffer_tail': es.buffer[-64:].numpy(),
              'buffer_size': np.array(es.buffer.numel())}
    names = list(es.params)
    for step in NOISE_STEPS:
        offs = es.offsets(step)
        arrays[f'step{step}/offsets'] = torch.stack([offs[n] for n in names]).numpy()
        if step == NOISE_STEPS[0]:
            nz = es.noise(offs, torch.tensor(NOISE_DIRECTIONS))
            for n in NOISE_PARAMS:
                v = nz[n]
                if isinstance(v, (tuple, list)):
                    arrays[f'noise/{n}/a'], arrays[f'noise/{n}/b'] = v[0].numpy(), v[1].numpy()
                else:
                    arrays[f'noise/{n}/eps'] = v.numpy()
    np.savez_compressed(HERE / 'golden_noise.npz', **arrays)
    print(json.dumps({k: list(v.shape) for k, v in arrays.items()}))


if __name__ == '__main__':
    root = Path(sys.argv[1] if len(sys.argv) > 1 else '/root/reference')
    if '--autocast' in sys.argv:
        autocast_losses(root)
    elif '--scoring' in sys.argv:
        scoring_losses(root)
    elif '--noise' in sys.argv:
        noise_source(root)
    elif '--sensitive-small' in sys.argv:
        sensitive_small_sigma(root)
    else:
        main(root)
