"""Benchmark: perturbed member-tokens/s of one MI355X on the full EGGROLL population step.

    python bench.py [--steps K] [--warmup W] [--members 3072] [--no-cpu] [--no-extra]
    python bench.py --probe-mlp      # for rocprofv3 --pmc: a copy of known size, then the fused MLP
    python bench.py --probe-attention  # for rocprofv3 --pmc: the attention launches of one chunk
    python bench.py --probe-step     # for rocprofv3 --pmc: a copy of known size, then one step at 512 members
    python bench.py --probe-cycle    # the readout probe kernels (cycle_derivatives), own JSON line
    python bench.py --probe-chain    # chain_chunk (attention held) at the Cut estimator's shape, own JSON line
    python bench.py --probe-chain --own routed   # the same with the routed own-query moves
    python bench.py --probe-chain --own window   # ... or with own-query moves over whole key windows

Workload (config 4 of the baseline): one GPU's share of the population -- 3072 members (1536
antithetic pairs) of the 37.7M-parameter model, rank-1 perturbations on every matrix and
embedding and eps on the mixing scalars, sigma = 1e-3, one 2048-token Zipf(1.1) sequence -- then
the rank-normalised fitness, the rank-1 gradient rebuild and an AdamW update of all weights. A step is one
`Eggroll.step`. Weights are the seeded initialisation; tokens are synthetic.

Printed: one JSON line. `value` = members * tokens * steps / wall time of the timed steps (inputs
resident in HBM). `roofline` is for the dominant kernel, the fused relu^2 MLP (`mlp_fused`: the
attention c_proj with its rank-1 term into the residual rows, then norm, c_fc with its rank-1
term, relu^2, c_proj with its rank-1 term and the residual add in one launch, the hidden kept on
chip, and the next layer's mix_norm on the finished rows): algorithmic FLOPs per launch / its
mean duration, timed live with HIP events on the launch stream.
`mlp_only` is the MLP alone (config 1's kernel: no attention c_proj, no next-layer norm) at the same
rows, timed the same way. `head_split` is one more step with the head's product on fp32-accurate
weights (bf16 hi + lo halves), after the timed steps. `cpu_baseline` times the CPU oracle
(oracle/model_ref.py, float32) on a bounded sample of the same workload on this host.
"""
import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

import torch

PEAK_BF16 = 2.5e15  # dense bf16 MFMA, MI355X
ROOT = Path(__file__).resolve().parent
TRAFFIC_FILE = ROOT / 'profiles' / 'mlp_fused_traffic.md'


def mlp_flops(rows, d=512, f=2048, attn=True):
    """Algorithmic FLOPs of one fused-MLP launch over `rows` member-token rows: both GEMMs (2 d f
    each) plus the two rank-1 terms (2 f + 2 d), per row; with `attn`, also the attention c_proj
    the launch runs first (2 d d and its rank-1 term 2 d per row)."""
    return rows * (4 * d * f + 2 * (d + f) + (2 * d * d + 2 * d if attn else 0))


def step_flops(members, T=2048, d=512, f=2048, V=4096, layers=8, windows=(1024, 1024, 1024, 2048) * 2):
    """Algorithmic FLOPs of the population forward per step (GEMMs, attention products, head)."""
    per_tok = 0
    for w in windows[:layers]:
        keys = sum(min(t, w) + 1 for t in range(T)) / T
        per_tok += 2 * d * 3 * d + 2 * d * d + 4 * d * f + 4 * 64 * 8 * keys
    per_tok += 2 * d * V
    return members * T * per_tok


def mlp_traffic(rows):
    """HBM bytes per fused-MLP launch of `rows` rows: the bytes per launch measured with rocprofv3
    --pmc FETCH_SIZE / WRITE_SIZE (scaled by the same counters on a copy of known size) at the row
    count recorded beside them in the profile summary, scaled to `rows` (a workgroup moves the same
    bytes per row at any launch size)."""
    if not TRAFFIC_FILE.exists():
        return None
    text = TRAFFIC_FILE.read_text()
    m = re.search(r'^traffic_bytes_per_launch:\s*([0-9]+)', text, re.M)
    n = re.search(r'^traffic_rows_per_launch:\s*([0-9]+)', text, re.M)
    return round(int(m.group(1)) * rows / int(n.group(1))) if m and n else None


def mlp_inputs(rows=512 * 2048, d=512, f=2048, seed=0):
    """The fused MLP's inputs at the bench shape: 512 members x 2048 tokens of an N(0, 1) fp32
    stream, N(0, 1/fan_in) weights, pair-shared N(0, 1) noise rows, sigma = 1e-3."""
    from noise_amd import kernels as K
    from noise_amd.kernels import NoiseRows
    dev = torch.device('cuda', 0)
    g = torch.Generator(device=dev).manual_seed(seed)
    members, T = rows // 2048, 2048
    nrows = members // 2
    w_fc32 = torch.randn(f, d, device=dev, generator=g) / d ** 0.5
    w_pr32 = torch.randn(d, f, device=dev, generator=g) / f ** 0.5
    w_fc = torch.empty(K.MLP_PACKED_ELEMS, device=dev, dtype=torch.bfloat16)
    w_pr = torch.empty(K.MLP_PACKED_ELEMS, device=dev, dtype=torch.bfloat16)
    K.mlp_pack(w_fc32, w_fc, w_pr32, w_pr)
    sign = torch.tensor([1e-3, -1e-3], device=dev).repeat(members // 2)
    fc = NoiseRows(a=torch.randn(nrows, f, device=dev, generator=g), b=torch.randn(nrows, d, device=dev, generator=g),
                   shift=1)
    pr = NoiseRows(a=torch.randn(nrows, d, device=dev, generator=g), b=torch.randn(nrows, f, device=dev, generator=g),
                   shift=1)
    x = torch.randn(rows, d, device=dev, generator=g)
    return dict(x=x, T=T, members=members, w_fc=w_fc, w_pr=w_pr, sign=sign, fc=fc, pr=pr)


def next_mix_norm(a, seed=1):
    """The record of the next layer's mix_norm as the step hands it to mlp_fused, for a layer with
    a value embedding: x0 mixing with perturbed lambdas, h, the q/k/v dots and the gate."""
    from noise_amd import kernels as K
    from noise_amd.kernels import NoiseRows
    x = a['x']
    dev, M, rows, shift = x.device, x.shape[0], a['fc'].a.shape[0], a['fc'].shift
    g = torch.Generator(device=dev).manual_seed(seed)
    a['x0'] = torch.randn(M, 512, device=dev, generator=g)
    a['h'] = torch.empty(M, 512, dtype=torch.bfloat16, device=dev)
    a['u3'] = torch.empty(M, 3, device=dev)
    a['gate'] = torch.empty(M, 8, device=dev)
    a['bs'] = tuple(torch.randn(rows, 512, device=dev, generator=g) for _ in range(3))
    a['lam'] = torch.tensor([1.1, 0.2], device=dev)
    a['eps'] = torch.randn(rows, 2, device=dev, generator=g)
    a['gw'] = torch.randn(8, 32, device=dev, generator=g) * 0.1
    a['gnz'] = NoiseRows(a=torch.randn(rows, 8, device=dev, generator=g), b=torch.randn(rows, 32, device=dev, generator=g),
                         shift=shift)
    return K.mix_norm_args(x, a['h'], a['T'], a['sign'], a['x0'], a['lam'][0], a['lam'][1], a['eps'][:, 0],
                           a['eps'][:, 1], shift, bs=a['bs'], u=a['u3'], gate_w=a['gw'], gate_nz=a['gnz'],
                           gate=a['gate'])


def attention_proj(a, seed=2, parts=8):
    """The attention c_proj operands the step folds into mlp_fused: y [M, 512] bf16 (the attention
    output), w_o [512, 512] bf16, the per-head parts of y . b_o [M, 8] and the c_proj noise rows."""
    from noise_amd.kernels import NoiseRows
    x = a['x']
    dev, M, rows, shift = x.device, x.shape[0], a['fc'].a.shape[0], a['fc'].shift
    g = torch.Generator(device=dev).manual_seed(seed)
    y = torch.randn(M, 512, device=dev, generator=g).to(torch.bfloat16)
    w_o = (torch.randn(512, 512, device=dev, generator=g) / 512 ** 0.5).to(torch.bfloat16)
    u = torch.randn(M, parts, device=dev, generator=g)
    nz = NoiseRows(a=torch.randn(rows, 512, device=dev, generator=g), b=torch.randn(rows, 512, device=dev, generator=g),
                   shift=shift)
    return (y, w_o, u, nz)


def probe_mlp(reps=3):
    """Counter-collection workload: `reps` copies of a 1 GiB fp32 buffer (1 GiB read + 1 GiB
    written per dispatch), then `reps` fused-MLP launches at the bench shape (512 members x 2048
    tokens, pair-shared noise rows) as the step runs them: the attention c_proj into the residual
    rows, then the normed residual MLP with the next layer's mix_norm (a value-embedding layer's)
    in the epilogue."""
    import noise_amd  # noqa: F401  (loads the library)
    from noise_amd import _lib
    from noise_amd import kernels as K
    dev = torch.device('cuda', 0)
    g = torch.Generator(device=dev).manual_seed(0)
    src = torch.randn(1 << 28, device=dev, generator=g)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    del src, dst
    a = mlp_inputs()
    nxt = next_mix_norm(a)
    att = attention_proj(a)
    for _ in range(reps):
        K.mlp_fused(a['x'], a['x'], a['T'], a['members'], a['w_fc'], a['w_pr'], _lib.MLP_NORM | _lib.MLP_RESIDUAL,
                    a['sign'], a['fc'], a['pr'], next_norm=nxt, attn=att)
    torch.cuda.synchronize()
    print(f'probe-mlp: {reps} x copy 1 GiB, {reps} x mlp_fused (attention c_proj first, next mix_norm last) over '
          f'{a["x"].shape[0]} rows', flush=True)


def probe_step(members=512, T=2048):
    """Counter-collection workload for every kernel of the step: one copy of a 1 GiB fp32 buffer
    (the scale reference for FETCH_SIZE / WRITE_SIZE), then one `Eggroll.step` with `members`
    members (one batched forward of 512 members: every forward kernel once per layer), the rank
    fitness, the gradient rebuild and AdamW -- the bench's step at one chunk."""
    import noise_amd
    from noise_amd.synthetic import sequence
    dev = torch.device('cuda', 0)
    g = torch.Generator(device=dev).manual_seed(0)
    src = torch.randn(1 << 28, device=dev, generator=g)
    dst = torch.empty_like(src)
    dst.copy_(src)
    del src, dst
    model = noise_amd.make_model(dev, 0)
    opt = noise_amd.AdamW(model.parameters(), lr=1e-3, betas=(0.5, 0.95), eps=1e-8, weight_decay=0.0)
    es = noise_amd.Eggroll(model, members // 2, sigma=1e-3, chunk=256, fitness='ranks')
    idx, targets = sequence(T, seed=0)
    loss = es.step(idx[None].to(dev), targets[None].to(dev), opt, 1)
    torch.cuda.synchronize()
    print(f'probe-step: copy 1 GiB, one step of {members} members x {T} tokens, mean loss {loss:.6f}', flush=True)


def probe_attention(members=512, T=2048, reps=2):
    """Counter-collection workload: the window-1024 and window-2048 attention launches of one
    bench chunk (512 members x 2048 tokens x 8 heads, unit-rms q and k), `reps` times each."""
    import noise_amd  # noqa: F401  (loads the library)
    from noise_amd import kernels as K
    dev = torch.device('cuda', 0)
    g = torch.Generator(device=dev).manual_seed(0)
    M = members * T
    qkv = torch.empty(M, 1536, device=dev, dtype=torch.bfloat16)
    for i in range(3):  # q, k unit-rms per head; v N(0, 1)
        blk = torch.randn(M, 512, device=dev, generator=g)
        if i < 2:
            blk = blk.view(M, 8, 64)
            blk = (blk * torch.rsqrt(blk.square().mean(-1, keepdim=True))).view(M, 512)
        qkv[:, i * 512:(i + 1) * 512] = blk.bfloat16()
        del blk
    y = torch.empty(M, 512, device=dev, dtype=torch.bfloat16)
    b = torch.randn(members // 2, 512, device=dev, generator=g)
    uproj = torch.empty(M, 8, device=dev)
    for _ in range(reps):
        for w in (1024, 2048):
            K.window_attention(qkv, y, members, T, w, b, 1, uproj)
    torch.cuda.synchronize()
    print(f'probe-attention: {reps} x windows 1024 and 2048 over {members} members x {T} tokens', flush=True)


# cycle_derivatives: per (token, direction, vocabulary entry) 4 full-rate VALU instructions (2
# cycles per wave64 instruction) and 3 quarter-rate transcendentals (8 cycles) -> 32 SIMD cycles
# per 64 elements; 1024 SIMDs at 2.4 GHz.
PEAK_PROBE_ELEMS = 1024 * 2.4e9 * 64 / (4 * 2 + 3 * 8)


def _median_launch_ms(fn, reps=6):
    fn()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for e0, e1 in ev:
        e0.record()
        fn()
        e1.record()
    torch.cuda.synchronize()
    return sorted(e0.elapsed_time(e1) for e0, e1 in ev)[reps // 2]


def power_probe():
    """The same launches with the bench's random operands and with zeroed ones: the instruction
    stream is identical, so a shorter time with zeros is the power limit (MFMA switching energy
    falls with zero operands and the clock rises). Fused MLP alone at 512 members x 2048 tokens
    (zero packed weights: c_fc and with it the relu^2 operand of c_proj vanish), and the
    row-resident bf16 head at 1,048,576 rows x V = 4096 (zero weight, then zero rows too)."""
    from noise_amd import _lib
    from noise_amd import kernels as K
    from noise_amd.kernels import NoiseRows
    a = mlp_inputs()
    flags = _lib.MLP_NORM | _lib.MLP_RESIDUAL
    x0 = a['x'].clone()

    def mlp():
        a['x'].copy_(x0)
        K.mlp_fused(a['x'], a['x'], a['T'], a['members'], a['w_fc'], a['w_pr'], flags, a['sign'], a['fc'], a['pr'])

    copy = _median_launch_ms(lambda: a['x'].copy_(x0))
    out = {'kernel': 'mlp_fused_kernel<true, true, 0, false> (the MLP alone)', 'unit': 'ms per launch',
           'random_operands': _median_launch_ms(mlp) - copy}
    a['w_fc'].zero_()
    a['w_pr'].zero_()
    out['zero_weights'] = _median_launch_ms(mlp) - copy
    print(json.dumps(out), flush=True)
    del a, x0
    torch.cuda.empty_cache()
    dev = torch.device('cuda', 0)
    g = torch.Generator(device=dev).manual_seed(3)
    M, T, V = 512 * 2048, 2048, 4096
    h = torch.randn(M, 512, device=dev, generator=g).to(torch.bfloat16)
    W = (torch.randn(V, 512, device=dev, generator=g) * 0.05).to(torch.bfloat16)
    targets = torch.randint(0, V, (M,), device=dev, generator=g)
    ce = torch.empty(M, device=dev)
    sign = torch.tensor([1e-3, -1e-3], device=dev).repeat(256)
    nz = NoiseRows(a=torch.randn(256, V, device=dev, generator=g), shift=1)
    u = torch.randn(M, device=dev, generator=g)
    head = lambda: K.head_ce(h, W, None, T, targets, ce, sign, nz, u, targets_stride=T, ignore_index=-1)
    out = {'kernel': 'head_rr_kernel<false> (bf16 head)', 'unit': 'ms per launch', 'random_operands': _median_launch_ms(head)}
    W.zero_()
    out['zero_weights'] = _median_launch_ms(head)
    h.zero_()
    out['zero_weights_and_rows'] = _median_launch_ms(head)
    print(json.dumps(out), flush=True)


def bench_probe_cycle(steps, warmup, no_cpu, n=2048, P=512, V=4096):
    """The readout probe of the current records on one GPU: cycle_derivatives over one 2048-token
    sequence along a full cycle of 512 directions, V = 4096 (train/speedrun/run.py:250-265)."""
    from noise_amd import probes
    from noise_amd.synthetic import probe_inputs
    dev = torch.device('cuda', 0)
    torch.cuda.set_device(dev)
    d = {k: v.to(dev) for k, v in probe_inputs(n, 512, V, sigma=0.005, seed=0).items()}
    args = (d['base'], d['C'], d['y'], d['steps'], d['sq'], d['dots'], d['dir_sq'])
    for _ in range(warmup):
        probes.cycle_derivatives(*args)
    stream = torch.cuda.current_stream()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for a, b in events:
        a.record(stream)
        out = probes.cycle_derivatives(*args)
        b.record(stream)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    launch_ms = sum(a.elapsed_time(b) for a, b in events) / steps
    elems = n * P * V
    achieved = elems / (launch_ms / 1e3)
    line = {
        'metric': 'readout probe evaluations/sec on 1 GPU (cycle_derivatives: token x direction, soft-capped LSE over V)',
        'value': n * P * steps / elapsed, 'unit': 'probes/s', 'n_gpus': 1, 'steps': steps, 'warmup': warmup,
        'ms_per_step': elapsed / steps * 1e3, 'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None,
        'dtype': 'f32', 'data': 'synthetic (N(0,4) streams, N(0,9/512) head, sign-flipped Hadamard cycle, Zipf targets)',
        'config': {'workload': 'readout probe: 2048 tokens x 512 directions x V=4096', 'tokens': n, 'directions': P,
                   'vocab': V, 'width': 512, 'sigma': 0.005},
        'roofline': {'bound': 'valu', 'achieved': achieved / 1e9, 'peak': PEAK_PROBE_ELEMS / 1e9, 'unit': 'Gelem/s',
                     'frac': achieved / PEAK_PROBE_ELEMS, 'traffic': None,
                     'kernel': 'probe_kernel<4,4> + clean_sum_kernel (one cycle_derivatives call)',
                     'elements_per_launch': elems, 'launch_ms': launch_ms},
        'finite': bool(torch.isfinite(out).all()),
    }
    if not no_cpu:
        line['cpu_baseline'] = cpu_baseline_probe(n, P, V)
    print(json.dumps(line), flush=True)


def bench_probe_chain(steps, warmup, m=256, P=512, L=8, W=512, H=2048, k=128, V=4096, own=None, K=64, T=2048):
    """chain_chunk (train/val/run.py:307-351) for one chunk of the Cut estimator: 256 tokens x a full
    cycle of 512 moves of the raw embedding (site -1) through 8 blocks with 128 routed units each,
    then the head over V = 4096. own: every block also moves its own token's attention through its
    own query along its top K = 64 keys per head (own = 'routed', the estimator's default) or over
    its whole key window (own = 'window': the chunk of the last 256 positions of a 2048-token
    sequence, windows 1024 / 2048 by layer, key windows cut to multiples of 256 as the reference's
    own_query_window does)."""
    from noise_amd import probes
    dev = torch.device('cuda', 0)
    torch.cuda.set_device(dev)
    g = torch.Generator(device=dev).manual_seed(0)
    rn = lambda *s: torch.randn(*s, device=dev, generator=g)
    nrm = lambda x: x * torch.rsqrt(x.square().mean(-1, keepdim=True) + 1.1920929e-07)
    e = rn(m, W) * 2
    mids = [rn(m, W) * 3 for _ in range(L)]
    w_fc = [(rn(H, W) * 3 ** 0.5 / W ** 0.5).bfloat16() for _ in range(L)]
    w_out_t = [(rn(H, W) / H ** 0.5).bfloat16() for _ in range(L)]
    idx = [torch.argsort(rn(m, H), -1)[:, :k].contiguous() for _ in range(L)]
    hs = [torch.einsum('mkd,md->mk', w_fc[b].float()[idx[b]], nrm(mids[b])) for b in range(L)]
    xL = rn(m, W) * 4
    weight = rn(V, W) * 3 / W ** 0.5
    y = torch.randint(0, V, (m,), device=dev, generator=g)
    steps_ = 0.01 * e.square().mean(-1, keepdim=True).sqrt()
    args = dict(move=steps_.unsqueeze(-1) * rn(m, P, W), scale=steps_.expand(-1, P).contiguous(), e=e, x0=nrm(e),
                mids=mids, xL=xL, idx=idx, hs=hs, lam_r=torch.ones(L), lam_0=torch.full((L,), 0.1), w_fc=w_fc,
                w_out_t=w_out_t, weight_t=weight.T.bfloat16().contiguous(), base=xL @ weight.T,
                target_logit_w=weight[y], y=y)
    if own == 'window':
        heads = W // 64
        ang = torch.arange(T, device=dev)[:, None].float() * (1.0 / 1024 ** torch.linspace(0, 1, 32, device=dev))[None]
        windows = [1024, 1024, 1024, 2048, 1024, 1024, 1024, 2048][:L]
        t0, t1 = T - m, T
        rels, keys, vals = [], [], []
        for w in windows:
            length = min(T, -(-(t1 - max(0, t0 - w)) // 256) * 256)
            start = max(0, t1 - length)
            rels.append(torch.arange(t0, t1, device=dev) - start)
            k_ = rn(heads, length, 64)
            keys.append((k_ * torch.rsqrt(k_.square().mean(-1, keepdim=True))).bfloat16())
            vals.append(rn(heads, length, 64).bfloat16())
        args['own'] = ('window', torch.arange(t0, t1, device=dev), rels, [rn(m, W) * 3 for _ in range(L)],
                       [rn(W, W) / W ** 0.5 for _ in range(L)], keys, vals, [rn(W, W) / W ** 0.5 for _ in range(L)],
                       ang.cos(), ang.sin(), windows)
    elif own == 'routed':
        heads = W // 64
        ang = torch.arange(T, device=dev)[:, None].float() * (1.0 / 1024 ** torch.linspace(0, 1, 32, device=dev))[None]
        keys = []
        for _ in range(L):
            k_ = rn(m, heads, K, 64)
            keys.append((k_ * torch.rsqrt(k_.square().mean(-1, keepdim=True))).bfloat16())
        probs = [torch.softmax(rn(m, heads, K + 32) * 2, -1).sort(-1, descending=True).values[..., :K].contiguous()
                 for _ in range(L)]
        args['own'] = ('routed', torch.arange(m, device=dev) + (T - m), [rn(m, W) * 3 for _ in range(L)],
                       [rn(W, W) / W ** 0.5 for _ in range(L)], keys,
                       [rn(m, heads, K, 64).bfloat16() for _ in range(L)], probs,
                       [(1 - p.sum(-1, keepdim=True)) * rn(m, heads, 64) * 0.5 for p in probs],
                       [rn(W, W) / W ** 0.5 for _ in range(L)], (ang.cos(), ang.sin()))
    for _ in range(warmup):
        probes.chain_chunk(-1, **args)
    stream = torch.cuda.current_stream()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for a, b in events:
        a.record(stream)
        out = probes.chain_chunk(-1, **args)
        b.record(stream)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    call_ms = sum(a.elapsed_time(b) for a, b in events) / steps
    flops = 2 * m * P * W * k * 2 * L + 2 * m * P * W * V
    if own:  # per block: two float32 products as three bf16 MFMA products each, then per head the
        # routed 64-key products (2 x 64 x 64) or the window's two passes (3 x keys x 64, 64-key blocks)
        flops += L * (2 * (m * P + m) * W * 3 * W + 2 * m * P * W * 3 * W)
        if own == 'routed':
            flops += L * m * P * (W // 64) * 4 * 64 * 64
        else:
            keys_seen = sum(sum(-(-(min(int(r), S - 1) - max(0, int(r) - w) + 1) // 64) * 64
                                for r in rel.tolist()) for rel, w, S in
                            zip(args['own'][2], args['own'][10], [kk.shape[1] for kk in args['own'][5]]))
            flops += P * (W // 64) * 6 * 64 * keys_seen
    workload = {None: 'chain_chunk site -1, attention held: ', 'routed': 'chain_chunk site -1, own-query routed (K=64): ',
                'window': 'chain_chunk site -1, own-query over key windows (1024/2048): '}[own] + \
        '256 tokens x 512 moves, 8 blocks, k=128, V=4096'
    line = {
        'metric': 'chain_chunk moves/sec on 1 GPU (token x move through 8 routed blocks and the soft-capped head)',
        'value': m * P * steps / elapsed, 'unit': 'moves/s', 'n_gpus': 1, 'steps': steps, 'warmup': warmup,
        'ms_per_step': elapsed / steps * 1e3, 'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None,
        'dtype': 'bf16', 'data': 'synthetic (random streams, bf16 block weights, Gaussian moves)',
        'config': {'workload': workload, 'tokens': m, 'moves': P, 'blocks': L, 'routed_units': k, 'vocab': V,
                   'own': own},
        'roofline': {'bound': 'mfma', 'achieved': flops / (call_ms / 1e3) / 1e12, 'peak': PEAK_BF16 / 1e12,
                     'unit': 'TFLOP/s', 'frac': flops / (call_ms / 1e3) / PEAK_BF16, 'traffic': None,
                     'kernel': 'one chain_chunk call (start + 8 blocks + head)', 'flops_per_call': flops,
                     'call_ms': call_ms},
        'finite': bool(torch.isfinite(out).all()),
        'cpu_baseline': cpu_baseline_chain(args, P, tokens=2 if own == 'window' else 8),
    }
    print(json.dumps(line), flush=True)


def cpu_baseline_chain(args, P, tokens=8):
    """The oracle's chain_chunk (numpy float32 with the reference's bf16 casts) on the first
    `tokens` tokens of the same chunk, every move, the same own mode."""
    from oracle import probes_ref as R
    sl = slice(0, tokens)
    f = lambda t: t.detach().cpu().double().numpy() if t.is_floating_point() else t.detach().cpu().numpy()
    tok = {'move', 'scale', 'e', 'x0', 'xL', 'base', 'target_logit_w', 'y'}
    per_tok_lists = {'mids', 'idx', 'hs'}
    kw = {}
    for key, v in args.items():
        if key == 'own':
            continue
        if key in tok:
            kw[key] = f(v[sl])
        elif key in per_tok_lists:
            kw[key] = [f(t[sl]) for t in v]
        elif isinstance(v, list):
            kw[key] = [f(t) for t in v]
        else:
            kw[key] = f(v)
    own = args.get('own')
    if own is not None and own[0] == 'routed':
        _, pos, inputs, w_q, keys, vals, probs, rests, w_proj_t, (cos, sin) = own
        kw['own'] = ('routed', f(pos[sl]), [f(t[sl]) for t in inputs], [f(t) for t in w_q], [f(t[sl]) for t in keys],
                     [f(t[sl]) for t in vals], [f(t[sl]) for t in probs], [f(t[sl]) for t in rests],
                     [f(t) for t in w_proj_t], (f(cos), f(sin)))
    elif own is not None:
        _, pos, rels, inputs, w_q, keys, vals, w_proj_t, cos, sin, windows = own
        kw['own'] = ('window', f(pos[sl]), [f(t[sl]) for t in rels], [f(t[sl]) for t in inputs], [f(t) for t in w_q],
                     [f(t) for t in keys], [f(t) for t in vals], [f(t) for t in w_proj_t], f(cos), f(sin), windows)
    t0 = time.perf_counter()
    R.chain_chunk(-1, **kw, policy='build32')
    dt = time.perf_counter() - t0
    return {'value': tokens * P / dt, 'unit': 'moves/s', 'cores': os.cpu_count() or 1, 'kind': 'port',
            'sample': f'oracle chain_chunk in numpy float32 (bf16 casts kept) on {tokens} tokens x {P} moves of '
                      'the same chunk, same own mode; numpy may use every host core'}


def cpu_baseline_probe(n, P, V, tokens=768):
    import numpy as np
    from noise_amd.synthetic import probe_inputs
    from oracle import probes_ref as R
    d = probe_inputs(tokens, 512, V, probes=P, sigma=0.005, seed=0)
    args = [d[k].numpy() for k in ('base', 'C', 'y', 'steps', 'sq', 'dots', 'dir_sq')]
    R.cycle_derivatives(*[a[:1] if a.shape[0] == tokens else a for a in args], dtype=np.float32)
    t0 = time.perf_counter()
    R.cycle_derivatives(*args, dtype=np.float32, chunk=1)
    dt = time.perf_counter() - t0
    return {'value': tokens * P / dt, 'unit': 'probes/s', 'cores': 1, 'kind': 'port',
            'sample': f'oracle cycle_derivatives in numpy float32 on CPU, {tokens} tokens x {P} directions x V={V}'}


def _cpu_model():
    try:
        for line in open('/proc/cpuinfo'):
            if line.startswith('model name'):
                return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return 'unknown'


def _median_time(fn, seconds_budget, max_reps=5):
    t0 = time.perf_counter()
    fn()  # warmup
    first = time.perf_counter() - t0
    reps = max(1, min(max_reps, int(seconds_budget / max(first, 1e-3))))
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], reps


def cpu_baseline(seconds_budget=20.0):
    """The CPU oracle's fp32 population_loss on the host cores: the bench's own workload at
    T = 2048 (one antithetic pair, a bounded sample of the 3072 members) and config 0 of the
    baseline (8 members, T = 256, Zipf(1.1) tokens, seed-0 weights, sigma 1e-3)."""
    from noise_amd.synthetic import antithetic, pair_noise, sequence
    from oracle import model_ref as R
    threads = int(os.environ.get('OMP_NUM_THREADS') or 0) or (os.cpu_count() or 1)
    torch.set_num_threads(threads)
    params = R.init_params(0)
    idx, targets = sequence(2048, seed=0)
    noise, sign = antithetic(pair_noise(1, seed=1), 1e-3)
    med, reps = _median_time(lambda: R.population_loss(params, noise, sign, idx, targets, policy='fp32'),
                             seconds_budget)
    idx0, tg0 = sequence(256, seed=0)
    noise0, sign0 = antithetic(pair_noise(4, seed=1), 1e-3)
    med0, reps0 = _median_time(lambda: R.population_loss(params, noise0, sign0, idx0, tg0, policy='fp32'),
                               seconds_budget / 4)
    return {'value': 2 * 2048 / med, 'unit': 'member-tokens/s', 'cores': threads, 'kind': 'port',
            'sample': f'oracle population_loss fp32 on CPU, 2 members (1 antithetic pair) x 2048 tokens, '
                      f'median of {reps} after 1 warmup',
            'cpu_model': _cpu_model(),
            'config0': {'value': 8 * 256 / med0, 'unit': 'member-tokens/s',
                        'sample': f'config 0: 8 members (4 pairs) x 256 tokens, median of {reps0} after 1 warmup'}}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=3)
    ap.add_argument('--warmup', type=int, default=1)
    ap.add_argument('--members', type=int, default=3072)
    ap.add_argument('--tokens', type=int, default=2048)
    ap.add_argument('--chunk', type=int, default=512,
                    help='pairs per batched forward (a member\'s loss does not depend on it)')
    ap.add_argument('--no-cpu', action='store_true', help='skip the CPU baseline')
    ap.add_argument('--no-extra', action='store_true',
                    help='skip the measurements after the timed steps (MLP alone, fp32-accurate head step)')
    ap.add_argument('--probe-mlp', action='store_true', help='run the MLP counter-collection workload only')
    ap.add_argument('--probe-attention', action='store_true', help='run the attention counter-collection workload only')
    ap.add_argument('--probe-step', action='store_true', help='run the whole-step counter-collection workload only')
    ap.add_argument('--probe-cycle', action='store_true', help='bench the readout probe kernels (own JSON line)')
    ap.add_argument('--probe-chain', action='store_true', help='bench chain_chunk (own JSON line)')
    ap.add_argument('--power-probe', action='store_true',
                    help='the fused MLP and the head with their real operands and with zeros (own JSON lines)')
    ap.add_argument('--own', choices=['none', 'routed', 'window'], default='none',
                    help='--probe-chain: every attention held, the routed own-query moves, or over key windows')
    args = ap.parse_args()
    if args.gpus != 1:
        print(f'bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}). '
              'Run with --gpus 1.', file=sys.stderr)
        sys.exit(2)

    if args.probe_mlp:
        probe_mlp()
        return
    if args.probe_attention:
        probe_attention()
        return
    if args.probe_step:
        probe_step()
        return
    if args.probe_cycle:
        bench_probe_cycle(max(args.steps, 5), args.warmup, args.no_cpu)
        return
    if args.probe_chain:
        bench_probe_chain(max(args.steps, 5), args.warmup, own=None if args.own == 'none' else args.own)
        return
    if args.power_probe:
        power_probe()
        return

    import noise_amd
    from noise_amd.synthetic import sequence

    device = torch.device('cuda', 0)
    torch.cuda.set_device(device)
    pairs = args.members // 2
    T = args.tokens
    model = noise_amd.make_model(device, 0)
    opt = noise_amd.AdamW(model.parameters(), lr=1e-3, betas=(0.5, 0.95), eps=1e-8, weight_decay=0.0)
    es = noise_amd.Eggroll(model, pairs, sigma=1e-3, chunk=args.chunk, fitness='ranks')
    idx, targets = sequence(T, seed=0)
    x, y = idx[None].to(device), targets[None].to(device)

    for s in range(args.warmup):
        es.step(x, y, opt, s + 1)
    es.engine.probe = []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    losses = []
    for s in range(args.steps):
        losses.append(es.step(x, y, opt, args.warmup + s + 1))
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    probe, es.engine.probe = es.engine.probe, None

    mlp_ms = sum(a.elapsed_time(b) for a, b, _ in probe) / len(probe)
    rows = probe[0][2]
    flops = mlp_flops(rows, attn=es.engine.fused_mlp and es.engine.fuse_attn_proj)
    achieved = flops / (mlp_ms / 1e3) / 1e12
    members = 2 * pairs
    value = members * T * args.steps / elapsed
    out = {
        'metric': 'perturbed member-tokens/sec on 1 GPU; fused-MLP MFMA % of bf16 peak',
        'value': value,
        'unit': 'member-tokens/s',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': elapsed / args.steps * 1e3,
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'bf16',
        'data': 'synthetic (Zipf(1.1) tokens, seed-0 weights, N(0,1) noise buffer)',
        'config': {'workload': 'config 4: full EGGROLL population step (forward + rank-normalised fitness + '
                               'rank-1 gradient + AdamW)',
                   'members': members, 'pairs': pairs, 'seq_len': T, 'sigma': 1e-3, 'model': '37.7M (8x512, V=4096)',
                   'members_per_forward': 2 * args.chunk, 'parallelism': 'single GPU'},
        'roofline': {'bound': 'mfma', 'achieved': achieved, 'peak': PEAK_BF16 / 1e12, 'unit': 'TFLOP/s',
                     'frac': achieved * 1e12 / PEAK_BF16, 'traffic': mlp_traffic(rows),
                     'kernel': 'mlp_fused: attention c_proj + rank-1 into the residual rows, then norm + c_fc + '
                               'rank-1 + relu^2 + c_proj + rank-1 + residual, hidden on chip, then the next '
                               "layer's mix_norm (x0 mixing, norm, q/k/v dots, gate) in the epilogue",
                     'flops_per_launch': flops, 'rows_per_launch': rows, 'launch_ms': mlp_ms},
        'step_tflops': step_flops(members, T) / (elapsed / args.steps) / 1e12,
        'mean_loss': losses[-1],
    }
    # Outside the timed region: (1) the relu^2 MLP alone (config 1's kernel, no attention c_proj
    # fold, no next-layer norm) at the same rows, its fraction of peak for the MLP's own FLOPs;
    # (2) one step with the head as the fp32-weight product (bf16 hi + lo halves, config 4's
    # "fp32 head") instead of the trainer's bf16 autocast product.
    if not args.no_extra:
        out['mlp_only'] = mlp_only_roofline()
        from noise_amd.population import PreparedWeights
        es.weights = PreparedWeights(es.params, es.cfg, head_split=True)
        es.step(x, y, opt, args.warmup + args.steps + 1)  # warmup of the hi + lo head
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        es.step(x, y, opt, args.warmup + args.steps + 2)
        torch.cuda.synchronize()
        hs = time.perf_counter() - t0
        out['head_split'] = {'ms_per_step': hs * 1e3, 'value': members * T / hs, 'unit': 'member-tokens/s',
                             'steps': 1, 'warmup': 1,
                             'note': 'one step with the head product on fp32-accurate weights (bf16 hi + lo halves)'}
    if not args.no_cpu:
        out['cpu_baseline'] = cpu_baseline()
    print(json.dumps(out), flush=True)


def mlp_only_roofline(reps=5):
    """The fused relu^2 MLP alone (norm, c_fc + rank-1, relu^2, c_proj + rank-1, residual, the hidden
    on chip) at the bench's 512 members x 2048 tokens: mean launch time from HIP events on the
    launch stream, and its fraction of bf16 peak for rows * (4 d f + 2 (d + f)) FLOPs."""
    from noise_amd import _lib
    from noise_amd import kernels as K
    a = mlp_inputs()
    stream = torch.cuda.current_stream()
    launch = lambda: K.mlp_fused(a['x'], a['x'], a['T'], a['members'], a['w_fc'], a['w_pr'],
                                 _lib.MLP_NORM | _lib.MLP_RESIDUAL, a['sign'], a['fc'], a['pr'])
    launch()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for e0, e1 in events:
        e0.record(stream)
        launch()
        e1.record(stream)
    torch.cuda.synchronize()
    ms = sum(e0.elapsed_time(e1) for e0, e1 in events) / reps
    # the two-wave (producer/consumer) form of the same launch, bit-identical and opt-in
    os.environ['NOISE_MLP_TWO_WAVE'] = '1'
    try:
        launch()
        for e0, e1 in events:
            e0.record(stream)
            launch()
            e1.record(stream)
        torch.cuda.synchronize()
        ms2 = sum(e0.elapsed_time(e1) for e0, e1 in events) / reps
    finally:
        del os.environ['NOISE_MLP_TWO_WAVE']
    rows = a['x'].shape[0]
    flops = mlp_flops(rows, attn=False)
    del a
    torch.cuda.empty_cache()
    return {'launch_ms': ms, 'two_wave_launch_ms': ms2, 'flops_per_launch': flops, 'rows_per_launch': rows,
            'achieved': flops / (ms / 1e3) / 1e12, 'unit': 'TFLOP/s', 'frac': flops / (ms / 1e3) / PEAK_BF16,
            'kernel': 'mlp_fused alone (norm, c_fc, relu^2, c_proj, residual; no attention c_proj, no next norm)'}


if __name__ == '__main__':
    main()
