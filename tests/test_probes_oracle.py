"""Pins the probe oracle (oracle/probes_ref.py) by brute force, in float64 on the CPU.

Each closed form is checked against an evaluation that does not use it: the moved logits (or the
moved stream, its RMS norm and the head) are formed explicitly, one forward per probe, and the
loss comes from torch.nn.functional.cross_entropy. A dropped target correction, a wrong sign of
the cross term in |x + s D|^2, a missing mask or a transposed C fails these.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from noise_amd.synthetic import probe_inputs
from oracle import probes_ref as P

F64 = torch.float64
EPS = float(np.finfo(np.float32).eps)


def readout_loss(x, weight, y, width):
    """Soft-capped readout CE of streams x [.., width] (train/val/run.py:238-242), float64."""
    logits = x * torch.rsqrt(x.square().sum(-1, keepdim=True) / width + EPS) @ weight.T
    logits = 15 * torch.tanh(logits / 15)
    return F.cross_entropy(logits, y.clamp(min=0), reduction='none') * (y >= 0)


def capped_ce(raw, y):
    return F.cross_entropy(15 * torch.tanh(raw / 15), y.clamp(min=0), reduction='none') * (y >= 0)


@pytest.mark.parametrize('sigma', [0.1, 0.5])
def test_coordinate_differences_brute_force(sigma):
    g = torch.Generator().manual_seed(3)
    n, V = 6, 96
    raw = torch.randn(n, V, generator=g, dtype=F64) * 12     # many logits in the cap's bend
    raw[0, :8] = torch.tensor([60., -60., 40., 0., 14.9, -30., 200., 1e-3], dtype=F64)
    y = torch.randint(0, V, (n,), generator=g)
    y[2] = -1
    y[3] = 0
    want = torch.empty(n, V, dtype=F64)
    for v in range(V):
        e = torch.zeros(V, dtype=F64)
        e[v] = sigma
        want[:, v] = (capped_ce(raw + e, y) - capped_ce(raw - e, y)) / (2 * sigma)
    got = P.coordinate_differences(raw.numpy(), y.numpy(), sigma)
    np.testing.assert_allclose(got, want.numpy(), rtol=1e-9, atol=1e-12)
    assert np.all(got[2] == 0)


@pytest.mark.parametrize('dirs', ['hadamard', 'gaussian'])
def test_cycle_derivatives_brute_force(dirs):
    width, V, n = 32, 80, 7
    d = probe_inputs(n, width, V, sigma=0.05, dirs=dirs, probes=24 if dirs == 'gaussian' else None,
                     seed=5, dtype=F64)
    d['y'][4] = -1
    x, W, D, y, s = d['x'], d['weight'], d['D'], d['y'], d['steps']
    clean = readout_loss(x, W, y, width)
    want = torch.stack([(readout_loss(x + s[:, None] * D[:, j], W, y, width) - clean) / s
                        for j in range(D.shape[1])], 1)
    got = P.cycle_derivatives(d['base'], d['C'], y, s, d['sq'], d['dots'], d['dir_sq'], width=width)
    np.testing.assert_allclose(got, want.numpy(), rtol=1e-8, atol=1e-10)
    assert np.all(got[4] == 0)


def test_row_derivatives_brute_force_and_cycle():
    width, V, n, K = 32, 64, 9, 5
    d = probe_inputs(n, width, V, sigma=0.02, seed=7, dtype=F64)
    g = torch.Generator().manual_seed(1)
    rows = torch.stack([torch.randperm(width, generator=g)[:K] for _ in range(n)])
    x, W, D, y, s = d['x'], d['weight'], d['D'], d['y'], d['steps']
    dots, dir_sq = d['dots'].gather(1, rows), d['dir_sq'][rows]
    got = P.row_derivatives(d['base'], d['C'], rows, y, s, d['sq'], dots, dir_sq, width=width)
    full = P.cycle_derivatives(d['base'], d['C'], y, s, d['sq'], d['dots'], d['dir_sq'], width=width)
    np.testing.assert_allclose(got, np.take_along_axis(full, rows.numpy(), 1), rtol=1e-12, atol=1e-14)
    clean = readout_loss(x, W, y, width)
    for i in range(n):
        for k in range(K):
            moved = readout_loss(x[i:i + 1] + s[i] * D[:, rows[i, k]], W, y[i:i + 1], width)
            assert abs(got[i, k] - float((moved - clean[i]) / s[i])) <= 1e-8 * (1 + abs(got[i, k]))


def test_cycle_derivatives_small_step_is_gradient():
    """As the step shrinks the forward difference tends to the directional derivative of the
    readout loss (autograd in float64); O(step) agreement rules out a wrong 1/step scaling."""
    width, V, n = 32, 64, 4
    d = probe_inputs(n, width, V, sigma=1e-6, seed=9, dtype=F64)
    x = d['x'].clone().requires_grad_(True)
    readout_loss(x, d['weight'], d['y'], width).sum().backward()
    want = (x.grad @ d['D']).numpy()
    got = P.cycle_derivatives(d['base'], d['C'], d['y'], d['steps'], d['sq'], d['dots'], d['dir_sq'],
                              width=width)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-6)


def _chain_inputs(site, m=3, P_=5, W=32, H=64, k=8, V=48, L=3, seed=0):
    """A tiny attention-held chain: clean streams, routed units and their clean pre-activations
    (hs = W_fc[idx] norm(mid), as the reference captures them), head and moves."""
    g = torch.Generator().manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=g, dtype=F64)
    nrm = lambda x: x * torch.rsqrt(x.square().sum(-1, keepdim=True) / W + EPS)
    e = rn(m, W) * 2
    x0 = nrm(e)
    mids = [rn(m, W) * 1.5 for _ in range(L)]
    w_fc = [rn(H, W) / W ** 0.5 for _ in range(L)]
    w_out_t = [rn(H, W) / H ** 0.5 for _ in range(L)]
    idx = [torch.stack([torch.randperm(H, generator=g)[:k] for _ in range(m)]) for _ in range(L)]
    hs = [torch.einsum('mkd,md->mk', w_fc[b][idx[b]], nrm(mids[b])) for b in range(L)]
    xL = rn(m, W) * 2
    weight = rn(V, W) * 3 / W ** 0.5
    y = torch.randint(0, V, (m,), generator=g)
    y[1] = -1
    steps = 0.05 * (e if site < 0 else mids[site]).square().mean(-1).sqrt()
    move = steps[:, None, None] * rn(m, P_, W)
    scale = steps[:, None].expand(m, P_).clone()
    lam_r, lam_0 = 1 + 0.1 * rn(L), 0.1 + 0.05 * rn(L)
    return dict(move=move, scale=scale, e=e, x0=x0, mids=mids, xL=xL, idx=idx, hs=hs, lam_r=lam_r,
                lam_0=lam_0, w_fc=w_fc, w_out_t=w_out_t, weight_t=weight.T.contiguous(),
                base=xL @ weight.T, target_logit_w=weight[y.clamp(min=0)], y=y), nrm, weight


@pytest.mark.parametrize('site', [-1, 0, 2])
def test_chain_chunk_brute_force(site):
    """chain_chunk (train/val/run.py:307-351, every attention held) against explicit moved streams:
    norm(x + D) itself, the routed units' relu^2 at the moved pre-activations, the head's CE."""
    d, nrm, weight = _chain_inputs(site)
    m, P_, W = d['move'].shape
    L = len(d['mids'])
    ce = lambda x, yy: F.cross_entropy(15 * torch.tanh(nrm(x) @ weight.T / 15), yy.clamp(min=0), reduction='none')
    want = torch.zeros(m, P_, dtype=F64)
    for i in range(m):
        if d['y'][i] < 0:
            continue
        clean = ce(d['xL'][i:i + 1], d['y'][i:i + 1])
        for p in range(P_):
            if site < 0:
                dx0 = nrm(d['e'][i] + d['move'][i, p]) - d['x0'][i]
                D, first = (d['lam_r'][0] + d['lam_0'][0]) * dx0, 0
            else:
                D, first = d['move'][i, p], site
            for b in range(first, L):
                if b > first:
                    D = d['lam_r'][b] * D + (d['lam_0'][b] * dx0 if site < 0 else 0)
                rows = d['idx'][b][i]
                hp = d['w_fc'][b][rows] @ nrm(d['mids'][b][i] + D)
                h = d['hs'][b][i]
                D = D + (torch.relu(hp).square() - torch.relu(h).square()) @ d['w_out_t'][b][rows]
            want[i, p] = (ce(d['xL'][i:i + 1] + D, d['y'][i:i + 1]) - clean)[0] / d['scale'][i, p]
    got = P.chain_chunk(site, **{k: v for k, v in d.items()}, width=W)
    np.testing.assert_allclose(got, want.numpy(), rtol=1e-9, atol=1e-11)
    assert np.all(got[1] == 0)


def test_norm_difference_is_difference_of_norms():
    g = torch.Generator().manual_seed(4)
    x, dl = torch.randn(4, 16, generator=g, dtype=F64), torch.randn(4, 3, 16, generator=g, dtype=F64) * 0.1
    nrm = lambda v: v * torch.rsqrt(v.square().sum(-1, keepdim=True) / 16 + EPS)
    np.testing.assert_allclose(P.norm_difference(x.numpy(), dl.numpy(), 16),
                               (nrm(x[:, None] + dl) - nrm(x)[:, None]).numpy(), rtol=1e-12, atol=1e-14)


def _qc_case(m=3, P_=4, W=16, heads=2, S=6, K=3, T=10, seed=0, rotary=None):
    """Own-query inputs with explicit full key sets: clean queries from the block input, the clean
    softmax over S keys per head, the top K keys by clean probability and the held keys' share.
    rotary: (pos, cos, sin) shared by several blocks, else drawn here."""
    g = torch.Generator().manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=g, dtype=F64)
    d = W // heads
    nrm = lambda v, n: v * torch.rsqrt(v.square().sum(-1, keepdim=True) / n + EPS)
    x, w_q, w_proj_t = rn(m, W) * 2, rn(W, W) / W ** 0.5, rn(W, W) / W ** 0.5
    if rotary is None:
        pos = torch.randint(0, T, (m,), generator=g)
        ang = rn(T, d // 2)
        cos, sin = ang.cos(), ang.sin()
    else:
        pos, cos, sin = rotary
    keys, vals = nrm(rn(m, heads, S, d), d), rn(m, heads, S, d)

    def query(xx):  # q for stream(s) xx (..., W) of token i: norm, W_q, rotary, per-head RMS norm
        r = (nrm(xx, W) @ w_q.T).view(*xx.shape[:-1], heads, d)
        return r, lambda i: nrm(torch.cat([r[..., :d // 2] * cos[pos[i]] + r[..., d // 2:] * sin[pos[i]],
                                           r[..., :d // 2] * -sin[pos[i]] + r[..., d // 2:] * cos[pos[i]]], -1), d)
    probs = []
    for i in range(m):
        q0 = query(x[i])[1](i)                                     # (h, d)
        probs.append(torch.softmax(torch.einsum('hd,hsd->hs', q0, keys[i]) * d ** -0.5, -1))
    probs = torch.stack(probs)                                      # (m, h, S)
    top = probs.topk(K, -1).indices
    take = lambda z: torch.gather(z, 2, top[..., None].expand(-1, -1, -1, d))
    held = torch.ones_like(probs, dtype=torch.bool).scatter(2, top, False)
    rest = torch.einsum('mhs,mhsd->mhd', probs * held, vals)
    case = dict(pos=pos, w_q=w_q, top_keys=take(keys), top_values=take(vals), top_p=probs.gather(2, top), rest=rest,
                w_proj_t=w_proj_t, cos=cos, sin=sin)

    def brute(i, D):
        """Attention output change of token i, its stream moved by D, through c_proj: the top keys'
        logits recomputed with the moved query, every other logit held."""
        q0, q1 = query(x[i])[1](i), query(x[i] + D)[1](i)
        s0 = torch.einsum('hd,hsd->hs', q0, keys[i]) * d ** -0.5
        s1 = torch.where(held[i], s0, torch.einsum('hd,hsd->hs', q1, keys[i]) * d ** -0.5)
        out = lambda s: torch.einsum('hs,hsd->hd', torch.softmax(s, -1), vals[i])
        return (out(s1) - out(s0)).reshape(-1) @ w_proj_t
    return x, case, brute


def test_query_change_routed_brute_force():
    """query_change_routed (train/val/run.py:282-304) against the moved query's full softmax with the
    held keys' logits fixed: pins the qk-norm difference, dlse = log1p(sum p expm1(ds)) and the
    expm1(-dlse) rescaling of the held share."""
    m, P_, W = 3, 4, 16
    x, c, brute = _qc_case(m, P_, W)
    g = torch.Generator().manual_seed(1)
    delta = torch.randn(m, P_, W, generator=g, dtype=F64) * 0.3
    got = P.query_change_routed(x, delta, width=W, **c)
    want = torch.stack([torch.stack([brute(i, delta[i, p]) for p in range(P_)]) for i in range(m)])
    np.testing.assert_allclose(got, want.numpy(), rtol=1e-9, atol=1e-12)


@pytest.mark.parametrize('site', [-1, 1])
def test_chain_chunk_routed_brute_force(site):
    """chain_chunk with own = ('routed', ...) (train/val/run.py:326-331): at every block the move
    enters, its own token's attention output changes through its own query along its top keys
    (the explicit held-logit softmax of the test above) before that block's MLP."""
    d, nrm, weight = _chain_inputs(site)
    m, P_, W = d['move'].shape
    L = len(d['mids'])
    g = torch.Generator().manual_seed(7)
    T, dh = 10, W // 2
    ang = torch.randn(T, dh // 2, generator=g, dtype=F64)
    rotary = (torch.randint(0, T, (m,), generator=g), ang.cos(), ang.sin())
    blocks = [_qc_case(m, P_, W, heads=2, S=7, K=4, seed=20 + b, rotary=rotary) for b in range(L)]
    own = ('routed', rotary[0], [bl[0] for bl in blocks]) + tuple(
        [bl[1][k] for bl in blocks] for k in ('w_q', 'top_keys', 'top_values', 'top_p', 'rest', 'w_proj_t')) + (
        (rotary[1], rotary[2]),)
    ce = lambda x, yy: F.cross_entropy(15 * torch.tanh(nrm(x) @ weight.T / 15), yy.clamp(min=0), reduction='none')
    want = torch.zeros(m, P_, dtype=F64)
    for i in range(m):
        if d['y'][i] < 0:
            continue
        clean = ce(d['xL'][i:i + 1], d['y'][i:i + 1])
        for p in range(P_):
            if site < 0:
                dx0 = nrm(d['e'][i] + d['move'][i, p]) - d['x0'][i]
                D, first = (d['lam_r'][0] + d['lam_0'][0]) * dx0, 0
            else:
                D, first = d['move'][i, p], site
            for b in range(first, L):
                if b > first:
                    D = d['lam_r'][b] * D + (d['lam_0'][b] * dx0 if site < 0 else 0)
                if site < 0 or b > first:
                    D = D + blocks[b][2](i, D)
                rows = d['idx'][b][i]
                hp = d['w_fc'][b][rows] @ nrm(d['mids'][b][i] + D)
                h = d['hs'][b][i]
                D = D + (torch.relu(hp).square() - torch.relu(h).square()) @ d['w_out_t'][b][rows]
            want[i, p] = (ce(d['xL'][i:i + 1] + D, d['y'][i:i + 1]) - clean)[0] / d['scale'][i, p]
    got = P.chain_chunk(site, **d, own=own, width=W)
    np.testing.assert_allclose(got, want.numpy(), rtol=1e-9, atol=1e-11)
    none = P.chain_chunk(site, **d, width=W)
    assert np.abs(got - none)[[0, 2]].max() > 1e-3 * np.abs(none).max()   # the own-query term is live


def test_tf32_rounding():
    """_tf32 keeps 10 mantissa bits, rounding to nearest with ties away from zero."""
    u = 2.0 ** -10
    vals = np.array([1.0, 1 + u, 1 + u / 2, 1 + u / 2 - 2 ** -23, 1 + 3 * u / 2, -(1 + u / 2), 3.0, 1e-30])
    want = np.array([1.0, 1 + u, 1 + u, 1.0, 1 + 2 * u, -(1 + u), 3.0, 0.0])
    got = P._tf32(vals)
    np.testing.assert_array_equal(got[:-1], want[:-1])
    assert abs(got[-1] - 1e-30) <= 1e-30 * 2 ** -10


def _window_case(m=4, P_=3, W=16, heads=2, S=9, window=4, seed=3, rotary=None):
    """query_change inputs: one key window of S positions shared by the chunk's tokens (keys
    rotated and RMS-normed per head), tokens at relative positions rel (one with fewer than
    window + 1 keys before it), and a brute force over the explicit window softmax."""
    g = torch.Generator().manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=g, dtype=F64)
    d = W // heads
    nrm = lambda v, n: v * torch.rsqrt(v.square().sum(-1, keepdim=True) / n + EPS)
    x, w_q, w_proj_t = rn(m, W) * 2, rn(W, W) / W ** 0.5, rn(W, W) / W ** 0.5
    if rotary is None:
        T = 20
        ang = rn(T, d // 2)
        pos, cos, sin = torch.randint(0, T, (m,), generator=g), ang.cos(), ang.sin()
    else:
        pos, cos, sin = rotary
    keys, vals = nrm(rn(heads, S, d), d), rn(heads, S, d)
    rel = torch.tensor([S - 1, 2, S - 3, window][:m] + [S - 1] * max(0, m - 4))

    def query(xx, i):
        r = (nrm(xx, W) @ w_q.T).view(heads, d)
        return nrm(torch.cat([r[:, :d // 2] * cos[pos[i]] + r[:, d // 2:] * sin[pos[i]],
                              r[:, :d // 2] * -sin[pos[i]] + r[:, d // 2:] * cos[pos[i]]], -1), d)

    def brute(i, D):
        allowed = [t for t in range(S) if 0 <= int(rel[i]) - t <= window]
        kk, vv = keys[:, allowed], vals[:, allowed]
        out = lambda q: torch.einsum('hs,hsd->hd', torch.softmax(torch.einsum('hd,hsd->hs', q, kk) * d ** -0.5, -1), vv)
        return (out(query(x[i] + D, i)) - out(query(x[i], i))).reshape(-1) @ w_proj_t
    case = dict(pos=pos, rel=rel, w_q=w_q, keys=keys, values=vals, w_proj_t=w_proj_t, cos=cos, sin=sin, window=window)
    return x, case, brute


def test_query_change_brute_force():
    """query_change (train/val/run.py:256-281) against the moved query's explicit softmax over the
    token's window (lag 0..window, inclusive), every logit in it moving."""
    m, P_, W = 4, 3, 16
    x, c, brute = _window_case(m, P_, W)
    g = torch.Generator().manual_seed(2)
    delta = torch.randn(m, P_, W, generator=g, dtype=F64) * 0.3
    got = P.query_change(x, delta, width=W, **c)
    want = torch.stack([torch.stack([brute(i, delta[i, p]) for p in range(P_)]) for i in range(m)])
    np.testing.assert_allclose(got, want.numpy(), rtol=1e-9, atol=1e-12)


@pytest.mark.parametrize('site', [-1, 0])
def test_chain_chunk_window_brute_force(site):
    """chain_chunk with own = ('window', ...) (train/val/run.py:332-335) against explicit moved
    streams with the window attention change before every later MLP."""
    d, nrm, weight = _chain_inputs(site)
    m, P_, W = d['move'].shape
    L = len(d['mids'])
    g = torch.Generator().manual_seed(11)
    T, dh = 20, W // 2
    ang = torch.randn(T, dh // 2, generator=g, dtype=F64)
    rotary = (torch.randint(0, T, (m,), generator=g), ang.cos(), ang.sin())
    blocks = [_window_case(m, P_, W, heads=2, S=8 + b, window=3 + 2 * b, seed=30 + b, rotary=rotary)
              for b in range(L)]
    own = ('window', rotary[0], [bl[1]['rel'] for bl in blocks], [bl[0] for bl in blocks],
           [bl[1]['w_q'] for bl in blocks], [bl[1]['keys'] for bl in blocks], [bl[1]['values'] for bl in blocks],
           [bl[1]['w_proj_t'] for bl in blocks], rotary[1], rotary[2], [bl[1]['window'] for bl in blocks])
    ce = lambda x, yy: F.cross_entropy(15 * torch.tanh(nrm(x) @ weight.T / 15), yy.clamp(min=0), reduction='none')
    want = torch.zeros(m, P_, dtype=F64)
    for i in range(m):
        if d['y'][i] < 0:
            continue
        clean = ce(d['xL'][i:i + 1], d['y'][i:i + 1])
        for p in range(P_):
            if site < 0:
                dx0 = nrm(d['e'][i] + d['move'][i, p]) - d['x0'][i]
                D, first = (d['lam_r'][0] + d['lam_0'][0]) * dx0, 0
            else:
                D, first = d['move'][i, p], site
            for b in range(first, L):
                if b > first:
                    D = d['lam_r'][b] * D + (d['lam_0'][b] * dx0 if site < 0 else 0)
                if site < 0 or b > first:
                    D = D + blocks[b][2](i, D)
                rows = d['idx'][b][i]
                hp = d['w_fc'][b][rows] @ nrm(d['mids'][b][i] + D)
                h = d['hs'][b][i]
                D = D + (torch.relu(hp).square() - torch.relu(h).square()) @ d['w_out_t'][b][rows]
            want[i, p] = (ce(d['xL'][i:i + 1] + D, d['y'][i:i + 1]) - clean)[0] / d['scale'][i, p]
    got = P.chain_chunk(site, **d, own=own, width=W)
    np.testing.assert_allclose(got, want.numpy(), rtol=1e-9, atol=1e-11)
    none = P.chain_chunk(site, **d, width=W)
    assert np.abs(got - none)[[0, 2]].max() > 1e-3 * np.abs(none).max()
