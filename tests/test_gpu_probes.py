"""Parity of the probe kernels (libnoise_amd through noise_amd.probes) with the float64 oracle
(oracle/probes_ref.py), on the same seeded inputs.

Tolerances. The probes are differences of two soft-capped log-sum-exps over the vocabulary,
divided by the step: in float32 the reference's own formula (train/val/run.py:154-167) is off from
the exact value by up to ~4e-6 in (moved - clean) on these inputs (the oracle evaluated in
float32 shows it), i.e. ~4e-6 / step on a derivative. The kernels are held to
|gpu - exact| <= 8e-6 / step + 1e-5 |exact| per element and a mean error below 1.5e-6 / step.
coordinate_differences forms cap(raw +- sigma) - cap(raw) without cancellation and is held to
2e-6 + 1e-4 |exact|. chain_chunk carries the reference's bf16 casts: see its test.
"""
import numpy as np
import pytest
import torch

from noise_amd.synthetic import probe_inputs
from oracle import probes_ref as P

pytestmark = pytest.mark.gpu

ATOL_STEP, RTOL, MEAN_STEP = 8e-6, 1e-5, 1.5e-6


def _probes():
    from noise_amd import probes
    return probes


def _cuda(d, device):
    return {k: v.to(device) for k, v in d.items()}


def _check_probe(got, want, steps, mask_rows=(), nan_rows=()):
    got = got.cpu().double().numpy()
    s = steps.cpu().double().numpy().reshape(-1, 1)
    ok = np.ones(got.shape[0], bool)
    for i in mask_rows:
        assert np.all(got[i] == 0), i
        ok[i] = False
    for i in nan_rows:
        assert np.all(np.isnan(got[i])), i
        ok[i] = False
    err = np.abs(got[ok] - want[ok])
    bound = ATOL_STEP / s[ok] + RTOL * np.abs(want[ok])
    worst = np.unravel_index(np.argmax(err - bound), err.shape)
    assert np.all(err <= bound), (worst, got[ok][worst], want[ok][worst], err[worst], bound[worst])
    assert float((err * s[ok]).mean()) <= MEAN_STEP


@pytest.mark.parametrize('n,P_,V,dirs', [(37, 72, 4096, 'hadamard'), (5, 3, 4096, 'gaussian'),
                                        (64, 512, 4096, 'hadamard')])
def test_cycle_derivatives_matches_oracle(device, n, P_, V, dirs):
    d = probe_inputs(n, 512, V, probes=P_, sigma=0.005, dirs=dirs, seed=n + P_, masked=0.1)
    y = d['y'].clone()
    y[1] = -1
    nan_row = n - 1
    y[nan_row] = V                      # out of range: NaN row instead of a device fault
    g = _cuda(d, device)
    got = _probes().cycle_derivatives(g['base'], g['C'], y.to(device), g['steps'].view(-1, 1),
                                      g['sq'].view(-1, 1), g['dots'], g['dir_sq'])
    torch.cuda.synchronize()
    yy = y.clone()
    yy[nan_row] = 0
    want = P.cycle_derivatives(d['base'], d['C'], yy, d['steps'], d['sq'], d['dots'], d['dir_sq'])
    masked = [i for i in range(n) if y[i] < 0]
    _check_probe(got, want, d['steps'], masked, [nan_row])


def test_cycle_derivatives_full_cycle_sampled(device):
    """The bench shape (one 2048-token sequence, a full cycle of 512, V = 4096), checked on a
    sample of 12 tokens spread over the sequence."""
    d = probe_inputs(2048, 512, 4096, sigma=0.005, seed=11)
    g = _cuda(d, device)
    got = _probes().cycle_derivatives(g['base'], g['C'], g['y'], g['steps'], g['sq'], g['dots'], g['dir_sq'])
    torch.cuda.synchronize()
    rows = np.linspace(0, 2047, 12).astype(int)
    want = P.cycle_derivatives(d['base'][rows], d['C'], d['y'][rows], d['steps'][rows], d['sq'][rows],
                               d['dots'][rows], d['dir_sq'])
    assert torch.isfinite(got).all()
    _check_probe(got[rows], want, d['steps'][rows])


def test_cycle_derivatives_unaligned_rows(device):
    """V = 1001 and rows at odd strides: the scalar-load path with a partial last chunk."""
    n, P_, V = 9, 10, 1001
    d = probe_inputs(n, 512, V, probes=P_, sigma=0.01, dirs='gaussian', seed=4)
    base = torch.empty(n, V + 3, device=device)[:, 1:V + 1]
    base.copy_(d['base'])
    C = torch.empty(P_, V + 1, device=device)[:, :V]
    C.copy_(d['C'])
    g = _cuda(d, device)
    got = _probes().cycle_derivatives(base, C, g['y'], g['steps'], g['sq'], g['dots'], g['dir_sq'])
    torch.cuda.synchronize()
    want = P.cycle_derivatives(d['base'], d['C'], d['y'], d['steps'], d['sq'], d['dots'], d['dir_sq'])
    _check_probe(got, want, d['steps'])


def test_row_derivatives_matches_oracle(device):
    n, P_, K, V = 33, 64, 21, 4096
    d = probe_inputs(n, 512, V, probes=P_, sigma=0.005, dirs='gaussian', seed=8)
    gen = torch.Generator().manual_seed(2)
    rows = torch.stack([torch.randperm(P_, generator=gen)[:K] for _ in range(n)])
    dots = d['dots'].gather(1, rows)
    dir_sq = d['dir_sq'][rows].contiguous()
    bad = rows.clone()
    bad[3, 5] = P_                          # an invalid row index: NaN in that slot only
    g = _cuda(d, device)
    got = _probes().row_derivatives(g['base'], g['C'], bad.to(device), g['y'], g['steps'], g['sq'],
                                    dots.to(device), dir_sq.to(device))
    torch.cuda.synchronize()
    want = P.row_derivatives(d['base'], d['C'], rows, d['y'], d['steps'], d['sq'], dots, dir_sq)
    got = got.cpu().double()
    assert torch.isnan(got[3, 5])
    got[3, 5] = float(want[3, 5])
    _check_probe(got, want, d['steps'])


@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
def test_coordinate_differences_matches_oracle(device, dtype):
    gen = torch.Generator().manual_seed(5)
    n, V, sigma = 23, 4096, 0.1
    raw = (torch.randn(n, V, generator=gen) * 8).to(dtype)
    raw[0, :6] = torch.tensor([80., -80., 30., 0., 15., -15.]).to(dtype)
    y = torch.randint(0, V, (n,), generator=gen)
    y[2] = -1
    y[4] = V
    got = _probes().coordinate_differences(raw.to(device), y.to(device), sigma)
    torch.cuda.synchronize()
    yy = y.clone()
    yy[4] = 0
    want = P.coordinate_differences(raw.double().numpy(), yy.numpy(), sigma)
    got = got.cpu().double().numpy()
    assert np.all(got[2] == 0)
    assert np.all(np.isnan(got[4]))
    keep = [i for i in range(n) if i not in (2, 4)]
    np.testing.assert_allclose(got[keep], want[keep], rtol=1e-4, atol=2e-6)


def test_coordinate_differences_reference_layout(device):
    """The reference's call: raw [b, t, V] bf16 (a slice of a padded head output), y [b, t]."""
    gen = torch.Generator().manual_seed(6)
    b, t, V = 2, 7, 4096
    padded = (torch.randn(b, t, V + 128, generator=gen) * 6).to(torch.bfloat16)
    raw = padded.to(device)[..., :V]
    y = torch.randint(-1, V, (b, t), generator=gen)
    got = _probes().coordinate_differences(raw, y.to(device), 0.1)
    torch.cuda.synchronize()
    assert got.shape == (b, t, V) and got.dtype == torch.float32
    want = P.coordinate_differences(padded[..., :V].double().reshape(-1, V).numpy(), y.reshape(-1).numpy(), 0.1)
    np.testing.assert_allclose(got.reshape(-1, V).cpu().double().numpy(), want, rtol=1e-4, atol=2e-6)


def _chain_case(site, m, P_, L, seed=0, W=512, H=2048, k=128, V=4096):
    """Chain inputs at the model's widths: bf16 block and head weights, routed units with their
    clean pre-activations W_fc[idx] norm(mid), moves of the size the Cut estimator takes."""
    g = torch.Generator().manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=g)
    nrm = lambda x: x * torch.rsqrt(x.square().mean(-1, keepdim=True) + 1.1920929e-07)
    e = rn(m, W) * 2
    x0 = nrm(e)
    mids = [rn(m, W) * 3 for _ in range(L)]
    w_fc = [(rn(H, W) * 3 ** 0.5 / W ** 0.5).bfloat16() for _ in range(L)]
    w_out_t = [(rn(H, W) / H ** 0.5).bfloat16() for _ in range(L)]
    idx = [torch.stack([torch.randperm(H, generator=g)[:k] for _ in range(m)]) for _ in range(L)]
    hs = [torch.einsum('mkd,md->mk', w_fc[b].float()[idx[b]], nrm(mids[b])) for b in range(L)]
    xL = rn(m, W) * 4
    weight = rn(V, W) * 3 / W ** 0.5
    y = torch.randint(0, V, (m,), generator=g)
    steps = 0.01 * (e if site < 0 else mids[site]).square().mean(-1, keepdim=True).sqrt()
    move = steps.unsqueeze(-1) * rn(m, P_, W)
    scale = steps.expand(-1, P_).contiguous()
    lam_r, lam_0 = 1 + 0.1 * rn(L), 0.1 + 0.05 * rn(L)
    return dict(move=move, scale=scale, e=e, x0=x0, mids=mids, xL=xL, idx=idx, hs=hs, lam_r=lam_r, lam_0=lam_0,
                w_fc=w_fc, w_out_t=w_out_t, weight_t=weight.T.bfloat16().contiguous(), base=xL @ weight.T,
                target_logit_w=weight[y.clamp(min=0)], y=y)


def _to(d, device):
    return {k: ([v.to(device) for v in x] if isinstance(x, list) else x.to(device)) for k, x in d.items()}


def _oracle_chain(site, d, rows, policy, own=None):
    sub = {k: ([v[rows] for v in x] if k in ('mids', 'idx', 'hs') else
               (x if k in ('lam_r', 'lam_0', 'w_fc', 'w_out_t', 'weight_t') else x[rows]))
           for k, x in d.items()}
    sub = {k: ([v.double().numpy() if v.is_floating_point() else v.numpy() for v in x] if isinstance(x, list)
               else (x.double().numpy() if x.is_floating_point() else x.numpy())) for k, x in sub.items()}
    return P.chain_chunk(site, **sub, own=own, policy=policy)


@pytest.mark.parametrize('site,m,P_,L', [(-1, 6, 40, 3), (1, 5, 37, 3), (0, 3, 516, 2)])
def test_chain_chunk_matches_oracle(device, site, m, P_, L):
    """chain_chunk against the oracle with the reference's bf16 cast points. A derivative here is
    (moved - clean) / step with bf16-rounded logit moves, so a product that lands on the other side
    of a bf16 rounding boundary moves it by ~1e-3 relative: the oracle's own float32 evaluation
    with the same casts (build32) drifts that far from its float64 one (build). The GPU is held to
    twice that envelope, max and mean."""
    d = _chain_case(site, m, P_, L, seed=m + P_)
    d['y'][1] = -1
    got = _probes().chain_chunk(site, **_to(d, device)).cpu().double().numpy()
    torch.cuda.synchronize()
    rows = np.arange(m)
    want = _oracle_chain(site, d, rows, 'build')
    env = np.abs(want - _oracle_chain(site, d, rows, 'build32'))
    assert np.all(got[1] == 0)
    ok = rows != 1
    err = np.abs(got[ok] - want[ok])
    scale = np.abs(want[ok]).max()
    print(f'chain site {site}: max |gpu - build| {err.max():.3e} (envelope {env[ok].max():.3e}), '
          f'mean {err.mean():.3e} (envelope {env[ok].mean():.3e}), max |want| {scale:.3e}')
    assert np.isfinite(got).all()
    assert err.max() <= 2 * env[ok].max() + 1e-4 * scale
    assert err.mean() <= 2 * env[ok].mean() + 1e-5 * scale


def _routed_own(m, L, K, seed, W=512, T=1024):
    """own = ('routed', ...) at the model's widths: per block input streams, fp32 c_q and c_proj
    weights, unit-RMS bf16 keys, bf16 values, top-K clean probabilities from a softmax over a wider
    key set and the held keys' share; positions and rotary tables over T."""
    g = torch.Generator().manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=g)
    heads = W // 64
    pos = torch.randint(0, T, (m,), generator=g)
    ang = torch.arange(T)[:, None].float() * (1.0 / 1024 ** torch.linspace(0, 1, 32))[None]
    inputs = [rn(m, W) * 3 for _ in range(L)]
    w_q = [rn(W, W) / W ** 0.5 for _ in range(L)]
    w_proj_t = [rn(W, W) / W ** 0.5 for _ in range(L)]
    keys, vals, probs, rests = [], [], [], []
    for _ in range(L):
        k_ = rn(m, heads, K, 64)
        keys.append((k_ * torch.rsqrt(k_.square().mean(-1, keepdim=True))).bfloat16())
        vals.append(rn(m, heads, K, 64).bfloat16())
        full = torch.softmax(rn(m, heads, K + 32) * 2, -1).sort(-1, descending=True).values
        probs.append(full[..., :K].contiguous())
        rests.append((1 - full[..., :K].sum(-1, keepdim=True)) * rn(m, heads, 64) * 0.5)
    return ('routed', pos, inputs, w_q, keys, vals, probs, rests, w_proj_t, (ang.cos(), ang.sin()))


def _own_to(own, device=None, rows=None):
    """own moved to a device, or sliced to `rows` and turned into float64 numpy for the oracle."""
    if device is not None:
        conv = lambda t: t.to(device)
    else:
        conv = lambda t: t.double().numpy() if t.is_floating_point() else t.numpy()
    sl = (lambda t: t[rows]) if rows is not None else (lambda t: t)
    _, pos, inputs, w_q, keys, vals, probs, rests, w_proj_t, (cos, sin) = own
    tok = lambda part: [conv(sl(t)) for t in part]   # per-token entries, sliced
    return ('routed', conv(sl(pos)), tok(inputs), [conv(t) for t in w_q], tok(keys), tok(vals), tok(probs),
            tok(rests), [conv(t) for t in w_proj_t], (conv(cos), conv(sin)))


@pytest.mark.parametrize('site,m,P_,L,K', [(-1, 5, 40, 3, 64), (1, 4, 37, 3, 20), (0, 3, 516, 2, 64)])
def test_chain_chunk_routed_matches_oracle(device, site, m, P_, L, K):
    """chain_chunk with own = ('routed', ...): each block the move enters first changes its own
    token's attention output through its own query along its top keys (train/val/run.py:284-304).
    The bar adds the own-query step's tf32 envelope (its float32 products on the reference's TF32
    inputs, see the step's own test) to the build / build32 one; the own-query term itself must
    move the result."""
    d = _chain_case(site, m, P_, L, seed=m + P_ + K)
    d['y'][1] = -1
    own = _routed_own(m, L, K, seed=K + m)
    got = _probes().chain_chunk(site, **_to(d, device), own=_own_to(own, device)).cpu().double().numpy()
    none = _probes().chain_chunk(site, **_to(d, device)).cpu().double().numpy()
    torch.cuda.synchronize()
    rows = np.arange(m)
    sub = _own_to(own, rows=rows)
    want = _oracle_chain(site, d, rows, 'build', own=sub)
    env = np.abs(want - _oracle_chain(site, d, rows, 'build32', own=sub))[rows != 1]
    etf = np.abs(want - _oracle_chain(site, d, rows, 'tf32', own=sub))[rows != 1]
    assert np.all(got[1] == 0)
    ok = rows != 1
    err = np.abs(got[ok] - want[ok])
    scale = np.abs(want[ok]).max()
    print(f'routed chain site {site} K {K}: max |gpu - build| {err.max():.3e} (envelopes {env.max():.3e}, '
          f'tf32 {etf.max():.3e}), mean {err.mean():.3e} (envelopes {env.mean():.3e}, tf32 {etf.mean():.3e}), '
          f'max |want| {scale:.3e}, own term {np.abs(got - none)[ok].max():.3e}')
    assert np.isfinite(got).all()
    assert err.max() <= 2 * max(env.max(), etf.max()) + 1e-4 * scale
    assert err.mean() <= 2 * env.mean() + 0.5 * etf.mean() + 1e-5 * scale
    assert np.abs(got - none)[ok].max() > 10 * (err.max() + 1e-6 * scale)


def test_chain_chunk_routed_bad_position_gives_nan(device):
    """A position outside the rotary tables gives NaN for that token's moves (the reference's
    index would fault on the device), the other tokens unchanged."""
    site, m, P_, L, K = -1, 3, 16, 2, 8
    d = _chain_case(site, m, P_, L, seed=3)
    own = _routed_own(m, L, K, seed=4)
    good = _probes().chain_chunk(site, **_to(d, device), own=_own_to(own, device)).cpu()
    own[1][2] = 5000
    bad = _probes().chain_chunk(site, **_to(d, device), own=_own_to(own, device)).cpu()
    assert torch.isnan(bad[2]).all()
    assert torch.equal(bad[:2], good[:2])


@pytest.mark.parametrize('m,P_,K,W', [(4, 70, 64, 512), (3, 300, 37, 512), (2, 5, 1, 512), (3, 40, 64, 256)])
def test_chain_query_step_matches_oracle(device, m, P_, K, W):
    """The own-query step alone (noise_chain_query, mix off): the change it adds to delta against
    query_change_routed with the reference's bf16 casts (build). The reference runs the step's
    three float32 products on TF32 inputs; the kernels run them as bf16 hi/lo triples (2^-16
    relative against TF32's 2^-11), so the GPU is held to twice the tf32 envelope |build - tf32|
    at its largest and to half of it on average."""
    own = _routed_own(m, 1, K, seed=m * P_ + K, W=W)
    g = torch.Generator().manual_seed(K)
    delta = torch.randn(m, P_, W, generator=g) * 0.05
    dev_delta = delta.reshape(m * P_, W).to(device)
    step = _probes()._routed_query(_own_to(own, device), m, P_, W, 1, dev_delta.device)
    step(0, dev_delta, None, 0, 1.0, 0.0)
    got = (dev_delta.cpu().double().reshape(m, P_, W) - delta.double()).numpy()
    torch.cuda.synchronize()
    sub = _own_to(own, rows=np.arange(m))
    args = (sub[2][0], delta.double().numpy(), sub[1], sub[3][0], sub[4][0], sub[5][0], sub[6][0], sub[7][0],
            sub[8][0], sub[9][0], sub[9][1], W)
    want = P.query_change_routed(*args, policy='build')
    env = np.abs(want - P.query_change_routed(*args, policy='tf32'))
    err = np.abs(got - want)
    scale = np.abs(want).max()
    print(f'query step m {m} P {P_} K {K} W {W}: max |gpu - build| {err.max():.3e} (tf32 envelope {env.max():.3e}), '
          f'mean {err.mean():.3e} (tf32 envelope {env.mean():.3e}), max |want| {scale:.3e}')
    assert err.max() <= 2 * env.max()
    assert err.mean() <= 0.5 * env.mean()


def _window_own(m, L, S, windows, seed, W=512, T=2048):
    """own = ('window', ...) at the model's widths: per block one key window of S positions
    (unit-RMS bf16 keys, bf16 values) shared by the chunk's tokens, at relative positions that
    cover the window's start (fewer than window + 1 keys), its inclusive bound and its end."""
    g = torch.Generator().manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=g)
    heads = W // 64
    ang = torch.arange(T)[:, None].float() * (1.0 / 1024 ** torch.linspace(0, 1, 32))[None]
    rels, keys, vals = [], [], []
    for b in range(L):
        w = windows[b]
        base = [0, 5, w - 1, w, w + 1, S - 1]
        rels.append(torch.tensor([max(0, min(S - 1, base[t % len(base)] + t // len(base))) for t in range(m)]))
        k_ = rn(heads, S, 64)
        keys.append((k_ * torch.rsqrt(k_.square().mean(-1, keepdim=True))).bfloat16())
        vals.append(rn(heads, S, 64).bfloat16())
    pos = rels[0] + (T - S)
    return ('window', pos, rels, [rn(m, W) * 3 for _ in range(L)], [rn(W, W) / W ** 0.5 for _ in range(L)], keys,
            vals, [rn(W, W) / W ** 0.5 for _ in range(L)], ang.cos(), ang.sin(), list(windows))


def _window_to(own, device=None):
    """own ('window', ...) moved to a device, or as float64 numpy for the oracle."""
    conv = (lambda t: t.to(device)) if device is not None else (
        lambda t: t.double().numpy() if t.is_floating_point() else t.numpy())
    _, pos, rels, inputs, w_q, keys, vals, w_proj_t, cos, sin, windows = own
    lst = lambda part: [conv(t) for t in part]
    return ('window', conv(pos), lst(rels), lst(inputs), lst(w_q), lst(keys), lst(vals), lst(w_proj_t), conv(cos),
            conv(sin), windows)


@pytest.mark.parametrize('m,P_,S,window,W', [(6, 70, 300, 128, 512), (4, 150, 1100, 1024, 512), (3, 5, 40, 0, 512),
                                            (3, 33, 50, 20, 256)])
def test_chain_query_window_step_matches_oracle(device, m, P_, S, window, W):
    """The key-window own-query step alone (noise_chain_query_window, mix off) against query_change
    with the reference's bf16 casts: windows of 129 and 1025 keys (17 blocks of 64), tokens at the
    window's start, bound and end. Bar as the routed step: twice the tf32 envelope at its largest,
    half of it on average. Window 0 (the token's own key only): a softmax over one key cannot
    change, so the step must add (float32 rounding of) nothing."""
    own = _window_own(m, 1, S, [window], seed=m * P_ + S, W=W)
    g = torch.Generator().manual_seed(S)
    delta = torch.randn(m, P_, W, generator=g) * 0.05
    dev_delta = delta.reshape(m * P_, W).to(device)
    step = _probes()._window_query(_window_to(own, device), m, P_, W, 1, dev_delta.device)
    step(0, dev_delta, None, 0, 1.0, 0.0)
    got = (dev_delta.cpu().double().reshape(m, P_, W) - delta.double()).numpy()
    torch.cuda.synchronize()
    o = _window_to(own)
    args = (o[3][0], delta.double().numpy(), o[1], o[2][0], o[4][0], o[5][0], o[6][0], o[7][0], o[8], o[9], window,
            W)
    want = P.query_change(*args, policy='build')
    if window == 0:
        print(f'window step m {m} P {P_} window 0: max |gpu| {np.abs(got).max():.3e}')
        assert np.abs(got).max() <= 1e-6
        return
    env = np.abs(want - P.query_change(*args, policy='tf32'))
    err = np.abs(got - want)
    scale = np.abs(want).max()
    print(f'window step m {m} P {P_} S {S} window {window}: max |gpu - build| {err.max():.3e} (tf32 envelope '
          f'{env.max():.3e}), mean {err.mean():.3e} (tf32 envelope {env.mean():.3e}), max |want| {scale:.3e}')
    assert np.isfinite(got).all()
    assert err.max() <= 2 * env.max()
    assert err.mean() <= 0.5 * env.mean()


@pytest.mark.parametrize('site,m,P_,L', [(-1, 5, 40, 3), (0, 4, 37, 2)])
def test_chain_chunk_window_matches_oracle(device, site, m, P_, L):
    """chain_chunk with own = ('window', ...) (train/val/run.py:332-335) against the oracle: the bar
    of the routed chain."""
    d = _chain_case(site, m, P_, L, seed=m + P_ + 7)
    d['y'][1] = -1
    own = _window_own(m, L, 300, [128, 256, 100][:L], seed=m + 17)
    got = _probes().chain_chunk(site, **_to(d, device), own=_window_to(own, device)).cpu().double().numpy()
    none = _probes().chain_chunk(site, **_to(d, device)).cpu().double().numpy()
    torch.cuda.synchronize()
    rows = np.arange(m)
    o = _window_to(own)
    want = _oracle_chain(site, d, rows, 'build', own=o)
    env = np.abs(want - _oracle_chain(site, d, rows, 'build32', own=o))[rows != 1]
    etf = np.abs(want - _oracle_chain(site, d, rows, 'tf32', own=o))[rows != 1]
    assert np.all(got[1] == 0)
    ok = rows != 1
    err = np.abs(got[ok] - want[ok])
    scale = np.abs(want[ok]).max()
    print(f'window chain site {site}: max |gpu - build| {err.max():.3e} (envelopes {env.max():.3e}, '
          f'tf32 {etf.max():.3e}), mean {err.mean():.3e} (envelopes {env.mean():.3e}, tf32 {etf.mean():.3e}), '
          f'max |want| {scale:.3e}, own term {np.abs(got - none)[ok].max():.3e}')
    assert np.isfinite(got).all()
    assert err.max() <= 2 * max(env.max(), etf.max()) + 1e-4 * scale
    assert err.mean() <= 2 * env.mean() + 0.5 * etf.mean() + 1e-5 * scale
    assert np.abs(got - none)[ok].max() > 10 * (err.max() + 1e-6 * scale)


def test_chain_query_window_without_keys_gives_nan(device):
    """A token whose window holds no key (rel < 0) gets NaN; the others are unchanged."""
    m, P_ = 3, 8
    own = _window_own(m, 1, 64, [16], seed=5)
    g = torch.Generator().manual_seed(1)
    delta = (torch.randn(m * P_, 512, generator=g) * 0.05).to(device)
    run = lambda o: (lambda dd: (_probes()._window_query(_window_to(o, device), m, P_, 512, 1, dd.device)(
        0, dd, None, 0, 1.0, 0.0), dd.cpu())[1])(delta.clone())
    good = run(own)
    own[2][0][2] = -1
    bad = run(own).reshape(m, P_, 512)
    assert torch.isnan(bad[2]).all()
    assert torch.equal(bad[:2], good.reshape(m, P_, 512)[:2])
