"""Soft-capped log-sum-exp probes of the readout head, on the HIP kernels of libnoise_amd.

Drop-in twins of four functions of the reference trainer, with the same arguments, shapes and
float32 results (device tensors in, device tensors out, asynchronous on the current stream):

* `coordinate_differences(raw, y, sigma)`  -- train/val/run.py:100-111 (speedrun/run.py:57-68)
* `cycle_derivatives(base, C, y, steps, sq, dots, dir_sq)`       -- train/val/run.py:154-167
* `row_derivatives(base, C, rows, y, steps, sq, dots, dir_sq)`   -- train/val/run.py:170-183
* `chain_chunk(site, move, scale, e, x0, mids, xL, idx, hs, lam_r, lam_0, w_fc, w_out_t,
  weight_t, base, target_logit_w, y, own=None)`                   -- train/val/run.py:307-351,
  with every attention held (own = None), with the routed own-query moves (own = ('routed', ...),
  query_change_routed, train/val/run.py:284-304) or over whole key windows (own = ('window', ...),
  query_change, train/val/run.py:256-281)

The reference reads the stream width from a module constant (WIDTH = 512); here it is the keyword
`width`. A target y < 0 masks its token (zeros, as the reference's `* (y >= 0)`); a target >= V
gives NaN for the token instead of the reference's device-side gather fault.
"""
import ctypes as C

import torch

from . import _lib
from ._lib import ChainBlock, ChainHead, ChainQuery, ChainQueryWindow, Probe

WIDTH = 512


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _need(cond, msg):
    if not cond:
        raise ValueError(msg)


def _f32_rows(t, name, cols=None):
    _need(t.is_cuda, f'{name}: libnoise_amd kernels take device tensors')
    _need(t.dtype == torch.float32, f'{name}: expected float32, got {t.dtype}')
    _need(t.dim() == 2, f'{name}: expected a 2-D tensor, got shape {tuple(t.shape)}')
    if cols is not None:
        _need(t.shape[1] == cols, f'{name}: expected {cols} columns, got {t.shape[1]}')
    return t if t.stride(1) == 1 else t.contiguous()


def _vec(t, n, name):
    _need(t.is_cuda and t.dtype == torch.float32, f'{name}: expected a float32 device tensor')
    _need(t.numel() == n, f'{name}: expected {n} values, got shape {tuple(t.shape)}')
    return t.reshape(n).contiguous()


def _targets(y, n):
    _need(y.is_cuda and not y.is_floating_point(), 'y: expected an integer device tensor')
    _need(y.numel() == n, f'y: expected {n} targets, got shape {tuple(y.shape)}')
    return y.reshape(n).to(torch.int64).contiguous()


def coordinate_differences(raw, y, sigma):
    """raw [..., V] logits (float32 or bfloat16), y [...] targets -> float32 [..., V]:
    d CE / d raw_v by central differences of step sigma, in closed form."""
    _need(raw.is_cuda, 'raw: libnoise_amd kernels take device tensors')
    _need(raw.dtype in (torch.float32, torch.bfloat16), f'raw: expected float32 or bfloat16, got {raw.dtype}')
    _need(tuple(y.shape) == tuple(raw.shape[:-1]), f'y {tuple(y.shape)} does not match raw {tuple(raw.shape)}')
    V = raw.shape[-1]
    lead = raw.shape[:-1]
    flat = raw.reshape(-1, V) if raw.dim() != 2 else raw
    if flat.stride(-1) != 1:
        flat = flat.contiguous()
    n = flat.shape[0]
    yy = _targets(y, n)
    out = torch.empty(n, V, dtype=torch.float32, device=raw.device)
    if n:
        _lib.call('noise_coordinate_differences', flat.data_ptr(), int(flat.dtype == torch.bfloat16),
                  flat.stride(0), yy.data_ptr(), n, V, float(sigma), out.data_ptr(), out.stride(0), _stream())
    return out.view(*lead, V)


def _probe(base, C_, y, steps, sq, dots, dir_sq, width, rows=None):
    base = _f32_rows(base, 'base')
    n, V = base.shape
    C_ = _f32_rows(C_, 'C', V)
    P = C_.shape[0]
    K = P if rows is None else rows.shape[1]
    dots = _f32_rows(dots, 'dots', K)
    _need(dots.shape[0] == n, f'dots: expected {n} rows, got {dots.shape[0]}')
    a = Probe()
    a.base, a.ld_base = base.data_ptr(), base.stride(0)
    a.C, a.ld_C = C_.data_ptr(), C_.stride(0)
    yy = _targets(y, n)
    st = _vec(steps, n, 'steps')
    sqv = _vec(sq, n, 'sq')
    a.y, a.steps, a.sq = yy.data_ptr(), st.data_ptr(), sqv.data_ptr()
    a.dots, a.ld_dots = dots.data_ptr(), dots.stride(0)
    keep = [base, C_, yy, st, sqv, dots]
    if rows is None:
        dsq = _vec(dir_sq, P, 'dir_sq')
        a.dir_sq, a.ld_dir_sq = dsq.data_ptr(), 0
        keep.append(dsq)
    else:
        _need(rows.is_cuda and not rows.is_floating_point() and rows.dim() == 2 and rows.shape[0] == n,
              f'rows: expected an integer device tensor [{n}, K], got {tuple(rows.shape)}')
        rr = rows.to(torch.int64).contiguous()
        dsq = _f32_rows(dir_sq, 'dir_sq', K)
        _need(dsq.shape[0] == n, f'dir_sq: expected {n} rows, got {dsq.shape[0]}')
        a.rows, a.ld_rows = rr.data_ptr(), rr.stride(0)
        a.dir_sq, a.ld_dir_sq = dsq.data_ptr(), dsq.stride(0)
        keep += [rr, dsq]
    a.n, a.P, a.K, a.V, a.width = n, P, K, V, int(width)
    clean = torch.empty(n, dtype=torch.float32, device=base.device)
    out = torch.empty(n, K, dtype=torch.float32, device=base.device)
    a.clean_sum, a.out, a.ld_out = clean.data_ptr(), out.data_ptr(), out.stride(0)
    if n:
        _lib.call('noise_row_derivatives' if rows is not None else 'noise_cycle_derivatives', C.byref(a), _stream())
    # `keep` holds the converted inputs until the launches are queued; torch's allocator reuses their
    # memory only for later work on this same stream, which runs after these kernels.
    return out


def cycle_derivatives(base, C, y, steps, sq, dots, dir_sq, width=WIDTH):
    """base [n, V] = W x; C [P, V] (row j = W D_j); y [n]; steps, sq [n, 1] or [n]; dots [n, P];
    dir_sq [P] -> float32 [n, P]: (loss(x + s D_j) - loss(x)) / s for every token and direction."""
    return _probe(base, C, y, steps, sq, dots, dir_sq, width)


def row_derivatives(base, C, rows, y, steps, sq, dots, dir_sq, width=WIDTH):
    """rows [n, K] indices into C's rows; dots, dir_sq [n, K] -> float32 [n, K]."""
    return _probe(base, C, y, steps, sq, dots, dir_sq, width, rows=rows)


def _dev_f32(t, shape, name):
    _need(t.is_cuda, f'{name}: libnoise_amd kernels take device tensors')
    _need(tuple(t.shape) == tuple(shape), f'{name}: expected shape {tuple(shape)}, got {tuple(t.shape)}')
    return t.float().contiguous()


def _dev_bf16(t, shape, name):
    _need(t.is_cuda, f'{name}: libnoise_amd kernels take device tensors')
    _need(tuple(t.shape) == tuple(shape), f'{name}: expected shape {tuple(shape)}, got {tuple(t.shape)}')
    t = t.to(torch.bfloat16).contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()  # the kernels read 16-byte pieces


def chain_chunk(site, move, scale, e, x0, mids, xL, idx, hs, lam_r, lam_0, w_fc, w_out_t, weight_t, base,
                target_logit_w, y, own=None):
    """Forward differences of each token's loss along every move of one site, attention held, MLPs
    restricted to each token's routed units (train/val/run.py:307-351). site: -1 for the raw
    embedding, else the block whose mid stream moves; move [m, P, W]; scale [m, P]; e, x0, xL
    [m, W]; mids, idx, hs per block ([m, W], [m, k], [m, k]); w_fc, w_out_t per block [H, W];
    weight_t [W, V]; base [m, V]; target_logit_w [m, W]; y [m]. own: None, or ('routed', pos,
    inputs, w_q, top_keys, top_values, top_p, rest, w_proj_t, (cos, sin)) as the reference's
    strong_keys builds it: pos [m]; per block inputs [m, W], w_q [W, W], top_keys and top_values
    [m, heads, K, 64], top_p [m, heads, K], rest [m, heads, 64], w_proj_t [W, W]; cos, sin
    [T, 32]; or ('window', pos, rels, inputs, w_q, keys, values, w_proj_t, cos, sin, windows) as
    own_query_window builds it: per block rels [m], keys and values [heads, S, 64], windows (int).
    Returns float32 [m, P]."""
    _need(own is None or own[0] in ('routed', 'window'), "own: expected None, ('routed', ...) or ('window', ...)")
    m, P, W = move.shape
    L = len(mids)
    V = weight_t.shape[1]
    H, k = w_fc[0].shape[0], idx[0].shape[1]
    dev = move.device
    _need(-1 <= site < L, f'site {site} outside [-1, {L})')
    mv = _dev_f32(move, (m, P, W), 'move').view(m * P, W)
    sc = _dev_f32(scale, (m, P), 'scale')
    e, x0, xL = (_dev_f32(t, (m, W), n) for t, n in ((e, 'e'), (x0, 'x0'), (xL, 'xL')))
    lr = [float(v) for v in torch.as_tensor(lam_r).reshape(-1).tolist()]
    l0 = [float(v) for v in torch.as_tensor(lam_0).reshape(-1).tolist()]
    _need(len(lr) >= L and len(l0) >= L, 'lam_r / lam_0: one value per block')
    weight = _dev_bf16(weight_t, (W, V), 'weight_t').t().contiguous()
    bs = _dev_f32(base, (m, V), 'base')
    tw = _dev_f32(target_logit_w, (m, W), 'target_logit_w')
    yy = _targets(y, m)
    out = torch.empty(m, P, dtype=torch.float32, device=dev)
    if m == 0:
        return out
    stream = _stream()
    if site < 0:
        dx0 = torch.empty(m * P, W, dtype=torch.float32, device=dev)
        delta = torch.empty_like(dx0)
        _lib.call('noise_chain_start', e.data_ptr(), x0.data_ptr(), mv.data_ptr(), m, P, W, lr[0] + l0[0],
                  dx0.data_ptr(), delta.data_ptr(), stream)
        first = 0
    else:
        dx0, delta, first = None, mv.clone(), site
    dz = torch.empty(m * P, W, dtype=torch.bfloat16, device=dev)
    wf = torch.empty(m, k, W, dtype=torch.bfloat16, device=dev)
    wo = torch.empty(m, W, k, dtype=torch.bfloat16, device=dev)
    g = torch.empty(m * P, k, dtype=torch.bfloat16, device=dev)
    query = None if own is None else (_routed_query if own[0] == 'routed' else _window_query)(own, m, P, W, L, dev)
    for b in range(first, L):
        mix = int(b > first)
        if query is not None and (site < 0 or b > first):
            # the move is at the block's input: its own query moves too (the step mixes first)
            query(b, delta, dx0, mix, lr[b], l0[b])
            mix = 0
        mid = _dev_f32(mids[b], (m, W), f'mids[{b}]')
        ib = idx[b].to(device=dev, dtype=torch.int64).contiguous()
        hb = _dev_f32(hs[b], (m, k), f'hs[{b}]')
        wfc = _dev_bf16(w_fc[b], (H, W), f'w_fc[{b}]')
        wot = _dev_bf16(w_out_t[b], (H, W), f'w_out_t[{b}]')
        _need(tuple(ib.shape) == (m, k), f'idx[{b}]: expected shape {(m, k)}, got {tuple(ib.shape)}')
        a = ChainBlock(delta=delta.data_ptr(), dx0=dx0.data_ptr() if dx0 is not None else None,
                       mix=mix, lam_r=lr[b], lam_0=l0[b], mid=mid.data_ptr(), idx=ib.data_ptr(),
                       ld_idx=k, hs=hb.data_ptr(), ld_hs=k, w_fc=wfc.data_ptr(), w_out_t=wot.data_ptr(),
                       m=m, P=P, W=W, k=k, H=H, dz=dz.data_ptr(), wf=wf.data_ptr(), wo=wo.data_ptr(),
                       g=g.data_ptr())
        _lib.call('noise_chain_block', C.byref(a), stream)
    dbf = torch.empty(m * P, W, dtype=torch.bfloat16, device=dev)
    inv = torch.empty(m * P, dtype=torch.float32, device=dev)
    zy = torch.empty_like(inv)
    clean = torch.empty(2 * m, dtype=torch.float32, device=dev)
    h = ChainHead(delta=delta.data_ptr(), xL=xL.data_ptr(), base=bs.data_ptr(), ld_base=V, weight=weight.data_ptr(),
                  target_w=tw.data_ptr(), y=yy.data_ptr(), scale=sc.data_ptr(), ld_scale=P, m=m, P=P, W=W, V=V,
                  out=out.data_ptr(), ld_out=P, dbf=dbf.data_ptr(), inv=inv.data_ptr(), zy=zy.data_ptr(),
                  clean=clean.data_ptr())
    _lib.call('noise_chain_head', C.byref(h), stream)
    return out


def _query_workspaces(m, P, W, dev):
    return (torch.empty(m * P + m, 3 * W, dtype=torch.bfloat16, device=dev),
            torch.empty(m * P + m, W, dtype=torch.float32, device=dev),
            torch.empty(W, 3 * W, dtype=torch.bfloat16, device=dev),
            torch.empty(W, 3 * W, dtype=torch.bfloat16, device=dev))


def _rotary(pos, cos, sin, m):
    _need(pos.is_cuda and not pos.is_floating_point() and pos.numel() == m, f'own pos: expected {m} device integers')
    _need(cos.dim() == 2 and cos.shape[1] == 32, f'own cos: expected [T, 32], got {tuple(cos.shape)}')
    T = cos.shape[0]
    return (pos.reshape(m).to(torch.int64).contiguous(), _dev_f32(cos, (T, 32), 'own cos'),
            _dev_f32(sin, (T, 32), 'own sin'), T)


def _window_query(own, m, P, W, L, dev):
    """Checks own = ('window', ...) and returns step(b, delta, dx0, mix, lam_r, lam_0), which runs
    the block's own-query step over each token's key window (noise_chain_query_window)."""
    _need(len(own) == 11, "own: expected ('window', pos, rels, inputs, w_q, keys, values, w_proj_t, cos, sin, "
                          'windows)')
    _, pos, rels, inputs, w_q, keys, values, w_proj_t, cos, sin, windows = own
    for name, v in (('rels', rels), ('inputs', inputs), ('w_q', w_q), ('keys', keys), ('values', values),
                    ('w_proj_t', w_proj_t), ('windows', windows)):
        _need(len(v) >= L, f'own {name}: one entry per block')
    _need(W % 64 == 0, f'own: width {W} is not a whole number of 64-wide heads')
    heads = W // 64
    ps, ct, st, T = _rotary(pos, cos, sin, m)
    a3, dr, wq3, wp3 = _query_workspaces(m, P, W, dev)

    def step(b, delta, dx0, mix, lam_r, lam_0):
        _need(keys[b].dim() == 3 and keys[b].shape[0] == heads and keys[b].shape[2] == 64,
              f'own keys[{b}]: expected [{heads}, S, 64], got {tuple(keys[b].shape)}')
        S = keys[b].shape[1]
        rb = rels[b]
        _need(rb.is_cuda and not rb.is_floating_point() and rb.numel() == m, f'own rels[{b}]: expected {m} device integers')
        rr = rb.reshape(m).to(torch.int64).contiguous()
        x = _dev_f32(inputs[b], (m, W), f'own inputs[{b}]')
        wq = _dev_f32(w_q[b], (W, W), f'own w_q[{b}]')
        kk = _dev_bf16(keys[b], (heads, S, 64), f'own keys[{b}]')
        vv = _dev_bf16(values[b], (heads, S, 64), f'own values[{b}]')
        wp = _dev_f32(w_proj_t[b], (W, W), f'own w_proj_t[{b}]')
        a = ChainQueryWindow(delta=delta.data_ptr(), dx0=dx0.data_ptr() if dx0 is not None else None, mix=mix,
                             lam_r=lam_r, lam_0=lam_0, x=x.data_ptr(), pos=ps.data_ptr(), rel=rr.data_ptr(),
                             w_q=wq.data_ptr(), keys=kk.data_ptr(), values=vv.data_ptr(), w_proj_t=wp.data_ptr(),
                             cos_t=ct.data_ptr(), sin_t=st.data_ptr(), T=T, m=m, P=P, W=W, heads=heads, S=S,
                             window=int(windows[b]), a3=a3.data_ptr(), dr=dr.data_ptr(), wq3=wq3.data_ptr(),
                             wp3=wp3.data_ptr())
        _lib.call('noise_chain_query_window', C.byref(a), _stream())
    return step


def _routed_query(own, m, P, W, L, dev):
    """Checks own = ('routed', ...) and returns step(b, delta, dx0, mix, lam_r, lam_0), which runs
    the block's own-query step (noise_chain_query) in place on delta."""
    _need(len(own) == 10, "own: expected ('routed', pos, inputs, w_q, top_keys, top_values, top_p, rest, "
                          'w_proj_t, (cos, sin))')
    _, pos, inputs, w_q, top_keys, top_values, top_p, rest, w_proj_t, cos_sin = own
    for name, v in (('inputs', inputs), ('w_q', w_q), ('top_keys', top_keys), ('top_values', top_values),
                    ('top_p', top_p), ('rest', rest), ('w_proj_t', w_proj_t)):
        _need(len(v) >= L, f'own {name}: one entry per block')
    _need(W % 64 == 0, f'own: width {W} is not a whole number of 64-wide heads')
    heads = W // 64
    _need(top_keys[0].dim() == 4 and tuple(top_keys[0].shape[:2]) == (m, heads) and top_keys[0].shape[3] == 64,
          f'own top_keys: expected [{m}, {heads}, K, 64], got {tuple(top_keys[0].shape)}')
    K = top_keys[0].shape[2]
    ps, ct, st, T = _rotary(pos, cos_sin[0], cos_sin[1], m)
    a3, dr, wq3, wp3 = _query_workspaces(m, P, W, dev)

    def step(b, delta, dx0, mix, lam_r, lam_0):
        x = _dev_f32(inputs[b], (m, W), f'own inputs[{b}]')
        wq = _dev_f32(w_q[b], (W, W), f'own w_q[{b}]')
        kk = _dev_bf16(top_keys[b], (m, heads, K, 64), f'own top_keys[{b}]')
        vv = _dev_bf16(top_values[b], (m, heads, K, 64), f'own top_values[{b}]')
        pp = _dev_f32(top_p[b], (m, heads, K), f'own top_p[{b}]')
        rr = _dev_f32(rest[b], (m, heads, 64), f'own rest[{b}]')
        wp = _dev_f32(w_proj_t[b], (W, W), f'own w_proj_t[{b}]')
        a = ChainQuery(delta=delta.data_ptr(), dx0=dx0.data_ptr() if dx0 is not None else None, mix=mix,
                       lam_r=lam_r, lam_0=lam_0, x=x.data_ptr(), pos=ps.data_ptr(), w_q=wq.data_ptr(),
                       top_keys=kk.data_ptr(), top_values=vv.data_ptr(), top_p=pp.data_ptr(), rest=rr.data_ptr(),
                       w_proj_t=wp.data_ptr(), cos_t=ct.data_ptr(), sin_t=st.data_ptr(), T=T, m=m, P=P, W=W,
                       heads=heads, K=K, a3=a3.data_ptr(), dr=dr.data_ptr(), wq3=wq3.data_ptr(),
                       wp3=wp3.data_ptr())
        _lib.call('noise_chain_query', C.byref(a), _stream())
    return step
