"""CPU oracle of the soft-capped log-sum-exp probe functions -- TEST INFRASTRUCTURE ONLY.

Only tests/ and bench.py's `cpu_baseline` leg may import this module, and only as the checker.
The shipped path (noise_amd/probes.py over libnoise_amd) never calls it.

Restatements in numpy float64 (float32 when asked) of six functions of the reference trainer:

* `coordinate_differences` -- train/val/run.py:100-111 (train/speedrun/run.py:57-68): central
  differences of each token's soft-capped cross-entropy along each of its own logits, in the
  closed form log1p(w_v expm1(cap(raw_v +- sigma) - cap(raw_v))) with the target correction;
* `cycle_derivatives`      -- train/val/run.py:154-167 (train/speedrun/run.py:90-103): forward
  differences of each token's readout loss along every direction of a cycle, the moved stream's
  RMS norm evaluated exactly from |x|^2, x.D_j and |D_j|^2;
* `row_derivatives`        -- train/val/run.py:170-183: the same along per-token rows of the
  direction set;
* `query_change_routed`    -- train/val/run.py:284-304: a token's attention output change when its
  own query moves and only its top keys' logits move;
* `query_change`           -- train/val/run.py:256-281: the same over every key of its window;
* `chain_chunk`            -- train/val/run.py:307-351 with own = None, ('routed', ...) or
  ('window', ...): moves of one site carried through the later blocks' routed MLPs (and
  own-query attention changes) to the head's loss.

cap(v) = 15 tanh(v / 15); norm(x) = x rsqrt(|x|^2 / width + eps), eps = float32 machine epsilon.

Pinning (tests/test_probes_oracle.py): each function against a brute-force evaluation that never
uses its closed form -- the moved streams / logits / queries are built explicitly and pushed
through torch.nn.functional.cross_entropy or an explicit softmax in float64 (one forward per
probe), and row_derivatives against cycle_derivatives gathered at the rows. The 'tf32' policy's
rounding is pinned against hand-computed values.
"""
import numpy as np

CAP = 15.0
EPS32 = float(np.finfo(np.float32).eps)


def cap(v):
    return CAP * np.tanh(v / CAP)


def _logsumexp(z, axis=-1):
    m = np.max(z, axis=axis, keepdims=True)
    return (m + np.log(np.sum(np.exp(z - m), axis=axis, keepdims=True))).squeeze(axis)


def coordinate_differences(raw, y, sigma, dtype=np.float64):
    """raw (n, V) logits before the cap, y (n,) targets (negative: masked), sigma the logit step.
    Returns (n, V): d loss / d raw_v by central differences (train/val/run.py:100-111)."""
    raw = np.asarray(raw, dtype)
    y = np.asarray(y)
    s = dtype(sigma)
    z, up, down = cap(raw), cap(raw + s), cap(raw - s)
    weight = np.exp(z - _logsumexp(z)[:, None])
    change = np.log1p(weight * np.expm1(up - z)) - np.log1p(weight * np.expm1(down - z))
    rows = np.arange(raw.shape[0])
    t = np.clip(y, 0, None)
    change[rows, t] -= (up - down)[rows, t]
    return change / (2 * s) * (y >= 0)[:, None]


def _head_terms(base, y, sq, width, dtype):
    t = np.clip(np.asarray(y), 0, None)
    base_y = base[np.arange(base.shape[0]), t]
    inv0 = 1.0 / np.sqrt(sq / dtype(width) + dtype(EPS32))
    clean = _logsumexp(cap(base * inv0[:, None])) - cap(base_y * inv0)
    return t, base_y, clean


def cycle_derivatives(base, C, y, steps, sq, dots, dir_sq, width=512, dtype=np.float64, chunk=32):
    """base (n, V) = W x of the clean streams; C (P, V) row j = W D_j; y (n,); steps (n,) step per
    token; sq (n,) |x|^2; dots (n, P) x . D_j; dir_sq (P,) |D_j|^2. Returns (n, P)
    (train/val/run.py:154-167)."""
    base, C = np.asarray(base, dtype), np.asarray(C, dtype)
    steps, sq = np.asarray(steps, dtype).reshape(-1), np.asarray(sq, dtype).reshape(-1)
    dots, dir_sq = np.asarray(dots, dtype), np.asarray(dir_sq, dtype).reshape(-1)
    y = np.asarray(y)
    t, base_y, clean = _head_terms(base, y, sq, width, dtype)
    out = np.empty((base.shape[0], C.shape[0]), dtype)
    for i0 in range(0, base.shape[0], chunk):
        sl = slice(i0, i0 + chunk)
        s = steps[sl, None]
        inv = 1.0 / np.sqrt((sq[sl, None] + 2 * s * dots[sl] + s * s * dir_sq[None]) / dtype(width) + dtype(EPS32))
        z = (base[sl, None, :] + s[..., None] * C[None]) * inv[..., None]
        dirs_y = C[:, t[sl]].T                                       # (m, P)
        moved = _logsumexp(cap(z)) - cap((base_y[sl, None] + s * dirs_y) * inv)
        out[sl] = (moved - clean[sl, None]) / s * (y[sl] >= 0)[:, None]
    return out


def row_derivatives(base, C, rows, y, steps, sq, dots, dir_sq, width=512, dtype=np.float64):
    """rows (n, K) indices into C's rows; dots, dir_sq (n, K). Returns (n, K)
    (train/val/run.py:170-183)."""
    base, C = np.asarray(base, dtype), np.asarray(C, dtype)
    rows = np.asarray(rows)
    steps, sq = np.asarray(steps, dtype).reshape(-1), np.asarray(sq, dtype).reshape(-1)
    dots, dir_sq = np.asarray(dots, dtype), np.asarray(dir_sq, dtype)
    y = np.asarray(y)
    t, base_y, clean = _head_terms(base, y, sq, width, dtype)
    dirs = C[rows]                                                   # (n, K, V)
    dirs_y = dirs[np.arange(base.shape[0]), :, t]                    # (n, K)
    s = steps[:, None]
    inv = 1.0 / np.sqrt((sq[:, None] + 2 * s * dots + s * s * dir_sq) / dtype(width) + dtype(EPS32))
    z = (base[:, None, :] + s[..., None] * dirs) * inv[..., None]
    moved = _logsumexp(cap(z)) - cap((base_y[:, None] + s * dirs_y) * inv)
    return (moved - clean[:, None]) / s * (y >= 0)[:, None]


# ---------------------------------------------------------------- chain_chunk (attention held)

def _bf16(x):
    """Round float64/32 numpy values to bfloat16 (round to nearest even), returned as float64."""
    import torch
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).bfloat16().double().numpy()


def _tf32(x):
    """Round to TF32 (10 explicit mantissa bits, round to nearest, ties away from zero), returned as
    float64: the input rounding of the reference's float32 products under
    torch.set_float32_matmul_precision('high') (train/val/run.py:1286)."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return (((b + 0x1000) & 0xFFFFE000).astype(np.uint32)).view(np.float32).astype(np.float64)


def _rms(x, width):
    return x / np.sqrt(np.sum(x * x, -1, keepdims=True) / width + EPS32)


def norm_difference(x, delta, width=512):
    """norm(x + delta) - norm(x) in the closed form of train/val/run.py:246-253: x (m, W),
    delta (m, P, W)."""
    sq = np.sum(x * x, -1)[:, None]
    dots = np.einsum('md,mpd->mp', x, delta)
    inv0 = 1.0 / np.sqrt(sq / width + EPS32)
    inv = 1.0 / np.sqrt((sq + 2 * dots + np.sum(delta * delta, -1)) / width + EPS32)
    return delta * inv[..., None] + x[:, None, :] * (inv - inv0)[..., None]


def _query_moves(x, delta, pos, w_q, cos, sin, heads, d, width, tf):
    """Clean rotated query r0 (m, 1, h, d) and its change dr (m, P, h, d), inv0, inv (qk-norm)."""
    m, P, _ = delta.shape
    c, s_ = cos[pos][:, None, None, :], sin[pos][:, None, None, :]
    rot = lambda u: np.concatenate([u[..., :d // 2] * c + u[..., d // 2:] * s_,
                                    u[..., :d // 2] * -s_ + u[..., d // 2:] * c], -1)
    r0 = rot((tf(_rms(x, width)) @ tf(w_q).T).reshape(m, 1, heads, d))
    dr = rot((tf(norm_difference(x, delta, width)) @ tf(w_q).T).reshape(m, P, heads, d))
    sq = np.sum(r0 * r0, -1, keepdims=True)
    inv0 = 1.0 / np.sqrt(sq / d + EPS32)
    inv = 1.0 / np.sqrt((sq + 2 * np.sum(r0 * dr, -1, keepdims=True) + np.sum(dr * dr, -1, keepdims=True)) / d + EPS32)
    return r0, dr, inv0, inv


def query_change(x, delta, pos, rel, w_q, keys, values, w_proj_t, cos, sin, window, width=512, policy='fp64'):
    """train/val/run.py:256-281: the change of each token's attention output, through the output
    projection, when only its own query moves, over every key of its window. keys, values
    (h, S, d) clean (keys rotated and normed) shared by the chunk's tokens; rel (m,) the tokens'
    positions within those S; a key t is allowed when 0 <= rel - t <= window. Policies as
    query_change_routed."""
    dt = np.float32 if policy == 'build32' else np.float64
    rb = (lambda v: _bf16(v).astype(dt)) if policy in ('build', 'build32', 'tf32') else (lambda v: v)
    tf = _tf32 if policy == 'tf32' else (lambda v: v)
    f = lambda v: np.asarray(v, dt)
    x, delta, w_q, keys, vals, w_proj_t, cos, sin = map(f, (x, delta, w_q, keys, values, w_proj_t, cos, sin))
    pos, rel = np.asarray(pos), np.asarray(rel)
    m, P, _ = delta.shape
    heads, S, d = keys.shape
    r0, dr, inv0, inv = _query_moves(x, delta, pos, w_q, cos, sin, heads, d, width, tf)
    q0, dq = r0 * inv0, dr * inv + r0 * (inv - inv0)
    lag = rel[:, None] - np.arange(S)[None]
    allowed = ((lag >= 0) & (lag <= window))[:, None, None, :]               # (m, 1, 1, S)
    scores = rb(np.einsum('mphd,htd->mpht', rb(q0), keys)) * d ** -0.5
    scores = np.where(allowed, scores, -np.inf)
    mx = np.max(scores, -1, keepdims=True)
    e = np.exp(scores - mx)
    p0 = e / np.sum(e, -1, keepdims=True)                                      # (m, 1, h, S)
    ds = rb(np.einsum('mphd,htd->mpht', rb(dq), keys)) * d ** -0.5
    dlse = np.log1p(np.sum(p0 * np.expm1(ds), -1, keepdims=True))
    dout = rb(np.einsum('mpht,htd->mphd', rb(p0 * np.expm1(ds - dlse)), vals))
    return tf(dout.reshape(m, P, heads * d)) @ tf(w_proj_t)


def query_change_routed(x, delta, pos, w_q, top_keys, top_values, top_p, rest, w_proj_t, cos, sin, width=512,
                        policy='fp64'):
    """train/val/run.py:282-304: the change of each token's attention output, through the output
    projection, when only its own query moves and only the logits of its top keys per head move.
    x (m, W) block input; delta (m, P, W); top_keys, top_values (m, h, K, d); top_p (m, h, K);
    rest (m, h, d); w_q (W, W); w_proj_t (W, W) = c_proj.weight^T; cos, sin (T, d / 2).
    'build' rounds where the reference casts to bf16 (dq, both einsum products, the weights);
    'tf32' also rounds the inputs of the three float32 products to TF32, as the reference's
    hardware does under its matmul precision setting (the envelope of its own arithmetic)."""
    dt = np.float32 if policy == 'build32' else np.float64
    rb = (lambda v: _bf16(v).astype(dt)) if policy in ('build', 'build32', 'tf32') else (lambda v: v)
    tf = _tf32 if policy == 'tf32' else (lambda v: v)
    f = lambda v: np.asarray(v, dt)
    x, delta, w_q, keys, vals, tp, rest, w_proj_t = map(f, (x, delta, w_q, top_keys, top_values, top_p, rest,
                                                           w_proj_t))
    cos, sin = f(cos), f(sin)
    pos = np.asarray(pos)
    m, P, _ = delta.shape
    _, heads, K, d = keys.shape
    c, s_ = cos[pos][:, None, None, :], sin[pos][:, None, None, :]
    rot = lambda u: np.concatenate([u[..., :d // 2] * c + u[..., d // 2:] * s_,
                                    u[..., :d // 2] * -s_ + u[..., d // 2:] * c], -1)
    r0 = rot((tf(_rms(x, width)) @ tf(w_q).T).reshape(m, 1, heads, d))
    dr = rot((tf(norm_difference(x, delta, width)) @ tf(w_q).T).reshape(m, P, heads, d))
    sq = np.sum(r0 * r0, -1, keepdims=True)
    inv0 = 1.0 / np.sqrt(sq / d + EPS32)
    inv = 1.0 / np.sqrt((sq + 2 * np.sum(r0 * dr, -1, keepdims=True) + np.sum(dr * dr, -1, keepdims=True)) / d + EPS32)
    dq = dr * inv + r0 * (inv - inv0)
    ds = rb(np.einsum('mphd,mhkd->mphk', rb(dq), keys)) * d ** -0.5
    p = tp[:, None]
    dlse = np.log1p(np.sum(p * np.expm1(ds), -1, keepdims=True))
    dout = rb(np.einsum('mphk,mhkd->mphd', rb(p * np.expm1(ds - dlse)), vals))
    dout = dout + np.expm1(-dlse) * rest[:, None]
    return tf(dout.reshape(m, P, heads * d)) @ tf(w_proj_t)


def chain_chunk(site, move, scale, e, x0, mids, xL, idx, hs, lam_r, lam_0, w_fc, w_out_t, weight_t,
                base, target_logit_w, y, own=None, width=512, policy='fp64'):
    """train/val/run.py:307-351 with own = None (every attention held), own = ('routed', pos,
    inputs, w_q, top_keys, top_values, top_p, rest, w_proj_t, (cos, sin)) (each move also changes
    its own token's attention through its own query, along its top keys) or own = ('window', pos,
    rels, inputs, w_q, keys, values, w_proj_t, cos, sin, windows) (the same over every key of its
    window; per-block lists as in the reference): forward differences of each token's loss along every move of one site, each
    later MLP restricted to the token's routed units. policy 'fp64': float64 throughout; 'build': float64 with bfloat16 rounding where the
    reference casts (dz, both routed products and their inputs, the head product and its input);
    'build32': the same casts in float32 arithmetic, so |build - build32| shows how far the casts
    alone let two correct evaluations drift (a product landing on the other side of a bf16
    rounding boundary); 'tf32': 'build' with the own-query step's float32 products on TF32 inputs
    (query_change_routed). Returns (m, P)."""
    dt = np.float32 if policy == 'build32' else np.float64
    rb = (lambda v: _bf16(v).astype(dt)) if policy in ('build', 'build32', 'tf32') else (lambda v: v)
    f = lambda v: np.asarray(v, dt)
    move, scale, e, x0, xL, base, tw = map(f, (move, scale, e, x0, xL, base, target_logit_w))
    lam_r, lam_0 = f(lam_r), f(lam_0)
    y = np.asarray(y)
    L = len(mids)
    if site < 0:
        dx0 = _rms(e[:, None, :] + move, width) - x0[:, None, :]
        delta, first = (lam_r[0] + lam_0[0]) * dx0, 0
    else:
        dx0, delta, first = None, move, site
    for b in range(first, L):
        if b > first:
            delta = lam_r[b] * delta + (lam_0[b] * dx0 if dx0 is not None else 0)
        if own is not None and (site < 0 or b > first):
            if own[0] == 'routed':
                _, pos, inputs, w_q, top_keys, top_values, top_p, rest, w_proj_t, cos_sin = own
                delta = delta + query_change_routed(inputs[b], delta, pos, w_q[b], top_keys[b], top_values[b],
                                                    top_p[b], rest[b], w_proj_t[b], cos_sin[0], cos_sin[1], width,
                                                    policy)
            else:
                assert own[0] == 'window'
                _, pos, rels, inputs, w_q, keys, values, w_proj_t, cos, sin, windows = own
                delta = delta + query_change(inputs[b], delta, pos, rels[b], w_q[b], keys[b], values[b],
                                             w_proj_t[b], cos, sin, windows[b], width, policy)
        dz = rb(norm_difference(f(mids[b]), delta.astype(dt), width))
        wf = f(w_fc[b])[np.asarray(idx[b])]                      # (m, k, W)
        dh = rb(np.einsum('mpd,mkd->mpk', dz, wf))
        h = f(hs[b])[:, None, :]
        up, down = np.maximum(h + dh, 0), np.maximum(h, 0)
        wo = f(w_out_t[b])[np.asarray(idx[b])]                   # (m, k, W)
        delta = delta + rb(np.einsum('mpk,mkd->mpd', rb((up - down) * (up + down)), wo))
    sq = np.sum(xL * xL, -1)[:, None]
    dots = np.einsum('md,mpd->mp', xL, delta)
    inv = 1.0 / np.sqrt((sq + 2 * dots + np.sum(delta * delta, -1)) / width + EPS32)
    t = np.clip(y, 0, None)
    moved_logits = rb(np.einsum('mpd,dv->mpv', rb(delta), f(weight_t)))
    z = (base[:, None, :] + moved_logits) * inv[..., None]
    base_y = base[np.arange(base.shape[0]), t]
    zy = (base_y[:, None] + np.einsum('mpd,md->mp', delta, tw)) * inv
    moved = _logsumexp(cap(z)) - cap(zy)
    inv0 = 1.0 / np.sqrt(sq / width + EPS32)
    clean = _logsumexp(cap(base * inv0)) - cap(base_y * inv0[:, 0])
    return (moved - clean[:, None]) / scale * (y >= 0)[:, None]
