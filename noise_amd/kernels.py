"""Thin torch-tensor wrappers over the C ABI of libnoise_amd (include/noise_amd.h).

Every wrapper checks devices, dtypes, shapes and strides on the host, then passes raw device
pointers and the current HIP stream. Launches are asynchronous; no wrapper synchronises.
"""
import ctypes as C

import torch

from . import _lib
from ._lib import Attention, Head, MixNorm, Mlp, Rank1, Rope


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _need(cond, msg):
    if not cond:
        raise ValueError(msg)


def _on_gpu(*ts):
    for t in ts:
        if t is not None:
            _need(t.is_cuda, 'libnoise_amd kernels take device tensors')


def _rows(t, width, dtype, name):
    """A 2-D (or row-strided) tensor whose rows are contiguous; returns its row stride."""
    _need(t.dtype == dtype, f'{name}: expected {dtype}, got {t.dtype}')
    _need(t.dim() == 2 and t.shape[1] >= width and t.stride(1) == 1,
          f'{name}: expected rows of {width} contiguous elements, got shape {tuple(t.shape)} '
          f'strides {t.stride()}')
    return t.stride(0)


class NoiseRows:
    """Perturbation vectors of one parameter for a chunk of members: a [rows, out] and b [rows, in]
    (row r of member p is p >> shift), or eps [rows, L] for a mixing-scalar vector."""

    __slots__ = ('a', 'b', 'eps', 'shift')

    def __init__(self, a=None, b=None, eps=None, shift=0):
        self.a, self.b, self.eps, self.shift = a, b, eps, shift


def rank1(sign, T, a_list, u_list, u_parts, ldu, shift):
    r = Rank1()
    if sign is None:
        return None
    r.sign = sign.data_ptr()
    r.rows_per_member = T
    r.member_shift = shift
    r.nseg = len(a_list)
    lda = a_list[0].stride(0)
    for s, (a, u) in enumerate(zip(a_list, u_list)):
        _need(a.dtype == torch.float32 and a.stride(1) == 1 and a.stride(0) == lda, 'rank1: a rows')
        r.a[s] = a.data_ptr()
        r.u[s] = u.data_ptr()
    r.seg_cols = a_list[0].shape[1]
    r.u_parts = u_parts
    r.lda = lda
    r.ldu = ldu
    r._keep = (sign, tuple(a_list), tuple(u_list))  # the struct holds raw pointers into these
    return r


def lowrank_gemm(A, W, r1, mode, C_out, b_next=None, u_next=None):
    """C = A W^T + rank-1 (see NOISE_EPI_*); A [M, K] bf16, W [N, K] bf16."""
    _on_gpu(A, W, C_out, b_next, u_next)
    M, K = A.shape
    N = W.shape[0]
    lda = _rows(A, K, torch.bfloat16, 'A')
    ldw = _rows(W, K, torch.bfloat16, 'W')
    cdt = torch.bfloat16 if mode in (_lib.EPI_BF16, _lib.EPI_RELU2_BF16) else torch.float32
    ldc = _rows(C_out, N, cdt, 'C')
    _need(C_out.shape[0] >= M, 'C has too few rows')
    ldb = b_next.stride(0) if b_next is not None else 0
    ldun = u_next.stride(0) if u_next is not None else 0
    _lib.call('noise_lowrank_gemm', _ptr(A), lda, _ptr(W), ldw, M, N, K,
              C.byref(r1) if r1 is not None else None, mode, _ptr(C_out), ldc,
              _ptr(b_next), ldb, _ptr(u_next), ldun, _stream())


MLP_PACKED_ELEMS = 2048 * 512  # bf16 elements of each packed MLP weight copy


def mlp_pack(w_fc=None, fc_packed=None, w_proj=None, proj_packed=None):
    """Packed bf16 copies of c_fc (fp32 [2048, 512]) and/or c_proj (fp32 [512, 2048]) weights in the
    operand layouts of mlp_fused."""
    for w, out, shape, name in ((w_fc, fc_packed, (2048, 512), 'c_fc'), (w_proj, proj_packed, (512, 2048), 'c_proj')):
        if out is None:
            continue
        _on_gpu(w, out)
        _need(w.dtype == torch.float32 and tuple(w.shape) == shape and w.stride(1) == 1,
              f'mlp_pack: {name} weight must be fp32 {list(shape)} with contiguous rows')
        _need(out.dtype == torch.bfloat16 and out.is_contiguous() and out.numel() == MLP_PACKED_ELEMS,
              f'mlp_pack: packed {name} must be a contiguous bf16 tensor of 2048 * 512 elements')
    _lib.call('noise_mlp_pack', _ptr(w_fc if fc_packed is not None else None),
              w_fc.stride(0) if fc_packed is not None else 0,
              _ptr(w_proj if proj_packed is not None else None), w_proj.stride(0) if proj_packed is not None else 0,
              _ptr(fc_packed), _ptr(proj_packed), _stream())


def mlp_fused(x_in, x_out, T, members, w_fc_packed, w_proj_packed, flags, sign=None, fc=None, proj=None,
              member_stride_in=None, member_stride_out=None, next_norm=None, attn=None):
    """x_out = [x_in +] c_proj(relu(c_fc(h) + rank-1)^2) + rank-1 with h = bf16(norm x_in) under
    MLP_NORM (else bf16(x_in)), in one launch. x_in / x_out: fp32 rows of 512; member p's rows
    start at p * member_stride (default T rows). fc / proj: NoiseRows of c_fc and c_proj.
    next_norm: a mix_norm_args record over x_out, run on the finished rows in the same launch.
    attn: (y, w_o, u, nz_o) -- the attention c_proj first, x_in + y w_o^T + s (u summed over its
    columns) a_o^T: y [members * T, 512] bf16, w_o [512, 512] bf16, u [members * T, parts] fp32
    and nz_o the c_proj NoiseRows (u and nz_o None when unperturbed)."""
    _on_gpu(x_in, x_out, w_fc_packed, w_proj_packed, sign)
    ld_in = _rows(x_in, 512, torch.float32, 'x_in')
    ld_out = _rows(x_out, 512, torch.float32, 'x_out')
    for w in (w_fc_packed, w_proj_packed):
        _need(w.dtype == torch.bfloat16 and w.numel() == MLP_PACKED_ELEMS and w.is_contiguous(),
              'mlp_fused: the weights must be packed bf16 copies (mlp_pack)')
    g = Mlp()
    g.in_, g.ld_in = x_in.data_ptr(), ld_in
    g.member_stride_in = T * ld_in if member_stride_in is None else member_stride_in
    g.out, g.ld_out = x_out.data_ptr(), ld_out
    g.member_stride_out = T * ld_out if member_stride_out is None else member_stride_out
    span_in = (members - 1) * g.member_stride_in + (T - 1) * ld_in + 512 if members else 0
    span_out = (members - 1) * g.member_stride_out + (T - 1) * ld_out + 512 if members else 0
    _need(span_in <= x_in.numel() and span_out <= x_out.numel(), 'mlp_fused: x_in / x_out have too few rows')
    g.T, g.members, g.flags = T, members, flags
    g.w_fc, g.w_proj = w_fc_packed.data_ptr(), w_proj_packed.data_ptr()
    if sign is not None:
        _need(sign.dtype == torch.float32 and sign.numel() >= members, 'mlp_fused: sign [members] fp32')
        need = ((members - 1) >> fc.shift) + 1 if members else 0
        for t, width, name in ((fc.a, 2048, 'c_fc a'), (fc.b, 512, 'c_fc b'), (proj.a, 512, 'c_proj a'),
                               (proj.b, 2048, 'c_proj b')):
            _on_gpu(t)
            _rows(t, width, torch.float32, name)
            _need(t.shape[0] >= need, f'mlp_fused: {name} has {t.shape[0]} noise rows, {need} needed')
        _need(proj.shift == fc.shift, 'mlp_fused: c_fc and c_proj noise rows must share member_shift')
        g.sign, g.member_shift = sign.data_ptr(), fc.shift
        g.a_fc, g.ld_a_fc = fc.a.data_ptr(), fc.a.stride(0)
        g.b_fc, g.ld_b_fc = fc.b.data_ptr(), fc.b.stride(0)
        g.a_proj, g.ld_a_proj = proj.a.data_ptr(), proj.a.stride(0)
        g.b_proj, g.ld_b_proj = proj.b.data_ptr(), proj.b.stride(0)
    if next_norm is not None:
        _need(isinstance(next_norm, MixNorm) and next_norm.x == x_out.data_ptr() and next_norm.M == members * T,
              'mlp_fused: next_norm must be a mix_norm_args record over the rows of x_out')
        g.next = C.pointer(next_norm)
    if attn is not None:
        y, w_o, u, nz_o = attn
        _on_gpu(y, w_o, u)
        ld_y = _rows(y, 512, torch.bfloat16, 'attn y')
        _need(y.shape[0] >= members * T, 'mlp_fused: attn y has too few rows')
        _need(w_o.dtype == torch.bfloat16 and tuple(w_o.shape) == (512, 512) and w_o.is_contiguous(),
              'mlp_fused: attn w_o must be a contiguous [512, 512] bf16 tensor')
        g.attn_y, g.ld_attn_y, g.attn_w = y.data_ptr(), ld_y, w_o.data_ptr()
        if sign is not None:
            _need(u is not None and nz_o is not None and u.dtype == torch.float32 and u.dim() == 2 and
                  u.stride(1) == 1 and u.shape[0] >= members * T, 'mlp_fused: attn u [rows, parts] fp32')
            _need(nz_o.shift == fc.shift, 'mlp_fused: the attention c_proj noise rows must share member_shift')
            _rows(nz_o.a, 512, torch.float32, 'attn a')
            g.attn_u, g.ld_attn_u, g.attn_parts = u.data_ptr(), u.stride(0), u.shape[1]
            g.attn_a, g.ld_attn_a = nz_o.a.data_ptr(), nz_o.a.stride(0)
    _lib.call('noise_mlp_fused', C.byref(g), _stream())


def embed_norm(table, idx, T, members, sign, nz, x0, x=None, idx_stride=0, next_norm=None):
    """x0 = norm(W[idx] + s a[idx] b) and x = x0 (when given), or, with next_norm (a mix_norm_args
    record mixing with this x0), the first layer's mix_norm on the rows in the same launch."""
    _on_gpu(table, idx, x0, x)
    _need(idx.dtype == torch.int64, 'idx must be int64')
    a = b = None
    lda = ldb = 0
    shift = 0
    if sign is not None:
        a, b, shift = nz.a, nz.b, nz.shift
        lda, ldb = a.stride(0), b.stride(0)
    head = (_ptr(table), table.stride(0), table.shape[0], table.shape[1], _ptr(idx), idx_stride, T, members,
            _ptr(sign), _ptr(a), lda, _ptr(b), ldb, shift, _ptr(x0))
    if next_norm is None:
        _lib.call('noise_embed_norm', *head, _ptr(x), _stream())
    else:
        _need(isinstance(next_norm, MixNorm) and x is None, 'embed_norm: next_norm replaces the copy x')
        _lib.call('noise_embed_mix_norm', *head, C.byref(next_norm), _stream())


def mix_norm(x, h, T, sign=None, x0=None, resid=None, mix=None, eps_r=None, eps_m=None, shift=0,
             bs=(), u=None, gate_w=None, gate_nz=None, gate=None, gain=None):
    """x = (lr + s er) x + (l0 + s e0) x0 (when x0 is given), h = bf16(norm x) (times `gain` [512]
    when given, F.rms_norm's weight), u[:, j] = h . bs[j], gate = 2 sigmoid(h[:32] (Wg + s a b^T)^T)
    (when gate_w is given), in one launch."""
    run_mix_norm(mix_norm_args(x, h, T, sign, x0, resid, mix, eps_r, eps_m, shift, bs, u, gate_w, gate_nz, gate,
                               gain))


def run_mix_norm(g):
    _lib.call('noise_mix_norm', C.byref(g), _stream())


def mix_norm_args(x, h, T, sign=None, x0=None, resid=None, mix=None, eps_r=None, eps_m=None, shift=0,
                  bs=(), u=None, gate_w=None, gate_nz=None, gate=None, gain=None):
    """The MixNorm launch record of `mix_norm`, for run_mix_norm or mlp_fused(next_norm=...)."""
    g = MixNorm()
    if gain is not None:
        _need(gain.dtype == torch.float32 and gain.shape == (512,) and gain.is_contiguous() and gain.device == x.device,
              'mix_norm: gain must be a contiguous float32 [512] tensor on the rows\' device')
        g.gain = gain.data_ptr()
    g.x, g.x0, g.M, g.T, g.member_shift = x.data_ptr(), _ptr(x0), x.shape[0], T, shift
    g.sign = _ptr(sign)
    g.resid, g.mix = _ptr(resid), _ptr(mix)
    if x0 is not None and sign is not None:
        g.eps_resid, g.eps_mix, g.ld_eps = eps_r.data_ptr(), eps_m.data_ptr(), eps_r.stride(0)
    g.h = h.data_ptr()
    g.nb = len(bs)
    for j, b in enumerate(bs):
        g.b[j] = b.data_ptr()
    if bs:
        g.ldb = bs[0].stride(0)
        g.u, g.ldu = u.data_ptr(), u.stride(0) if u.dim() == 2 else 1
    if gate_w is not None:
        g.gate_w, g.gate = gate_w.data_ptr(), gate.data_ptr()
        if sign is not None:
            g.gate_a, g.gate_b = gate_nz.a.data_ptr(), gate_nz.b.data_ptr()
            g.ld_gate_a, g.ld_gate_b = gate_nz.a.stride(0), gate_nz.b.stride(0)
    return g


def _rope_args(g, T, cos, sin, sign, gate, ve_table, idx, ve_nz, idx_stride):
    g.T = T
    g.cos, g.sin = cos.data_ptr(), sin.data_ptr()
    if gate is not None:
        g.gate, g.ve_table, g.idx, g.idx_stride, g.vocab = (gate.data_ptr(), ve_table.data_ptr(),
                                                            idx.data_ptr(), idx_stride, ve_table.shape[0])
        if sign is not None:
            g.sign = sign.data_ptr()
            g.member_shift = ve_nz.shift
            g.ve_a, g.ve_b = ve_nz.a.data_ptr(), ve_nz.b.data_ptr()
            g.ld_ve_a, g.ld_ve_b = ve_nz.a.stride(0), ve_nz.b.stride(0)
    return g


def qkv_rope_gemm(A, W, r1, out16, T, cos, sin, sign=None, gate=None, ve_table=None, idx=None, ve_nz=None,
                  idx_stride=0):
    """out16 [M, 1536] bf16 = rope_norm_ve(A W^T + rank-1) in one launch (W = [Wq; Wk; Wv])."""
    _on_gpu(A, W, out16, cos, sin, gate, ve_table, idx)
    M, K = A.shape
    _need(W.shape[0] == 1536 and W.shape[1] == K, 'qkv_rope_gemm: W must be [1536, K]')
    _need(out16.dtype == torch.bfloat16 and tuple(out16.shape) == (M, 1536) and out16.is_contiguous(),
          'qkv_rope_gemm: out must be a contiguous [M, 1536] bf16 tensor')
    lda = _rows(A, K, torch.bfloat16, 'A')
    ldw = _rows(W, K, torch.bfloat16, 'W')
    g = Rope()
    g.out, g.M = out16.data_ptr(), M
    _rope_args(g, T, cos, sin, sign, gate, ve_table, idx, ve_nz, idx_stride)
    _lib.call('noise_qkv_rope_gemm', _ptr(A), lda, _ptr(W), ldw, M, K,
              C.byref(r1) if r1 is not None else None, C.byref(g), _stream())


def rope_norm_ve(qkv32, out16, T, cos, sin, sign=None, gate=None, ve_table=None, idx=None, ve_nz=None,
                 idx_stride=0):
    g = Rope()
    g.qkv, g.out, g.M = qkv32.data_ptr(), out16.data_ptr(), qkv32.shape[0]
    _rope_args(g, T, cos, sin, sign, gate, ve_table, idx, ve_nz, idx_stride)
    _lib.call('noise_rope_norm_ve', C.byref(g), _stream())


def window_attention(qkv16, y, members, T, window, b_proj=None, shift=0, u_proj=None, moments=None,
                     scratch=None):
    g = Attention()
    g.qkv, g.ldqkv, g.y = qkv16.data_ptr(), qkv16.stride(0), y.data_ptr()
    g.members, g.T, g.heads, g.window, g.scale = members, T, 8, window, 0.125
    if b_proj is not None:
        g.b_proj, g.ld_b_proj, g.u_proj = b_proj.data_ptr(), b_proj.stride(0), u_proj.data_ptr()
    g.member_shift = shift
    g.moments, g.scratch = _ptr(moments), _ptr(scratch)
    _lib.call('noise_window_attention', C.byref(g), _stream())


def head_ce(h, w_hi, w_lo, T, targets, ce, sign=None, nz=None, u=None, targets_stride=0, ignore_index=-100,
            logits=None):
    """ce [M] (0 where the target is `ignore_index`); with `logits` [M, >= V] fp32 also the capped
    logits. w_lo None: the bf16 head alone; else h (w_hi + w_lo)^T, fp32-accurate."""
    g = Head()
    g.h, g.w_hi, g.w_lo = h.data_ptr(), w_hi.data_ptr(), _ptr(w_lo)
    g.M, g.V, g.T = h.shape[0], w_hi.shape[0], T
    if sign is not None:
        g.sign, g.a, g.lda, g.u, g.member_shift = (sign.data_ptr(), nz.a.data_ptr(), nz.a.stride(0),
                                                   u.data_ptr(), nz.shift)
    members = -(-g.M // T) if g.M else 0
    _need(targets.dtype == torch.int64 and targets.is_contiguous() and ce.numel() >= g.M and
          (members == 0 or targets.numel() >= (members - 1) * targets_stride + T),
          'head_ce: targets must be contiguous int64 covering (members - 1) * targets_stride + T entries '
          '(targets_stride 0: one sequence shared by every member), ce [M]')
    g.targets, g.targets_stride, g.ce = targets.data_ptr(), targets_stride, ce.data_ptr()
    g.ignore_index = ignore_index
    if logits is not None:
        _on_gpu(logits)
        _need(logits.dtype == torch.float32 and logits.dim() == 2 and logits.stride(1) == 1 and
              logits.shape[0] >= g.M and logits.shape[1] >= g.V, 'head_ce: logits must be fp32 [M, >= V] rows')
        g.logits, g.ld_logits = logits.data_ptr(), logits.stride(0)
    _lib.call('noise_head_ce', C.byref(g), _stream())


def member_mean(ce, members, T, out):
    _lib.call('noise_member_mean', _ptr(ce), members, T, _ptr(out), _stream())


def cast_bf16(x, hi, lo=None):
    _need(x.dtype == torch.float32 and x.is_contiguous() and hi.is_contiguous(), 'cast_bf16: contiguous fp32')
    _need(hi.numel() == x.numel() and (lo is None or lo.numel() == x.numel()), 'cast_bf16: sizes')
    _lib.call('noise_cast_bf16', _ptr(x), x.numel(), _ptr(hi), _ptr(lo), _stream())


def cast_bf16_many(items):
    """cast_bf16 over up to 64 (x, hi, lo or None) triples in one launch."""
    _need(0 < len(items) <= 64, 'cast_bf16_many: 1..64 buffers')
    for x, hi, lo in items:
        _on_gpu(x, hi, lo)
        _need(x.dtype == torch.float32 and x.is_contiguous() and hi.is_contiguous() and
              (lo is None or lo.is_contiguous()), 'cast_bf16_many: contiguous fp32')
        _need(hi.numel() == x.numel() and (lo is None or lo.numel() == x.numel()), 'cast_bf16_many: sizes')
    k = len(items)
    xs = (C.c_void_p * k)(*[x.data_ptr() for x, _, _ in items])
    ns = (C.c_int64 * k)(*[x.numel() for x, _, _ in items])
    his = (C.c_void_p * k)(*[hi.data_ptr() for _, hi, _ in items])
    los = (C.c_void_p * k)(*[None if lo is None else lo.data_ptr() for _, _, lo in items])
    _lib.call('noise_cast_bf16_many', k, xs, ns, his, los, _stream())


def pair_gather(buffer, offsets, directions, widths, starts, out):
    """out[d, starts[k] + i] = buffer[offsets[k, directions[d]] + min(i, widths[k] - 1)] for
    i < widths[k] rounded up to 4: every parameter's noise slice of the pairs `directions`, side by
    side (eggroll.py:122-128). offsets: int64 [params, pairs]; widths / starts: Python ints."""
    _on_gpu(buffer, offsets, directions, out)
    _need(buffer.dtype == torch.float32 and buffer.is_contiguous(), 'pair_gather: contiguous fp32 buffer')
    _need(offsets.dtype == torch.int64 and offsets.dim() == 2 and offsets.stride(1) == 1 and
          offsets.shape[0] == len(widths), 'pair_gather: offsets must be int64 [params, pairs] rows')
    _need(directions.dtype == torch.int64 and directions.is_contiguous(), 'pair_gather: int64 directions')
    _need(out.dtype == torch.float32 and out.dim() == 2 and out.stride(1) == 1 and
          out.shape[0] >= directions.numel(), 'pair_gather: out must be fp32 [n, cols] rows')
    n, k = directions.numel(), len(widths)
    w = (C.c_int * k)(*widths)
    st = (C.c_int * k)(*starts)
    _lib.call('noise_pair_gather', _ptr(buffer), buffer.numel(), _ptr(offsets), offsets.stride(0), offsets.shape[1],
              _ptr(directions), n, k, w, st, _ptr(out), out.stride(0), _stream())


def fitness(losses, pairs, weight, status, mode='zscore', ranked=None):
    """weight [pairs] from antithetic losses: the reference z-score (mode 'zscore') or centred ranks
    ('ranks'; `ranked` [len(losses) / 2] receives the per-pair values)."""
    _on_gpu(losses, weight, status, ranked)
    _need(losses.dtype == torch.float32 and losses.is_contiguous(), 'fitness: fp32 losses')
    _need(weight.dtype == torch.float32 and weight.is_contiguous() and weight.numel() >= pairs, 'fitness: weight')
    if mode == 'zscore':
        _lib.call('noise_fitness', _ptr(losses), losses.numel(), pairs, _ptr(weight), _ptr(status), _stream())
    elif mode == 'ranks':
        _need(ranked is not None and ranked.dtype == torch.float32 and ranked.is_contiguous() and
              ranked.numel() >= losses.numel() // 2, 'fitness: ranks mode needs ranked [len(losses) / 2] fp32')
        _lib.call('noise_fitness_ranks', _ptr(losses), losses.numel(), pairs, _ptr(weight), _ptr(ranked),
                  _ptr(status), _stream())
    else:
        raise ValueError(f"fitness mode must be 'zscore' or 'ranks', not {mode!r}")


def es_gradient_work(n, out, inn):
    """Floats of workspace with which es_gradient splits its pair sum over more workgroups."""
    return int(_lib.load().noise_es_gradient_work(n, out, inn))


def es_gradient(w, a_base, a_off, b_base, b_off, out, inn, scale, G, accumulate=False, work=None):
    _on_gpu(w, a_base, a_off, G)
    _need(work is None or (work.is_cuda and work.dtype == torch.float32 and work.is_contiguous()),
          'es_gradient: work must be a contiguous fp32 device tensor')
    _lib.call('noise_es_gradient', _ptr(w), w.numel(), _ptr(a_base), _ptr(a_off), _ptr(b_base), _ptr(b_off),
              out, inn, scale, int(accumulate), _ptr(G), _ptr(work), 0 if work is None else work.numel(),
              _stream())


def es_gradient_params(w, buffer, offsets, shapes, grads, scale, accumulate=False):
    """grads[k] = scale * sum_j w_j a_kj b_kj^T for every parameter k in one launch
    (eggroll.py:155-163): pair j's noise for parameter k is buffer[offsets[k, j]:][:out + in], split
    into a (out) and b (in; b = 1 for a vector parameter, shape (out,)). offsets: int64
    [params, >= pairs] rows; shapes: one (out,) or (out, in) per parameter; grads: contiguous fp32
    device tensors of those shapes."""
    _on_gpu(w, buffer, offsets, *grads)
    _need(w.dtype == torch.float32 and w.is_contiguous(), 'es_gradient_params: contiguous fp32 w')
    _need(buffer.dtype == torch.float32 and buffer.is_contiguous(), 'es_gradient_params: contiguous fp32 buffer')
    _need(offsets.dtype == torch.int64 and offsets.dim() == 2 and offsets.stride(1) == 1 and
          offsets.shape[0] == len(shapes) and offsets.shape[1] >= w.numel(),
          'es_gradient_params: offsets must be int64 [params, >= pairs] rows')
    _need(len(grads) == len(shapes), 'es_gradient_params: one gradient per shape')
    for g, s in zip(grads, shapes):
        _need(g.dtype == torch.float32 and g.is_contiguous() and tuple(g.shape) == tuple(s),
              f'es_gradient_params: gradient {tuple(g.shape)} for shape {tuple(s)}')
        _need(len(s) == 1 or (len(s) == 2 and s[1] > 1),
              f'es_gradient_params: shape {tuple(s)}: a vector is (out,), a matrix (out, in > 1)')
    k = len(shapes)
    outs = (C.c_int * k)(*[s[0] for s in shapes])
    ins = (C.c_int * k)(*[s[1] if len(s) == 2 else 1 for s in shapes])
    ptrs = (C.c_void_p * k)(*[g.data_ptr() for g in grads])
    _lib.call('noise_es_gradient_params', _ptr(w), w.numel(), _ptr(buffer), buffer.numel(), _ptr(offsets),
              offsets.stride(0), k, outs, ins, ptrs, scale, int(accumulate), _stream())


def adamw(param, grad, exp_avg, exp_avg_sq, lr, beta1, beta2, eps, weight_decay, step, unless=None):
    """One AdamW update; with `unless` (a device int32 status) it is skipped on the device when the
    status is not NOISE_OK."""
    for t in (param, grad, exp_avg, exp_avg_sq):
        _need(t.is_cuda and t.dtype == torch.float32 and t.is_contiguous(), 'adamw: contiguous fp32 device tensors')
    if unless is None:
        _lib.call('noise_adamw', _ptr(param), _ptr(grad), _ptr(exp_avg), _ptr(exp_avg_sq), param.numel(), lr, beta1,
                  beta2, eps, weight_decay, step, _stream())
        return
    _need(unless.is_cuda and unless.dtype == torch.int32 and unless.numel() >= 1, 'adamw: unless is a device int32')
    _lib.call('noise_adamw_unless', _ptr(param), _ptr(grad), _ptr(exp_avg), _ptr(exp_avg_sq), param.numel(), lr,
              beta1, beta2, eps, weight_decay, step, _ptr(unless), _stream())
