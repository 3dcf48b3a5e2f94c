"""Kernel-level parity of libnoise_amd on the GPU against float64 references of the same op on the
same (bf16-rounded) inputs. Tolerances: fp32 outputs to accumulation-order error; bf16 outputs
within 1e-2 relative (and almost all elements bit-identical to the rounded reference)."""
import math

import pytest
import torch

from noise_amd import _lib
from noise_amd import kernels as nk
from noise_amd.kernels import NoiseRows
from oracle import model_ref as R

pytestmark = pytest.mark.gpu


EPS32 = torch.finfo(torch.float32).eps


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _bf(x):
    return x.to(torch.bfloat16)


def _close_bf16(got, ref, rtol=1e-2, exact_frac=0.99):
    got = got.double().cpu()
    ref_r = ref.to(torch.bfloat16).double()
    err = (got - ref).abs()
    assert (err <= rtol * ref.abs() + 1e-2 * rtol * ref.abs().max()).all(), float(err.max())
    assert (got == ref_r).double().mean() >= exact_frac


GEMM_CASES = [
    # M, N, K, T, nseg, parts, shift
    (512, 256, 64, 256, 1, 1, 0),
    (1000, 512, 512, 256, 1, 8, 0),      # row tail
    (768, 1536, 512, 100, 3, 1, 1),      # 3 segments, tiles straddling members, pair rows
    (512, 2048, 512, 512, 1, 1, 0),
    (256, 512, 2048, 128, 1, 16, 1),
    (300, 128, 128, 64, 1, 1, 0),        # one column tile, row tail
    (300, 384, 128, 64, 3, 2, 1),        # 128-column segments
    (512, 512, 512, 256, 1, 8, 1),       # K = 512, 128-row aligned members (the step's attention c_proj shape)
    (1024, 1536, 512, 128, 1, 2, 0),     # N = 1536 with one rank-1 segment
]


@pytest.mark.parametrize('M,N,K,T,nseg,parts,shift', GEMM_CASES)
@pytest.mark.parametrize('mode', [_lib.EPI_BF16, _lib.EPI_F32, _lib.EPI_ADD_F32, _lib.EPI_RELU2_BF16])
def test_lowrank_gemm(device, M, N, K, T, nseg, parts, shift, mode):
    g = _gen(M + N + K + mode)
    members = (M + T - 1) // T
    rows = (members >> shift) + 1
    A = _bf(torch.randn(M, K, generator=g))
    W = _bf(torch.randn(N, K, generator=g) / math.sqrt(K))
    sign = torch.randn(members, generator=g) * 0.1
    seg = N // nseg
    a = [torch.randn(rows, seg, generator=g) for _ in range(nseg)]
    u = [torch.randn(M, parts, generator=g) for _ in range(nseg)]
    p = torch.arange(M) // T
    ref = A.double() @ W.double().t()
    for s in range(nseg):
        ref[:, s * seg:(s + 1) * seg] += (sign[p] * u[s].sum(1)).double()[:, None] * a[s][p >> shift].double()
    dA, dW, dsign = A.to(device), W.to(device), sign.to(device)
    da = [x.to(device) for x in a]
    du = [x.to(device) for x in u]
    r1 = nk.rank1(dsign, T, da, du, parts, parts, shift)
    if mode == _lib.EPI_F32:
        C = torch.empty(M, N, device=device)
        nk.lowrank_gemm(dA, dW, r1, mode, C)
        torch.testing.assert_close(C.cpu().double(), ref, rtol=1e-5, atol=1e-4)
    elif mode == _lib.EPI_ADD_F32:
        C0 = torch.randn(M, N, generator=g)
        C = C0.to(device)
        nk.lowrank_gemm(dA, dW, r1, mode, C)
        torch.testing.assert_close(C.cpu().double(), ref + C0.double(), rtol=1e-5, atol=1e-4)
    elif mode == _lib.EPI_BF16:
        C = torch.empty(M, N, dtype=torch.bfloat16, device=device)
        nk.lowrank_gemm(dA, dW, r1, mode, C)
        _close_bf16(C, ref)
    else:
        bnext = torch.randn(rows, N, generator=g)
        C = torch.empty(M, N, dtype=torch.bfloat16, device=device)
        un = torch.full((M, N // 64), float("nan"), device=device)
        nk.lowrank_gemm(dA, dW, r1, mode, C, bnext.to(device), un)
        hid = torch.relu(ref).square()
        _close_bf16(C, hid)
        got = C.cpu().double()  # the partial dots use the stored bf16 values
        want = (got * bnext[p >> shift].double()).view(M, N // 64, 64).sum(-1)
        torch.testing.assert_close(un.cpu().double(), want, rtol=1e-5, atol=1e-3)


def test_lowrank_gemm_unperturbed_and_errors(device):
    g = _gen(3)
    A = _bf(torch.randn(300, 128, generator=g)).to(device)
    W = _bf(torch.randn(256, 128, generator=g)).to(device)
    C = torch.empty(300, 256, device=device)
    nk.lowrank_gemm(A, W, None, _lib.EPI_F32, C)
    torch.testing.assert_close(C.cpu().double(), A.cpu().double() @ W.cpu().double().t(), rtol=1e-5, atol=1e-4)
    with pytest.raises(ValueError):
        nk.lowrank_gemm(A, W[:100], None, _lib.EPI_F32, C)     # N not a multiple of 128
    with pytest.raises(ValueError):
        nk.lowrank_gemm(A[:, :100], W[:, :100], None, _lib.EPI_F32, C)  # K not a multiple of 64


def test_embed_norm(device):
    g = _gen(4)
    V, T, m = 4096, 96, 6
    table = torch.randn(V, 512, generator=g)
    idx = torch.randint(0, V, (T,), generator=g)
    a, b = torch.randn(3, V, generator=g), torch.randn(3, 512, generator=g)
    sign = torch.tensor([0.5, -0.5, 0.1, -0.1, 0.02, -0.02])
    x0 = torch.empty(m * T, 512, device=device)
    x = torch.empty_like(x0)
    nk.embed_norm(table.to(device), idx.to(device), T, m, sign.to(device),
                 NoiseRows(a=a.to(device), b=b.to(device), shift=1), x0, x)
    ref = R.rms_norm(R.lowrank_embed(table.double(), a.double().repeat_interleave(2, 0),
                                     b.double().repeat_interleave(2, 0), idx, sign.double())).reshape(m * T, 512)
    torch.testing.assert_close(x0.cpu().double(), ref, rtol=1e-5, atol=1e-5)
    assert torch.equal(x0, x)
    bad = idx.clone()
    bad[5] = V
    nk.embed_norm(table.to(device), bad.to(device), T, m, None, None, x0)
    rows = x0.cpu().view(m, T, 512)
    assert torch.isnan(rows[:, 5]).all() and not torch.isnan(rows[:, 4]).any()


@pytest.mark.parametrize('pert,gate', [(True, True), (False, True), (True, False)])
def test_embed_mix_norm_matches_two_launches(device, pert, gate):
    """embed_norm with the first layer's mix_norm in the same launch equals embed_norm (x = x0)
    followed by mix_norm on the same inputs: x0 bit-exact, the rest to fp32 rounding."""
    g = _gen(41)
    V, T, m = 4096, 66, 4
    M = m * T
    table = torch.randn(V, 512, generator=g).to(device)
    idx = torch.randint(0, V, (T,), generator=g).to(device)
    sign = torch.tensor([0.5, -0.5, 0.1, -0.1], device=device) if pert else None
    nz = NoiseRows(a=torch.randn(2, V, generator=g).to(device), b=torch.randn(2, 512, generator=g).to(device), shift=1)
    lam = torch.tensor([1.1, 0.2], device=device)
    eps = torch.randn(2, 8, generator=g).to(device), torch.randn(2, 8, generator=g).to(device)
    bs = tuple(torch.randn(2, 512, generator=g).to(device) for _ in range(3)) if pert else ()
    gw = torch.randn(8, 32, generator=g).to(device) if gate else None
    gnz = NoiseRows(a=torch.randn(2, 8, generator=g).to(device), b=torch.randn(2, 32, generator=g).to(device),
                    shift=1) if gate and pert else None
    outs = []
    for fused in (False, True):
        x0 = torch.full((M, 512), float('nan'), device=device)
        x = torch.full_like(x0, float('nan'))
        h = torch.full((M, 512), float('nan'), dtype=torch.bfloat16, device=device)
        u = torch.full((M, 3), float('nan'), device=device)
        gt = torch.full((M, 8), float('nan'), device=device)
        rec = nk.mix_norm_args(x, h, T, sign, x0, lam[0], lam[1], eps[0][:, 2] if pert else None,
                               eps[1][:, 2] if pert else None, 1, bs=bs, u=u, gate_w=gw, gate_nz=gnz, gate=gt)
        if fused:
            nk.embed_norm(table, idx, T, m, sign, nz, x0, None, next_norm=rec)
        else:
            nk.embed_norm(table, idx, T, m, sign, nz, x0, x)
            nk.run_mix_norm(rec)
        outs.append((x0, x, h, u, gt))
    (x0a, xa, ha, ua, ga), (x0b, xb, hb, ub, gb) = outs
    assert torch.equal(x0a, x0b)
    torch.testing.assert_close(xb, xa, rtol=1e-6, atol=1e-6)
    hd = (hb.float() - ha.float()).abs()
    assert (hd <= 2.0 ** -7 * ha.float().abs()).all() and (hd == 0).double().mean() >= 0.999
    # x agrees to fp32 rounding, so an odd h value may round to the other bf16 neighbour: the dots
    # and the gate are checked against float64 on each path's own h
    nrow = (torch.arange(M) // T) >> 1
    s64 = sign.double().cpu()[torch.arange(M) // T] if pert else None
    for hh, uu, gg in ((ha, ua, ga), (hb, ub, gb)):
        h64 = hh.double().cpu()
        if pert:
            want = torch.stack([(h64 * b.double().cpu()[nrow]).sum(1) for b in bs], 1)
            torch.testing.assert_close(uu.double().cpu(), want, rtol=1e-5, atol=1e-4)
        if gate:
            z = h64[:, :32] @ gw.double().cpu().t()
            if pert:
                nd = (h64[:, :32] * gnz.b.double().cpu()[nrow]).sum(1)
                z = z + (s64 * nd)[:, None] * gnz.a.double().cpu()[nrow]
            torch.testing.assert_close(gg.double().cpu(), 2 * torch.sigmoid(z), rtol=1e-5, atol=1e-5)
    with pytest.raises(ValueError, match='same members'):
        bad = nk.mix_norm_args(xb, hb, T, sign, x0a, lam[0], lam[1], eps[0][:, 2] if pert else None,
                               eps[1][:, 2] if pert else None, 1)
        nk.embed_norm(table, idx, T, m, sign, nz, x0b, None, next_norm=bad)


@pytest.mark.parametrize('T', [64, 66])  # 4 rows per wave / one row per wave (T % 4 != 0)
def test_mix_norm(device, T):
    g = _gen(5)
    m = 4
    M = T * m
    x, x0 = torch.randn(M, 512, generator=g), torch.randn(M, 512, generator=g)
    lam = torch.tensor([1.1, 0.2])
    eps_r, eps_m = torch.randn(2, 8, generator=g), torch.randn(2, 8, generator=g)
    sign = torch.tensor([0.3, -0.3, 0.05, -0.05])
    bs = [torch.randn(2, 512, generator=g) for _ in range(3)]
    gw = torch.randn(8, 32, generator=g)
    ga, gb = torch.randn(2, 8, generator=g), torch.randn(2, 32, generator=g)
    dx = x.to(device)
    h = torch.empty(M, 512, dtype=torch.bfloat16, device=device)
    u = torch.empty(M, 3, device=device)
    gate = torch.empty(M, 8, device=device)
    dl = lam.to(device)
    nk.mix_norm(dx, h, T, sign.to(device), x0.to(device), dl[0], dl[1], eps_r.to(device)[:, 3], eps_m.to(device)[:, 3], 1,
               bs=tuple(b.to(device) for b in bs), u=u, gate_w=gw.to(device),
               gate_nz=NoiseRows(a=ga.to(device), b=gb.to(device), shift=1), gate=gate)
    p = torch.arange(M) // T
    s = sign[p].double()[:, None]
    mixed = (lam[0] + s * eps_r[p >> 1, 3, None]) * x.double() + (lam[1] + s * eps_m[p >> 1, 3, None]) * x0.double()
    torch.testing.assert_close(dx.cpu().double(), mixed, rtol=1e-6, atol=1e-5)
    hn = R.rms_norm(mixed)
    _close_bf16(h, hn)
    hb = h.cpu().double()
    for j in range(3):
        torch.testing.assert_close(u[:, j].cpu().double(), (hb * bs[j][p >> 1].double()).sum(1), rtol=1e-5, atol=1e-4)
    z = hb[:, :32] @ gw.double().t() + s * (hb[:, :32] * gb[p >> 1].double()).sum(1, keepdim=True) * ga[p >> 1].double()
    torch.testing.assert_close(gate.cpu().double(), 2 * torch.sigmoid(z), rtol=1e-5, atol=1e-5)


def test_rope_norm_ve(device):
    g = _gen(6)
    T, m, V = 48, 4, 4096
    M = T * m
    qkv = torch.randn(M, 1536, generator=g)
    gate = torch.rand(M, 8, generator=g) * 2
    table = torch.randn(V, 512, generator=g)
    idx = torch.randint(0, V, (T,), generator=g)
    a, b = torch.randn(m, V, generator=g), torch.randn(m, 512, generator=g)
    sign = torch.tensor([0.2, -0.2, 0.7, -0.7])
    cos, sin = R.rotary_tables(T)
    out = torch.empty(M, 1536, dtype=torch.bfloat16, device=device)
    nk.rope_norm_ve(qkv.to(device), out, T, cos.to(device), sin.to(device), sign.to(device), gate.to(device),
                   table.to(device), idx.to(device), NoiseRows(a=a.to(device), b=b.to(device), shift=0))
    q = qkv[:, :512].double().view(m, T, 8, 64)
    k = qkv[:, 512:1024].double().view(m, T, 8, 64)
    rq = R.rms_norm(R.rotary(q, cos.double(), sin.double())).reshape(M, 512)
    rk = R.rms_norm(R.rotary(k, cos.double(), sin.double())).reshape(M, 512)
    ve = R.lowrank_embed(table.double(), a.double(), b.double(), idx, sign.double()).reshape(M, 512)
    v = qkv[:, 1024:].double() + gate.double().repeat_interleave(64, 1) * ve
    got = out.cpu()
    _close_bf16(got[:, :512], rq)
    _close_bf16(got[:, 512:1024], rk)
    _close_bf16(got[:, 1024:], v)


@pytest.mark.parametrize('T,members,shift,ve,pert', [
    (256, 4, 1, True, True), (100, 5, 0, True, True), (2048, 1, 0, False, True), (64, 8, 1, True, False),
    (300, 2, 1, False, False), (256, 2, 0, True, False), (512, 2, 0, False, False)])
def test_qkv_rope_gemm_matches_unfused(device, T, members, shift, ve, pert):
    """The fused q|k|v projection equals lowrank_gemm (fp32 out) followed by rope_norm_ve on the
    same inputs: the same fp32 arithmetic up to the order of the norm's sum of squares."""
    g = _gen(T * 7 + members)
    M, K, V = T * members, 512, 4096
    rows = (members >> shift) + 1
    A = _bf(torch.randn(M, K, generator=g)).to(device)
    W = _bf(torch.randn(1536, K, generator=g) / math.sqrt(K)).to(device)
    sign = (torch.randn(members, generator=g) * 0.3).to(device) if pert else None
    a = [torch.randn(rows, 512, generator=g).to(device) for _ in range(3)]
    u = [torch.randn(M, 1, generator=g).to(device) for _ in range(3)]
    r1 = nk.rank1(sign, T, a, u, 1, 1, shift) if pert else None
    cos, sin = (x.to(device) for x in R.rotary_tables(T))
    gate = (torch.rand(M, 8, generator=g) * 2).to(device) if ve else None
    table = torch.randn(V, 512, generator=g).to(device)
    idx = torch.randint(0, V, (T,), generator=g).to(device)
    nz = NoiseRows(a=torch.randn(rows, V, generator=g).to(device), b=torch.randn(rows, 512, generator=g).to(device),
                   shift=shift)
    fused = torch.empty(M, 1536, dtype=torch.bfloat16, device=device)
    nk.qkv_rope_gemm(A, W, r1, fused, T, cos, sin, sign, gate, table if ve else None, idx, nz if ve else None)
    qkv32 = torch.empty(M, 1536, device=device)
    nk.lowrank_gemm(A, W, nk.rank1(sign, T, a, u, 1, 1, shift) if pert else None, _lib.EPI_F32, qkv32)
    ref = torch.empty(M, 1536, dtype=torch.bfloat16, device=device)
    nk.rope_norm_ve(qkv32, ref, T, cos, sin, sign, gate, table if ve else None, idx, nz if ve else None)
    got, want = fused.cpu().double(), ref.cpu().double()
    assert float((got == want).double().mean()) >= 0.99
    assert float((got - want).abs().max()) <= 2 ** -7 * max(1.0, float(want.abs().max()))


@pytest.mark.parametrize('T,members,shift,ve', [(256, 4, 1, True), (128, 3, 0, False), (2048, 1, 0, True),
                                                 (512, 3, 1, False), (384, 2, 0, True),
                                                 (32, 5, 0, False), (96, 3, 1, False), (64, 8, 1, False)])
def test_qkv_row_resident_matches_oracle(device, T, members, shift, ve):
    """The q|k|v projection against the float64 oracle directly: R.lowrank for each of q, k, v
    (rank-1 through the given x . b dots), R.rotary and R.rms_norm per head for q and k, and
    v + gate * R.lowrank_embed. The two-waves-per-SIMD row-resident kernel runs where T and the
    row count are multiples of 256 (T = 256, 2048, 512), the one-wave form where they are multiples
    of 128 (T = 128, 384), the 256 x 256 tile GEMM with the same epilogue elsewhere (T = 32, 96, 64)."""
    g = _gen(T + 31 * members)
    M, K, V = T * members, 512, 4096
    rows = (members >> shift) + 1
    A = _bf(torch.randn(M, K, generator=g))
    W = _bf(torch.randn(1536, K, generator=g) / math.sqrt(K))
    sign = torch.randn(members, generator=g) * 0.3
    a = [torch.randn(rows, 512, generator=g) for _ in range(3)]
    b = [torch.randn(rows, K, generator=g) for _ in range(3)]
    pr = torch.arange(members) >> shift
    x = A.double().view(members, T, K)
    u = [(x * b[k].double()[pr][:, None, :]).sum(-1).reshape(M, 1).float() for k in range(3)]
    cos, sin = R.rotary_tables(T)
    gate = torch.rand(M, 8, generator=g) * 2
    table = torch.randn(V, 512, generator=g)
    idx = torch.randint(0, V, (T,), generator=g)
    nz = NoiseRows(a=torch.randn(rows, V, generator=g), b=torch.randn(rows, 512, generator=g), shift=shift)
    dv = lambda z: z.to(device)
    r1 = nk.rank1(dv(sign), T, [dv(z) for z in a], [dv(z) for z in u], 1, 1, shift)
    out = torch.empty(M, 1536, dtype=torch.bfloat16, device=device)
    nk.qkv_rope_gemm(dv(A), dv(W), r1, out, T, dv(cos), dv(sin), dv(sign), dv(gate) if ve else None,
                     dv(table) if ve else None, dv(idx),
                     NoiseRows(a=dv(nz.a), b=dv(nz.b), shift=shift) if ve else None)
    s = sign.double()
    proj = [R.lowrank(x, W.double()[512 * k:512 * (k + 1)], a[k].double()[pr], b[k].double()[pr], s)
            for k in range(3)]
    rq = R.rms_norm(R.rotary(proj[0].view(members, T, 8, 64), cos.double(), sin.double())).reshape(M, 512)
    rk = R.rms_norm(R.rotary(proj[1].view(members, T, 8, 64), cos.double(), sin.double())).reshape(M, 512)
    v = proj[2].reshape(M, 512)
    if ve:
        emb = R.lowrank_embed(table.double(), nz.a.double()[pr], nz.b.double()[pr], idx, s).reshape(M, 512)
        v = v + gate.double().repeat_interleave(64, 1) * emb
    got = out.cpu()
    _close_bf16(got[:, :512], rq)
    _close_bf16(got[:, 512:1024], rk)
    _close_bf16(got[:, 1024:], v)


@pytest.mark.parametrize('T,members,pert', [(256, 2, True), (256, 2, False), (128, 2, True)])
def test_qkv_row_resident_invalid_tokens(device, T, members, pert):
    """A token outside [0, vocab) makes the value-embedding term, and so the row's v, NaN; its q and
    k and every other row stay finite. T = 256 runs the two-waves-per-SIMD kernel, T = 128 the
    one-wave form."""
    g = _gen(T + 7 * members + pert)
    M, K, V = T * members, 512, 4096
    A = _bf(torch.randn(M, K, generator=g)).to(device)
    W = _bf(torch.randn(1536, K, generator=g) / math.sqrt(K)).to(device)
    sign = (torch.randn(members, generator=g) * 0.3).to(device) if pert else None
    a = [torch.randn(members, 512, generator=g).to(device) for _ in range(3)]
    u = [torch.randn(M, 1, generator=g).to(device) for _ in range(3)]
    r1 = nk.rank1(sign, T, a, u, 1, 1, 0) if pert else None
    cos, sin = (x.to(device) for x in R.rotary_tables(T))
    gate = (torch.rand(M, 8, generator=g) * 2).to(device)
    table = torch.randn(V, 512, generator=g).to(device)
    idx = torch.randint(0, V, (T,), generator=g)
    bad = torch.tensor([0, 5, T // 2, T - 1])
    idx[bad] = torch.tensor([-1, V, V + 7, -100])
    nz = NoiseRows(a=torch.randn(members, V, generator=g).to(device), b=torch.randn(members, 512, generator=g).to(device),
                   shift=0)
    out = torch.empty(M, 1536, dtype=torch.bfloat16, device=device)
    nk.qkv_rope_gemm(A, W, r1, out, T, cos, sin, sign, gate, table, idx.to(device), nz)
    got = out.cpu().float().view(members, T, 1536)
    is_bad = torch.zeros(T, dtype=torch.bool)
    is_bad[bad] = True
    assert torch.isfinite(got[:, :, :1024]).all()
    assert torch.isnan(got[:, is_bad, 1024:]).all()
    assert torch.isfinite(got[:, ~is_bad, 1024:]).all()


@pytest.mark.parametrize('T,window,members,unit', [
    (96, 16, 2, True), (128, 64, 3, True), (256, 1024, 2, True), (300, 100, 2, True),
    (2048, 1024, 1, True), (2048, 2048, 1, True), (520, 0, 1, True), (700, 300, 2, False),
    (2048, 1024, 1, False)])
def test_window_attention(device, T, window, members, unit):
    """Against exact softmax attention (bf16 output tolerance) and against the build's rounding
    model (constant shift, bf16 probabilities); unit-rms q, k as the model feeds them, or raw
    N(0, 1) rows as in the attention-only workload."""
    g = _gen(T + window)
    M = members * T
    q = torch.randn(M, 8, 64, generator=g)
    k = torch.randn(M, 8, 64, generator=g)
    if unit:
        q, k = R.rms_norm(q), R.rms_norm(k)
    v = torch.randn(M, 512, generator=g)
    qkv = _bf(torch.cat([q.reshape(M, 512), k.reshape(M, 512), v], 1))
    bp = torch.randn(members, 512, generator=g)
    y = torch.empty(M, 512, dtype=torch.bfloat16, device=device)
    uproj = torch.empty(M, 8, device=device)
    mom = torch.empty(members, 8, 2, 64, device=device)
    scratch = torch.empty(members * 8 * ((T + 255) // 256) * 128, device=device)
    nk.window_attention(qkv.to(device), y, members, T, window, bp.to(device), 0, uproj, mom, scratch)
    qd, kd, vd = (qkv[:, i * 512:(i + 1) * 512].double().view(members, T, 8, 64) for i in range(3))
    ref = R.window_attention(qd, kd, vd, window).reshape(M, 512)
    got = y.cpu().double()
    err = (got - ref).abs()
    assert float(err.max()) < 2e-2 * max(1.0, float(ref.abs().max())), float(err.max())
    assert float(err.mean()) < 2e-3
    model = R.window_attention_shifted(qd, kd, vd, window).reshape(M, 512)
    assert float((got - model).abs().max()) < 2 ** -7 * max(1.0, float(model.abs().max()))
    p = torch.arange(M) // T
    torch.testing.assert_close(uproj.cpu().double(), (got * bp[p].double()).view(M, 8, 64).sum(-1), rtol=1e-5, atol=1e-4)
    gy = got.view(members, T, 8, 64)
    want = torch.stack([gy.mean(1), gy.square().mean(1)], 2)  # [members, 8, 2, 64]
    torch.testing.assert_close(mom.cpu().double(), want, rtol=1e-5, atol=1e-5)


def _head_weights(W, device, split):
    """bf16 hi (+ lo when split) copies of W, and the fp64 weight the kernel's product equals."""
    hi = torch.empty(W.shape[0], 512, dtype=torch.bfloat16, device=device)
    lo = torch.empty_like(hi) if split else None
    nk.cast_bf16(W.to(device), hi, lo)
    return hi, lo, (W.double() if split else W.to(torch.bfloat16).double())


@pytest.mark.parametrize('split', [False, True])  # the bf16 head / the fp32-weight hi + lo head
def test_head_ce(device, split):
    g = _gen(7)
    T, m, V = 64, 4, 4096
    M = T * m
    h = _bf(R.rms_norm(torch.randn(M, 512, generator=g)))
    W = torch.randn(V, 512, generator=g) * 0.06
    a = torch.randn(m, V, generator=g)
    u = torch.randn(M, generator=g)
    sign = torch.tensor([0.01, -0.01, 0.002, -0.002])
    targets = torch.randint(0, V, (T,), generator=g)
    hi, lo, Wd = _head_weights(W, device, split)
    ce = torch.empty(M, device=device)
    nk.head_ce(h.to(device), hi, lo, T, targets.to(device), ce, sign.to(device),
              NoiseRows(a=a.to(device), shift=0), u.to(device))
    p = torch.arange(M) // T
    z = h.double() @ Wd.t() + (sign[p] * u).double()[:, None] * a[p].double()
    ref = R.softcap_ce(z, targets.repeat(m))
    torch.testing.assert_close(ce.cpu().double(), ref, rtol=0, atol=2e-5)
    losses = torch.empty(m, device=device)
    nk.member_mean(ce, m, T, losses)
    torch.testing.assert_close(losses.cpu().double(), ce.cpu().double().view(m, T).mean(1), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize('T,split', [(256, False), (300, False), (256, True)])
def test_head_ce_ignore_index_and_logits(device, T, split):
    """F.cross_entropy's ignore_index in the fused head: a target equal to it scores 0, any other
    target outside [0, V) scores NaN (torch raises there); the optional capped-logits output
    matches 15 tanh(z / 15) of the fp64 product, and asking for it leaves ce unchanged. T = 300
    takes the ragged-row kernel and a partial last tile."""
    g = _gen(17)
    m, V = 2, 4096
    M = T * m
    h = _bf(R.rms_norm(torch.randn(M, 512, generator=g)))
    W = torch.randn(V, 512, generator=g) * 0.06
    a = torch.randn(m, V, generator=g)
    u = torch.randn(M, generator=g)
    sign = torch.tensor([0.01, -0.01])
    targets = torch.randint(0, V, (m, T), generator=g)
    targets[0, 3], targets[1, 7], targets[0, T - 1] = -1, -1, -1
    targets[1, 11], targets[0, 20] = -100, V + 5
    hi, lo, Wd = _head_weights(W, device, split)
    dh, dt, ds, du = h.to(device), targets.to(device), sign.to(device), u.to(device)
    nz = NoiseRows(a=a.to(device), shift=0)
    p = torch.arange(M) // T
    z = h.double() @ Wd.t() + (sign[p] * u).double()[:, None] * a[p].double()
    tf = targets.reshape(-1)
    valid = (tf >= 0) & (tf < V)
    ref = torch.zeros(M, dtype=torch.float64)
    ref[valid] = R.softcap_ce(z[valid], tf[valid])
    for ignore in (-1, -100):
        ce = torch.empty(M, device=device)
        nk.head_ce(dh, hi, lo, T, dt, ce, ds, nz, du, targets_stride=T, ignore_index=ignore)
        c = ce.cpu().double()
        torch.testing.assert_close(c[valid], ref[valid], rtol=0, atol=2e-5)
        assert torch.all(c[tf == ignore] == 0)
        assert torch.all(torch.isnan(c[~valid & (tf != ignore)]))
        logits = torch.full((M, V + 64), 7.0, device=device)
        ce2 = torch.empty(M, device=device)
        nk.head_ce(dh, hi, lo, T, dt, ce2, ds, nz, du, targets_stride=T, ignore_index=ignore, logits=logits)
        # with logits out the tile kernel runs; without, at T = 256, the row-resident one
        torch.testing.assert_close(ce2.cpu()[valid], ce.cpu()[valid], rtol=0, atol=2e-5)
        assert torch.equal(torch.isnan(ce2.cpu()), torch.isnan(ce.cpu()))
        lg = logits.cpu().double()
        torch.testing.assert_close(lg[:, :V], 15 * torch.tanh(z / 15), rtol=0, atol=2e-5)
        assert torch.all(lg[:, V:] == 7.0)  # the row padding past V is never written
    with pytest.raises(Exception, match='ignore_index'):
        nk.head_ce(dh, hi, lo, T, dt, ce, ds, nz, du, targets_stride=T, ignore_index=5)


@pytest.mark.parametrize('T,m,V,shift,pert,split', [
    (256, 4, 4096, 1, True, False), (256, 4, 4096, 1, True, True), (512, 2, 1024, 0, True, False),
    (256, 2, 64, 0, False, True), (256, 3, 4096, 0, False, False)])
def test_head_row_resident_matches_oracle(device, T, m, V, shift, pert, split):
    """The row-resident head (whole 256-row workgroups of one member, V % 64 == 0, no logits out)
    against the float64 soft-capped cross-entropy: pair-shared noise rows, the fp32-accurate hi + lo
    weight and the bf16 one, small vocabularies (a single pair of 32-entry chunks at V = 64), an
    ignored target (0) and out-of-range ones (NaN) next to valid ones."""
    g = _gen(T + 7 * m + V)
    M = T * m
    rows = (m >> shift) + 1
    h = _bf(R.rms_norm(torch.randn(M, 512, generator=g)) * 1.5)
    W = torch.randn(V, 512, generator=g) * 0.08
    a = torch.randn(rows, V, generator=g)
    u = torch.randn(M, generator=g)
    sign = torch.randn(m, generator=g) * 0.05
    targets = torch.randint(0, V, (m, T), generator=g)
    targets[0, 5], targets[m - 1, T - 1], targets[1, 0] = -1, V, -7
    hi, lo, Wd = _head_weights(W, device, split)
    ce = torch.empty(M, device=device)
    nk.head_ce(h.to(device), hi, lo, T, targets.to(device), ce, sign.to(device) if pert else None,
               NoiseRows(a=a.to(device), shift=shift) if pert else None, u.to(device) if pert else None,
               targets_stride=T, ignore_index=-1)
    p = torch.arange(M) // T
    z = h.double() @ Wd.t()
    if pert:
        z = z + (sign[p] * u).double()[:, None] * a[p >> shift].double()
    tf = targets.reshape(-1)
    valid = (tf >= 0) & (tf < V)
    got = ce.cpu().double()
    # logits up to |z| ~ 12 here (cross-entropies ~ 10.5): fp32 rounding of the product, of the
    # 4096-term sum and of the soft cap leaves a few 1e-6 relative
    torch.testing.assert_close(got[valid], R.softcap_ce(z[valid], tf[valid]), rtol=4e-6, atol=1e-5)
    assert torch.all(got[tf == -1] == 0)
    assert torch.all(torch.isnan(got[~valid & (tf != -1)]))


def test_cast_bf16_round_to_nearest_even(device):
    g = _gen(8)
    x = torch.randn(100003, generator=g) * 10
    x[:4] = torch.tensor([1.00390625, 1.01171875, -3.0078125, 0.0])  # exact ties
    hi = torch.empty(x.numel(), dtype=torch.bfloat16, device=device)
    lo = torch.empty_like(hi)
    nk.cast_bf16(x.to(device), hi, lo)
    assert torch.equal(hi.cpu(), x.to(torch.bfloat16))
    assert torch.equal(lo.cpu(), (x - x.to(torch.bfloat16).float()).to(torch.bfloat16))


def test_cast_bf16_many_matches_single_casts(device):
    """One launch over ragged buffers (sizes not multiples of 4, one empty, one much larger, lo on
    some) gives bit for bit what one cast_bf16 per buffer gives, and nothing past each buffer."""
    g = _gen(18)
    sizes = [5, 0, 1 << 20, 4099, 262144, 3]
    xs = [(torch.randn(n, generator=g) * 10).to(device) for n in sizes]
    los = [i % 2 == 0 for i in range(len(sizes))]
    his = [torch.full((n + 8,), float('nan'), dtype=torch.bfloat16, device=device) for n in sizes]
    lo_t = [torch.full((n + 8,), float('nan'), dtype=torch.bfloat16, device=device) if l else None
            for n, l in zip(sizes, los)]
    nk.cast_bf16_many([(x, h[:x.numel()], l[:x.numel()] if l is not None else None)
                       for x, h, l in zip(xs, his, lo_t)])
    for x, h, l in zip(xs, his, lo_t):
        n = x.numel()
        h1 = torch.empty(n, dtype=torch.bfloat16, device=device)
        l1 = torch.empty_like(h1)
        if n:
            nk.cast_bf16(x, h1, l1)
        assert torch.equal(h[:n], h1) and torch.isnan(h[n:]).all()
        if l is not None:
            assert torch.equal(l[:n], l1) and torch.isnan(l[n:]).all()


def _gather_layout(shapes):
    widths = [sum(s) for s in shapes.values()]
    padded = [-(-w // 4) * 4 for w in widths]
    return widths, [sum(padded[:k]) for k in range(len(padded))], sum(padded)


def test_pair_gather(device):
    """noise_pair_gather against torch indexing and the oracle's `noise` (eggroll.py:122-128), bit
    for bit, on the model's 60 parameter slices: repeated and out-of-order pairs, the last
    admissible offset, the pad columns (the slice's last value), and NaN for a pair index outside
    the table or a slice past the buffer's end."""
    from noise_amd.config import param_shapes
    from oracle import es_ref
    shapes = dict(param_shapes())
    widths, starts, total = _gather_layout(shapes)
    size, pairs = 1 << 20, 9
    g = _gen(21)
    buf = torch.randn(size, generator=g).to(device)
    offs = {n: torch.randint(0, size - w, (pairs,), generator=g) for n, w in zip(shapes, widths)}
    offs['lm_head.weight'][2] = size - widths[list(shapes).index('lm_head.weight')]  # ends at the last float
    table = torch.stack(list(offs.values())).to(device)
    dirs = torch.tensor([0, 8, 2, 2, 5], device=device)
    out = torch.full((dirs.numel(), total + 8), 7.0, device=device)
    nk.pair_gather(buf, table, dirs, widths, starts, out)
    ref = es_ref.noise(buf.cpu(), offs, shapes, dirs.cpu())
    got = out.cpu()
    for (name, shape), st, w in zip(shapes.items(), starts, widths):
        v = ref[name]
        want = torch.cat(v, 1) if isinstance(v, tuple) else v
        assert torch.equal(got[:, st:st + w], want), name
        pw = -(-w // 4) * 4
        assert torch.equal(got[:, st + w:st + pw], want[:, -1:].expand(-1, pw - w)), name  # pad columns
    assert (got[:, total:] == 7.0).all()  # nothing past the layout
    # a pair index outside [0, pairs), a slice past the buffer: NaN rows / columns, no read
    bad = table.clone()
    bad[0, 1] = size - 4  # resid_lambdas (8 wide) would end 4 floats past the buffer
    dirs2 = torch.tensor([1, pairs, -1], device=device)
    out2 = torch.zeros(3, total, device=device)
    nk.pair_gather(buf, bad, dirs2, widths, starts, out2)
    o2 = out2.cpu()
    assert torch.isnan(o2[0, :8]).all() and not torch.isnan(o2[0, 8:]).any()
    assert torch.isnan(o2[1:]).all()
    with pytest.raises(ValueError):
        nk.pair_gather(buf, table, dirs, widths, [s + 1 for s in starts], out)  # misaligned columns


def test_pair_rows_match_noise(device):
    """Eggroll's per-chunk gather (the HIP kernel) against Eggroll.noise, the reference's slicing,
    on the device buffer and the device generator's offsets of a step."""
    from noise_amd import make_model
    from noise_amd.eggroll import Eggroll
    model = make_model(device, 0)
    es = Eggroll(model, 6)
    offsets = es.offsets(3)
    table = torch.stack([offsets[n] for n in es.shapes])
    dirs = torch.tensor([5, 0, 3, 3, 1], device=device)
    rows = es._pair_rows(table, dirs)
    ref = es.noise(offsets, dirs)
    for name, v in ref.items():
        r = rows[name]
        if isinstance(v, (tuple, list)):
            assert torch.equal(r.a, v[0]) and torch.equal(r.b, v[1]), name
        else:
            assert torch.equal(r.eps, v), name


def test_fitness_gradient_adamw(device):
    from oracle import es_ref
    g = _gen(9)
    pairs, out, inn = 37, 70, 90
    losses = torch.randn(2 * pairs, generator=g) + 8
    w_ref, n = es_ref.fitness(losses.double(), pairs)
    w = torch.empty(pairs, device=device)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    nk.fitness(losses.to(device), pairs, w, status)
    torch.testing.assert_close(w.cpu().double(), w_ref, rtol=1e-5, atol=1e-5)
    assert int(status.item()) == 0
    bad = losses.clone()
    bad[3] = float('inf')
    nk.fitness(bad.to(device), pairs, w, status)
    assert int(status.item()) == _lib.NOISE_ENONFINITE

    buf = torch.randn(10000, generator=g)
    off = torch.randint(0, 10000 - out - inn, (pairs,), generator=g)
    w_in = torch.randn(pairs, generator=g)
    a = torch.stack([buf[o:o + out] for o in off.tolist()])
    b = torch.stack([buf[o + out:o + out + inn] for o in off.tolist()])
    ref = es_ref.gradient(w_in.double(), {'m': (a, b), 'v': a[:, :8]}, n)
    G = torch.empty(out, inn, device=device)
    dbuf, doff = buf.to(device), off.to(device)
    nk.es_gradient(w_in.to(device), dbuf, doff, dbuf, doff + out, out, inn, -1.0 / n, G)
    torch.testing.assert_close(G.cpu().double(), ref['m'], rtol=1e-5, atol=1e-6)
    Gv = torch.empty(8, device=device)
    nk.es_gradient(w_in.to(device), dbuf, doff, None, None, 8, 1, -1.0 / n, Gv)
    torch.testing.assert_close(Gv.cpu().double(), ref['v'], rtol=1e-5, atol=1e-6)

    p0 = torch.randn(1000, generator=g)
    refp = p0.clone().requires_grad_(True)
    opt = torch.optim.AdamW([refp], lr=1e-3, betas=(0.5, 0.95), eps=1e-8, weight_decay=0.0)
    dp, dm, dv = p0.to(device), torch.zeros(1000, device=device), torch.zeros(1000, device=device)
    for step in range(1, 4):
        grad = torch.randn(1000, generator=g) * 1e-3
        refp.grad = grad.clone()
        opt.step()
        nk.adamw(dp, grad.to(device), dm, dv, 1e-3, 0.5, 0.95, 1e-8, 0.0, step)
    torch.testing.assert_close(dp.cpu(), refp.detach(), rtol=0, atol=1e-6)


def test_adamw_unless_status(device):
    """noise_adamw_unless: with the status at NOISE_OK the same update as noise_adamw, bit for bit;
    with it set (as noise_fitness sets it for a non-finite loss) parameters and moments unchanged."""
    g = _gen(23)
    p0, grad = torch.randn(4099, generator=g), torch.randn(4099, generator=g) * 1e-3
    m0, v0 = torch.randn(4099, generator=g) * 1e-3, torch.rand(4099, generator=g) * 1e-6
    ref = [t.to(device) for t in (p0, m0, v0)]
    nk.adamw(*ref[:1], grad.to(device), *ref[1:], 1e-3, 0.9, 0.95, 1e-8, 0.1, 3)
    for code, want in ((0, ref), (_lib.NOISE_ENONFINITE, [t.to(device) for t in (p0, m0, v0)])):
        st = torch.tensor([code], dtype=torch.int32, device=device)
        got = [t.to(device) for t in (p0, m0, v0)]
        nk.adamw(got[0], grad.to(device), got[1], got[2], 1e-3, 0.9, 0.95, 1e-8, 0.1, 3, unless=st)
        for a, b in zip(got, want):
            assert torch.equal(a, b), code


def test_adamw_state_dict_round_trip(device):
    """noise_amd.AdamW keeps torch.optim.AdamW's state format: after two one-launch steps on a GPT
    whose parameters and gradients tile flat buffers, state_dict() holds every moment and the step;
    an optimizer restored from it takes the same next step bit for bit, torch.optim.AdamW loads the
    same state dict and takes the same step, and the per-parameter path (gradients that do not
    tile) continues from the same moments."""
    import copy
    import noise_amd
    from noise_amd.optim import AdamW
    g = _gen(13)

    def model_with_grads():
        m = noise_amd.make_model(device, 0)
        ps = list(m.parameters())
        flat = torch.empty(sum(p.numel() for p in ps), device=device)
        off = 0
        for p in ps:
            p.grad = flat[off:off + p.numel()].view_as(p)
            off += p.numel()
        return m, ps, flat

    hyper = dict(lr=1e-3, betas=(0.5, 0.95), eps=1e-8, weight_decay=0.01)
    m1, ps1, g1 = model_with_grads()
    opt1 = AdamW(m1.parameters(), **hyper)
    grads = [torch.randn(g1.numel(), generator=g).to(device) * 1e-3 for _ in range(4)]
    for k in range(2):
        g1.copy_(grads[k])
        opt1.step()
    sd = copy.deepcopy(opt1.state_dict())
    assert len(sd['state']) == len(ps1)
    assert all(float(st['step']) == 2 and st['exp_avg'].shape == ps1[i].shape and bool(st['exp_avg_sq'].any())
               for i, st in sd['state'].items())

    m2, ps2, g2 = model_with_grads()
    with torch.no_grad():
        for a, b in zip(ps2, ps1):
            a.copy_(b)
    opt2 = AdamW(m2.parameters(), **hyper)
    opt2.load_state_dict(sd)
    ref = [p.detach().clone().requires_grad_(True) for p in ps1]
    opt_t = torch.optim.AdamW(ref, **hyper)
    opt_t.load_state_dict(copy.deepcopy(sd))
    g1.copy_(grads[2])
    g2.copy_(grads[2])
    opt1.step()
    opt2.step()
    off = 0
    for r in ref:
        r.grad = grads[2][off:off + r.numel()].view_as(r).clone()
        off += r.numel()
    opt_t.step()
    for a, b, r in zip(ps1, ps2, ref):
        assert torch.equal(a, b)
        torch.testing.assert_close(a, r.detach(), rtol=0, atol=1e-6)

    # The per-parameter path (separate gradient tensors) on optimizer 2 follows optimizer 1's flat step.
    for p, gg in zip(ps2, torch.split(grads[3], [p.numel() for p in ps2])):
        p.grad = gg.view_as(p).clone()
    g1.copy_(grads[3])
    opt1.step()
    opt2.step()
    for a, b in zip(ps1, ps2):
        torch.testing.assert_close(a, b, rtol=0, atol=1e-7)


def test_fitness_ranks_bit_exact(device):
    """Centred-rank fitness on 3072 losses (1536 pairs) with planted ties -- equal differences,
    +0.0 / -0.0, duplicated blocks -- bit-exact to the oracle's stable-argsort ranks, including the
    wrap into fewer pair slots and the non-finite status."""
    from oracle import es_ref
    g = _gen(12)
    pairs = 1536
    losses = torch.randn(2 * pairs, generator=g) * 0.01 + 8
    losses[2 * 100 + 1] = losses[2 * 100]                  # f = +0
    losses[2 * 101 + 1], losses[2 * 101] = 8.0, 8.0        # f = 0 again
    losses[2 * 102 + 1], losses[2 * 102] = -0.0, 0.0       # f = -0.0
    losses[2 * 300:2 * 340] = losses[2 * 500:2 * 540]      # 40 duplicated differences
    q = (torch.randint(0, 9, (pairs,), generator=g) * 2 ** -10).float()  # coarse grid: many ties
    losses[1:2 * 900:2][:600] = losses[0:2 * 900:2][:600] + q[:600]
    for slots in (pairs, 1000):
        w_ref, r_ref, n = es_ref.fitness_ranks(losses, slots)
        w = torch.empty(slots, device=device)
        ranked = torch.empty(n, device=device)
        status = torch.full((1,), 7, dtype=torch.int32, device=device)
        nk.fitness(losses.to(device), slots, w, status, mode='ranks', ranked=ranked)
        assert torch.equal(ranked.cpu(), r_ref)
        assert torch.equal(w.cpu(), w_ref)
        assert int(status.item()) == 0
    bad = losses.clone()
    bad[5] = float('nan')
    w = torch.empty(pairs, device=device)
    nk.fitness(bad.to(device), pairs, w, status, mode='ranks', ranked=ranked)
    assert int(status.item()) == _lib.NOISE_ENONFINITE
    _, r_nan, _ = es_ref.fitness_ranks(bad, pairs)
    assert torch.equal(ranked.cpu(), r_nan)  # NaN sorts last, as torch.argsort does


@pytest.mark.parametrize('out,inn', [(512, 512), (70, 90), (300, 1)])
def test_es_gradient_split_pairs(device, out, inn):
    """The gradient with the pair sum split over more workgroups (1536 pairs, as the population
    step has them) against float64 sums, against the one-pass path, and identical on a second call."""
    from oracle import es_ref
    g = _gen(out + inn)
    pairs = 1536
    buf = torch.randn(200000, generator=g)
    off = torch.randint(0, buf.numel() - out - inn, (pairs,), generator=g)
    w_in = torch.randn(pairs, generator=g)
    a = torch.stack([buf[o:o + out] for o in off.tolist()])
    b = torch.stack([buf[o + out:o + out + inn] for o in off.tolist()]) if inn > 1 else None
    ref = es_ref.gradient(w_in.double(), {'m': (a, b) if b is not None else a}, pairs)['m']
    work = torch.empty(max(nk.es_gradient_work(pairs, out, inn), 1), device=device)
    assert nk.es_gradient_work(pairs, out, inn) > 0
    dbuf, doff, dw = buf.to(device), off.to(device), w_in.to(device)
    bb, bo = (dbuf, doff + out) if inn > 1 else (None, None)
    G1, G2, G0 = (torch.empty(out, inn, device=device) for _ in range(3))
    nk.es_gradient(dw, dbuf, doff, bb, bo, out, inn, -1.0 / pairs, G1, work=work)
    nk.es_gradient(dw, dbuf, doff, bb, bo, out, inn, -1.0 / pairs, G2, work=work)
    nk.es_gradient(dw, dbuf, doff, bb, bo, out, inn, -1.0 / pairs, G0)
    torch.testing.assert_close(G1.cpu().double(), ref.reshape(out, inn), rtol=1e-5, atol=1e-6)
    assert torch.equal(G1, G2)
    torch.testing.assert_close(G1, G0, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize('pairs', [1536, 37, 0])
def test_es_gradient_params_one_launch(device, pairs):
    """Every parameter's gradient in one launch (ragged matrices, a vector, one shape spanning many
    tiles) against float64 sums of the reference's noise() slices (eggroll.py:122-128, 155-163);
    bit-identical to the one-pass noise_es_gradient of each; accumulate adds; a slice past the
    buffer's end makes that parameter's gradient NaN and leaves the others finite."""
    from oracle import es_ref
    g = _gen(pairs + 11)
    shapes = [(8,), (70, 90), (512, 512), (300,), (129, 65), (2048, 512)]
    buf = torch.randn(300000, generator=g)
    table = torch.stack([torch.randint(0, buf.numel() - sum(s), (max(pairs, 1),), generator=g) for s in shapes])
    w_in = torch.randn(pairs, generator=g)
    dbuf, dtab, dw = buf.to(device), table.to(device), w_in.to(device)
    grads = [torch.full(s, float('nan'), device=device) for s in shapes]
    nk.es_gradient_params(dw, dbuf, dtab, shapes, grads, -1.0 / max(pairs, 1))
    for k, s in enumerate(shapes):
        rows = torch.stack([buf[o:o + sum(s)] for o in table[k, :pairs].tolist()]) if pairs else \
            torch.zeros(0, sum(s))
        v = (rows[:, :s[0]], rows[:, s[0]:]) if len(s) == 2 else rows
        ref = es_ref.gradient(w_in.double(), {'p': v}, max(pairs, 1))['p']
        torch.testing.assert_close(grads[k].cpu().double(), ref, rtol=1e-5, atol=1e-6)
        if pairs == 0:  # noise_es_gradient takes no empty pair list: the sum is zero
            assert not grads[k].any()
            continue
        one = torch.full(s, float('nan'), device=device)
        off = dtab[k, :pairs].contiguous()
        if len(s) == 2:
            nk.es_gradient(dw, dbuf, off, dbuf, off + s[0], s[0], s[1], -1.0 / max(pairs, 1), one)
        else:
            nk.es_gradient(dw, dbuf, off, None, None, s[0], 1, -1.0 / max(pairs, 1), one)
        assert torch.equal(one, grads[k]), s
    if pairs == 0:
        return
    twice = [t.clone() for t in grads]
    nk.es_gradient_params(dw, dbuf, dtab, shapes, twice, -1.0 / pairs, accumulate=True)
    for a, b in zip(twice, grads):
        torch.testing.assert_close(a, 2 * b, rtol=1e-6, atol=1e-7)
    bad = dtab.clone()
    bad[1, pairs // 2] = buf.numel() - sum(shapes[1]) + 1  # one float past the end
    nk.es_gradient_params(dw, dbuf, bad, shapes, grads, -1.0 / pairs)
    assert torch.isnan(grads[1]).all()
    assert all(torch.isfinite(t).all() for k, t in enumerate(grads) if k != 1)


@pytest.mark.parametrize('window', [1024, 2048])
def test_config2_attention_full_size(device, window):
    """Config 2 at its full shape: q, k, v [256 members, 8 heads, 2048 tokens, 64] ~ N(0, 1) bf16.
    64 sampled (member, head, query) outputs against exact float64 attention over their visible
    keys; the moments of 4 sampled (member, head) pairs against the kernel's own output (mean over
    tokens of y and y^2: an identity independent of size)."""
    members, T = 256, 2048
    M = members * T
    g = torch.Generator(device=device).manual_seed(window)
    qkv = torch.randn(M, 1536, device=device, generator=g).to(torch.bfloat16)
    y = torch.empty(M, 512, dtype=torch.bfloat16, device=device)
    mom = torch.empty(members, 8, 2, 64, device=device)
    scratch = torch.empty(members * 8 * (T // 256) * 128, device=device)
    nk.window_attention(qkv, y, members, T, window, moments=mom, scratch=scratch)
    torch.cuda.synchronize()
    gc = _gen(window + 1)
    ps = torch.randint(0, members, (64,), generator=gc)
    hs = torch.randint(0, 8, (64,), generator=gc)
    ts = torch.randint(0, T, (64,), generator=gc)
    ts[:4] = torch.tensor([0, 1, min(window, T - 1), T - 1])
    for p, h, t in zip(ps.tolist(), hs.tolist(), ts.tolist()):
        lo = max(0, t - window)
        rows = qkv[p * T + lo:p * T + t + 1].double().cpu()
        q = qkv[p * T + t, h * 64:(h + 1) * 64].double().cpu()
        k = rows[:, 512 + h * 64:512 + (h + 1) * 64]
        v = rows[:, 1024 + h * 64:1024 + (h + 1) * 64]
        w = torch.softmax(k @ q / 8.0, 0)
        ref = w @ v
        got = y[p * T + t, h * 64:(h + 1) * 64].double().cpu()
        assert float((got - ref).abs().max()) <= 2e-2 * max(1.0, float(ref.abs().max())), (p, h, t)
    for p, h in [(0, 0), (17, 3), (128, 7), (255, 5)]:
        yy = y[p * T:(p + 1) * T, h * 64:(h + 1) * 64].double().cpu()
        want = torch.stack([yy.mean(0), yy.square().mean(0)])
        torch.testing.assert_close(mom[p, h].double().cpu(), want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize('split', [False, True])
def test_config3_norm_gain_then_head(device, split):
    """Config 3's RMSNorm with a gain ~ U(0.9, 1.1) (F.rms_norm's weight; the reference's own `norm`,
    utils/model.py:46-47, has none): mix_norm with `gain` forms h = bf16(norm(x) gain) and the
    head's dot u = h . b, then the head's CE on h. h against the float64 F.rms_norm within one bf16
    rounding, u and the CE of 256 sampled rows against float64 on the kernel's h; 64 members x 2048
    tokens, perturbed (sigma = 1e-3), Zipf targets."""
    from noise_amd.synthetic import zipf_tokens
    members, T, V = 64, 2048, 4096
    M = members * T
    g = torch.Generator(device=device).manual_seed(31)
    x = torch.randn(M, 512, device=device, generator=g) * 3.0
    gc = _gen(34)
    gain = (torch.rand(512, generator=gc) * 0.2 + 0.9)
    W = torch.randn(V, 512, generator=gc) / math.sqrt(512)
    a = torch.randn(members // 2, V, generator=gc)
    b = torch.randn(members // 2, 512, generator=gc)
    sign = torch.tensor([1e-3, -1e-3]).repeat(members // 2)
    targets = zipf_tokens(T, seed=6)
    h = torch.empty(M, 512, dtype=torch.bfloat16, device=device)
    u = torch.empty(M, 1, device=device)
    nk.mix_norm(x, h, T, sign.to(device), shift=1, bs=(b.to(device),), u=u, gain=gain.to(device))
    hi = torch.empty(V, 512, dtype=torch.bfloat16, device=device)
    lo = torch.empty_like(hi) if split else None
    nk.cast_bf16(W.to(device), hi, lo)
    ce = torch.empty(M, device=device)
    # one target sequence shared by every member (stride 0)
    nk.head_ce(h, hi, lo, T, targets.to(device), ce, sign.to(device), NoiseRows(a=a.to(device), shift=1), u.view(-1))
    torch.cuda.synchronize()
    rows = torch.randint(0, M, (256,), generator=gc)
    xr = x[rows.to(device)].double().cpu()
    want_h = torch.nn.functional.rms_norm(xr, (512,), weight=gain.double(), eps=EPS32)
    closed = xr * torch.rsqrt(xr.square().mean(1, keepdim=True) + EPS32) * gain.double()
    torch.testing.assert_close(want_h, closed, rtol=1e-12, atol=0)  # the weight multiplies the normed rows
    hr = h[rows.to(device)].double().cpu()
    assert float(((hr - want_h).abs() / want_h.abs().clamp_min(1e-30)).max()) <= 2 ** -8
    assert float((hr - want_h.to(torch.bfloat16).double()).abs().gt(0).double().mean()) < 0.01
    p = rows // T
    torch.testing.assert_close(u[rows.to(device), 0].double().cpu(), (hr * b[p // 2].double()).sum(1), rtol=1e-5, atol=1e-4)
    Wd = W.double() if split else W.to(torch.bfloat16).double()
    z = hr @ Wd.t() + (sign[p].double() * u[rows.to(device), 0].double().cpu())[:, None] * a[p // 2].double()
    torch.testing.assert_close(ce[rows.to(device)].double().cpu(), R.softcap_ce(z, targets[rows % T]), rtol=0, atol=5e-5)


@pytest.mark.parametrize('split', [False, True])
def test_config3_head_full_size(device, split):
    """Config 3 at its full shape: h [512 members x 2048 tokens, 512] bf16 N(0, 1) normalised,
    W [4096, 512] fp32 ~ N(0, 1/512) with a rank-1 perturbation (sigma = 1e-3, a, b ~ N(0, 1)),
    Zipf targets. 256 sampled rows against float64 (split: of W itself; else of bf16(W), the
    product of the bf16 head), and the per-member means against the kernel's own per-token losses."""
    from noise_amd.synthetic import zipf_tokens
    members, T, V = 512, 2048, 4096
    M = members * T
    g = torch.Generator(device=device).manual_seed(3)
    h = torch.randn(M, 512, device=device, generator=g)
    h = (h * torch.rsqrt(h.square().mean(1, keepdim=True))).to(torch.bfloat16)
    gc = _gen(33)
    W = torch.randn(V, 512, generator=gc) / math.sqrt(512)
    a = torch.randn(members // 2, V, generator=gc)
    b = torch.randn(members // 2, 512, generator=gc)
    sign = torch.tensor([1e-3, -1e-3]).repeat(members // 2)
    targets = zipf_tokens(T, seed=5)
    db = b.to(device)
    Wd = W.double() if split else W.to(torch.bfloat16).double()
    u = torch.empty(M, device=device)
    for p0 in range(0, members, 64):  # u = h . b of each member's noise row, in slices
        rows = h[p0 * T:(p0 + 64) * T].float().view(64, T, 512)
        u[p0 * T:(p0 + 64) * T] = torch.einsum('ptd,pd->pt', rows, db[torch.arange(p0, p0 + 64, device=device) // 2]).reshape(-1)
    hi = torch.empty(V, 512, dtype=torch.bfloat16, device=device)
    lo = torch.empty_like(hi) if split else None
    nk.cast_bf16(W.to(device), hi, lo)
    ce = torch.empty(M, device=device)
    nk.head_ce(h, hi, lo, T, targets.to(device), ce, sign.to(device), NoiseRows(a=a.to(device), shift=1), u)
    losses = torch.empty(members, device=device)
    nk.member_mean(ce, members, T, losses)
    torch.cuda.synchronize()
    rows = torch.randint(0, M, (256,), generator=gc)
    hr = h[rows.to(device)].double().cpu()
    p = rows // T
    z = hr @ Wd.t() + (sign[p].double() * u[rows.to(device)].double().cpu())[:, None] * a[p // 2].double()
    ref = R.softcap_ce(z, targets[rows % T])
    torch.testing.assert_close(ce[rows.to(device)].double().cpu(), ref, rtol=0, atol=5e-5)
    torch.testing.assert_close(losses.double().cpu(), ce.double().view(members, T).mean(1).cpu(), rtol=1e-6, atol=1e-6)
    assert float((losses.cpu() - math.log(V)).abs().max()) < 1.0  # near-uniform logits at this scale
