"""Host-side checks that need no GPU: the C ABI library loads and exports what include/noise_amd.h
declares, argument validation rejects bad shapes before anything is launched, and the parameter
container round-trips the fixed model's strict state dict (utils/eval.py:24-31)."""
import ctypes as C
import re
from pathlib import Path

import pytest
import torch

import noise_amd
from noise_amd import _lib
from noise_amd.config import param_shapes

ROOT = Path(__file__).resolve().parents[1]


def header_functions():
    text = (ROOT / 'include' / 'noise_amd.h').read_text()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return sorted(set(re.findall(r'^\s*(?:const\s+)?\w+\*?\s+\*?(noise_\w+)\s*\(', text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = header_functions()
    assert len(declared) >= 12
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_lib.exported_symbols())
    assert lib.noise_abi_version() == 2  # 2: noise_mixnorm_t.gain


def test_argument_errors_raise_before_launch():
    lib = _lib.load()
    # N = 100 is not a multiple of 128: rejected on the host with a ValueError.
    fake = C.c_void_p(256)
    st = lib.noise_lowrank_gemm(fake, 64, fake, 64, 10, 100, 64, None, 0, fake, 100, None, 0, None, 0, None)
    assert st == _lib.NOISE_EINVAL
    with pytest.raises(ValueError, match='multiple of 128'):
        _lib.check(st)
    st = lib.noise_embed_norm(fake, 500, 4096, 500, fake, 0, 8, 1, None, None, 0, None, 0, 0, fake, None, None)
    assert st == _lib.NOISE_EINVAL
    st = lib.noise_fitness(fake, 7, 3, fake, None, None)
    assert st == _lib.NOISE_EINVAL
    st = lib.noise_adamw(fake, fake, fake, fake, 10, 1e-3, 0.9, 0.99, 1e-8, 0.0, 0, None)
    assert st == _lib.NOISE_EINVAL
    with pytest.raises(FloatingPointError):
        _lib.check(_lib.NOISE_ENONFINITE)
    # Probe entry points: a non-positive sigma, short row strides and a NULL C are rejected; an
    # empty batch is a no-op.
    y = C.c_void_p(512)
    assert lib.noise_coordinate_differences(fake, 0, 64, y, 4, 64, 0.0, fake, 64, None) == _lib.NOISE_EINVAL
    assert lib.noise_coordinate_differences(fake, 0, 32, y, 4, 64, 0.1, fake, 64, None) == _lib.NOISE_EINVAL
    assert lib.noise_coordinate_differences(fake, 0, 64, y, 0, 64, 0.1, fake, 64, None) == _lib.NOISE_OK
    a = _lib.Probe(base=256, ld_base=32, C=256, ld_C=64, y=512, steps=256, sq=256, dots=256, ld_dots=8,
                   dir_sq=256, n=4, P=8, K=0, V=64, width=512, clean_sum=256, out=256, ld_out=8)
    assert lib.noise_cycle_derivatives(C.byref(a), None) == _lib.NOISE_EINVAL      # ld_base < V
    a.n = 0
    assert lib.noise_cycle_derivatives(C.byref(a), None) == _lib.NOISE_OK
    a.n, a.ld_base, a.K = 4, 64, 3
    assert lib.noise_row_derivatives(C.byref(a), None) == _lib.NOISE_EINVAL        # rows is NULL
    with pytest.raises(ValueError, match='rows'):
        _lib.check(_lib.NOISE_EINVAL)
    # Own-query step: width not 64 per head, K outside [1, 64], a NULL key set; m = 0 is a no-op.
    q = _lib.ChainQuery(delta=256, x=256, pos=512, w_q=256, top_keys=256, top_values=256, top_p=256, rest=256,
                        w_proj_t=256, cos_t=256, sin_t=256, T=16, m=2, P=4, W=512, heads=4, K=8, a3=256, dr=256,
                        wq3=256, wp3=256)
    assert lib.noise_chain_query(C.byref(q), None) == _lib.NOISE_EINVAL            # W != 64 heads
    q.heads, q.K = 8, 65
    assert lib.noise_chain_query(C.byref(q), None) == _lib.NOISE_EINVAL            # K > 64
    q.K, q.top_keys = 64, None
    assert lib.noise_chain_query(C.byref(q), None) == _lib.NOISE_EINVAL            # NULL keys
    with pytest.raises(ValueError, match='NULL'):
        _lib.check(_lib.NOISE_EINVAL)
    q.m = 0
    assert lib.noise_chain_query(C.byref(q), None) == _lib.NOISE_OK
    w = _lib.ChainQueryWindow(delta=256, x=256, pos=512, rel=512, w_q=256, keys=256, values=256, w_proj_t=256,
                              cos_t=256, sin_t=256, T=16, m=2, P=4, W=512, heads=8, S=32, window=4096, a3=256,
                              dr=256, wq3=256, wp3=256)
    assert lib.noise_chain_query_window(C.byref(w), None) == _lib.NOISE_EINVAL   # window + 1 > 4096 keys
    w.window, w.rel = 1024, None
    assert lib.noise_chain_query_window(C.byref(w), None) == _lib.NOISE_EINVAL   # NULL rel
    w.m = 0
    assert lib.noise_chain_query_window(C.byref(w), None) == _lib.NOISE_OK
    # es_gradient: a workspace size without a workspace is rejected; the split sizing rule gives
    # up to 16 pair splits per 64 x 64 tile and none for a handful of pairs.
    assert lib.noise_es_gradient(fake, 1536, fake, fake, fake, fake, 512, 512, -1.0, 0, fake, None, 10,
                                 None) == _lib.NOISE_EINVAL
    assert lib.noise_es_gradient_work(1536, 512, 512) == 16 * 512 * 512
    assert lib.noise_es_gradient_work(1536, 4096, 512) == 4 * 4096 * 512
    assert lib.noise_es_gradient_work(37, 70, 90) == 0
    assert lib.noise_es_gradient_work(0, 70, 90) == 0


def _rejects(st, match):
    assert st == _lib.NOISE_EINVAL
    with pytest.raises(ValueError, match=match):
        _lib.check(st)


def test_step_entry_points_reject_bad_arguments():
    """Every entry point of the population step validates its arguments on the host: each call
    here is either refused before any device call or an empty batch that returns at once (the
    pointers are placeholders that no call dereferences)."""
    lib = _lib.load()
    fake, odd = 256, 264  # 16-byte aligned; 8-byte but not 16-byte aligned

    head = _lib.Head(h=fake, w_hi=fake, M=1024, V=100, T=256, targets=fake, targets_stride=256, ce=fake,
                     ignore_index=-1)
    _rejects(lib.noise_head_ce(C.byref(head), None), 'multiple of 64')
    head.V, head.T = 192, 300  # V % 64 == 0, but the ragged rows take the tile kernel (V % 256)
    _rejects(lib.noise_head_ce(C.byref(head), None), 'multiple of 256')
    head.V, head.T, head.ignore_index = 4096, 256, 5
    _rejects(lib.noise_head_ce(C.byref(head), None), 'class index')
    head.ignore_index, head.h = -1, odd
    _rejects(lib.noise_head_ce(C.byref(head), None), '16-byte aligned')
    head.h, head.sign = fake, fake
    _rejects(lib.noise_head_ce(C.byref(head), None), 'perturbation needs')
    head.sign, head.M = None, 0
    assert lib.noise_head_ce(C.byref(head), None) == _lib.NOISE_OK

    mn = _lib.MixNorm(x=fake, M=256, T=256, h=fake, gain=odd)
    _rejects(lib.noise_mix_norm(C.byref(mn), None), 'gain must be 16-byte aligned')
    mn.gain, mn.M = fake, 0
    assert lib.noise_mix_norm(C.byref(mn), None) == _lib.NOISE_OK
    # the fused MLP's epilogue does not take a gain (the reference's norm has none)
    mn.M, mn.T = 512, 256
    mlp_next = _lib.Mlp(in_=fake, ld_in=512, member_stride_in=256 * 512, out=fake, ld_out=512,
                        member_stride_out=256 * 512, T=256, members=2,
                        flags=_lib.MLP_NORM | _lib.MLP_RESIDUAL, w_fc=fake, w_proj=fake, next=C.pointer(mn))
    mn.x = fake
    _rejects(lib.noise_mlp_fused(C.byref(mlp_next), None), 'gain')

    att = _lib.Attention(qkv=fake, ldqkv=1536, y=fake, members=2, T=256, heads=4, window=1024, scale=0.125)
    _rejects(lib.noise_window_attention(C.byref(att), None), 'heads == 8')
    att.heads, att.scale = 8, 0.5
    _rejects(lib.noise_window_attention(C.byref(att), None), 'scale')
    att.scale, att.ldqkv = 0.125, 1540
    _rejects(lib.noise_window_attention(C.byref(att), None), 'ldqkv')
    att.ldqkv, att.moments = 1536, fake
    _rejects(lib.noise_window_attention(C.byref(att), None), 'scratch')
    att.moments, att.members = None, 0
    assert lib.noise_window_attention(C.byref(att), None) == _lib.NOISE_OK

    mlp = _lib.Mlp(in_=fake, ld_in=512, member_stride_in=512 * 256, out=fake, ld_out=512,
                   member_stride_out=512 * 256, T=256, members=2, flags=8, w_fc=fake, w_proj=fake)
    _rejects(lib.noise_mlp_fused(C.byref(mlp), None), 'unknown flags')
    mlp.flags, mlp.in_ = 0, odd
    _rejects(lib.noise_mlp_fused(C.byref(mlp), None), 'aligned')
    mlp.in_, mlp.member_stride_out = fake, 0  # every member would write the same rows
    _rejects(lib.noise_mlp_fused(C.byref(mlp), None), 'overlap')
    mlp.member_stride_out, mlp.member_stride_in = 512 * 256, 0  # in place over shared input rows
    _rejects(lib.noise_mlp_fused(C.byref(mlp), None), 'in-place')
    mlp.out = 1 << 20  # distinct output rows: shared input rows are fine
    mlp.members = 0
    assert lib.noise_mlp_fused(C.byref(mlp), None) == _lib.NOISE_OK
    mlp.out, mlp.member_stride_in, mlp.members = fake, 512 * 256, 2
    mlp.in_, mlp.members = fake, 0
    assert lib.noise_mlp_fused(C.byref(mlp), None) == _lib.NOISE_OK
    _rejects(lib.noise_mlp_pack(None, 0, None, 0, fake, None, None), 'c_fc needs')
    assert lib.noise_mlp_pack(None, 0, None, 0, None, None, None) == _lib.NOISE_OK

    # pair_gather: two parameters of 512 and 100 floats per row, laid out at columns 0 and 512
    # (the second padded to 104), so a row needs 616 columns.
    widths = (C.c_int * 2)(512, 100)

    def gather(starts, n=4, nparams=2, out=fake, ld_out=616):
        return lib.noise_pair_gather(fake, 1 << 28, fake, 8, 8, fake, n, nparams, widths,
                                     (C.c_int * 2)(*starts), out, ld_out, None)

    _rejects(gather((0, 512), nparams=0), 'nparams')
    _rejects(gather((0, 514)), 'pair_gather')      # a start that is not a multiple of 4
    _rejects(gather((0, 256)), 'pair_gather')      # overlapping slices
    _rejects(gather((0, 512), ld_out=600), 'columns')
    _rejects(gather((0, 512), out=odd), '16-byte')
    assert gather((0, 512), n=0) == _lib.NOISE_OK

    _rejects(lib.noise_fitness_ranks(fake, 7, 3, fake, fake, None, None), 'even')
    _rejects(lib.noise_member_mean(fake, 4, 0, fake, None), 'member_mean')
    assert lib.noise_member_mean(fake, 0, 256, fake, None) == _lib.NOISE_OK
    _rejects(lib.noise_cast_bf16(fake + 4, 64, fake, None, None), 'cast_bf16')
    assert lib.noise_cast_bf16(fake, 0, fake, None, None) == _lib.NOISE_OK

    mix = _lib.MixNorm(x=fake, h=fake, M=512, T=256, nb=4)
    _rejects(lib.noise_mix_norm(C.byref(mix), None), 'nb=4')
    mix.nb, mix.u, mix.ldb, mix.ldu = 1, fake, 512, 1
    _rejects(lib.noise_mix_norm(C.byref(mix), None), r'null b\[0\]')
    mix.nb, mix.x0 = 0, fake
    _rejects(lib.noise_mix_norm(C.byref(mix), None), 'lambda scalars')
    mix.x0, mix.M = None, 0
    assert lib.noise_mix_norm(C.byref(mix), None) == _lib.NOISE_OK
    _rejects(lib.noise_embed_mix_norm(fake, 512, 4096, 512, fake, 256, 256, 2, None, None, 0, None, 0, 0, fake,
                                      None, None), 'null mix_norm')

    rope = _lib.Rope(qkv=fake, out=fake, M=512, T=256, cos=fake, sin=fake, gate=fake)
    _rejects(lib.noise_rope_norm_ve(C.byref(rope), None), 'gate needs')
    rope.gate = None
    _rejects(lib.noise_qkv_rope_gemm(fake, 512, fake, 512, 1024, 512, None, C.byref(rope), None), 'must equal')
    rope.M = 0
    assert lib.noise_rope_norm_ve(C.byref(rope), None) == _lib.NOISE_OK

    # The one-launch gradient of many parameters checks its table before launching.
    outs, ins = (C.c_int * 65)(*([512] * 65)), (C.c_int * 65)(*([512] * 65))
    ptrs = (C.c_void_p * 65)(*([fake] * 65))
    _rejects(lib.noise_es_gradient_params(fake, 1536, fake, 1 << 20, fake, 1536, 65, outs, ins, ptrs, -1.0, 0, None),
             'nparams=65')
    _rejects(lib.noise_es_gradient_params(fake, 1536, fake, 1 << 20, fake, 1024, 2, outs, ins, ptrs, -1.0, 0, None),
             'bad sizes')
    ins[1] = 0
    _rejects(lib.noise_es_gradient_params(fake, 1536, fake, 1 << 20, fake, 1536, 2, outs, ins, ptrs, -1.0, 0, None),
             'parameter 1')
    ins[1], ptrs[0] = 512, None
    _rejects(lib.noise_es_gradient_params(fake, 1536, fake, 1 << 20, fake, 1536, 2, outs, ins, ptrs, -1.0, 0, None),
             'parameter 0')

    # The status-guarded AdamW needs its status.
    _rejects(lib.noise_adamw_unless(fake, fake, fake, fake, 10, 1e-3, 0.9, 0.99, 1e-8, 0.0, 1, None, None),
             'null status')

    # The grouped bf16 cast checks its list: at most 64 buffers, each aligned.
    xs, his = (C.c_void_p * 65)(*([fake] * 65)), (C.c_void_p * 65)(*([fake] * 65))
    ns = (C.c_int64 * 65)(*([16] * 65))
    _rejects(lib.noise_cast_bf16_many(65, xs, ns, his, None, None), 'count=65')
    xs[1] = odd
    _rejects(lib.noise_cast_bf16_many(2, xs, ns, his, None, None), 'buffer 1 misaligned')

    # The allocation-free gradient refuses a split that would not fit its fixed array.
    need = lib.noise_es_gradient_work(1536, 4096, 768)
    assert need > lib.noise_es_gradient_noalloc_capacity()
    _rejects(lib.noise_es_gradient_noalloc(fake, 1536, fake, fake, fake, fake, 4096, 768, -1.0, 0, fake, None),
             'beyond the fixed')


def test_state_dict_strict_round_trip():
    a = noise_amd.make_model('cpu', 0)
    sd = a.state_dict()
    assert [(k, tuple(v.shape)) for k, v in sd.items()] == [(n, tuple(s)) for n, s in param_shapes()]
    b = noise_amd.GPT()
    b.load_state_dict(sd, strict=True)
    assert all(torch.equal(b.state_dict()[k], v) for k, v in sd.items())
    assert torch.equal(a.flat, b.flat)
    bad = dict(sd)
    bad.pop('lm_head.weight')
    with pytest.raises(RuntimeError):
        b.load_state_dict(bad, strict=True)
    bad = dict(sd)
    bad['extra.weight'] = torch.zeros(1)
    with pytest.raises(RuntimeError):
        b.load_state_dict(bad, strict=True)


def test_params_tile_one_flat_buffer():
    m = noise_amd.make_model('cpu', 1)
    off = 0
    for name, p in m.named_parameters():
        assert p.data_ptr() == m.flat.data_ptr() + 4 * off, name
        off += p.numel()
    assert off == m.flat.numel() == 37_749_776
    from noise_amd.optim import _flat_base
    base = _flat_base(list(m.parameters()))
    assert base is not None and base.numel() == off and base.data_ptr() == m.flat.data_ptr()


def test_population_loss_rejects_cpu_tensors():
    p = {n: torch.zeros(s) for n, s in param_shapes()}
    with pytest.raises(ValueError, match='GPU'):
        noise_amd.population_loss(None, p, {}, torch.zeros(2), torch.zeros(4, dtype=torch.long),
                                  torch.zeros(4, dtype=torch.long))


def test_eval_rows_and_hash(tmp_path):
    """load_rows (utils/prepare_data.py:39-47): shape check, sha256 of the int32 bytes against the
    pinned digest for a file named in the table, int64 out."""
    from noise_amd import evaluate as E
    x = torch.arange(3 * E.ROW_TOKENS, dtype=torch.int64).view(3, E.ROW_TOKENS) % 4096
    assert E.token_hash(x) == __import__('hashlib').sha256(x.to(torch.int32).numpy().tobytes()).hexdigest()
    torch.save(x.to(torch.int32), tmp_path / 'rows.pt')
    got = E.load_rows(tmp_path / 'rows.pt', 3)
    assert got.dtype == torch.int64 and torch.equal(got, x)
    with pytest.raises(ValueError, match='token tensor'):
        E.load_rows(tmp_path / 'rows.pt', 4)
    torch.save(x, tmp_path / 'val.pt')  # the pinned name, wrong tokens
    with pytest.raises(ValueError, match='sha256 mismatch'):
        E.load_rows(tmp_path / 'val.pt', 3)
    assert torch.equal(E.load_rows(tmp_path / 'val.pt', 3, expected=None), x)
    # contiguous per-rank shards cover every row exactly once, sizes within one
    split = E.TokenSplit(tmp_path / 'val.pt', torch.arange(544 * 2).view(544, 2))
    for world in (1, 3, 8, 7):
        parts = [split.shard(r, world) for r in range(world)]
        assert torch.equal(torch.cat(parts), split.tokens)
        assert max(len(q) for q in parts) - min(len(q) for q in parts) <= 1


def test_eval_cli_rejects_wrong_split(tmp_path):
    """The CLI refuses a split whose sha256 differs from the pinned val.pt, before any GPU work."""
    from noise_amd import evaluate as E
    torch.save(torch.zeros(E.VAL_ROWS, E.ROW_TOKENS, dtype=torch.int32), tmp_path / 'val.pt')
    with pytest.raises(ValueError, match='sha256 mismatch'):
        E.TokenSplit.open(tmp_path / 'val.pt', E.VAL_ROWS)
