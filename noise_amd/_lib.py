"""ctypes binding of libnoise_amd.so (declarations in include/noise_amd.h).

The library is loaded from this package directory only. There is no fallback: if the library is
missing or fails to load, every entry point raises, so the population forward never silently runs
anywhere but the HIP kernels.
"""
import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / 'libnoise_amd.so'

NOISE_OK, NOISE_EINVAL, NOISE_EHIP, NOISE_ENONFINITE = 0, 1, 2, 3
EPI_BF16, EPI_F32, EPI_ADD_F32, EPI_RELU2_BF16 = 0, 1, 2, 3
MLP_NORM, MLP_RESIDUAL = 1, 2

P = C.c_void_p
I64 = C.c_int64
INT = C.c_int
F32 = C.c_float


class Rank1(C.Structure):
    _fields_ = [('sign', P), ('rows_per_member', INT), ('member_shift', INT), ('seg_cols', INT),
                ('nseg', INT), ('u_parts', INT), ('lda', I64), ('ldu', I64),
                ('a', P * 3), ('u', P * 3)]


class MixNorm(C.Structure):
    _fields_ = [('x', P), ('x0', P), ('M', INT), ('T', INT), ('member_shift', INT), ('sign', P),
                ('resid', P), ('mix', P), ('eps_resid', P), ('eps_mix', P), ('ld_eps', I64),
                ('h', P), ('nb', INT), ('b', P * 3), ('ldb', I64), ('u', P), ('ldu', I64),
                ('gate_w', P), ('gate_a', P), ('gate_b', P), ('ld_gate_a', I64), ('ld_gate_b', I64),
                ('gate', P), ('gain', P)]


class Rope(C.Structure):
    _fields_ = [('qkv', P), ('out', P), ('M', INT), ('T', INT), ('member_shift', INT), ('cos', P),
                ('sin', P), ('gate', P), ('ve_table', P), ('idx', P), ('idx_stride', I64), ('vocab', INT), ('sign', P),
                ('ve_a', P), ('ve_b', P), ('ld_ve_a', I64), ('ld_ve_b', I64)]


class Mlp(C.Structure):
    _fields_ = [('in_', P), ('ld_in', I64), ('member_stride_in', I64), ('out', P), ('ld_out', I64),
                ('member_stride_out', I64), ('T', INT), ('members', INT), ('flags', INT), ('w_fc', P),
                ('w_proj', P), ('sign', P), ('member_shift', INT), ('a_fc', P), ('ld_a_fc', I64), ('b_fc', P),
                ('ld_b_fc', I64), ('a_proj', P), ('ld_a_proj', I64), ('b_proj', P), ('ld_b_proj', I64),
                ('next', C.POINTER(MixNorm)), ('attn_y', P), ('ld_attn_y', I64), ('attn_w', P), ('attn_u', P),
                ('ld_attn_u', I64), ('attn_parts', INT), ('attn_a', P), ('ld_attn_a', I64)]


class Attention(C.Structure):
    _fields_ = [('qkv', P), ('ldqkv', I64), ('y', P), ('members', INT), ('T', INT), ('heads', INT),
                ('window', INT), ('scale', F32), ('b_proj', P), ('ld_b_proj', I64), ('member_shift', INT),
                ('u_proj', P), ('moments', P), ('scratch', P)]


class Head(C.Structure):
    _fields_ = [('h', P), ('w_hi', P), ('w_lo', P), ('M', INT), ('V', INT), ('T', INT),
                ('member_shift', INT), ('sign', P), ('a', P), ('lda', I64), ('u', P), ('targets', P),
                ('targets_stride', I64), ('ce', P), ('ignore_index', I64), ('logits', P), ('ld_logits', I64)]


class Probe(C.Structure):
    _fields_ = [('base', P), ('ld_base', I64), ('C', P), ('ld_C', I64), ('rows', P), ('ld_rows', I64),
                ('y', P), ('steps', P), ('sq', P), ('dots', P), ('ld_dots', I64), ('dir_sq', P),
                ('ld_dir_sq', I64), ('n', INT), ('P', INT), ('K', INT), ('V', INT), ('width', INT),
                ('clean_sum', P), ('out', P), ('ld_out', I64)]


class ChainBlock(C.Structure):
    _fields_ = [('delta', P), ('dx0', P), ('mix', INT), ('lam_r', F32), ('lam_0', F32), ('mid', P),
                ('idx', P), ('ld_idx', I64), ('hs', P), ('ld_hs', I64), ('w_fc', P), ('w_out_t', P),
                ('m', INT), ('P', INT), ('W', INT), ('k', INT), ('H', INT),
                ('dz', P), ('wf', P), ('wo', P), ('g', P)]


class ChainQuery(C.Structure):
    _fields_ = [('delta', P), ('dx0', P), ('mix', INT), ('lam_r', F32), ('lam_0', F32), ('x', P), ('pos', P),
                ('w_q', P), ('top_keys', P), ('top_values', P), ('top_p', P), ('rest', P), ('w_proj_t', P),
                ('cos_t', P), ('sin_t', P), ('T', INT), ('m', INT), ('P', INT), ('W', INT), ('heads', INT),
                ('K', INT), ('a3', P), ('dr', P), ('wq3', P), ('wp3', P)]


class ChainQueryWindow(C.Structure):
    _fields_ = [('delta', P), ('dx0', P), ('mix', INT), ('lam_r', F32), ('lam_0', F32), ('x', P), ('pos', P),
                ('rel', P), ('w_q', P), ('keys', P), ('values', P), ('w_proj_t', P), ('cos_t', P), ('sin_t', P),
                ('T', INT), ('m', INT), ('P', INT), ('W', INT), ('heads', INT), ('S', INT), ('window', INT),
                ('a3', P), ('dr', P), ('wq3', P), ('wp3', P)]


class ChainHead(C.Structure):
    _fields_ = [('delta', P), ('xL', P), ('base', P), ('ld_base', I64), ('weight', P), ('target_w', P),
                ('y', P), ('scale', P), ('ld_scale', I64), ('m', INT), ('P', INT), ('W', INT), ('V', INT),
                ('out', P), ('ld_out', I64), ('dbf', P), ('inv', P), ('zy', P), ('clean', P)]


# name -> (restype, argtypes); every function returns an int status.
SIGNATURES = {
    'noise_abi_version': [],
    'noise_lowrank_gemm': [P, I64, P, I64, INT, INT, INT, C.POINTER(Rank1), INT, P, I64, P, I64, P, I64, P],
    'noise_mlp_fused': [C.POINTER(Mlp), P],
    'noise_mlp_pack': [P, I64, P, I64, P, P, P],
    'noise_embed_norm': [P, I64, INT, INT, P, I64, INT, INT, P, P, I64, P, I64, INT, P, P, P],
    'noise_embed_mix_norm': [P, I64, INT, INT, P, I64, INT, INT, P, P, I64, P, I64, INT, P, C.POINTER(MixNorm), P],
    'noise_mix_norm': [C.POINTER(MixNorm), P],
    'noise_rope_norm_ve': [C.POINTER(Rope), P],
    'noise_qkv_rope_gemm': [P, I64, P, I64, INT, INT, C.POINTER(Rank1), C.POINTER(Rope), P],
    'noise_window_attention': [C.POINTER(Attention), P],
    'noise_head_ce': [C.POINTER(Head), P],
    'noise_member_mean': [P, INT, INT, P, P],
    'noise_pair_gather': [P, I64, P, I64, I64, P, INT, INT, P, P, P, I64, P],
    'noise_fitness': [P, INT, INT, P, P, P],
    'noise_fitness_ranks': [P, INT, INT, P, P, P, P],
    'noise_es_gradient': [P, INT, P, P, P, P, INT, INT, F32, INT, P, P, I64, P],
    'noise_es_gradient_work': [INT, INT, INT],
    'noise_es_gradient_params': [P, INT, P, I64, P, I64, INT, P, P, P, F32, INT, P],
    'noise_es_gradient_noalloc': [P, INT, P, P, P, P, INT, INT, F32, INT, P, P],
    'noise_es_gradient_noalloc_capacity': [],
    'noise_adamw': [P, P, P, P, I64, F32, F32, F32, F32, F32, INT, P],
    'noise_adamw_unless': [P, P, P, P, I64, F32, F32, F32, F32, F32, INT, P, P],
    'noise_cast_bf16': [P, I64, P, P, P],
    'noise_cast_bf16_many': [INT, P, P, P, P, P],
    'noise_coordinate_differences': [P, INT, I64, P, INT, INT, F32, P, I64, P],
    'noise_cycle_derivatives': [C.POINTER(Probe), P],
    'noise_row_derivatives': [C.POINTER(Probe), P],
    'noise_chain_start': [P, P, P, INT, INT, INT, F32, P, P, P],
    'noise_chain_block': [C.POINTER(ChainBlock), P],
    'noise_chain_head': [C.POINTER(ChainHead), P],
    'noise_chain_query': [C.POINTER(ChainQuery), P],
    'noise_chain_query_window': [C.POINTER(ChainQueryWindow), P],
}

_lib = None


def load():
    """Load (once) and return the CDLL; raises ImportError if the library is absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(f'{LIB_PATH} is not built; run `python -m noise_amd.build`')
    lib = C.CDLL(str(LIB_PATH))
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = INT
    lib.noise_last_error.argtypes = []
    lib.noise_last_error.restype = C.c_char_p
    lib.noise_es_gradient_work.restype = I64  # a size, not a status
    lib.noise_es_gradient_noalloc_capacity.restype = I64
    _lib = lib
    return lib


def exported_symbols():
    return ['noise_last_error', *SIGNATURES]


def check(status, what=''):
    if status == NOISE_OK:
        return
    msg = load().noise_last_error().decode(errors='replace')
    if what:
        msg = f'{what}: {msg}'
    if status == NOISE_EINVAL:
        raise ValueError(msg)
    if status == NOISE_ENONFINITE:
        raise FloatingPointError(msg)
    raise RuntimeError(msg)


def call(name, *args):
    check(getattr(load(), name)(*args), name)
