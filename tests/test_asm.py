"""The kernels with inline asm (their own, or the MFMA tiles of mma_tile.h) checked on their gfx950 assembly, on the CPU: see
tests/asm_checks.py for the three properties. A variant that uses none of its prefetched values
(so that the compiler may reuse their registers while the loads are in flight) must fail the
load check, and an asm MFMA whose result the compiler reads at once must fail the result check:
each check sees the failure it exists for."""
import shutil

import pytest

from noise_amd import build as B
from tests import asm_checks as A

pytestmark = pytest.mark.skipif(shutil.which('hipcc') is None and not (B.Path('/opt/rocm/bin/hipcc').exists()),
                                reason='hipcc not available')


@pytest.mark.parametrize('name', ['proj', 'mlp', 'mlp_pc', 'head', 'attention', 'chain', 'gemm'])
def test_inline_asm_kernels_are_hazard_free(name, tmp_path):
    asm = A.device_asm(B.CSRC / f'{name}.hip', tmp_path)
    assert asm.count('v_mfma') > 0
    assert A.mfma_hazards(asm) == []
    assert A.async_load_touches(asm) == []
    assert A.lds_load_touches(asm) == []
    assert A.mfma_result_touches(asm) == []


# Spill budgets (.vgpr_spill_count) of the kernels the population step launches (for the fused MLP
# the step's two instances, with the attention c_proj and the next mix_norm or final norm, and the
# plain one bench.py times alone): the fused MLP spills a few prologue/epilogue values (its waves
# hold 512 registers), its two-wave form (256 registers a wave) some around its edge steps, the
# two-wave q|k|v projection some addresses around its prologue and between its chunk loops, the
# others none or a few; none inside a loop.
SPILL_BUDGET = {'mlp_fused_kernelILb1ELb1ELi2ELb1E': 16, 'mlp_fused_kernelILb1ELb1ELi1ELb1E': 16,
                'mlp_fused_kernelILb1ELb1ELi0ELb0E': 16, 'qkv_proj_kernel': 0, 'window_attention_kernel': 2,
                'qkv_rr_kernelILb0E': 20, 'qkv_rr_kernelILb1E': 24, 'head_rr_kernel': 4,
                'head_ce_kernelILb1ELb0E': 0, 'embed_norm_kernel': 0, 'es_gradient_kernel': 0,
                'es_gradient_params_kernel': 0,
                'mlp_pc_kernel': 128}


@pytest.mark.parametrize('name', ['mlp', 'mlp_pc', 'proj', 'attention', 'head', 'norm', 'es'])
def test_step_kernels_spill_within_budget_and_never_in_a_loop(name, tmp_path):
    asm = A.device_asm(B.CSRC / f'{name}.hip', tmp_path)
    spills = A.kernel_spills(asm)
    checked = 0
    for kernel, n in spills.items():
        for key, budget in SPILL_BUDGET.items():
            if key in kernel:
                assert n <= budget, (kernel, n)
                checked += 1
    assert checked > 0
    loops, bad = A.loop_scratch(asm)
    assert loops > 0 or name == 'norm'  # norm.hip's row kernels are straight-line code
    assert [b for b in bad if any(key in b[0] for key in SPILL_BUDGET)] == []


@pytest.mark.parametrize('name', ['proj', 'head', 'mlp_pc'])
def test_stage_barriers_cover_the_stage(name, tmp_path):
    """The step barriers of the one-ahead pipelines (q|k|v projection, head, two-wave MLP) wait for their stage's
    direct loads, whatever stores or table loads were issued after them."""
    asm = A.device_asm(B.CSRC / f'{name}.hip', tmp_path)
    checked, bad = A.step_barrier_waits(asm)
    assert checked > 0 and bad == []


def test_stage_barrier_check_catches_a_short_wait(tmp_path):
    src = tmp_path / 'short_wait.hip'
    src.write_text('''
#include <hip/hip_runtime.h>
__global__ void k(const float* p, float* o) {
  __shared__ float s[1024];
  __builtin_amdgcn_global_load_lds(p + threadIdx.x * 4, s, 16, 0, 0);
  o[threadIdx.x] = 1.f;
  __asm__ volatile("s_waitcnt vmcnt(2)\\n\\ts_barrier" ::: "memory");
  o[threadIdx.x + 64] = s[threadIdx.x];
}
''')
    asm = A.device_asm(src, tmp_path)
    checked, bad = A.step_barrier_waits(asm)
    assert checked == 1 and bad != []


def test_load_check_catches_reused_destinations(tmp_path):
    # an in-repo stand-in for the failure: asm loads whose results are never used
    src = tmp_path / 'dead_loads.hip'
    src.write_text('''
#include <hip/hip_runtime.h>
typedef float floatx4 __attribute__((ext_vector_type(4)));
__global__ void k(const float* p, float* o, int n) {
  float acc = 0.f;
  for (int i = 0; i < n; ++i) {
    floatx4 dead;
    const float* q = p + (i * 64 + threadIdx.x) * 4;
    __asm__ volatile("global_load_dwordx4 %0, %1, off" : "=v"(dead) : "v"(q));
    acc += q[1024];
  }
  o[threadIdx.x] = acc;
}
''')
    asm = A.device_asm(src, tmp_path)
    assert A.async_load_touches(asm) != []


def test_lds_check_catches_reused_destinations(tmp_path):
    # asm LDS reads whose results are never used: the compiler may hand their registers to other
    # values while the reads are in flight
    src = tmp_path / 'dead_lds.hip'
    src.write_text('''
#include <hip/hip_runtime.h>
typedef float floatx4 __attribute__((ext_vector_type(4)));
__global__ void k(const float* p, float* o, int n) {
  __shared__ float s[4096];
  for (int i = threadIdx.x; i < 4096; i += 64) s[i] = p[i];
  __syncthreads();
  const unsigned a = (unsigned)(unsigned long)(__attribute__((address_space(3))) float*)s + threadIdx.x * 16;
  float acc = 0.f;
  for (int i = 0; i < n; ++i) {
    floatx4 dead;
    __asm__ volatile("ds_read_b128 %0, %1 offset:1024" : "=v"(dead) : "v"(a));
    acc += p[i * 64 + threadIdx.x] * acc + 1.f;
  }
  __asm__ volatile("s_waitcnt lgkmcnt(0)");
  o[threadIdx.x] = acc;
}
''')
    asm = A.device_asm(src, tmp_path)
    assert A.lds_load_touches(asm) != []


def test_loop_scratch_check_catches_spills_in_a_loop(tmp_path):
    # 200 live values per lane at 1024 threads per workgroup: the loop body spills
    src = tmp_path / 'spill_loop.hip'
    src.write_text('''
#include <hip/hip_runtime.h>
__global__ void __launch_bounds__(1024) k(const float* p, float* o, int n) {
  float v[200];
#pragma unroll
  for (int j = 0; j < 200; ++j) v[j] = p[threadIdx.x + j * 1024];
  for (int i = 0; i < n; ++i) {
#pragma unroll
    for (int j = 0; j < 200; ++j) v[j] = v[j] * v[(j + 1) % 200] + p[i * 200 + j];
    __asm__ volatile("" ::: "memory");
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 200; ++j) s += v[j];
  o[threadIdx.x] = s;
}
''')
    asm = A.device_asm(src, tmp_path)
    loops, bad = A.loop_scratch(asm)
    assert loops == 1 and bad != []


def test_result_check_catches_early_reads(tmp_path):
    # an asm MFMA followed at once by compiler code that reads its accumulator
    src = tmp_path / 'early_read.hip'
    src.write_text('''
#include <hip/hip_runtime.h>
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
__global__ void k(const bf16x8* a, float* o) {
  floatx16 acc = {};
  bf16x8 x = a[threadIdx.x];
  __asm__ volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %1, %0" : "+a"(acc) : "v"(x));
  o[threadIdx.x] = acc[0] + acc[15];
}
''')
    asm = A.device_asm(src, tmp_path)
    assert A.mfma_result_touches(asm) != []
