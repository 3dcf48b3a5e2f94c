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


@pytest.mark.parametrize('name', ['proj', 'mlp', 'head', 'attention', 'chain', 'gemm'])
def test_inline_asm_kernels_are_hazard_free(name, tmp_path):
    asm = A.device_asm(B.CSRC / f'{name}.hip', tmp_path)
    assert asm.count('v_mfma') > 0
    assert A.mfma_hazards(asm) == []
    assert A.async_load_touches(asm) == []
    assert A.mfma_result_touches(asm) == []


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
