// Shared device helpers for the gfx950 kernels of libnoise_amd.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "noise_amd.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define NOISE_DEV __device__ __forceinline__

// Round-to-nearest-even float -> bfloat16 bits (v_cvt_pk_bf16_f32 on gfx950).
NOISE_DEV uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
NOISE_DEV float bf2f(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
// Two floats -> packed bf16 pair (lo in bits 0-15), one v_cvt_pk_bf16_f32 with both operands; the
// element-wise form costs two conversions plus a shift and an or.
NOISE_DEV uint32_t pack_bf2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((floatx2){lo, hi}, bf16x2));
}
NOISE_DEV float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
NOISE_DEV float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

NOISE_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

NOISE_DEV float group_sum(float v, int width) {
  for (int o = width >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Sum over the 32 lanes of each half-wave of 64 per-lane values; lane q of a half ends with the
// totals of values 2q and 2q+1 (62 exchanges instead of 5 x 64 for a butterfly per value).
NOISE_DEV void halfwave_transpose_sum(float (&v)[64], int lane) {
  const int q = lane & 31;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const bool up = q & 16;
    float send = up ? v[i] : v[i + 32];
    float keep = up ? v[i + 32] : v[i];
    v[i] = keep + __shfl_xor(send, 16, 64);
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const bool up = q & 8;
    float send = up ? v[i] : v[i + 16];
    float keep = up ? v[i + 16] : v[i];
    v[i] = keep + __shfl_xor(send, 8, 64);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const bool up = q & 4;
    float send = up ? v[i] : v[i + 8];
    float keep = up ? v[i + 8] : v[i];
    v[i] = keep + __shfl_xor(send, 4, 64);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool up = q & 2;
    float send = up ? v[i] : v[i + 4];
    float keep = up ? v[i + 4] : v[i];
    v[i] = keep + __shfl_xor(send, 2, 64);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const bool up = q & 1;
    float send = up ? v[i] : v[i + 2];
    float keep = up ? v[i + 2] : v[i];
    v[i] = keep + __shfl_xor(send, 1, 64);
  }
}

// Host-side error reporting shared by every entry point (defined in capi.hip).
namespace noise {
int set_error(int status, const char* fmt, ...);
int check_launch(const char* what);
// The row-resident q|k|v projection (proj.hip): launched and true when the shapes allow it.
bool proj_qkv_launch(const uint16_t* A, int64_t lda, const uint16_t* W, int64_t ldw, int M, int K,
                     const noise_rank1_t& r1, const noise_rope_t& rope, hipStream_t stream);
}  // namespace noise

#define NOISE_REQUIRE(cond, ...)                                      \
  do {                                                                \
    if (!(cond)) return noise::set_error(NOISE_EINVAL, __VA_ARGS__);  \
  } while (0)
