// Soft-capped log-sum-exp helpers shared by the readout probe kernels: cap(v) = 15 tanh(v / 15).
#pragma once
#include <math.h>

#include "common.h"

namespace noise {

constexpr float CAP_K1 = 0.19235933878519514f;      // 2 log2(e) / 15
constexpr float CAP_K2INV = -0.023104906018664842f; // 1 / (-30 log2(e))
constexpr float CAP_EPS32 = 1.1920928955078125e-07f;  // float32 machine epsilon

// exp(cap(u * inv) - 15) with ik = inv * CAP_K1: exp(-30 / (1 + e^(2 z / 15))), z = u inv, as
// v_exp_f32, v_rcp_f32, v_exp_f32. Every term lies in [e^-30, 1] (the cap's maximum is the shift).
NOISE_DEV float capexp(float u, float ik) {
  const float e = __builtin_amdgcn_exp2f(u * ik);
  return __builtin_amdgcn_exp2f(__builtin_amdgcn_rcpf(fmaf(e, CAP_K2INV, CAP_K2INV)));
}

NOISE_DEV float cap(float z) { return 15.f * tanhf(z / 15.f); }

// e^x - 1 for the small logit changes of the own-query steps: the Taylor series to x^8 / 8! in
// Horner form for |x| <= 0.5 (truncation below 1.1e-8 relative; about 2 ulp measured in float32
// without fma), expf(x) - 1 beyond (no cancellation there: |e^x - 1| >= 0.39).
NOISE_DEV float expm1_series(float x) {
  float r = fmaf(x, 1.f / 40320.f, 1.f / 5040.f);
  r = fmaf(x, r, 1.f / 720.f);
  r = fmaf(x, r, 1.f / 120.f);
  r = fmaf(x, r, 1.f / 24.f);
  r = fmaf(x, r, 1.f / 6.f);
  r = fmaf(x, r, 0.5f);
  r = fmaf(x, r, 1.f);
  return r * x;
}

NOISE_DEV float expm1_small(float x) { return fabsf(x) <= 0.5f ? expm1_series(x) : expf(x) - 1.f; }

// The same on 16 values with one branch: the series everywhere, then expf(x) - 1 where |x| > 0.5
// (or NaN) only if some lane of the wave has such a value.
NOISE_DEV floatx16 expm1_small16(floatx16 x) {
  floatx16 r;
  bool big = false;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    r[j] = expm1_series(x[j]);
    big |= !(fabsf(x[j]) <= 0.5f);
  }
  if (big) {
#pragma unroll
    for (int j = 0; j < 16; ++j) r[j] = fabsf(x[j]) <= 0.5f ? r[j] : expf(x[j]) - 1.f;
  }
  return r;
}

// cap(z1) - cap(z0), accurate when z1 is close to z0: tanh(a) - tanh(b) = tanh(a - b)(1 - tanh a tanh b).
NOISE_DEV float cap_difference(float z1, float z0) {
  return 15.f * tanhf((z1 - z0) / 15.f) * (1.f - tanhf(z1 / 15.f) * tanhf(z0 / 15.f));
}

// One wave: sum over the row of exp(cap(row[v] * inv) - 15), V entries (float4 loads if VEC).
template <bool VEC>
NOISE_DEV float row_capexp_sum(const float* row, int V, float inv, int lane) {
  const float ik = inv * CAP_K1;
  float acc = 0.f;
  if constexpr (VEC) {
    for (int v = lane * 4; v < V; v += 256) {
      const float4 b = *reinterpret_cast<const float4*>(row + v);
      acc += (capexp(b.x, ik) + capexp(b.y, ik)) + (capexp(b.z, ik) + capexp(b.w, ik));
    }
  } else {
    for (int v = lane; v < V; v += 64) acc += capexp(row[v], ik);
  }
  return wave_sum(acc);
}

}  // namespace noise
