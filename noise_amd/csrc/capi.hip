// Error reporting and the small utility entry points of libnoise_amd.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace noise {

static thread_local char g_error[512] = "";

int set_error(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return status;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(NOISE_EHIP, "%s: %s", what, hipGetErrorString(e));
  return NOISE_OK;
}

}  // namespace noise

extern "C" const char* noise_last_error(void) { return noise::g_error; }
extern "C" int noise_abi_version(void) { return 2; }

namespace {
// hi = bf16(x), lo = bf16(x - hi) (lo optional) for the elements i, i + stride, .. of x[0, n), four at
// a time (x 16-byte, hi and lo 8-byte aligned)
__device__ void cast_span(const float* __restrict__ x, int64_t n, uint16_t* __restrict__ hi,
                          uint16_t* __restrict__ lo, int64_t i, int64_t stride) {
  for (; i < n; i += stride) {
    if (i + 4 <= n) {
      float4 v = *reinterpret_cast<const float4*>(x + i);
      float f[4] = {v.x, v.y, v.z, v.w};
      uint16_t h[4], l[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        h[k] = f2bf(f[k]);
        l[k] = f2bf(f[k] - bf2f(h[k]));
      }
      *reinterpret_cast<uint2*>(hi + i) =
          make_uint2(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16));
      if (lo)
        *reinterpret_cast<uint2*>(lo + i) =
            make_uint2(l[0] | ((uint32_t)l[1] << 16), l[2] | ((uint32_t)l[3] << 16));
    } else {
      for (int64_t k = i; k < n; ++k) {
        uint16_t h = f2bf(x[k]);
        hi[k] = h;
        if (lo) lo[k] = f2bf(x[k] - bf2f(h));
      }
    }
  }
}

constexpr int CAST_MAX = 64;
struct CastList {
  const float* x[CAST_MAX];
  uint16_t* hi[CAST_MAX];
  uint16_t* lo[CAST_MAX];
  int64_t n[CAST_MAX];
};
}  // namespace

__global__ void cast_bf16_kernel(const float* __restrict__ x, int64_t n, uint16_t* __restrict__ hi,
                                 uint16_t* __restrict__ lo) {
  cast_span(x, n, hi, lo, ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4, (int64_t)gridDim.x * blockDim.x * 4);
}

// blockIdx.y = the buffer; the blocks along x stride over it
__global__ void cast_bf16_many_kernel(const CastList l) {
  const int k = blockIdx.y;
  cast_span(l.x[k], l.n[k], l.hi[k], l.lo[k], ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4,
            (int64_t)gridDim.x * blockDim.x * 4);
}

extern "C" int noise_cast_bf16(const float* x, int64_t n, uint16_t* hi, uint16_t* lo, void* stream) {
  NOISE_REQUIRE(n >= 0 && x && hi, "cast_bf16: bad arguments (n=%lld)", (long long)n);
  NOISE_REQUIRE(((uintptr_t)x % 16) == 0 && ((uintptr_t)hi % 8) == 0 && (!lo || ((uintptr_t)lo % 8) == 0),
                "cast_bf16: misaligned buffers");
  if (n == 0) return NOISE_OK;
  int64_t blocks = (n / 4 + 255) / 256 + 1;
  if (blocks > 16384) blocks = 16384;
  cast_bf16_kernel<<<(int)blocks, 256, 0, (hipStream_t)stream>>>(x, n, hi, lo);
  return noise::check_launch("cast_bf16");
}

extern "C" int noise_cast_bf16_many(int count, const float* const* x, const int64_t* n, uint16_t* const* hi,
                                    uint16_t* const* lo, void* stream) {
  NOISE_REQUIRE(count > 0 && count <= CAST_MAX, "cast_bf16_many: count=%d must be in 1..%d", count, CAST_MAX);
  NOISE_REQUIRE(x && n && hi, "cast_bf16_many: null argument");
  CastList l;
  int64_t blocks = 1;
  for (int k = 0; k < count; ++k) {
    uint16_t* lk = lo ? lo[k] : nullptr;
    NOISE_REQUIRE(n[k] >= 0 && (n[k] == 0 || (x[k] && hi[k])), "cast_bf16_many: buffer %d: bad arguments (n=%lld)",
                  k, (long long)n[k]);
    NOISE_REQUIRE(((uintptr_t)x[k] % 16) == 0 && ((uintptr_t)hi[k] % 8) == 0 && ((uintptr_t)lk % 8) == 0,
                  "cast_bf16_many: buffer %d misaligned", k);
    l.x[k] = x[k];
    l.hi[k] = hi[k];
    l.lo[k] = lk;
    l.n[k] = n[k];
    const int64_t b = (n[k] / 4 + 255) / 256 + 1;
    blocks = b > blocks ? b : blocks;
  }
  if (blocks > 512) blocks = 512;
  cast_bf16_many_kernel<<<dim3((unsigned)blocks, (unsigned)count), 256, 0, (hipStream_t)stream>>>(l);
  return noise::check_launch("cast_bf16_many");
}

// One workgroup per member: fixed-order tree sum of its T per-token losses.
__global__ void member_mean_kernel(const float* __restrict__ ce, int T, float* __restrict__ out) {
  __shared__ float part[256];
  const float* row = ce + (int64_t)blockIdx.x * T;
  float s = 0.f;
  for (int t = threadIdx.x; t < T; t += 256) s += row[t];
  part[threadIdx.x] = s;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) part[threadIdx.x] += part[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[blockIdx.x] = part[0] / (float)T;
}

extern "C" int noise_member_mean(const float* ce, int members, int T, float* out, void* stream) {
  NOISE_REQUIRE(ce && out && members >= 0 && T > 0, "member_mean: bad arguments");
  if (members == 0) return NOISE_OK;
  member_mean_kernel<<<members, 256, 0, (hipStream_t)stream>>>(ce, T, out);
  return noise::check_launch("member_mean");
}
