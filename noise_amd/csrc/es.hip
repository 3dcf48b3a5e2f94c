// EGGROLL update kernels: fitness -> rank-1 gradient rebuild -> AdamW.
//
// * fitness (train/val/eggroll.py:151-154): f_j = L[2j+1] - L[2j], f /= unbiased std(f) + 1e-8,
//   weight[i] = sum over j with j % pairs == i of f_j. One workgroup, fixed reduction order, so
//   every process that holds the same losses computes bit-identical weights. fitness_ranks: the
//   centred-rank variant of the same differences.
// * es_gradient (eggroll.py:155-163): G = scale * sum_j w_j a_j b_j^T, an fp32 GEMM whose
//   reduction dimension is the pair index; a_j and b_j are addressed through per-pair offsets, so
//   the same kernel reads materialised [pairs, out] noise or slices of one shared noise buffer.
// * adamw (eggroll.py:164-167 with the torch.optim.AdamW of eggroll.py:205): one pass over a flat
//   fp32 parameter buffer.
// * pair_gather (eggroll.py:122-128, `Eggroll.noise`): the perturbation rows of a batch of pairs,
//   every parameter's [out + in] slice of the shared noise buffer side by side in one block.
#include <mutex>

#include "common.h"

namespace {

constexpr int FT = 1024;
__device__ const float kOne = 1.0f;  // the b value of a vector parameter, read like a noise value

NOISE_DEV float block_sum(float v, float* red) {
  const int tid = threadIdx.x;
  red[tid] = v;
  __syncthreads();
  for (int o = FT / 2; o > 0; o >>= 1) {
    if (tid < o) red[tid] += red[tid + o];
    __syncthreads();
  }
  const float r = red[0];
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(FT) void fitness_kernel(const float* __restrict__ losses, int n, int pairs,
                                                     float* __restrict__ weight, int* status) {
  __shared__ float red[FT];
  const int tid = threadIdx.x;
  float s = 0.f, bad = 0.f;
  for (int j = tid; j < n; j += FT) {
    const float lp = losses[2 * j], lm = losses[2 * j + 1];
    if (!isfinite(lp) || !isfinite(lm)) bad = 1.f;
    s += lm - lp;
  }
  const float mean = block_sum(s, red) / (float)n;
  const float nbad = block_sum(bad, red);
  float q = 0.f;
  for (int j = tid; j < n; j += FT) {
    const float d = (losses[2 * j + 1] - losses[2 * j]) - mean;
    q += d * d;
  }
  const float var = block_sum(q, red) / (float)(n - 1);
  const float inv = 1.0f / (sqrtf(var) + 1e-8f);
  for (int i = tid; i < pairs; i += FT) {
    float acc = 0.f;
    for (int j = i; j < n; j += pairs) acc += (losses[2 * j + 1] - losses[2 * j]) * inv;
    weight[i] = acc;
  }
  if (tid == 0 && status) *status = nbad > 0.f ? NOISE_ENONFINITE : NOISE_OK;
}

// Centred-rank fitness: the same antithetic differences f_j = L[2j+1] - L[2j], replaced by
// rank(f_j) / (n - 1) - 0.5 with the rank of a stable ascending sort (ties keep index order, NaN
// sorts after every number), then summed into the pair slots like the z-score. The rank is the
// count #{k : f_k < f_j} + #{k < j : f_k == f_j}, so it equals torch.argsort(stable=True) without
// sorting; the differences stream through LDS in tiles of FT. One workgroup; fixed order.
NOISE_DEV bool rank_before(float a, int ia, float b, int ib) {  // a sorts before b
  const bool na = a != a, nb = b != b;
  if (na || nb) return !na ? true : (!nb ? false : ia < ib);
  return a < b || (a == b && ia < ib);
}

__global__ __launch_bounds__(FT) void fitness_ranks_kernel(const float* __restrict__ losses, int n, int pairs,
                                                           float* __restrict__ weight, float* __restrict__ ranked,
                                                           int* status) {
  __shared__ float tile[FT];
  __shared__ float red[FT];
  const int tid = threadIdx.x;
  float bad = 0.f;
  const float denom = (float)(n > 1 ? n - 1 : 1);
  for (int j0 = 0; j0 < n; j0 += FT) {  // the differences this pass ranks: j0 + tid
    const int j = j0 + tid;
    const float fj = j < n ? losses[2 * j + 1] - losses[2 * j] : 0.f;
    if (j < n && (!isfinite(losses[2 * j]) || !isfinite(losses[2 * j + 1]))) bad = 1.f;
    int rank = 0;
    for (int k0 = 0; k0 < n; k0 += FT) {
      __syncthreads();
      const int k = k0 + tid;
      tile[tid] = k < n ? losses[2 * k + 1] - losses[2 * k] : 0.f;
      __syncthreads();
      const int kn = n - k0 < FT ? n - k0 : FT;
      for (int t = 0; t < kn; ++t) rank += rank_before(tile[t], k0 + t, fj, j) ? 1 : 0;
    }
    if (j < n) ranked[j] = (float)rank / denom - 0.5f;
  }
  const float nbad = block_sum(bad, red);  // its barriers also order the `ranked` writes
  for (int i = tid; i < pairs; i += FT) {
    float acc = 0.f;
    for (int j = i; j < n; j += pairs) acc += ranked[j];
    weight[i] = acc;
  }
  if (tid == 0 && status) *status = nbad > 0.f ? NOISE_ENONFINITE : NOISE_OK;
}

// 64 x 64 output tile per workgroup of 256 threads (four waves of 32 x 32, fp32 MFMA), 32 pairs
// per stage. The next stage's scaled noise goes global -> registers while the current one is
// summed from one of two LDS buffers (one barrier per stage). Every output sums its pairs in a
// fixed order (ascending pairs, two per MFMA).
// With splits > 1, workgroup z sums pairs [z per, (z + 1) per) into its own slice of `partial`
// and es_gradient_reduce_kernel adds the slices in order: the same sums on every run.
__global__ __launch_bounds__(256) void es_gradient_kernel(const float* __restrict__ w, int n,
                                                          const float* __restrict__ a_base,
                                                          const int64_t* __restrict__ a_off,
                                                          const float* __restrict__ b_base,
                                                          const int64_t* __restrict__ b_off, int out,
                                                          int in, float scale, int accumulate,
                                                          float* __restrict__ G, int per,
                                                          float* __restrict__ partial) {
  constexpr int SJ = 32;
  __shared__ __attribute__((aligned(16))) float As[2][SJ][64];
  __shared__ __attribute__((aligned(16))) float Bs[2][SJ][64];
  const int tid = threadIdx.x;
  const int o0 = blockIdx.y * 64, i0 = blockIdx.x * 64;
  // wave (wo, wi) owns the 32 x 32 output block (o0 + 32 wo, i0 + 32 wi): v_mfma_f32_32x32x2_f32,
  // fp32 products and fp32 sums, two pairs per MFMA (lane l: A row l % 32 / B column l % 32 at
  // pair 2 kk + l / 32; accumulator v: row 8 (v / 4) + 4 (l / 32) + v % 4, column l % 32)
  const int lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6), wo = wv >> 1, wi = wv & 1;
  floatx16 acc = {};
  const int jb = blockIdx.z * per, je = min(n, jb + per);  // this workgroup's pairs
  // loader: wave wv fetches pairs wv, wv + 4, .., wv + 28 of a stage, lane = column. Branch-free
  // (the pair index and the columns clamped into range, padding pairs entering with multiplier 0,
  // a missing b read as 1 from kOne), so a stage's loads are in flight together; fetch only issues them and
  // stash, after the stage before has run its MFMAs, applies the multipliers and writes LDS.
  const bool a_col = o0 + lane < out, b_col = b_base ? i0 + lane < in : lane == 0;
  const int ac = a_col ? o0 + lane : out - 1, bc = b_col ? i0 + lane : in - 1;
  float av[8], bv[8], am[8], bm[8];
  auto fetch = [&](int j0) {
    int64_t ao[8], bo[8];
    float wj[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int j = j0 + wv + 4 * e, jc = j < je ? j : je - 1;
      ao[e] = a_off[jc];
      bo[e] = b_base ? b_off[jc] : 0;
      wj[e] = w[jc];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bool live = j0 + wv + 4 * e < je;
      av[e] = a_base[ao[e] + ac];
      bv[e] = *(b_base ? b_base + bo[e] + bc : &kOne);
      am[e] = live ? wj[e] : 0.f;
      bm[e] = live ? 1.0f : 0.f;
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      As[buf][wv + 4 * e][lane] = a_col ? am[e] * av[e] : 0.f;
      Bs[buf][wv + 4 * e][lane] = b_col ? bm[e] * bv[e] : 0.f;
    }
  };
  if (jb < je) fetch(jb);
  for (int j0 = jb, buf = 0; j0 < je; j0 += SJ, buf ^= 1) {
    stash(buf);
    if (j0 + SJ < je) fetch(j0 + SJ);
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < SJ / 2; ++kk)
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(As[buf][2 * kk + (lane >> 5)][wo * 32 + (lane & 31)],
                                                  Bs[buf][2 * kk + (lane >> 5)][wi * 32 + (lane & 31)], acc, 0, 0, 0);
  }
  const int i = i0 + wi * 32 + (lane & 31);
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int o = o0 + wo * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
    if (o >= out || i >= in) continue;
    if (partial) {
      partial[((int64_t)blockIdx.z * out + o) * in + i] = acc[v];
    } else {
      float* dst = G + (int64_t)o * in + i;
      const float x = scale * acc[v];
      *dst = accumulate ? *dst + x : x;
    }
  }
}

__global__ __launch_bounds__(256) void es_gradient_reduce_kernel(const float* __restrict__ partial, int splits,
                                                                 int64_t elems, float scale, int accumulate,
                                                                 float* __restrict__ G) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= elems) return;
  float s = 0.f;
  for (int z = 0; z < splits; ++z) s += partial[z * elems + e];
  const float v = scale * s;
  G[e] = accumulate ? G[e] + v : v;
}

// Pair splits for an (out, in) gradient: enough workgroups to fill the chip (the pair loop of a
// lone workgroup is latency-bound), at least two 32-pair stages each.
int es_splits(int n, int out, int in) {
  const int64_t wgs = (int64_t)((in + 63) / 64) * ((out + 63) / 64);
  int split = (int)((2048 + wgs - 1) / wgs);
  split = split < 16 ? split : 16;
  const int max_by_pairs = n / 64 > 1 ? n / 64 : 1;
  return split < max_by_pairs ? split : max_by_pairs;
}

NOISE_DEV float lerp_torch(float start, float end, float weight) {
  const float diff = end - start;
  return weight < 0.5f ? start + weight * diff : end - diff * (1.0f - weight);
}

__global__ __launch_bounds__(256) void adamw_kernel(float* __restrict__ param, const float* __restrict__ grad,
                                                    float* __restrict__ m, float* __restrict__ v, int64_t n,
                                                    float decay, float w1, float beta2, float w2,
                                                    float step_size, float bc2_sqrt, float eps,
                                                    const int* __restrict__ skip) {
  if (skip && *skip != NOISE_OK) return;  // the caller's status says the gradient is not to be applied
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) {
    const float g = grad[i];
    float p = param[i] * decay;
    const float mi = lerp_torch(m[i], g, w1);
    const float vi = v[i] * beta2 + w2 * g * g;
    const float denom = sqrtf(vi) / bc2_sqrt + eps;
    p = p - step_size * (mi / denom);
    param[i] = p;
    m[i] = mi;
    v[i] = vi;
  }
}

}  // namespace

extern "C" int noise_fitness(const float* losses, int n_losses, int pairs, float* weight, int* status_out,
                             void* stream) {
  NOISE_REQUIRE(losses && weight && pairs > 0, "fitness: bad arguments");
  NOISE_REQUIRE(n_losses >= 2 && n_losses % 2 == 0, "fitness: n_losses=%d must be even and >= 2", n_losses);
  fitness_kernel<<<1, FT, 0, (hipStream_t)stream>>>(losses, n_losses / 2, pairs, weight, status_out);
  return noise::check_launch("fitness");
}

extern "C" int noise_fitness_ranks(const float* losses, int n_losses, int pairs, float* weight, float* ranked,
                                   int* status_out, void* stream) {
  NOISE_REQUIRE(losses && weight && ranked && pairs > 0, "fitness_ranks: bad arguments");
  NOISE_REQUIRE(n_losses >= 2 && n_losses % 2 == 0, "fitness_ranks: n_losses=%d must be even and >= 2", n_losses);
  fitness_ranks_kernel<<<1, FT, 0, (hipStream_t)stream>>>(losses, n_losses / 2, pairs, weight, ranked, status_out);
  return noise::check_launch("fitness_ranks");
}

extern "C" int64_t noise_es_gradient_work(int n, int out, int in) {
  if (n <= 0 || out <= 0 || in <= 0) return 0;
  const int split = es_splits(n, out, in);
  return split > 1 ? (int64_t)split * out * in : 0;
}

extern "C" int noise_es_gradient(const float* w, int n, const float* a_base, const int64_t* a_off,
                                 const float* b_base, const int64_t* b_off, int out, int in, float scale,
                                 int accumulate, float* G, float* work, int64_t work_elems, void* stream) {
  NOISE_REQUIRE(w && a_base && a_off && G && n >= 0 && out > 0 && in > 0, "es_gradient: bad arguments");
  NOISE_REQUIRE(!b_base || b_off, "es_gradient: b_base needs b_off");
  NOISE_REQUIRE(b_base || in == 1, "es_gradient: a vector parameter (no b) needs in == 1");
  NOISE_REQUIRE(work_elems >= 0 && (work || work_elems == 0), "es_gradient: work_elems without work");
  const hipStream_t st = (hipStream_t)stream;
  const int64_t elems = (int64_t)out * in;
  int split = es_splits(n, out, in);
  if (split > 1 && work_elems < split * elems) split = 1;  // no room: one pass over every pair
  const int per = split > 1 ? ((n + split - 1) / split + 31) / 32 * 32 : (n > 0 ? n : 1);
  split = split > 1 ? (n + per - 1) / per : 1;
  dim3 grid((in + 63) / 64, (out + 63) / 64, split);
  NOISE_REQUIRE(grid.y < 65536, "es_gradient: out=%d too large", out);
  es_gradient_kernel<<<grid, 256, 0, st>>>(w, n, a_base, a_off, b_base, b_off, out, in, scale, accumulate, G, per,
                                           split > 1 ? work : nullptr);
  if (int e = noise::check_launch("es_gradient")) return e;
  if (split == 1) return NOISE_OK;
  es_gradient_reduce_kernel<<<(unsigned)((elems + 255) / 256), 256, 0, st>>>(work, split, elems, scale, accumulate,
                                                                             G);
  return noise::check_launch("es_gradient");
}

// ---- allocation-free variant of noise_es_gradient -------------------------------------------
// The split pair sum keeps its partial tiles in `scratch`, a file-scope device array each GPU holds
// for the life of the process. Host code never passes the array's name to a kernel (on the host it
// is only a stand-in for the symbol): the device address comes from hipGetSymbolAddress, once per
// device, with that device current, and is kept per device.
namespace {
constexpr int64_t ES_SCRATCH_FLOATS = int64_t(8) << 20;  // 32 MiB: the 1536-pair split of a [4096, 512] gradient
constexpr int ES_MAX_DEVICES = 64;
__device__ __align__(256) float scratch[ES_SCRATCH_FLOATS];
std::mutex g_scratch_mu;
float* g_scratch_ptr[ES_MAX_DEVICES] = {};

int device_scratch(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return noise::set_error(NOISE_EHIP, "es_gradient_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= ES_MAX_DEVICES)
    return noise::set_error(NOISE_EINVAL, "es_gradient_noalloc: device %d beyond the %d supported", dev, ES_MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return noise::set_error(NOISE_EHIP, "es_gradient_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                              hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return NOISE_OK;
}
}  // namespace

extern "C" int64_t noise_es_gradient_noalloc_capacity(void) { return ES_SCRATCH_FLOATS; }

extern "C" int noise_es_gradient_noalloc(const float* w, int n, const float* a_base, const int64_t* a_off,
                                         const float* b_base, const int64_t* b_off, int out, int in, float scale,
                                         int accumulate, float* G, void* stream) {
  NOISE_REQUIRE(out > 0 && in > 0 && n >= 0, "es_gradient_noalloc: bad arguments");
  const int split = es_splits(n, out, in);
  const int64_t need = split > 1 ? (int64_t)split * out * in : 0;
  NOISE_REQUIRE(need <= ES_SCRATCH_FLOATS,
                "es_gradient_noalloc: %d pairs over a [%d, %d] gradient need %lld scratch floats, beyond the fixed "
                "%lld (use noise_es_gradient with a workspace)",
                n, out, in, (long long)need, (long long)ES_SCRATCH_FLOATS);
  float* work = nullptr;
  if (need > 0)
    if (int rc = device_scratch(&work)) return rc;
  // The same kernels and split as noise_es_gradient with a workspace of `need` floats: every partial
  // tile the reduction reads is written by this call first, so the array needs no clearing.
  return noise_es_gradient(w, n, a_base, a_off, b_base, b_off, out, in, scale, accumulate, G, work, need, stream);
}

// ---- every parameter's gradient in one launch -------------------------------------------------
// One workgroup per 64 x 64 tile of any parameter (parameter k owns tiles tile0[k] .. tile0[k + 1]
// - 1, row-major over its [out, in] grid); each sums all n pairs in one pass, in the order of
// es_gradient_kernel without a split (ascending pairs, two per MFMA, the same products), so
// parameter k's result is bit-identical to noise_es_gradient's one-pass result for it. Pair j's
// noise for parameter k is the slice buffer[o .. o + out + in), o = offsets[k, j]: a_j its first
// out values, b_j the next in (b_j = 1 for a vector parameter, in == 1); a slice outside the
// buffer makes the pair's terms NaN instead of a read.
namespace {
constexpr int GP_MAX = 64;
struct GradLayout {
  float* G[GP_MAX];
  int out[GP_MAX];
  int in[GP_MAX];
  int tiles_x[GP_MAX];
  int tile0[GP_MAX + 1];
};

__global__ __launch_bounds__(256) void es_gradient_params_kernel(const float* __restrict__ w, int n,
                                                                 const float* __restrict__ buffer,
                                                                 int64_t buffer_len,
                                                                 const int64_t* __restrict__ offsets,
                                                                 int64_t ld_offsets, int nparams,
                                                                 const GradLayout lay, float scale,
                                                                 int accumulate) {
  constexpr int SJ = 32;
  __shared__ __attribute__((aligned(16))) float As[2][SJ][64];
  __shared__ __attribute__((aligned(16))) float Bs[2][SJ][64];
  // Consecutive workgroups are dealt to the 8 XCDs in turn; XCD x takes the x-th contiguous run of
  // tiles, so the workgroups sharing an L2 mostly share a parameter and its noise rows.
  const int nb = gridDim.x, bx = blockIdx.x, q = nb >> 3, rem = nb & 7, xcd = bx & 7;
  const int t = xcd * q + (xcd < rem ? xcd : rem) + (bx >> 3);
  int lo = 0, hi = nparams;  // tile0[lo] <= t < tile0[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (lay.tile0[mid] <= t) lo = mid;
    else hi = mid;
  }
  const int k = lo, out = lay.out[k], in = lay.in[k], tt = t - lay.tile0[k];
  const int o0 = (tt / lay.tiles_x[k]) * 64, i0 = (tt % lay.tiles_x[k]) * 64;
  const int64_t* off = offsets + (int64_t)k * ld_offsets;
  const int64_t last = buffer_len - ((int64_t)out + (in > 1 ? in : 0));  // the largest valid slice start
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6), wo = wv >> 1, wi = wv & 1;
  // loader: wave wv fetches pairs wv, wv + 4, .., wv + 28 of a stage, lane = column (each load
  // instruction reads 64 consecutive floats of one pair's row). Branch-free, so that a stage's 16
  // loads are in flight together: the pair index and the columns are clamped into range (the host
  // checks that the buffer holds a slice), a vector parameter's b (the constant 1) is read from
  // kOne like a noise value, and the pair's status enters through its multipliers: 0 past the last
  // pair, NaN for a slice outside the buffer.
  const bool vec = in == 1, a_col = o0 + lane < out, b_col = vec ? lane == 0 : i0 + lane < in;
  const int ac = a_col ? o0 + lane : out - 1;
  const int bc = vec ? 0 : (b_col ? out + i0 + lane : out + in - 1);
  // fetch only issues a stage's loads (and forms its multipliers); stash, after the stage before
  // has run its MFMAs, applies them and writes LDS, so the loads' latency hides under those MFMAs
  float av[8], bv[8], am[8], bm[8];
  auto fetch = [&](int j0) {
    int64_t o[8];
    float wj[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int j = j0 + wv + 4 * e;
      o[e] = off[j < n ? j : n - 1];
      wj[e] = w[j < n ? j : n - 1];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bool live = j0 + wv + 4 * e < n, ok = o[e] >= 0 && o[e] <= last;
      const float* src = buffer + (ok ? o[e] : 0);
      av[e] = src[ac];
      bv[e] = *(vec ? &kOne : src + bc);
      am[e] = !live ? 0.f : ok ? wj[e] : __builtin_nanf("");
      bm[e] = !live ? 0.f : ok ? 1.0f : __builtin_nanf("");
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      As[buf][wv + 4 * e][lane] = a_col ? am[e] * av[e] : 0.f;
      Bs[buf][wv + 4 * e][lane] = b_col ? bm[e] * bv[e] : 0.f;
    }
  };
  floatx16 acc = {};
  if (n > 0) fetch(0);
  for (int j0 = 0, buf = 0; j0 < n; j0 += SJ, buf ^= 1) {
    stash(buf);
    if (j0 + SJ < n) fetch(j0 + SJ);
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < SJ / 2; ++kk)
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(As[buf][2 * kk + (lane >> 5)][wo * 32 + (lane & 31)],
                                                  Bs[buf][2 * kk + (lane >> 5)][wi * 32 + (lane & 31)], acc, 0, 0, 0);
  }
  float* const G = lay.G[k];
  const int i = i0 + wi * 32 + (lane & 31);
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int o = o0 + wo * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
    if (o >= out || i >= in) continue;
    float* dst = G + (int64_t)o * in + i;
    const float x = scale * acc[v];
    *dst = accumulate ? *dst + x : x;
  }
}
}  // namespace

extern "C" int noise_es_gradient_params(const float* w, int n, const float* buffer, int64_t buffer_len,
                                        const int64_t* offsets, int64_t ld_offsets, int nparams, const int* outs,
                                        const int* ins, float* const* grads, float scale, int accumulate,
                                        void* stream) {
  NOISE_REQUIRE((w || n == 0) && buffer && offsets && outs && ins && grads, "es_gradient_params: null argument");
  NOISE_REQUIRE(nparams > 0 && nparams <= GP_MAX, "es_gradient_params: nparams=%d must be in 1..%d", nparams, GP_MAX);
  NOISE_REQUIRE(n >= 0 && ld_offsets >= n && buffer_len > 0,
                "es_gradient_params: bad sizes (n=%d ld_offsets=%lld buffer_len=%lld)", n, (long long)ld_offsets,
                (long long)buffer_len);
  GradLayout lay;
  int64_t tiles = 0;
  for (int k = 0; k < nparams; ++k) {
    NOISE_REQUIRE(grads[k] && outs[k] > 0 && ins[k] > 0, "es_gradient_params: parameter %d: [%d, %d] at %p", k,
                  outs[k], ins[k], (void*)grads[k]);
    NOISE_REQUIRE((int64_t)outs[k] + (ins[k] > 1 ? ins[k] : 0) <= buffer_len,
                  "es_gradient_params: parameter %d: a [%d, %d] slice is longer than the buffer (%lld)", k, outs[k],
                  ins[k], (long long)buffer_len);
    lay.G[k] = grads[k];
    lay.out[k] = outs[k];
    lay.in[k] = ins[k];
    lay.tiles_x[k] = (ins[k] + 63) / 64;
    lay.tile0[k] = (int)tiles;
    tiles += (int64_t)lay.tiles_x[k] * ((outs[k] + 63) / 64);
    NOISE_REQUIRE(tiles < (int64_t)1 << 31, "es_gradient_params: more than 2^31 tiles");
  }
  for (int k = nparams; k <= GP_MAX; ++k) lay.tile0[k] = (int)tiles;
  es_gradient_params_kernel<<<(unsigned)tiles, 256, 0, (hipStream_t)stream>>>(w, n, buffer, buffer_len, offsets,
                                                                               ld_offsets, nparams, lay, scale,
                                                                               accumulate);
  return noise::check_launch("es_gradient_params");
}

// One workgroup per (parameter k, pair row d): out[d, start_k + i] = buffer[o + min(i, w_k - 1)]
// for i < pad4(w_k), o = offsets[k, directions[d]] -- a contiguous slice copied with coalesced
// 4-byte reads (o is any index) into a 16-byte-aligned column range. Indices that fall outside
// the buffer or the offsets table give NaN columns instead of a read.
constexpr int PG_MAX = 64;
struct PairLayout {
  int widths[PG_MAX];
  int starts[PG_MAX];
};

__global__ __launch_bounds__(256) void pair_gather_kernel(const float* __restrict__ buffer, int64_t buffer_len,
                                                          const int64_t* __restrict__ offsets, int64_t ld_offsets,
                                                          int64_t pairs, const int64_t* __restrict__ directions,
                                                          const PairLayout lay, float* __restrict__ out,
                                                          int64_t ld_out) {
  const int k = blockIdx.x, d = blockIdx.y;
  const int w = lay.widths[k], pw = (w + 3) & ~3;
  const int64_t dir = directions[d];
  const bool dir_ok = dir >= 0 && dir < pairs;
  const int64_t o = dir_ok ? offsets[k * ld_offsets + dir] : -1;
  const bool ok = dir_ok && o >= 0 && o + w <= buffer_len;
  float* dst = out + (int64_t)d * ld_out + lay.starts[k];
  for (int i = threadIdx.x; i < pw; i += 256) dst[i] = ok ? buffer[o + (i < w ? i : w - 1)] : __builtin_nanf("");
}

extern "C" int noise_pair_gather(const float* buffer, int64_t buffer_len, const int64_t* offsets,
                                 int64_t ld_offsets, int64_t pairs, const int64_t* directions, int n,
                                 int nparams, const int* widths, const int* starts, float* out, int64_t ld_out,
                                 void* stream) {
  NOISE_REQUIRE(buffer && offsets && directions && out && widths && starts, "pair_gather: null argument");
  NOISE_REQUIRE(nparams > 0 && nparams <= PG_MAX, "pair_gather: nparams=%d must be in 1..%d", nparams, PG_MAX);
  NOISE_REQUIRE(n >= 0 && n < 65536 && pairs > 0 && ld_offsets >= pairs && buffer_len > 0,
                "pair_gather: bad sizes (n=%d pairs=%lld ld_offsets=%lld)", n, (long long)pairs,
                (long long)ld_offsets);
  NOISE_REQUIRE(((uintptr_t)out % 16) == 0 && ld_out % 4 == 0, "pair_gather: out rows must be 16-byte aligned");
  PairLayout lay;
  int64_t end = 0;
  for (int k = 0; k < nparams; ++k) {
    NOISE_REQUIRE(widths[k] > 0 && starts[k] >= end && starts[k] % 4 == 0,
                  "pair_gather: parameter %d: width %d at column %d (columns must be 4-aligned, in order, disjoint)",
                  k, widths[k], starts[k]);
    end = (int64_t)starts[k] + ((widths[k] + 3) & ~3);
    lay.widths[k] = widths[k];
    lay.starts[k] = starts[k];
  }
  NOISE_REQUIRE(end <= ld_out, "pair_gather: the layout needs %lld columns, ld_out=%lld", (long long)end,
                (long long)ld_out);
  if (n == 0) return NOISE_OK;
  pair_gather_kernel<<<dim3(nparams, n), 256, 0, (hipStream_t)stream>>>(buffer, buffer_len, offsets, ld_offsets, pairs,
                                                                       directions, lay, out, ld_out);
  return noise::check_launch("pair_gather");
}

static int adamw_launch(float* param, const float* grad, float* exp_avg, float* exp_avg_sq, int64_t n, float lr,
                        float beta1, float beta2, float eps, float weight_decay, int step, const int* skip,
                        void* stream) {
  NOISE_REQUIRE(param && grad && exp_avg && exp_avg_sq && n >= 0, "adamw: bad arguments");
  NOISE_REQUIRE(step >= 1, "adamw: step=%d must count from 1", step);
  if (n == 0) return NOISE_OK;
  const double bias1 = 1.0 - __builtin_pow((double)beta1, step);
  const double bias2 = 1.0 - __builtin_pow((double)beta2, step);
  const float step_size = (float)(lr / bias1);
  const float bc2_sqrt = (float)__builtin_sqrt(bias2);
  int64_t blocks = (n + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  adamw_kernel<<<(int)blocks, 256, 0, (hipStream_t)stream>>>(param, grad, exp_avg, exp_avg_sq, n,
                                                              1.0f - lr * weight_decay, 1.0f - beta1, beta2,
                                                              1.0f - beta2, step_size, bc2_sqrt, eps, skip);
  return noise::check_launch("adamw");
}

extern "C" int noise_adamw(float* param, const float* grad, float* exp_avg, float* exp_avg_sq, int64_t n,
                           float lr, float beta1, float beta2, float eps, float weight_decay, int step,
                           void* stream) {
  return adamw_launch(param, grad, exp_avg, exp_avg_sq, n, lr, beta1, beta2, eps, weight_decay, step, nullptr, stream);
}

extern "C" int noise_adamw_unless(float* param, const float* grad, float* exp_avg, float* exp_avg_sq, int64_t n,
                                  float lr, float beta1, float beta2, float eps, float weight_decay, int step,
                                  const int* status, void* stream) {
  NOISE_REQUIRE(status, "adamw_unless: null status");
  return adamw_launch(param, grad, exp_avg, exp_avg_sq, n, lr, beta1, beta2, eps, weight_decay, step, status, stream);
}
