// Soft-capped log-sum-exp probes of the readout head (train/val/run.py:100-111, 154-183;
// train/speedrun/run.py:57-68, 90-103).
//
// cycle / row derivatives: for token i and direction j, the moved logits are
//   z_v = (base_iv + s_i C_jv) inv_ij,  inv_ij = rsqrt((|x_i|^2 + 2 s_i x_i.D_j + s_i^2 |D_j|^2) / width + eps)
// and the probe needs LSE_v(cap(z_v)) over the whole vocabulary: n * P * V soft-cap exponentials,
// nothing GEMM-shaped, so the kernel is bound by VALU issue. Each element costs
//   u = fma(s, C, base); E = exp2(u * inv * 2 log2(e) / 15); q = rcp(fma(E, c, c)); g = exp2(q); acc += g
// with c = -1 / (30 log2(e)), which gives g = exp(cap(z) - 15) = exp(-30 / (1 + e^(2 z / 15))):
// four full-rate VALU instructions and three quarter-rate transcendentals (v_exp_f32, v_rcp_f32,
// v_exp_f32). The constant shift by 15 (the cap's maximum) keeps every term in [e^-30, 1], so no
// running maximum is needed.
//
// Tiling: a workgroup of four waves owns TI tokens x TJ directions; its waves split the vocabulary
// in chunks of 256 (each lane a float4 of 4 consecutive entries, rows read coalesced straight from
// L2 into registers, the next chunk's loads in flight while this one computes). The per-pair
// scalars (s_i, inv_ij) are wave-uniform and live in SGPRs, so the element loop holds only
// accumulators and loaded rows in VGPRs. A lane-transpose sum then an LDS sum over the four waves
// give one total per pair, and one lane per pair forms
//   out = (log(S_ij / S0_i) - (cap(z_y) - cap(z0_y))) / s_i,
// the clean sums S0 coming from a first launch over the n clean rows. Workgroup ids run over the
// direction tiles fastest, so with a multiple of 8 direction tiles each XCD's L2 holds one eighth
// of C.
#include "softcap.h"

namespace {

using noise::cap;
using noise::cap_difference;
using noise::capexp;
constexpr float K1 = noise::CAP_K1;
constexpr float EPS32 = noise::CAP_EPS32;
constexpr int CHUNK = 256;                      // vocabulary entries per wave per step

NOISE_DEV float uniform(float x) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x)));
}

NOISE_DEV float block_sum256(float v, float* red) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

// Sum over the 64 lanes of N per-lane values (N a power of two <= 64): lane l ends with the total
// of value l >> (6 - log2 N) in v[0].
template <int N>
NOISE_DEV void lanes_transpose_sum(float (&v)[N], int lane) {
  constexpr int LOG2N = __builtin_ctz(N);
#pragma unroll
  for (int k = 0; k < LOG2N; ++k) {
    const int m = 32 >> k, half = (N >> k) / 2;
    const bool up = lane & m;
#pragma unroll
    for (int i = 0; i < half; ++i) {
      // Select between two finished sums rather than between two array slots: a select of slots
      // becomes a lane-dependent index, which would keep v out of registers.
      const float x = v[i] + __shfl_xor(v[i], m, 64);
      const float y = v[i + half] + __shfl_xor(v[i + half], m, 64);
      v[i] = up ? y : x;
    }
  }
#pragma unroll
  for (int k = LOG2N; k < 6; ++k) v[0] += __shfl_xor(v[0], 32 >> k, 64);
}

// ---------------------------------------------------------------- coordinate differences

template <bool BF16>
NOISE_DEV float load_raw(const void* raw, int64_t off) {
  if constexpr (BF16) return bf2f(static_cast<const uint16_t*>(raw)[off]);
  else return static_cast<const float*>(raw)[off];
}

// One workgroup per row: the row's soft-capped LSE, then every coordinate's central difference.
// cap(raw +- sigma) - cap(raw) is formed as +-15 tanh(sigma / 15)(1 - tanh(a +- sigma/15) tanh(a)),
// a = raw / 15, so it keeps its relative accuracy however small it is.
template <bool BF16>
__global__ __launch_bounds__(256) void coordinate_differences_kernel(
    const void* __restrict__ raw, int64_t ld_raw, const int64_t* __restrict__ y, int V, float sigma,
    float step15, float ts, float* __restrict__ out, int64_t ld_out) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int64_t target = y[row];
  float* o = out + row * ld_out;
  if (target < 0) {
    for (int v = threadIdx.x; v < V; v += 256) o[v] = 0.f;
    return;
  }
  const int64_t base = row * ld_raw;
  float s = 0.f;
  for (int v = threadIdx.x; v < V; v += 256) s += expf(cap(load_raw<BF16>(raw, base + v)) - 15.f);
  const float lse = 15.f + logf(block_sum256(s, red));
  const bool bad = target >= V;
  const float inv2s = 0.5f / sigma;
  for (int v = threadIdx.x; v < V; v += 256) {
    const float a = load_raw<BF16>(raw, base + v) / 15.f;
    const float t = tanhf(a);
    const float w = expf(15.f * t - lse);
    const float up = 15.f * ts * (1.f - tanhf(a + step15) * t);
    const float down = -15.f * ts * (1.f - tanhf(a - step15) * t);
    float change = log1pf(w * expm1f(up)) - log1pf(w * expm1f(down));
    if (v == target) change -= up - down;
    o[v] = bad ? __builtin_nanf("") : change * inv2s;
  }
}

// ---------------------------------------------------------------- clean sums

// One wave per token: S0_i = sum_v exp(cap(base_iv inv0_i) - 15).
template <bool VEC>
__global__ __launch_bounds__(256) void clean_sum_kernel(noise_probe_t a) {
  const int lane = threadIdx.x & 63;
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= a.n) return;
  const float inv0 = rsqrtf(a.sq[i] / (float)a.width + EPS32);
  const float acc = noise::row_capexp_sum<VEC>(a.base + (int64_t)i * a.ld_base, a.V, inv0, lane);
  if (lane == 0) a.clean_sum[i] = acc;
}

// ---------------------------------------------------------------- probes

template <int TI, int TJ, bool ROWS, bool VEC>
__global__ __launch_bounds__(256, 2) void probe_kernel(noise_probe_t a, int tiles_j, int64_t tiles,
                                                       int vsplit) {
  constexpr int NP = TI * TJ;              // (token, direction) pairs of a tile
  constexpr int NC = ROWS ? NP : TJ;       // distinct rows of C a tile reads
  static_assert(NP <= 64 && (NP & (NP - 1)) == 0, "pairs per tile: a power of two <= 64");
  __shared__ float part[4][NP];
  __shared__ float pair_ik[4][NP], pair_inv[4][NP];
  __shared__ int pair_row[4][NP];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // vsplit waves share a tile, each taking every vsplit-th chunk of the vocabulary.
  const int sub = wave % vsplit;
  const int64_t tile = (int64_t)blockIdx.x * (4 / vsplit) + wave / vsplit;
  const bool live = tile < tiles;
  const int i0 = live ? (int)(tile / tiles_j) * TI : 0, j0 = live ? (int)(tile % tiles_j) * TJ : 0;
  const int lim = ROWS ? a.K : a.P;

  // Pair scalars, once per wave, so the loop and the epilogue use the same values.
  if (lane < NP) {
    const int p = lane;
    const int gi = min(i0 + p / TJ, a.n - 1), gj = min(j0 + p % TJ, lim - 1);
    const float s = a.steps[gi], sq = a.sq[gi];
    const float dot = a.dots[(int64_t)gi * a.ld_dots + gj];
    const float dsq = ROWS ? a.dir_sq[(int64_t)gi * a.ld_dir_sq + gj] : a.dir_sq[gj];
    const float inv = rsqrtf((sq + 2.f * s * dot + s * s * dsq) / (float)a.width + EPS32);
    pair_inv[wave][p] = inv;
    pair_ik[wave][p] = inv * K1;
    int r = gj;
    if constexpr (ROWS) {
      const int64_t rr = a.rows[(int64_t)gi * a.ld_rows + gj];
      r = (rr >= 0 && rr < a.P) ? (int)rr : -1;
    }
    pair_row[wave][p] = r;
  }
  __syncthreads();

  float s[TI], ik[NP];
  int brow[TI], crow[NC];
#pragma unroll
  for (int i = 0; i < TI; ++i) {
    brow[i] = min(i0 + i, a.n - 1);
    s[i] = uniform(a.steps[brow[i]]);
  }
#pragma unroll
  for (int p = 0; p < NP; ++p) ik[p] = uniform(pair_ik[wave][p]);
#pragma unroll
  for (int c = 0; c < NC; ++c) crow[c] = __builtin_amdgcn_readfirstlane(max(pair_row[wave][c], 0));

  float acc[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) acc[p] = 0.f;

  const int V = a.V;
  const int nch = live ? (V + CHUNK - 1) / CHUNK : 0;
  const float* __restrict__ B = a.base;
  const float* __restrict__ Cm = a.C;

  auto load = [&](int ch, float4 (&bv)[TI], float4 (&cv)[NC]) __attribute__((always_inline)) {
    const int v = ch * CHUNK + lane * 4;
    if constexpr (VEC) {
      const int vv = v < V ? v : 0;
#pragma unroll
      for (int i = 0; i < TI; ++i)
        bv[i] = *reinterpret_cast<const float4*>(B + (int64_t)brow[i] * a.ld_base + vv);
#pragma unroll
      for (int c = 0; c < NC; ++c)
        cv[c] = *reinterpret_cast<const float4*>(Cm + (int64_t)crow[c] * a.ld_C + vv);
    } else {
      float t[4];
#pragma unroll
      for (int i = 0; i < TI; ++i) {
        const float* row = B + (int64_t)brow[i] * a.ld_base;
#pragma unroll
        for (int k = 0; k < 4; ++k) t[k] = row[v + k < V ? v + k : 0];
        bv[i] = make_float4(t[0], t[1], t[2], t[3]);
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const float* row = Cm + (int64_t)crow[c] * a.ld_C;
#pragma unroll
        for (int k = 0; k < 4; ++k) t[k] = row[v + k < V ? v + k : 0];
        cv[c] = make_float4(t[0], t[1], t[2], t[3]);
      }
    }
  };

  auto compute = [&](const float4 (&bv)[TI], const float4 (&cv)[NC]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < TI; ++i) {
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        const int p = i * TJ + j;
        const float4 c = cv[ROWS ? p : j];
        acc[p] += (capexp(fmaf(s[i], c.x, bv[i].x), ik[p]) + capexp(fmaf(s[i], c.y, bv[i].y), ik[p])) +
                  (capexp(fmaf(s[i], c.z, bv[i].z), ik[p]) + capexp(fmaf(s[i], c.w, bv[i].w), ik[p]));
      }
    }
  };

  // Partial chunk (or unaligned rows): entries past V contribute nothing. Their loads read entry 0
  // of the same rows, so the 0/1 weights never meet a value that is not already in the sum.
  auto compute_masked = [&](const float4 (&bv)[TI], const float4 (&cv)[NC], int ch) __attribute__((always_inline)) {
    const int v = ch * CHUNK + lane * 4;
    const float k0 = v < V ? 1.f : 0.f, k1 = v + 1 < V ? 1.f : 0.f;
    const float k2 = v + 2 < V ? 1.f : 0.f, k3 = v + 3 < V ? 1.f : 0.f;
#pragma unroll
    for (int i = 0; i < TI; ++i) {
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        const int p = i * TJ + j;
        const float4 c = cv[ROWS ? p : j];
        acc[p] += (k0 * capexp(fmaf(s[i], c.x, bv[i].x), ik[p]) + k1 * capexp(fmaf(s[i], c.y, bv[i].y), ik[p])) +
                  (k2 * capexp(fmaf(s[i], c.z, bv[i].z), ik[p]) + k3 * capexp(fmaf(s[i], c.w, bv[i].w), ik[p]));
      }
    }
  };

  auto step = [&](const float4 (&bv)[TI], const float4 (&cv)[NC], int ch) __attribute__((always_inline)) {
    if (VEC && (ch + 1) * CHUNK <= V) compute(bv, cv);
    else compute_masked(bv, cv, ch);
  };

  // Chunks sub, sub + vsplit, ...; two register sets alternate, one being filled while the other
  // is consumed. The loads are unconditional (past the wave's last chunk they re-read it), so the
  // only wait before a step is for that step's own loads.
  if (sub < nch) {
    const int last = sub + (nch - 1 - sub) / vsplit * vsplit;
    float4 b0[TI], c0[NC], b1[TI], c1[NC];
    load(sub, b0, c0);
    for (int ch = sub;; ch += 2 * vsplit) {
      load(min(ch + vsplit, last), b1, c1);
      step(b0, c0, ch);
      if (ch + vsplit >= nch) break;
      load(min(ch + 2 * vsplit, last), b0, c0);
      step(b1, c1, ch + vsplit);
      if (ch + 2 * vsplit >= nch) break;
    }
  }

  lanes_transpose_sum<NP>(acc, lane);
  constexpr int SPREAD = 64 / NP;
  if ((lane & (SPREAD - 1)) == 0) part[wave][lane / SPREAD] = acc[0];
  __syncthreads();
  if (!live || sub != 0 || lane >= NP) return;

  const int p = lane;
  const int gi = i0 + p / TJ, gj = j0 + p % TJ;
  if (gi >= a.n || gj >= lim) return;
  float* o = a.out + (int64_t)gi * a.ld_out + gj;
  const int64_t target = a.y[gi];
  if (target < 0) {
    *o = 0.f;
    return;
  }
  const int r = pair_row[wave][p];
  if (target >= V || r < 0) {
    *o = __builtin_nanf("");
    return;
  }
  float S = part[wave][p];
  for (int k = 1; k < vsplit; ++k) S += part[wave + k][p];
  const float S0 = a.clean_sum[gi];
  const float st = a.steps[gi];
  const float inv0 = rsqrtf(a.sq[gi] / (float)a.width + EPS32);
  const float base_y = a.base[(int64_t)gi * a.ld_base + target];
  const float zy = (base_y + st * a.C[(int64_t)r * a.ld_C + target]) * pair_inv[wave][p];
  const float moved_minus_clean = logf(S / S0) - cap_difference(zy, base_y * inv0);
  *o = moved_minus_clean / st;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int probe_launch(const noise_probe_t* a, bool rows, void* stream) {
  const char* what = rows ? "row_derivatives" : "cycle_derivatives";
  NOISE_REQUIRE(a, "%s: args is NULL", what);
  const int lim = rows ? a->K : a->P;
  NOISE_REQUIRE(a->n >= 0 && a->P >= 0 && a->V > 0 && a->width > 0 && (!rows || a->K >= 0),
                "%s: bad sizes (n=%d P=%d K=%d V=%d width=%d)", what, a->n, a->P, a->K, a->V, a->width);
  if (a->n == 0) return NOISE_OK;
  NOISE_REQUIRE(a->base && a->y && a->steps && a->sq && a->clean_sum && a->out,
                "%s: NULL base / y / steps / sq / clean_sum / out", what);
  NOISE_REQUIRE(a->ld_base >= a->V, "%s: ld_base %lld < V %d", what, (long long)a->ld_base, a->V);
  if (lim > 0) {
    NOISE_REQUIRE(a->P > 0 && a->C && a->dots && a->dir_sq, "%s: NULL C / dots / dir_sq or P = 0", what);
    NOISE_REQUIRE(a->ld_C >= a->V && a->ld_dots >= lim && a->ld_out >= lim,
                  "%s: row strides too small (ld_C=%lld ld_dots=%lld ld_out=%lld)", what,
                  (long long)a->ld_C, (long long)a->ld_dots, (long long)a->ld_out);
    NOISE_REQUIRE(!rows || (a->rows && a->ld_rows >= a->K && a->ld_dir_sq >= a->K),
                  "%s: NULL rows or ld_rows / ld_dir_sq < K", what);
  }
  // Tiles: TI tokens x TJ directions (cycle) or one token x 16 of its rows. Waves per tile: enough
  // waves to fill 256 CUs at two waves per SIMD and no more, since every extra wave on a tile adds
  // a transpose sum.
  const int TI = rows ? 1 : 4, TJ = rows ? 16 : 4;
  const int tiles_j = (lim + TJ - 1) / TJ;
  const int64_t tiles = (int64_t)((a->n + TI - 1) / TI) * tiles_j;
  const int vsplit = tiles >= 8192 ? 1 : tiles >= 4096 ? 2 : 4;
  const int64_t blocks = (tiles * vsplit + 3) / 4;
  NOISE_REQUIRE(blocks < (1ll << 31), "%s: too many tiles (%lld)", what, (long long)tiles);

  const bool vec_base = a->V % 4 == 0 && a->ld_base % 4 == 0 && aligned16(a->base);
  const hipStream_t st = (hipStream_t)stream;
  const int cblocks = (a->n + 3) / 4;
  if (vec_base) clean_sum_kernel<true><<<cblocks, 256, 0, st>>>(*a);
  else clean_sum_kernel<false><<<cblocks, 256, 0, st>>>(*a);
  if (int e = noise::check_launch(what)) return e;
  if (lim == 0) return NOISE_OK;
  const bool vec = vec_base && a->ld_C % 4 == 0 && aligned16(a->C);
  const dim3 grid((unsigned)blocks);
  if (rows) {
    if (vec) probe_kernel<1, 16, true, true><<<grid, 256, 0, st>>>(*a, tiles_j, tiles, vsplit);
    else probe_kernel<1, 16, true, false><<<grid, 256, 0, st>>>(*a, tiles_j, tiles, vsplit);
  } else {
    if (vec) probe_kernel<4, 4, false, true><<<grid, 256, 0, st>>>(*a, tiles_j, tiles, vsplit);
    else probe_kernel<4, 4, false, false><<<grid, 256, 0, st>>>(*a, tiles_j, tiles, vsplit);
  }
  return noise::check_launch(what);
}

}  // namespace

extern "C" int noise_coordinate_differences(const void* raw, int raw_is_bf16, int64_t ld_raw,
                                            const int64_t* y, int n, int V, float sigma, float* out,
                                            int64_t ld_out, void* stream) {
  NOISE_REQUIRE(n >= 0 && V > 0, "coordinate_differences: bad sizes (n=%d V=%d)", n, V);
  NOISE_REQUIRE(sigma > 0.f && isfinite(sigma), "coordinate_differences: sigma must be positive");
  if (n == 0) return NOISE_OK;
  NOISE_REQUIRE(raw && y && out, "coordinate_differences: NULL raw / y / out");
  NOISE_REQUIRE(ld_raw >= V && ld_out >= V, "coordinate_differences: row strides below V");
  const float step15 = sigma / 15.f;
  const float ts = (float)tanh((double)sigma / 15.0);
  const hipStream_t st = (hipStream_t)stream;
  if (raw_is_bf16)
    coordinate_differences_kernel<true><<<n, 256, 0, st>>>(raw, ld_raw, y, V, sigma, step15, ts, out, ld_out);
  else
    coordinate_differences_kernel<false><<<n, 256, 0, st>>>(raw, ld_raw, y, V, sigma, step15, ts, out, ld_out);
  return noise::check_launch("coordinate_differences");
}

extern "C" int noise_cycle_derivatives(const noise_probe_t* args, void* stream) {
  return probe_launch(args, false, stream);
}

extern "C" int noise_row_derivatives(const noise_probe_t* args, void* stream) {
  return probe_launch(args, true, stream);
}
