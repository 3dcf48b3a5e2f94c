// Chain moves of the attention-cut estimator with every attention held (train/val/run.py:307-351,
// own = None): moves of one site's stream carried through the later blocks' routed MLPs to the
// head, and the forward difference of each token's soft-capped loss.
//
// Rows are (token i, move p) pairs, row = i * P + p, each W wide. Per chunk:
//   start   (site < 0)  dx0 = norm(e_i + move) - x0_i, delta = (lam_r[0] + lam_0[0]) dx0
//   block b             delta = lam_r[b] delta + lam_0[b] dx0 (after the first block), then
//                       dz = norm(mid_i + delta) - norm(mid_i) in closed form, rounded to bf16;
//                       dh = bf16(dz W_fc[idx_i]^T)      (P x k per token: batched MFMA GEMM)
//                       g = bf16((relu(h + dh) - relu(h)) (relu(h + dh) + relu(h)))
//                       delta += bf16(g W_out_t[idx_i])  (P x W per token: batched MFMA GEMM)
//   head                z = (base_i + bf16(bf16(delta) W^T)) inv, LSE over the vocabulary fused into
//                       the GEMM's epilogue (a workgroup owns 256 rows and sweeps V), minus the
//                       clean LSE, the target term by tanh differences, divided by the step.
// The bf16 roundings are the reference's own (bmm / matmul of bf16 tensors return bf16). The
// gathered weights W_fc[idx_i] (k x W) and W_out_t[idx_i]^T (W x k) are materialised per token,
// as the reference does, so that both routed products are plain K-contiguous MFMA GEMMs.
#include "mma_tile.h"
#include "softcap.h"

namespace {

using noise::CAP_EPS32;
using noise::CAP_K1;

// One wave per row of W (a multiple of 256, at most 2048) floats: lane l holds the float4s at
// 4 l + 256 t, t < W / 256.
constexpr int MAXT = 8;

NOISE_DEV float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
NOISE_DEV void st4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }
NOISE_DEV float dot4(float4 a, float4 b) { return (a.x * b.x + a.y * b.y) + (a.z * b.z + a.w * b.w); }

__global__ __launch_bounds__(256) void chain_start_kernel(const float* __restrict__ e,
                                                          const float* __restrict__ x0,
                                                          const float* __restrict__ move, int rows, int P,
                                                          int W, float mix, float* __restrict__ dx0,
                                                          float* __restrict__ delta) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int64_t i = r / P;
  const int nt = W / 256;
  float4 u[MAXT];
  float sq = 0.f;
#pragma unroll
  for (int t = 0; t < MAXT; ++t)
    if (t < nt) {
      const float4 a = ld4(e + i * W + 4 * lane + 256 * t), b = ld4(move + r * W + 4 * lane + 256 * t);
      u[t] = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
      sq += dot4(u[t], u[t]);
    }
  const float inv = rsqrtf(wave_sum(sq) / (float)W + CAP_EPS32);
#pragma unroll
  for (int t = 0; t < MAXT; ++t)
    if (t < nt) {
      const float4 c = ld4(x0 + i * W + 4 * lane + 256 * t);
      const float4 d = make_float4(u[t].x * inv - c.x, u[t].y * inv - c.y, u[t].z * inv - c.z, u[t].w * inv - c.w);
      st4(dx0 + r * W + 4 * lane + 256 * t, d);
      st4(delta + r * W + 4 * lane + 256 * t, make_float4(mix * d.x, mix * d.y, mix * d.z, mix * d.w));
    }
}

// delta = lam_r delta + lam_0 dx0 (when mix), then dz = norm_difference(mid_i, delta) in bf16
// (train/val/run.py:246-253): delta inv + mid (inv - inv0).
__global__ __launch_bounds__(256) void chain_pre_kernel(float* __restrict__ delta,
                                                        const float* __restrict__ dx0,
                                                        const float* __restrict__ mid, int rows, int P, int W,
                                                        int mix, float lam_r, float lam_0,
                                                        uint16_t* __restrict__ dz) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int64_t i = r / P;
  const int nt = W / 256;
  float4 d[MAXT], x[MAXT];
  float sq = 0.f, dot = 0.f, dsq = 0.f;
#pragma unroll
  for (int t = 0; t < MAXT; ++t)
    if (t < nt) {
      const int64_t o = r * W + 4 * lane + 256 * t;
      float4 v = ld4(delta + o);
      if (mix) {
        const float4 z = dx0 ? ld4(dx0 + o) : make_float4(0.f, 0.f, 0.f, 0.f);
        v = make_float4(lam_r * v.x + lam_0 * z.x, lam_r * v.y + lam_0 * z.y, lam_r * v.z + lam_0 * z.z,
                        lam_r * v.w + lam_0 * z.w);
        st4(delta + o, v);
      }
      d[t] = v;
      x[t] = ld4(mid + i * W + 4 * lane + 256 * t);
      sq += dot4(x[t], x[t]);
      dot += dot4(x[t], v);
      dsq += dot4(v, v);
    }
  sq = wave_sum(sq);
  dot = wave_sum(dot);
  dsq = wave_sum(dsq);
  const float inv0 = rsqrtf(sq / (float)W + CAP_EPS32);
  const float inv = rsqrtf((sq + 2.f * dot + dsq) / (float)W + CAP_EPS32);
  const float dinv = inv - inv0;
#pragma unroll
  for (int t = 0; t < MAXT; ++t)
    if (t < nt) {
      const float4 a = d[t], b = x[t];
      *reinterpret_cast<uint2*>(dz + r * W + 4 * lane + 256 * t) =
          make_uint2(pack_bf2(a.x * inv + b.x * dinv, a.y * inv + b.y * dinv),
                     pack_bf2(a.z * inv + b.z * dinv, a.w * inv + b.w * dinv));
    }
}

// wf[i][kk][:] = w_fc[idx[i][kk]][:]  and  wo[i][n][kk] = w_out_t[idx[i][kk]][n], through LDS in
// blocks of 64 columns, in 16-byte pieces (8 bf16) both ways. An index outside [0, H) gathers NaN.
__global__ __launch_bounds__(256) void chain_gather_kernel(const uint16_t* __restrict__ w_fc,
                                                           const uint16_t* __restrict__ w_out_t,
                                                           const int64_t* __restrict__ idx, int64_t ld_idx,
                                                           int k, int H, int W, uint16_t* __restrict__ wf,
                                                           uint16_t* __restrict__ wo) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[256][72];  // [unit][column], padded rows
  const int64_t i = blockIdx.y;
  const int c0 = blockIdx.x * 64;
  const int tid = threadIdx.x;
  const uint4 NAN8 = make_uint4(0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u);
  for (int kb = 0; kb < k; kb += 256) {
    const int kn = min(256, k - kb);  // a multiple of 8 (k is a multiple of 128)
    for (int e = tid; e < kn * 8; e += 256) {  // unit kk, 8-column piece c8
      const int kk = e >> 3, c8 = (e & 7) * 8;
      const int64_t u = idx[i * ld_idx + kb + kk];
      const bool ok = u >= 0 && u < H;
      const uint4 a = ok ? *reinterpret_cast<const uint4*>(w_fc + u * W + c0 + c8) : NAN8;
      const uint4 b = ok ? *reinterpret_cast<const uint4*>(w_out_t + u * W + c0 + c8) : NAN8;
      *reinterpret_cast<uint4*>(wf + (i * k + kb + kk) * W + c0 + c8) = a;
      *reinterpret_cast<uint4*>(&tile[kk][c8]) = b;
    }
    __syncthreads();
    for (int e = tid; e < 64 * (kn >> 3); e += 256) {  // column c, 8-unit piece k8
      const int c = e / (kn >> 3), k8 = (e % (kn >> 3)) * 8;
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) w[j] = (uint32_t)tile[k8 + 2 * j][c] | ((uint32_t)tile[k8 + 2 * j + 1][c] << 16);
      *reinterpret_cast<uint4*>(wo + (i * W + c0 + c) * k + kb + k8) = make_uint4(w[0], w[1], w[2], w[3]);
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- routed MLP products

// RELUDIFF: G = the relu-square difference of bf16(acc); ADDROUND: delta += bf16(acc); ADD and
// STORE (the own-query step's fp32 products): delta += acc, delta = acc.
constexpr int MODE_RELUDIFF = 0, MODE_ADDROUND = 1, MODE_ADD = 2, MODE_STORE = 3;

struct ChainGemm {
  const uint16_t* A;   // [m * P, K] rows of the batch at i * P
  const uint16_t* B;   // per batch [N, K] at i * N * K
  int P, N, K;
  const float* hs;     // MODE_RELUDIFF: [m, ld_hs] clean pre-activations
  int64_t ld_hs;
  uint16_t* G;         // MODE_RELUDIFF out [m * P, N] bf16
  float* delta;        // MODE_ADDROUND, MODE_ADD in/out, MODE_STORE out [m * P, N] fp32
};

template <int MODE, int BN>
__global__ void __attribute__((amdgpu_flat_work_group_size(2 * BN, 2 * BN), amdgpu_waves_per_eu(2, 2)))
chain_gemm_kernel(const ChainGemm g) {
  constexpr int NSTG = BN == 256 ? 2 : 3, KDEPTH = BN == 256 ? 64 : 32;
  using Cfg = noise::TileCfg<BN, NSTG, KDEPTH>;
  __shared__ __attribute__((aligned(16))) uint16_t smem[Cfg::SMEM_ELEMS];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr int WN = BN / 64;
  const int wm = wave / WN, wn = wave % WN;
  const int64_t i = blockIdx.z;
  const int p0 = blockIdx.x * 256, n0 = blockIdx.y * BN;
  floatx16 acc[4][2];
  noise::zero_acc(acc);
  noise::mma_tile<BN, NSTG, KDEPTH>(g.A + (i * g.P + p0) * g.K, g.K, g.P - p0,
                                    g.B + (i * g.N + n0) * g.K, g.K, g.K, smem, acc);
  if constexpr (MODE == MODE_RELUDIFF) {
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int ni = 0; ni < 2; ++ni) {
        const int col = n0 + wn * 64 + ni * 32 + (lane & 31);
        const float h = g.hs[i * g.ld_hs + col];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int p = p0 + wm * 128 + mi * 32 + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
          if (p >= g.P) continue;
          const float c = bf2f(f2bf(acc[mi][ni][j]));
          const float up = fmaxf(h + c, 0.f), dn = fmaxf(h, 0.f);
          g.G[(i * g.P + p) * g.N + col] = f2bf((up - dn) * (up + dn));
        }
      }
  } else {
    // Four rounds of 64 rows (32 per row half): each wave stages its 32 x 64 block of bf16-rounded
    // products in LDS, then every thread adds float4s of the round's 64 x BN block into delta.
    constexpr int SLD = 68;
    float* stage = reinterpret_cast<float*>(smem);  // [waves][32][SLD]
    constexpr int NT = 2 * BN;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
      for (int j = 0; j < 16; ++j)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
          stage[(wave * 32 + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3)) * SLD + ni * 32 + (lane & 31)] =
              MODE == MODE_ADDROUND ? bf2f(f2bf(acc[mi][ni][j])) : acc[mi][ni][j];
      __syncthreads();
#pragma unroll
      for (int q = 0; q < (64 * BN / 4) / NT; ++q) {
        const int id = q * NT + threadIdx.x, rr = id / (BN / 4), c4 = (id % (BN / 4)) * 4;
        const int h = rr >> 5, r = rr & 31;  // row half (wm) and row within the round
        const int p = p0 + h * 128 + mi * 32 + r;
        if (p < g.P) {
          const float4 v = ld4(stage + ((h * WN + (c4 >> 6)) * 32 + r) * SLD + (c4 & 63));
          float* o = g.delta + (i * g.P + p) * g.N + n0 + c4;
          if constexpr (MODE == MODE_STORE) {
            st4(o, v);
          } else {
            float4 d = ld4(o);
            d.x += v.x; d.y += v.y; d.z += v.z; d.w += v.w;
            st4(o, d);
          }
        }
      }
      if (mi < 3) __syncthreads();
    }
  }
}

// ---------------------------------------------------------------- own-query step

// fp32 operands of the own-query products enter the bf16 MFMA as hi + lo halves: with
// A3 = [a_hi | a_lo | a_hi] and B3 = [b_hi | b_hi | b_lo] along K, A3 B3^T = a_hi b_hi + a_lo b_hi +
// a_hi b_lo, which leaves out only a_lo b_lo (relative 2^-16 per product).
NOISE_DEV void split3(uint16_t* o, int64_t W, int64_t c, float v, bool a_side) {
  const uint16_t hi = f2bf(v), lo = f2bf(v - bf2f(hi));
  o[c] = hi;
  o[W + c] = a_side ? lo : hi;
  o[2 * W + c] = a_side ? hi : lo;
}

// hi and lo bf16 halves of four floats, packed for one 8-byte store each.
NOISE_DEV void split4(float4 v, uint2& hi, uint2& lo) {
  hi = make_uint2(pack_bf2(v.x, v.y), pack_bf2(v.z, v.w));
  lo = make_uint2(pack_bf2(v.x - bf_lo(hi.x), v.y - bf_hi(hi.x)), pack_bf2(v.z - bf_lo(hi.y), v.w - bf_hi(hi.y)));
}

// B3 rows of an fp32 weight read as B[n][k] = w[n * s_n + k * s_k] (N = K = W).
__global__ __launch_bounds__(256) void chain_split_weight_kernel(const float* __restrict__ w, int64_t s_n,
                                                                 int64_t s_k, int W, uint16_t* __restrict__ out) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= (int64_t)W * W) return;
  const int64_t n = e / W, k = e % W;
  split3(out + n * 3 * W, W, k, w[n * s_n + k * s_k], false);
}

// Row r < m P: the optional mix of delta, then A3 of norm_difference(x_i, delta_r) (the query
// product's input, train/val/run.py:294).
__global__ __launch_bounds__(256) void chain_query_pre_kernel(float* __restrict__ delta,
                                                              const float* __restrict__ dx0,
                                                              const float* __restrict__ x, int m, int P, int W,
                                                              int mix, float lam_r, float lam_0,
                                                              uint16_t* __restrict__ a3) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t rows = (int64_t)m * P;
  if (r >= rows) return;
  const int64_t i = r / P;
  const int nt = W / 256;
  float4 d[MAXT], xv[MAXT];
  float sq = 0.f, dot = 0.f, dsq = 0.f;
#pragma unroll
  for (int t = 0; t < MAXT; ++t)
    if (t < nt) {
      const int64_t o = r * W + 4 * lane + 256 * t;
      float4 v = ld4(delta + o);
      if (mix) {
        const float4 z = dx0 ? ld4(dx0 + o) : make_float4(0.f, 0.f, 0.f, 0.f);
        v = make_float4(lam_r * v.x + lam_0 * z.x, lam_r * v.y + lam_0 * z.y, lam_r * v.z + lam_0 * z.z,
                        lam_r * v.w + lam_0 * z.w);
        st4(delta + o, v);
      }
      d[t] = v;
      xv[t] = ld4(x + i * W + 4 * lane + 256 * t);
      sq += dot4(xv[t], xv[t]);
      dot += dot4(xv[t], v);
      dsq += dot4(v, v);
    }
  sq = wave_sum(sq);
  dot = wave_sum(dot);
  dsq = wave_sum(dsq);
  const float inv0 = rsqrtf(sq / (float)W + CAP_EPS32);
  const float inv = rsqrtf((sq + 2.f * dot + dsq) / (float)W + CAP_EPS32);
  const float a = inv, b = inv - inv0;  // delta inv + x (inv - inv0)
  uint16_t* o = a3 + r * 3 * W;
#pragma unroll
  for (int t = 0; t < MAXT; ++t)
    if (t < nt) {
      const int c = 4 * lane + 256 * t;
      uint2 hi, lo;
      split4(make_float4(d[t].x * a + xv[t].x * b, d[t].y * a + xv[t].y * b, d[t].z * a + xv[t].z * b,
                         d[t].w * a + xv[t].w * b), hi, lo);
      *reinterpret_cast<uint2*>(o + c) = hi;
      *reinterpret_cast<uint2*>(o + W + c) = lo;
      *reinterpret_cast<uint2*>(o + 2 * W + c) = hi;
    }
}

// The clean query products r0_i = norm(x_i) W_q^T (train/val/run.py:293) in float32 on VALU,
// written to rows m P + i of dr. Workgroup: 8 tokens x 64 outputs; lane l of wave w forms the
// outputs 64 blockIdx.x + 16 w + l % 16 for tokens 8 blockIdx.y + l / 16 and + 4.
__global__ __launch_bounds__(256) void chain_query_clean_kernel(const float* __restrict__ x,
                                                                const float* __restrict__ w_q, int m, int W,
                                                                float* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) float xs[8][256 * MAXT];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int t0 = blockIdx.y * 8;
  const int nt = W / 256;
  for (int tt = wave; tt < 8; tt += 4) {  // norm(x) of tokens t0 + tt into LDS
    const int tok = min(t0 + tt, m - 1);
    float4 v[MAXT];
    float sq = 0.f;
#pragma unroll
    for (int t = 0; t < MAXT; ++t)
      if (t < nt) {
        v[t] = ld4(x + (int64_t)tok * W + 4 * lane + 256 * t);
        sq += dot4(v[t], v[t]);
      }
    const float inv0 = rsqrtf(wave_sum(sq) / (float)W + CAP_EPS32);
#pragma unroll
    for (int t = 0; t < MAXT; ++t)
      if (t < nt)
        st4(&xs[tt][4 * lane + 256 * t], make_float4(v[t].x * inv0, v[t].y * inv0, v[t].z * inv0, v[t].w * inv0));
  }
  __syncthreads();
  const int n = blockIdx.x * 64 + wave * 16 + (lane & 15), ta = lane >> 4;
  const float* wr = w_q + (int64_t)n * W;
  float s0 = 0.f, s1 = 0.f;
  for (int k = 0; k < W; k += 4) {
    const float4 wv = ld4(wr + k);
    s0 += dot4(wv, ld4(&xs[ta][k]));
    s1 += dot4(wv, ld4(&xs[ta + 4][k]));
  }
  if (t0 + ta < m) out[(int64_t)(t0 + ta) * W + n] = s0;
  if (t0 + ta + 4 < m) out[(int64_t)(t0 + ta + 4) * W + n] = s1;
}

struct ChainQuery {
  const float* dr;       // [m P + m, W] query products: moves' changes, then the clean rows
  const int64_t* pos;    // [m]
  const float* cos_t;    // [T, 32]
  const float* sin_t;
  const uint16_t* keys;  // [m, heads, K, 64]
  const uint16_t* vals;  // [m, heads, K, 64]
  const float* top_p;    // [m, heads, K]
  const float* rest;     // [m, heads, 64]
  int T, m, P, W, heads, K;
  uint16_t* a3;          // out [m P, 3 W]: A3 of the attention output changes
};

constexpr int QLD = 72;  // LDS row of a 64-wide bf16 tile, padded by 16 bytes (conflict-free reads)

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

// Value tiles [64 keys][64 dims] with chunk c (8 dims) of row r at c ^ (2 (r & 3)): the
// transposing reads below (16 lanes: 4 consecutive keys x 2 adjacent chunks) touch 8 distinct
// chunk positions.
NOISE_DEV int vswz(int row, int chunk) { return row * 64 + ((chunk ^ (2 * (row & 3))) << 3); }

// Workgroup (row tile, head h, token i), four waves of 32 moves each (train/val/run.py:290-303):
//   dr, r0 rotated; inv0, inv from |r0|^2, r0.dr, |dr|^2; dq = bf16(dr inv + r0 (inv - inv0))
//   ds = bf16(dq k_t) / 8 for the token's K <= 64 top keys (zero-padded to 64, p = 0 there),
//   formed transposed, ds^T = K dq^T, so a lane owns one move and 16 keys of each 32-key half
//   dlse = log1p(sum_t p_t expm1(ds_t)), w = bf16(p expm1(ds - dlse)) packed in registers as the
//   B operand of dout^T = V^T w^T (V^T read with ds_read_b64_tr_b16, as in the window step)
//   dout = bf16(w V) + expm1(-dlse) rest
// written as A3 of the output projection's product. A position outside [0, T) gives NaN.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 4))) void chain_query_attn_kernel(const ChainQuery g) {
  __shared__ __attribute__((aligned(16))) uint16_t kt[64 * QLD];     // keys [key][dim], padded rows
  __shared__ __attribute__((aligned(16))) uint16_t vts[64 * 64];     // values [key][dim], vswz chunks
  __shared__ __attribute__((aligned(16))) uint16_t at[4][32 * QLD];  // per wave: dq
  __shared__ __attribute__((aligned(16))) float ps[64];
  __shared__ float r0s[64], rs[64], cs[32], sn[32], inv0s;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = blockIdx.z, h = blockIdx.y;
  const int pw = blockIdx.x * 128 + wave * 32;  // first move of this wave
  const int64_t pos = g.pos[i];
  const bool pos_ok = pos >= 0 && pos < g.T;
  const int64_t pc = pos_ok ? pos : 0;
  const int64_t ih = (int64_t)i * g.heads + h;
  const int64_t kv0 = ih * g.K * 64;
  for (int e = tid; e < 64 * 8; e += 256) {
    const int k = e >> 3, c = e & 7;
    uint4 kv = make_uint4(0u, 0u, 0u, 0u), vv = kv;
    if (k < g.K) {
      kv = *reinterpret_cast<const uint4*>(g.keys + kv0 + k * 64 + 8 * c);
      vv = *reinterpret_cast<const uint4*>(g.vals + kv0 + k * 64 + 8 * c);
    }
    *reinterpret_cast<uint4*>(kt + k * QLD + 8 * c) = kv;
    *reinterpret_cast<uint4*>(vts + vswz(k, c)) = vv;
  }
  if (tid < 64) {
    ps[tid] = tid < g.K ? g.top_p[ih * g.K + tid] : 0.f;
    rs[tid] = g.rest[ih * 64 + tid];
  } else if (tid < 96) {
    cs[tid - 64] = g.cos_t[pc * 32 + tid - 64];
    sn[tid - 64] = g.sin_t[pc * 32 + tid - 64];
  }
  __syncthreads();
  if (tid < 64) {  // the clean rotated query of this head and |r0|^2
    const float* cr = g.dr + ((int64_t)g.m * g.P + i) * g.W + h * 64;
    const int c = tid & 31;
    const float u1 = cr[c], u2 = cr[c + 32];
    const float v = tid < 32 ? u1 * cs[c] + u2 * sn[c] : -u1 * sn[c] + u2 * cs[c];
    r0s[tid] = v;
    const float sq = wave_sum(v * v);
    if (tid == 0) inv0s = sq;
  }
  __syncthreads();
  const float sq = inv0s, inv0 = rsqrtf(sq / 64.f + CAP_EPS32);

  // dq: lanes 2 q and 2 q + 1 hold move q's dims c, c + 32 for c in [0, 16) and [16, 32)
  {
    const int q = lane >> 1, c0 = (lane & 1) * 16;
    const int p = min(pw + q, g.P - 1);
    const float* src = g.dr + ((int64_t)i * g.P + p) * g.W + h * 64;
    float u1[16], u2[16];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float4 a = ld4(src + c0 + 4 * t), b = ld4(src + 32 + c0 + 4 * t);
      u1[4 * t] = a.x; u1[4 * t + 1] = a.y; u1[4 * t + 2] = a.z; u1[4 * t + 3] = a.w;
      u2[4 * t] = b.x; u2[4 * t + 1] = b.y; u2[4 * t + 2] = b.z; u2[4 * t + 3] = b.w;
    }
    float dot = 0.f, dsq = 0.f;
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const int c = c0 + t;
      const float v1 = u1[t] * cs[c] + u2[t] * sn[c], v2 = -u1[t] * sn[c] + u2[t] * cs[c];
      u1[t] = v1;
      u2[t] = v2;
      dot += r0s[c] * v1 + r0s[c + 32] * v2;
      dsq += v1 * v1 + v2 * v2;
    }
    dot += noise::dpp_row<0xB1>(dot);
    dsq += noise::dpp_row<0xB1>(dsq);
    const float inv = rsqrtf((sq + 2.f * dot + dsq) / 64.f + CAP_EPS32), dinv = inv - inv0;
    uint16_t* dst = at[wave] + q * QLD;
#pragma unroll
    for (int t = 0; t < 16; t += 8) {
      uint4 w1, w2;
      uint32_t* p1 = reinterpret_cast<uint32_t*>(&w1);
      uint32_t* p2 = reinterpret_cast<uint32_t*>(&w2);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int a = t + 2 * j, c = c0 + a;
        p1[j] = pack_bf2(u1[a] * inv + r0s[c] * dinv, u1[a + 1] * inv + r0s[c + 1] * dinv);
        p2[j] = pack_bf2(u2[a] * inv + r0s[c + 32] * dinv, u2[a + 1] * inv + r0s[c + 33] * dinv);
      }
      *reinterpret_cast<uint4*>(dst + c0 + t) = w1;
      *reinterpret_cast<uint4*>(dst + 32 + c0 + t) = w2;
    }
  }
  __syncthreads();  // dq tiles complete
  const int fr = lane & 31, half = lane >> 5, fk = 8 * half;
  bf16x8 qf[4];  // B operand: move fr, dims 16 ks + 8 half .. + 7
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) qf[ks] = *reinterpret_cast<const bf16x8*>(at[wave] + fr * QLD + 16 * ks + fk);
  // ds^T of both 32-key halves: key 32 kb2 + 8 (j / 4) + 4 half + j % 4 for move fr
  floatx16 ds[2];
#pragma unroll
  for (int kb2 = 0; kb2 < 2; ++kb2) {
#pragma unroll
    for (int j = 0; j < 16; ++j) ds[kb2][j] = 0.f;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(kt + (32 * kb2 + fr) * QLD + 16 * ks + fk);
      ds[kb2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[ks], ds[kb2], 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) ds[kb2][j] = bf2f(f2bf(ds[kb2][j])) * 0.125f;
  }
  float es = 0.f;
#pragma unroll
  for (int kb2 = 0; kb2 < 2; ++kb2) {
    const floatx16 em = noise::expm1_small16(ds[kb2]);
    const float* pp = ps + 32 * kb2 + 4 * half;
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const float4 p = *reinterpret_cast<const float4*>(pp + 8 * g4);
      es += p.x * em[4 * g4] + p.y * em[4 * g4 + 1] + p.z * em[4 * g4 + 2] + p.w * em[4 * g4 + 3];
    }
  }
  const float dl = log1pf(es + __shfl_xor(es, 32, 64));
  // V^T fragment offsets: as in the window step
  int vfo[2];
  {
    const int s16 = lane & 15, a = s16 & 3, e = s16 >> 2, gq = lane >> 4;
    const int key = 4 * (gq >> 1) + e;
#pragma unroll
    for (int db = 0; db < 2; ++db) vfo[db] = vswz(key, 4 * db + 2 * (gq & 1) + (a >> 1)) + 4 * (a & 1);
  }
  floatx16 o[2];
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int j = 0; j < 16; ++j) o[db][j] = 0.f;
#pragma unroll
  for (int kb2 = 0; kb2 < 2; ++kb2) {
    floatx16 x = ds[kb2];
#pragma unroll
    for (int j = 0; j < 16; ++j) x[j] -= dl;
    const floatx16 em = noise::expm1_small16(x);
    const float* pp = ps + 32 * kb2 + 4 * half;
    bf16x8 pf[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const float4 pa = *reinterpret_cast<const float4*>(pp + 16 * kk);
      const float4 pb = *reinterpret_cast<const float4*>(pp + 16 * kk + 8);
      const int j0 = 8 * kk;
      u32x4 pk;
      pk[0] = pack_bf2(pa.x * em[j0], pa.y * em[j0 + 1]);
      pk[1] = pack_bf2(pa.z * em[j0 + 2], pa.w * em[j0 + 3]);
      pk[2] = pack_bf2(pb.x * em[j0 + 4], pb.y * em[j0 + 5]);
      pk[3] = pack_bf2(pb.z * em[j0 + 6], pb.w * em[j0 + 7]);
      pf[kk] = __builtin_bit_cast(bf16x8, pk);
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        const uint16_t* a0 = vts + 32 * kb2 * 64 + 16 * kk * 64 + vfo[db];
        const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(a0));
        const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(a0 + 8 * 64));
        u32x4 u;
        u[0] = __builtin_bit_cast(u32x2, lo)[0];
        u[1] = __builtin_bit_cast(u32x2, lo)[1];
        u[2] = __builtin_bit_cast(u32x2, hi)[0];
        u[3] = __builtin_bit_cast(u32x2, hi)[1];
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, u), pf[kk], o[db], 0, 0, 0);
      }
  }
  // lane: move fr, dims 32 db + 8 (j / 4) + 4 half + j % 4; the hi and lo halves go through LDS
  // (at for hi; kt or vts, free once every wave is past its products, for lo) for 16-byte stores
  __syncthreads();
  {
    const float nan = __builtin_nanf("");
    const float em = noise::expm1_small(-dl);
    uint16_t* hi_t = at[wave];
    uint16_t* lo_t = wave < 2 ? kt + (wave & 1) * 32 * QLD : vts + (wave & 1) * 32 * 64;
    const int lls = wave < 2 ? QLD : 64;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d0 = 32 * db + 8 * g4 + 4 * half;
        float4 v;
        v.x = pos_ok ? bf2f(f2bf(o[db][4 * g4])) + em * rs[d0] : nan;
        v.y = pos_ok ? bf2f(f2bf(o[db][4 * g4 + 1])) + em * rs[d0 + 1] : nan;
        v.z = pos_ok ? bf2f(f2bf(o[db][4 * g4 + 2])) + em * rs[d0 + 2] : nan;
        v.w = pos_ok ? bf2f(f2bf(o[db][4 * g4 + 3])) + em * rs[d0 + 3] : nan;
        uint2 hv, lv;
        split4(v, hv, lv);
        *reinterpret_cast<uint2*>(hi_t + fr * QLD + d0) = hv;
        *reinterpret_cast<uint2*>(lo_t + fr * lls + d0) = lv;
      }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int row = (lane >> 3) + 8 * t, c = (lane & 7) * 8;
      const int p = pw + row;
      if (p >= g.P) continue;
      const uint4 hv = *reinterpret_cast<const uint4*>(hi_t + row * QLD + c);
      const uint4 lv = *reinterpret_cast<const uint4*>(lo_t + row * lls + c);
      uint16_t* q = g.a3 + ((int64_t)i * g.P + p) * 3 * g.W + h * 64 + c;
      *reinterpret_cast<uint4*>(q) = hv;
      *reinterpret_cast<uint4*>(q + g.W) = lv;
      *reinterpret_cast<uint4*>(q + 2 * g.W) = hv;
    }
  }
}

struct ChainQueryWin {
  const float* dr;       // [m P + m, W] query products: moves' changes, then the clean rows
  const int64_t* pos;    // [m]
  const int64_t* rel;    // [m] positions within the key window
  const float* cos_t;    // [T, 32]
  const float* sin_t;
  const uint16_t* keys;  // [heads, S, 64]
  const uint16_t* vals;  // [heads, S, 64]
  int T, m, P, W, heads, S, window;
  uint16_t* a3;          // out [m P, 3 W]
};

constexpr int QWMAX = 4096;  // keys of one token's window (clean probabilities held in LDS)

NOISE_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}


// Workgroup (row tile, head h, token i), four waves of 32 moves each, over the n keys t with
// 0 <= rel_i - t <= window (train/val/run.py:264-281):
//   q0 = bf16(r0 inv0); p0 = softmax over the window of bf16(q0 K^T) / 8   (per token, on VALU)
//   dq as in the routed step. Scores are formed transposed, ds^T = K dq^T (MFMA, K the A operand
//   from LDS, dq the B operand held in registers), so a lane owns one move and 16 keys of every
//   32-key half-block: per-move sums need no cross-lane traffic until the end.
//   pass 1 over 64-key blocks: dlse = log1p(sum_t p0 expm1(ds_t)), ds = bf16(dq k_t) / 8;
//   pass 2 recomputes ds, packs w = bf16(p0 expm1(ds - dlse)) in registers as the B operand of
//   dout^T += V^T w^T, V^T read from the row-major value tile with ds_read_b64_tr_b16 (lane
//   4a + b of each 16-lane group receives element b of the rows addressed by lanes a, a + 4,
//   a + 8, a + 12) in the key order the score accumulators hold.
// dout = bf16(sum) is written as A3 of the output projection's product. A position outside
// [0, T) or a window with no key gives NaN.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 3))) void chain_query_window_kernel(const ChainQueryWin g) {
  __shared__ __attribute__((aligned(16))) uint16_t kts[2][64 * QLD];  // keys [key][dim], padded rows
  __shared__ __attribute__((aligned(16))) uint16_t vts[2][64 * 64];   // values [key][dim], vswz chunks
  __shared__ __attribute__((aligned(16))) float p0s[QWMAX + 64];
  // per wave: the dq tile, in the key buffers (free until the first key block lands)
  uint16_t(*at)[32 * QLD] = reinterpret_cast<uint16_t(*)[32 * QLD]>(&kts[0][0]);
  __shared__ float r0s[64], cs[32], sn[32], red[8], inv0s;
  __shared__ __attribute__((aligned(16))) uint16_t q0s[64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = blockIdx.z, h = blockIdx.y;
  const int pw = blockIdx.x * 128 + wave * 32;
  const int64_t pos = g.pos[i], rl = g.rel[i];
  const int64_t lo64 = rl - g.window > 0 ? rl - g.window : 0;
  const int64_t hi64 = rl < g.S - 1 ? rl : g.S - 1;
  const int n = hi64 >= lo64 ? (int)(hi64 - lo64 + 1) : 0;  // <= window + 1 <= QWMAX
  const int nb = (n + 63) & ~63;                               // keys swept, in blocks of 64
  const bool ok = pos >= 0 && pos < g.T && n > 0;
  const int64_t pc = ok ? pos : 0;
  const int64_t kbase = ((int64_t)h * g.S + (n > 0 ? lo64 : 0)) * 64;
  if (tid < 32) {
    cs[tid] = g.cos_t[pc * 32 + tid];
    sn[tid] = g.sin_t[pc * 32 + tid];
  }
  __syncthreads();
  if (tid < 64) {  // the clean rotated query of this head, inv0 and q0 = bf16(r0 inv0)
    const float* cr = g.dr + ((int64_t)g.m * g.P + i) * g.W + h * 64;
    const int c = tid & 31;
    const float u1 = cr[c], u2 = cr[c + 32];
    const float v = tid < 32 ? u1 * cs[c] + u2 * sn[c] : -u1 * sn[c] + u2 * cs[c];
    r0s[tid] = v;
    const float sq = wave_sum(v * v);
    q0s[tid] = f2bf(v * rsqrtf(sq / 64.f + CAP_EPS32));
    if (tid == 0) inv0s = sq;
  }
  __syncthreads();
  // clean scores of the window, then its softmax (zeros past the window up to nb)
  float mx = -INFINITY;
  for (int t = tid; t < n; t += 256) {
    const uint16_t* kr = g.keys + kbase + (int64_t)t * 64;
    float sc = 0.f;
#pragma unroll
    for (int c = 0; c < 64; c += 8) {
      const uint4 kv = *reinterpret_cast<const uint4*>(kr + c);
      const uint4 qv = *reinterpret_cast<const uint4*>(q0s + c);
      sc += bf_lo(qv.x) * bf_lo(kv.x) + bf_hi(qv.x) * bf_hi(kv.x) + bf_lo(qv.y) * bf_lo(kv.y) +
            bf_hi(qv.y) * bf_hi(kv.y) + bf_lo(qv.z) * bf_lo(kv.z) + bf_hi(qv.z) * bf_hi(kv.z) +
            bf_lo(qv.w) * bf_lo(kv.w) + bf_hi(qv.w) * bf_hi(kv.w);
    }
    sc = bf2f(f2bf(sc)) * 0.125f;
    p0s[t] = sc;
    mx = fmaxf(mx, sc);
  }
  mx = wave_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float z = 0.f;
  for (int t = tid; t < n; t += 256) {
    const float e = expf(p0s[t] - mx);
    p0s[t] = e;
    z += e;
  }
  z = wave_sum(z);
  if (lane == 0) red[4 + wave] = z;
  __syncthreads();
  z = (red[4] + red[5]) + (red[6] + red[7]);
  for (int t = tid; t < nb; t += 256) p0s[t] = t < n ? p0s[t] / z : 0.f;
  const float sq = inv0s, inv0 = rsqrtf(sq / 64.f + CAP_EPS32);

  // dq: lanes 2 q and 2 q + 1 hold move q's dims c, c + 32 for c in [0, 16) and [16, 32)
  {
    const int q = lane >> 1, c0 = (lane & 1) * 16;
    const int p = min(pw + q, g.P - 1);
    const float* src = g.dr + ((int64_t)i * g.P + p) * g.W + h * 64;
    float u1[16], u2[16];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float4 a = ld4(src + c0 + 4 * t), b = ld4(src + 32 + c0 + 4 * t);
      u1[4 * t] = a.x; u1[4 * t + 1] = a.y; u1[4 * t + 2] = a.z; u1[4 * t + 3] = a.w;
      u2[4 * t] = b.x; u2[4 * t + 1] = b.y; u2[4 * t + 2] = b.z; u2[4 * t + 3] = b.w;
    }
    float dot = 0.f, dsq = 0.f;
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const int c = c0 + t;
      const float v1 = u1[t] * cs[c] + u2[t] * sn[c], v2 = -u1[t] * sn[c] + u2[t] * cs[c];
      u1[t] = v1;
      u2[t] = v2;
      dot += r0s[c] * v1 + r0s[c + 32] * v2;
      dsq += v1 * v1 + v2 * v2;
    }
    dot += noise::dpp_row<0xB1>(dot);
    dsq += noise::dpp_row<0xB1>(dsq);
    const float inv = rsqrtf((sq + 2.f * dot + dsq) / 64.f + CAP_EPS32), dinv = inv - inv0;
    uint16_t* dst = at[wave] + q * QLD;
#pragma unroll
    for (int t = 0; t < 16; t += 8) {
      uint4 w1, w2;
      uint32_t* p1 = reinterpret_cast<uint32_t*>(&w1);
      uint32_t* p2 = reinterpret_cast<uint32_t*>(&w2);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int a = t + 2 * j, c = c0 + a;
        p1[j] = pack_bf2(u1[a] * inv + r0s[c] * dinv, u1[a + 1] * inv + r0s[c + 1] * dinv);
        p2[j] = pack_bf2(u2[a] * inv + r0s[c + 32] * dinv, u2[a + 1] * inv + r0s[c + 33] * dinv);
      }
      *reinterpret_cast<uint4*>(dst + c0 + t) = w1;
      *reinterpret_cast<uint4*>(dst + 32 + c0 + t) = w2;
    }
  }
  __syncthreads();  // dq tiles and p0 complete
  const int fr = lane & 31, half = lane >> 5, fk = 8 * half;
  bf16x8 qf[4];  // B operand: this lane's move fr, dims 16 ks + 8 half .. + 7
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) qf[ks] = *reinterpret_cast<const bf16x8*>(at[wave] + fr * QLD + 16 * ks + fk);
  __syncthreads();  // every wave holds its dq fragments: the key buffers take key blocks from here
  // V^T fragment offsets (within the value tile): in 16-lane group gq, lane a + 4 e addresses
  // key 4 (gq >> 1) + e (+ 16 kk + 32 kb2, + 8 for the second read), dims 32 db + 16 (gq & 1) + 4 a;
  // the lane then holds dim 32 db + lane % 32 for the keys its w values hold.
  int vfo[2];
  {
    const int s16 = lane & 15, a = s16 & 3, e = s16 >> 2, gq = lane >> 4;
    const int key = 4 * (gq >> 1) + e;
#pragma unroll
    for (int db = 0; db < 2; ++db) vfo[db] = vswz(key, 4 * db + 2 * (gq & 1) + (a >> 1)) + 4 * (a & 1);
  }
  // ds^T of one 32-key half-block: key 32 kb2 + 8 (j / 4) + 4 half + j % 4 for move fr
  auto scores = [&](const uint16_t* kt, int kb2) {
    floatx16 acc;
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = 0.f;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(kt + (32 * kb2 + fr) * QLD + 16 * ks + fk);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[ks], acc, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = bf2f(f2bf(acc[j])) * 0.125f;
    return acc;
  };
  // Blocks of 64 keys go global -> registers one block ahead, then into one of two LDS buffers
  // (one barrier per block). Thread tid moves chunk tid % 8 of keys tid / 8 and tid / 8 + 32.
  uint4 rk[2], rv[2];
  auto fetch = [&](int k0, bool with_values) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int k = (tid >> 3) + 32 * r, c = tid & 7;
      const bool in = k0 + k < n;
      const int64_t o = kbase + (int64_t)(in ? k0 + k : 0) * 64 + 8 * c;
      rk[r] = *reinterpret_cast<const uint4*>(g.keys + o);
      if (with_values) rv[r] = *reinterpret_cast<const uint4*>(g.vals + o);
      if (!in) rk[r] = rv[r] = make_uint4(0u, 0u, 0u, 0u);
    }
  };
  auto stash = [&](int buf, bool with_values) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int k = (tid >> 3) + 32 * r, c = tid & 7;
      *reinterpret_cast<uint4*>(kts[buf] + k * QLD + 8 * c) = rk[r];
      if (with_values) *reinterpret_cast<uint4*>(vts[buf] + vswz(k, c)) = rv[r];
    }
  };

  // pass 1
  float es = 0.f;
  if (nb) fetch(0, false);
  for (int k0 = 0, buf = 0; k0 < nb; k0 += 64, buf ^= 1) {
    stash(buf, false);
    if (k0 + 64 < nb) fetch(k0 + 64, false);
    __syncthreads();
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2) {
      const floatx16 em = noise::expm1_small16(scores(kts[buf], kb2));
      const float* pp = p0s + k0 + 32 * kb2 + 4 * half;
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const float4 p = *reinterpret_cast<const float4*>(pp + 8 * g4);
        es += p.x * em[4 * g4] + p.y * em[4 * g4 + 1] + p.z * em[4 * g4 + 2] + p.w * em[4 * g4 + 3];
      }
    }
  }
  const float dl = log1pf(es + __shfl_xor(es, 32, 64));

  // pass 2
  floatx16 o[2];
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int j = 0; j < 16; ++j) o[db][j] = 0.f;
  __syncthreads();  // pass 1 is done with both key buffers
  if (nb) fetch(0, true);
  for (int k0 = 0, buf = 0; k0 < nb; k0 += 64, buf ^= 1) {
    stash(buf, true);
    if (k0 + 64 < nb) fetch(k0 + 64, true);
    __syncthreads();
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2) {
      floatx16 ds = scores(kts[buf], kb2);
#pragma unroll
      for (int j = 0; j < 16; ++j) ds[j] -= dl;
      const floatx16 em = noise::expm1_small16(ds);
      const float* pp = p0s + k0 + 32 * kb2 + 4 * half;
      bf16x8 pf[2];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const float4 pa = *reinterpret_cast<const float4*>(pp + 16 * kk);
        const float4 pb = *reinterpret_cast<const float4*>(pp + 16 * kk + 8);
        const int j0 = 8 * kk;
        u32x4 pk;
        pk[0] = pack_bf2(pa.x * em[j0], pa.y * em[j0 + 1]);
        pk[1] = pack_bf2(pa.z * em[j0 + 2], pa.w * em[j0 + 3]);
        pk[2] = pack_bf2(pb.x * em[j0 + 4], pb.y * em[j0 + 5]);
        pk[3] = pack_bf2(pb.z * em[j0 + 6], pb.w * em[j0 + 7]);
        pf[kk] = __builtin_bit_cast(bf16x8, pk);
      }
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int db = 0; db < 2; ++db) {
          const uint16_t* a0 = vts[buf] + 32 * kb2 * 64 + 16 * kk * 64 + vfo[db];
          const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(a0));
          const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(a0 + 8 * 64));
          u32x4 u;
          u[0] = __builtin_bit_cast(u32x2, lo)[0];
          u[1] = __builtin_bit_cast(u32x2, lo)[1];
          u[2] = __builtin_bit_cast(u32x2, hi)[0];
          u[3] = __builtin_bit_cast(u32x2, hi)[1];
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, u), pf[kk], o[db], 0, 0, 0);
        }
    }
  }
  // lane: move fr, dims 32 db + 8 (j / 4) + 4 half + j % 4; the hi and lo halves go through LDS
  // (the key buffers for hi, the value buffers for lo, once every wave is past its products) for
  // 16-byte stores
  __syncthreads();
  {
    const float nan = __builtin_nanf("");
    uint16_t* hi_t = at[wave];
    uint16_t* lo_t = &vts[0][0] + wave * 32 * 64;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d0 = 32 * db + 8 * g4 + 4 * half;
        float4 v;
        v.x = ok ? bf2f(f2bf(o[db][4 * g4])) : nan;
        v.y = ok ? bf2f(f2bf(o[db][4 * g4 + 1])) : nan;
        v.z = ok ? bf2f(f2bf(o[db][4 * g4 + 2])) : nan;
        v.w = ok ? bf2f(f2bf(o[db][4 * g4 + 3])) : nan;
        uint2 hv, lv;
        split4(v, hv, lv);
        *reinterpret_cast<uint2*>(hi_t + fr * QLD + d0) = hv;
        *reinterpret_cast<uint2*>(lo_t + fr * 64 + d0) = lv;
      }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int row = (lane >> 3) + 8 * t, c = (lane & 7) * 8;
      const int p = pw + row;
      if (p >= g.P) continue;
      const uint4 hv = *reinterpret_cast<const uint4*>(hi_t + row * QLD + c);
      const uint4 lv = *reinterpret_cast<const uint4*>(lo_t + row * 64 + c);
      uint16_t* q = g.a3 + ((int64_t)i * g.P + p) * 3 * g.W + h * 64 + c;
      *reinterpret_cast<uint4*>(q) = hv;
      *reinterpret_cast<uint4*>(q + g.W) = lv;
      *reinterpret_cast<uint4*>(q + 2 * g.W) = hv;
    }
  }
}

// ---------------------------------------------------------------- head

// Per row: inv = rsqrt((|xL|^2 + 2 xL.delta + |delta|^2) / W + eps), zy = (base_y + delta.tw) inv
// (the reference's target term, in fp32), bf16(delta) for the head product.
__global__ __launch_bounds__(256) void chain_head_prep_kernel(const float* __restrict__ delta,
                                                              const float* __restrict__ xL,
                                                              const float* __restrict__ base, int64_t ld_base,
                                                              const float* __restrict__ tw,
                                                              const int64_t* __restrict__ y, int rows, int P,
                                                              int W, int V, uint16_t* __restrict__ dbf,
                                                              float* __restrict__ inv_out,
                                                              float* __restrict__ zy_out) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int64_t i = r / P;
  const int nt = W / 256;
  float sq = 0.f, dot = 0.f, dsq = 0.f, ty = 0.f;
#pragma unroll
  for (int t = 0; t < MAXT; ++t)
    if (t < nt) {
      const float4 d = ld4(delta + r * W + 4 * lane + 256 * t), x = ld4(xL + i * W + 4 * lane + 256 * t);
      sq += dot4(x, x);
      dot += dot4(x, d);
      dsq += dot4(d, d);
      ty += dot4(d, ld4(tw + i * W + 4 * lane + 256 * t));
      *reinterpret_cast<uint2*>(dbf + r * W + 4 * lane + 256 * t) = make_uint2(pack_bf2(d.x, d.y), pack_bf2(d.z, d.w));
    }
  sq = wave_sum(sq);
  dot = wave_sum(dot);
  dsq = wave_sum(dsq);
  ty = wave_sum(ty);
  if (lane == 0) {
    const float inv = rsqrtf((sq + 2.f * dot + dsq) / (float)W + CAP_EPS32);
    const int64_t t = y[i];
    const int64_t tc = t < 0 ? 0 : (t < V ? t : 0);
    inv_out[r] = inv;
    zy_out[r] = (base[i * ld_base + tc] + ty) * inv;
  }
}

// One wave per token: the clean sum S0_i = sum_v exp(cap(base_iv inv0_i) - 15) into clean[i] and the
// clean target logit z0_y = base_iy inv0_i into clean[m + i].
__global__ __launch_bounds__(256) void chain_clean_kernel(const float* __restrict__ base, int64_t ld_base,
                                                          const float* __restrict__ xL,
                                                          const int64_t* __restrict__ y, int m, int W, int V,
                                                          float* __restrict__ clean) {
  const int lane = threadIdx.x & 63;
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= m) return;
  float sq = 0.f;
  for (int c = lane; c < W; c += 64) sq += xL[(int64_t)i * W + c] * xL[(int64_t)i * W + c];
  const float inv0 = rsqrtf(wave_sum(sq) / (float)W + CAP_EPS32);
  const float s = noise::row_capexp_sum<false>(base + (int64_t)i * ld_base, V, inv0, lane);
  const int64_t t = y[i];
  const int64_t tc = t < 0 ? 0 : (t < V ? t : 0);
  if (lane == 0) {
    clean[i] = s;
    clean[m + i] = base[(int64_t)i * ld_base + tc] * inv0;
  }
}

struct ChainHead {
  const uint16_t* dbf;   // [m * P, W] bf16 moves
  const uint16_t* w;     // [V, W] bf16 head weight (weight_t transposed)
  const float* base;     // [m, ld_base]
  int64_t ld_base;
  const float* inv;      // [m * P]
  const float* zy;       // [m * P]
  const float* clean;    // [2 m]: clean sums, then clean target logits
  const float* scale;    // [m, ld_scale]
  int64_t ld_scale;
  const int64_t* y;      // [m]
  int m, P, W, V;
  float* out;            // [m, ld_out]
  int64_t ld_out;
};

constexpr int HBN = 256, HWN = HBN / 64, HNS = 2, HKB = 64;
using HCfg = noise::TileCfg<HBN, HNS, HKB>;

// A workgroup owns 256 rows and sweeps the vocabulary in 256-column tiles of mma_tile, keeping per
// row the running sum of exp(cap(z) - 15), z = (base + bf16(acc)) inv.
__global__ void __attribute__((amdgpu_flat_work_group_size(HCfg::THREADS, HCfg::THREADS), amdgpu_waves_per_eu(2, 2)))
chain_head_kernel(const ChainHead g) {
  constexpr int ROWS_BYTES = (2 + HWN) * 256 * 4;
  __shared__ __attribute__((aligned(16))) unsigned char lds[ROWS_BYTES + 2 * HCfg::SMEM_ELEMS];
  float* ik_s = reinterpret_cast<float*>(lds);
  int* tok_s = reinterpret_cast<int*>(lds + 1024);
  float(*sum_s)[256] = reinterpret_cast<float(*)[256]>(lds + 2048);
  uint16_t* smem = reinterpret_cast<uint16_t*>(lds + ROWS_BYTES);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / HWN, wn = wave % HWN;
  const int M = g.m * g.P;
  const int m0 = blockIdx.x * 256;
  if (tid < 256) {
    const int row = m0 + tid < M ? m0 + tid : M - 1;
    ik_s[tid] = g.inv[row] * CAP_K1;
    tok_s[tid] = row / g.P;
  }
  // (the per-row arrays are read after the main loop's first barrier)
  float rsum[4] = {0.f, 0.f, 0.f, 0.f};
  const uint16_t* A = g.dbf + (int64_t)m0 * g.W;
  for (int n0 = 0; n0 < g.V; n0 += HBN) {
    floatx16 acc[4][2];
    noise::zero_acc(acc);
    noise::mma_tile<HBN, HNS, HKB>(A, g.W, M - m0, g.w + (int64_t)n0 * g.W, g.W, g.W, smem, acc);
    const int colbase = n0 + wn * 64 + (lane & 31);
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      float es[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int rl = wm * 128 + mi * 32 + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
        const float ik = ik_s[rl];
        const float* brow = g.base + (int64_t)tok_s[rl] * g.ld_base + colbase;
        es[j] = noise::capexp(brow[0] + bf2f(f2bf(acc[mi][0][j])), ik) +
                noise::capexp(brow[32] + bf2f(f2bf(acc[mi][1][j])), ik);
      }
      rsum[mi] += noise::halfwave_transpose_sum16(es, lane);
    }
  }
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
    const int jj = (lane & 31) >> 1;
    const int rl = wm * 128 + mi * 32 + 8 * (jj >> 2) + 4 * (lane >> 5) + (jj & 3);
    if ((lane & 1) == 0) sum_s[wn][rl] = rsum[mi];
  }
  __syncthreads();
  if (tid < 256 && m0 + tid < M) {
    const int row = m0 + tid, i = row / g.P, p = row - i * g.P;
    float S = 0.f;
#pragma unroll
    for (int c = 0; c < HWN; ++c) S += sum_s[c][tid];
    const int64_t t = g.y[i];
    float* o = g.out + (int64_t)i * g.ld_out + p;
    if (t < 0) {
      *o = 0.f;
    } else if (t >= g.V) {
      *o = __builtin_nanf("");
    } else {
      const float mmc = logf(S / g.clean[i]) - noise::cap_difference(g.zy[row], g.clean[g.m + i]);
      *o = mmc / g.scale[(int64_t)i * g.ld_scale + p];
    }
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

extern "C" int noise_chain_start(const float* e, const float* x0, const float* move, int m, int P, int W,
                                 float mix, float* dx0, float* delta, void* stream) {
  NOISE_REQUIRE(m >= 0 && P > 0 && W > 0 && W % 256 == 0 && W <= 256 * MAXT,
                "chain_start: bad sizes (m=%d P=%d W=%d; W a multiple of 256 up to 2048)", m, P, W);
  if (m == 0) return NOISE_OK;
  NOISE_REQUIRE(e && x0 && move && dx0 && delta, "chain_start: NULL argument");
  const int rows = m * P;
  chain_start_kernel<<<(rows + 3) / 4, 256, 0, (hipStream_t)stream>>>(e, x0, move, rows, P, W, mix, dx0, delta);
  return noise::check_launch("chain_start");
}

extern "C" int noise_chain_block(const noise_chain_block_t* a, void* stream) {
  NOISE_REQUIRE(a, "chain_block: args is NULL");
  NOISE_REQUIRE(a->m >= 0 && a->P > 0 && a->W > 0 && a->W % 256 == 0 && a->W <= 256 * MAXT && a->k > 0 &&
                    a->k % 128 == 0 && a->H > 0,
                "chain_block: bad sizes (m=%d P=%d W=%d k=%d H=%d; W a multiple of 256 up to 2048, k of 128)",
                a->m, a->P, a->W, a->k, a->H);
  if (a->m == 0) return NOISE_OK;
  NOISE_REQUIRE(a->delta && a->mid && a->idx && a->hs && a->w_fc && a->w_out_t && a->dz && a->wf && a->wo && a->g,
                "chain_block: NULL argument");
  NOISE_REQUIRE(a->ld_idx >= a->k && a->ld_hs >= a->k, "chain_block: ld_idx / ld_hs below k");
  NOISE_REQUIRE(aligned16(a->dz) && aligned16(a->wf) && aligned16(a->wo) && aligned16(a->g),
                "chain_block: workspace buffers must be 16-byte aligned");
  NOISE_REQUIRE(aligned16(a->w_fc) && aligned16(a->w_out_t), "chain_block: w_fc and w_out_t must be 16-byte aligned");
  NOISE_REQUIRE(a->m <= 65535 && (int64_t)a->m * a->P < (1ll << 31), "chain_block: at most 65535 tokens per call");
  const hipStream_t st = (hipStream_t)stream;
  const int rows = a->m * a->P;
  const int64_t tiles_p = (a->P + 255) / 256;
  chain_pre_kernel<<<(rows + 3) / 4, 256, 0, st>>>(a->delta, a->dx0, a->mid, rows, a->P, a->W, a->mix,
                                                    a->lam_r, a->lam_0, a->dz);
  if (int e = noise::check_launch("chain_block")) return e;
  chain_gather_kernel<<<dim3(a->W / 64, a->m), 256, 0, st>>>(a->w_fc, a->w_out_t, a->idx, a->ld_idx, a->k,
                                                              a->H, a->W, a->wf, a->wo);
  if (int e = noise::check_launch("chain_block")) return e;
  ChainGemm g1{a->dz, a->wf, a->P, a->k, a->W, a->hs, a->ld_hs, a->g, nullptr};
  chain_gemm_kernel<MODE_RELUDIFF, 128><<<dim3((unsigned)tiles_p, a->k / 128, a->m), 256, 0, st>>>(g1);
  if (int e = noise::check_launch("chain_block")) return e;
  ChainGemm g2{a->g, a->wo, a->P, a->W, a->k, nullptr, 0, nullptr, a->delta};
  chain_gemm_kernel<MODE_ADDROUND, 256><<<dim3((unsigned)tiles_p, a->W / 256, a->m), 512, 0, st>>>(g2);
  return noise::check_launch("chain_block");
}

namespace {

// The parts of an own-query step around its attention kernel: the weights' hi/lo triples, the
// clean query products (rows m P + i of dr), the mix and A3 rows of the moves, and their
// dr = A3 W_q3^T.
int query_products(float* delta, const float* dx0, int mix, float lam_r, float lam_0, const float* x,
                   const float* w_q, const float* w_proj_t, int m, int P, int W, uint16_t* a3, float* dr,
                   uint16_t* wq3, uint16_t* wp3, hipStream_t st) {
  const int64_t rows = (int64_t)m * P;
  const unsigned wblocks = (unsigned)(((int64_t)W * W + 255) / 256);
  chain_split_weight_kernel<<<wblocks, 256, 0, st>>>(w_q, W, 1, W, wq3);
  if (int e = noise::check_launch("chain_query")) return e;
  chain_split_weight_kernel<<<wblocks, 256, 0, st>>>(w_proj_t, 1, W, W, wp3);
  if (int e = noise::check_launch("chain_query")) return e;
  chain_query_clean_kernel<<<dim3(W / 64, (unsigned)((m + 7) / 8)), 256, 0, st>>>(x, w_q, m, W, dr + rows * W);
  if (int e = noise::check_launch("chain_query")) return e;
  chain_query_pre_kernel<<<(unsigned)((rows + 3) / 4), 256, 0, st>>>(delta, dx0, x, m, P, W, mix, lam_r, lam_0, a3);
  if (int e = noise::check_launch("chain_query")) return e;
  ChainGemm g1{a3, wq3, (int)rows, W, 3 * W, nullptr, 0, nullptr, dr};
  chain_gemm_kernel<MODE_STORE, 256><<<dim3((unsigned)((rows + 255) / 256), W / 256, 1), 512, 0, st>>>(g1);
  return noise::check_launch("chain_query");
}

// delta += dout c_proj^T (fp32), over the moves' rows of A3.
int query_output(float* delta, const uint16_t* a3, const uint16_t* wp3, int m, int P, int W, hipStream_t st) {
  const int64_t rows = (int64_t)m * P;
  ChainGemm g2{a3, wp3, (int)rows, W, 3 * W, nullptr, 0, nullptr, delta};
  chain_gemm_kernel<MODE_ADD, 256><<<dim3((unsigned)((rows + 255) / 256), W / 256, 1), 512, 0, st>>>(g2);
  return noise::check_launch("chain_query");
}

}  // namespace

#define CHAIN_QUERY_COMMON_CHECKS(a, name)                                                                   \
  NOISE_REQUIRE(a->delta && a->x && a->pos && a->w_q && a->w_proj_t && a->cos_t && a->sin_t && a->a3 &&      \
                    a->dr && a->wq3 && a->wp3,                                                               \
                name ": NULL argument");                                                                     \
  NOISE_REQUIRE(aligned16(a->delta) && (!a->dx0 || aligned16(a->dx0)) && aligned16(a->x) && aligned16(a->dr) && \
                    aligned16(a->a3) && aligned16(a->wq3) && aligned16(a->wp3),                              \
                name ": delta, dx0, x and the workspaces must be 16-byte aligned");                          \
  NOISE_REQUIRE(a->m <= 65535 && (int64_t)a->m * a->P + a->m < (1ll << 31), name ": at most 65535 tokens per call")

extern "C" int noise_chain_query(const noise_chain_query_t* a, void* stream) {
  NOISE_REQUIRE(a, "chain_query: args is NULL");
  NOISE_REQUIRE(a->m >= 0 && a->P > 0 && a->W > 0 && a->W % 256 == 0 && a->W <= 256 * MAXT && a->heads > 0 &&
                    a->W == 64 * a->heads && a->K >= 1 && a->K <= 64 && a->T > 0,
                "chain_query: bad sizes (m=%d P=%d W=%d heads=%d K=%d T=%d; W = 64 heads, a multiple of 256 up "
                "to 2048, 1 <= K <= 64)",
                a->m, a->P, a->W, a->heads, a->K, a->T);
  if (a->m == 0) return NOISE_OK;
  NOISE_REQUIRE(a->top_keys && a->top_values && a->top_p && a->rest, "chain_query: NULL argument");
  NOISE_REQUIRE(aligned16(a->top_keys) && aligned16(a->top_values), "chain_query: keys and values must be 16-byte aligned");
  CHAIN_QUERY_COMMON_CHECKS(a, "chain_query");
  const hipStream_t st = (hipStream_t)stream;
  if (int e = query_products(a->delta, a->dx0, a->mix, a->lam_r, a->lam_0, a->x, a->w_q, a->w_proj_t, a->m, a->P,
                             a->W, a->a3, a->dr, a->wq3, a->wp3, st))
    return e;
  ChainQuery q{a->dr, a->pos, a->cos_t, a->sin_t, a->top_keys, a->top_values, a->top_p, a->rest,
               a->T, a->m, a->P, a->W, a->heads, a->K, a->a3};
  chain_query_attn_kernel<<<dim3((unsigned)((a->P + 127) / 128), a->heads, a->m), 256, 0, st>>>(q);
  if (int e = noise::check_launch("chain_query")) return e;
  return query_output(a->delta, a->a3, a->wp3, a->m, a->P, a->W, st);
}

extern "C" int noise_chain_query_window(const noise_chain_query_window_t* a, void* stream) {
  NOISE_REQUIRE(a, "chain_query_window: args is NULL");
  NOISE_REQUIRE(a->m >= 0 && a->P > 0 && a->W > 0 && a->W % 256 == 0 && a->W <= 256 * MAXT && a->heads > 0 &&
                    a->W == 64 * a->heads && a->S > 0 && a->window >= 0 && a->window < QWMAX && a->T > 0,
                "chain_query_window: bad sizes (m=%d P=%d W=%d heads=%d S=%d window=%d T=%d; W = 64 heads, a "
                "multiple of 256 up to 2048, 0 <= window < %d)",
                a->m, a->P, a->W, a->heads, a->S, a->window, a->T, QWMAX);
  if (a->m == 0) return NOISE_OK;
  NOISE_REQUIRE(a->rel && a->keys && a->values, "chain_query_window: NULL argument");
  NOISE_REQUIRE(aligned16(a->keys) && aligned16(a->values), "chain_query_window: keys and values must be 16-byte aligned");
  CHAIN_QUERY_COMMON_CHECKS(a, "chain_query_window");
  const hipStream_t st = (hipStream_t)stream;
  if (int e = query_products(a->delta, a->dx0, a->mix, a->lam_r, a->lam_0, a->x, a->w_q, a->w_proj_t, a->m, a->P,
                             a->W, a->a3, a->dr, a->wq3, a->wp3, st))
    return e;
  ChainQueryWin q{a->dr, a->pos, a->rel, a->cos_t, a->sin_t, a->keys, a->values,
                  a->T, a->m, a->P, a->W, a->heads, a->S, a->window, a->a3};
  chain_query_window_kernel<<<dim3((unsigned)((a->P + 127) / 128), a->heads, a->m), 256, 0, st>>>(q);
  if (int e = noise::check_launch("chain_query_window")) return e;
  return query_output(a->delta, a->a3, a->wp3, a->m, a->P, a->W, st);
}

extern "C" int noise_chain_head(const noise_chain_head_t* a, void* stream) {
  NOISE_REQUIRE(a, "chain_head: args is NULL");
  NOISE_REQUIRE(a->m >= 0 && a->P > 0 && a->W > 0 && a->W % 256 == 0 && a->W <= 256 * MAXT && a->V > 0 &&
                    a->V % 256 == 0,
                "chain_head: bad sizes (m=%d P=%d W=%d V=%d; W a multiple of 256 up to 2048, V of 256)", a->m,
                a->P, a->W, a->V);
  if (a->m == 0) return NOISE_OK;
  NOISE_REQUIRE(a->delta && a->xL && a->base && a->weight && a->target_w && a->y && a->scale && a->out &&
                    a->dbf && a->inv && a->zy && a->clean,
                "chain_head: NULL argument");
  NOISE_REQUIRE(a->ld_base >= a->V && a->ld_scale >= a->P && a->ld_out >= a->P, "chain_head: row strides too small");
  NOISE_REQUIRE(aligned16(a->dbf) && aligned16(a->weight), "chain_head: dbf and weight must be 16-byte aligned");
  NOISE_REQUIRE((int64_t)a->m * a->P < (1ll << 31), "chain_head: too many rows");
  const hipStream_t st = (hipStream_t)stream;
  const int rows = a->m * a->P;
  chain_head_prep_kernel<<<(rows + 3) / 4, 256, 0, st>>>(a->delta, a->xL, a->base, a->ld_base, a->target_w, a->y,
                                                         rows, a->P, a->W, a->V, a->dbf, a->inv, a->zy);
  if (int e = noise::check_launch("chain_head")) return e;
  chain_clean_kernel<<<(a->m + 3) / 4, 256, 0, st>>>(a->base, a->ld_base, a->xL, a->y, a->m, a->W, a->V, a->clean);
  if (int e = noise::check_launch("chain_head")) return e;
  ChainHead h{a->dbf, a->weight, a->base, a->ld_base, a->inv, a->zy, a->clean, a->scale, a->ld_scale,
              a->y, a->m, a->P, a->W, a->V, a->out, a->ld_out};
  chain_head_kernel<<<(rows + 255) / 256, HCfg::THREADS, 0, st>>>(h);
  return noise::check_launch("chain_head");
}
