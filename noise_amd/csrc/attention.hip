// Windowed causal attention of the population forward, with its fused epilogues.
//
// Reference semantics: attention/window_mask (utils/model.py:17-31) as called by population_loss
// (train/val/eggroll.py:91): softmax(q k^T / sqrt(64)) over keys j with i >= j >= i - window, on
// the normalised, rotated q and k. The epilogue also forms (a) u_proj[r, h] = y_h . b_h, the
// per-head parts of the dot that the c_proj rank-1 term needs (eggroll.py:58, 92), and (b) the
// per-(member, head) first and second moments of y over tokens ("credit moments").
//
// gfx950 mapping: one workgroup = 2 waves = 128 queries of one (member, head); each wave owns 64
// queries as two 32-query MFMA blocks. Scores are formed transposed, S^T = K Q^T with
// v_mfma_f32_32x32x16_bf16, so a lane holds one query and 16 keys of every 32-key block: the
// running max needs one cross-half exchange per block and the running sum none until the end.
// The probabilities are reused in-register as the B operand of O^T = V^T P^T (the key order inside
// an MFMA's K dimension only has to agree between the operands), with V staged transposed in LDS.
// Key blocks wholly outside a wave's window are skipped.
#include "common.h"

namespace {

constexpr int BQ = 128, BKEY = 64, LDS = 72;

__global__ __launch_bounds__(128) void window_attention_kernel(const noise_attention_t g) {
  __shared__ __attribute__((aligned(16))) uint16_t Ks[BKEY][LDS];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[64][LDS];
  __shared__ float mom_s[2][2][64];

  const int T = g.T;
  const int nqb = (T + BQ - 1) / BQ;
  int bid = blockIdx.x;
  const int qblk = bid % nqb;
  bid /= nqb;
  const int h = bid % g.heads;
  const int p = bid / g.heads;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int half = lane >> 5, q32 = lane & 31;
  const int q0 = qblk * BQ;
  const int64_t rowbase = (int64_t)p * T;
  const int64_t ld = g.ldqkv;
  const uint16_t* Qg = g.qkv + h * 64;
  const uint16_t* Kg = g.qkv + 512 + h * 64;
  const uint16_t* Vg = g.qkv + 1024 + h * 64;

  bf16x8 qf[2][4];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    int qi = q0 + w * 64 + qb * 32 + q32;
    qi = qi < T ? qi : T - 1;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qf[qb][ks] = __builtin_bit_cast(
          bf16x8, *reinterpret_cast<const u32x4*>(Qg + (rowbase + qi) * ld + ks * 16 + half * 8));
  }

  floatx16 o[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int j = 0; j < 16; ++j) o[a][b][j] = 0.f;
  float mrow[2] = {-INFINITY, -INFINITY}, lrow[2] = {0.f, 0.f};

  const float sl2 = g.scale * 1.4426950408889634f;
  const int wq_lo = q0 + w * 64;
  const int wq_hi = (q0 + w * 64 + 63 < T ? q0 + w * 64 + 63 : T - 1);
  const int q_last = (q0 + BQ - 1 < T ? q0 + BQ - 1 : T - 1);
  int kstart = q0 - g.window;
  kstart = kstart < 0 ? 0 : (kstart / BKEY) * BKEY;

  for (int kb = kstart; kb <= q_last; kb += BKEY) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int chunk = tid + i * 128;
      const int key = chunk >> 3, c8 = (chunk & 7) * 8;
      int kj = kb + key;
      kj = kj < T ? kj : T - 1;
      const u32x4 kv = *reinterpret_cast<const u32x4*>(Kg + (rowbase + kj) * ld + c8);
      const u32x4 vv = *reinterpret_cast<const u32x4*>(Vg + (rowbase + kj) * ld + c8);
      *reinterpret_cast<u32x4*>(&Ks[key][c8]) = kv;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        Vt[c8 + 2 * e][key] = (uint16_t)(vv[e] & 0xffff);
        Vt[c8 + 2 * e + 1][key] = (uint16_t)(vv[e] >> 16);
      }
    }
    __syncthreads();
    const bool active = wq_lo < T && kb <= wq_hi && wq_lo - g.window <= kb + BKEY - 1;
    if (!active) continue;

    floatx16 s[2][2];  // [key block][query block]
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int j = 0; j < 16; ++j) s[a][b][j] = 0.f;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2) {
        const bf16x8 kf = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const u32x4*>(&Ks[kb2 * 32 + q32][ks * 16 + half * 8]));
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
          s[kb2][qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[qb][ks], s[kb2][qb], 0, 0, 0);
      }
    }

#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const int qi = q0 + w * 64 + qb * 32 + q32;
      float mx = -INFINITY;
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int kj = kb + kb2 * 32 + 8 * (j >> 2) + 4 * half + (j & 3);
          const bool ok = kj <= qi && qi - kj <= g.window && kj < T;
          const float v = ok ? s[kb2][qb][j] * sl2 : -INFINITY;
          s[kb2][qb][j] = v;
          mx = fmaxf(mx, v);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mnew = fmaxf(mrow[qb], mx);
      const float muse = mnew == -INFINITY ? 0.f : mnew;
      const float alpha = exp2f(mrow[qb] - muse);
      mrow[qb] = mnew;
      float ls = 0.f;
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const float pv = exp2f(s[kb2][qb][j] - muse);
          s[kb2][qb][j] = pv;
          ls += pv;
        }
      lrow[qb] = lrow[qb] * alpha + ls;
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int j = 0; j < 16; ++j) o[qb][db][j] *= alpha;
    }

#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int kb2 = ks >> 1, jb = (ks & 1) * 8;
      bf16x8 pf[2];
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        u32x4 pk;
#pragma unroll
        for (int e = 0; e < 4; ++e) pk[e] = pack_bf2(s[kb2][qb][jb + 2 * e], s[kb2][qb][jb + 2 * e + 1]);
        pf[qb] = __builtin_bit_cast(bf16x8, pk);
      }
      const int kbase = kb2 * 32 + 16 * (ks & 1) + 4 * half;
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        const int dim = db * 32 + q32;
        const u32x2 lo = *reinterpret_cast<const u32x2*>(&Vt[dim][kbase]);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(&Vt[dim][kbase + 8]);
        u32x4 vk;
        vk[0] = lo[0]; vk[1] = lo[1]; vk[2] = hi[0]; vk[3] = hi[1];
        const bf16x8 vf = __builtin_bit_cast(bf16x8, vk);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
          o[qb][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[qb], o[qb][db], 0, 0, 0);
      }
    }
  }

  // ---- epilogue: normalise, store bf16 y, dot with b_proj, moments ----
  float mom[64];
#pragma unroll
  for (int i = 0; i < 64; ++i) mom[i] = 0.f;
  const int64_t pn = p >> g.member_shift;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int qi = q0 + w * 64 + qb * 32 + q32;
    const float lt = lrow[qb] + __shfl_xor(lrow[qb], 32, 64);
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
    const bool valid = qi < T;
    float dot = 0.f;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int jg = 0; jg < 4; ++jg) {
        const int dim = db * 32 + 8 * jg + 4 * half;
        float y[4];
        uint32_t pk[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          pk[e] = pack_bf2(o[qb][db][jg * 4 + 2 * e] * inv, o[qb][db][jg * 4 + 2 * e + 1] * inv);
          y[2 * e] = bf_lo(pk[e]);
          y[2 * e + 1] = bf_hi(pk[e]);
        }
        if (valid) {
          *reinterpret_cast<uint2*>(g.y + (rowbase + qi) * 512 + h * 64 + dim) = make_uint2(pk[0], pk[1]);
          if (g.b_proj) {
            const float4 bv = *reinterpret_cast<const float4*>(g.b_proj + pn * g.ld_b_proj + h * 64 + dim);
            dot += y[0] * bv.x + y[1] * bv.y + y[2] * bv.z + y[3] * bv.w;
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            mom[db * 16 + jg * 4 + e] += y[e];
            mom[32 + db * 16 + jg * 4 + e] += y[e] * y[e];
          }
        }
      }
    if (g.b_proj) {
      dot += __shfl_xor(dot, 32, 64);
      if (valid && half == 0) g.u_proj[(rowbase + qi) * g.heads + h] = dot;
    }
  }
  if (g.moments) {
    halfwave_transpose_sum(mom, lane);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int i = 2 * q32 + e;
      const int which = i >> 5, r = i & 31;
      const int dim = (r >> 4) * 32 + 8 * ((r & 15) >> 2) + 4 * half + (r & 3);
      mom_s[w][which][dim] = mom[e];
    }
    __syncthreads();
    float* dst = g.scratch + (((int64_t)p * g.heads + h) * nqb + qblk) * 128;
    dst[tid] = mom_s[0][tid >> 6][tid & 63] + mom_s[1][tid >> 6][tid & 63];
  }
}

__global__ __launch_bounds__(128) void moments_finalize_kernel(const float* __restrict__ scratch, int nqb,
                                                               int T, float* __restrict__ moments) {
  const float* src = scratch + (int64_t)blockIdx.x * nqb * 128 + threadIdx.x;
  float s = 0.f;
  for (int q = 0; q < nqb; ++q) s += src[q * 128];
  moments[(int64_t)blockIdx.x * 128 + threadIdx.x] = s / (float)T;
}

}  // namespace

extern "C" int noise_window_attention(const noise_attention_t* args, void* stream) {
  NOISE_REQUIRE(args && args->qkv && args->y, "window_attention: null qkv or y");
  const noise_attention_t& g = *args;
  NOISE_REQUIRE(g.members >= 0 && g.T > 0 && g.heads == 8 && g.window >= 0,
                "window_attention: need heads == 8, T > 0, window >= 0 (got heads=%d T=%d window=%d)",
                g.heads, g.T, g.window);
  NOISE_REQUIRE(g.ldqkv >= 1536 && g.ldqkv % 8 == 0, "window_attention: ldqkv must be >= 1536, multiple of 8");
  NOISE_REQUIRE(!g.b_proj || (g.u_proj && g.ld_b_proj >= 512 && g.ld_b_proj % 4 == 0),
                "window_attention: b_proj needs u_proj and a 4-float aligned row stride >= 512");
  NOISE_REQUIRE(!g.moments || g.scratch, "window_attention: moments need scratch");
  const int nqb = (g.T + BQ - 1) / BQ;
  const int64_t blocks = (int64_t)g.members * g.heads * nqb;
  NOISE_REQUIRE(blocks < (1ll << 31), "window_attention: too many workgroups");
  if (blocks == 0) return NOISE_OK;
  hipStream_t st = (hipStream_t)stream;
  window_attention_kernel<<<(int)blocks, 128, 0, st>>>(g);
  int rc = noise::check_launch("window_attention");
  if (rc || !g.moments) return rc;
  moments_finalize_kernel<<<g.members * g.heads, 128, 0, st>>>(g.scratch, nqb, g.T, g.moments);
  return noise::check_launch("window_attention moments");
}
