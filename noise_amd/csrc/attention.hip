// Windowed causal attention of the population forward, with its fused epilogues.
//
// Reference semantics: attention/window_mask (utils/model.py:17-31) as called by population_loss
// (train/val/eggroll.py:91): softmax(q k^T / sqrt(64)) over keys j with i >= j >= i - window, on
// the normalised, rotated q and k. The epilogue also forms (a) u_proj[r, h] = y_h . b_h, the
// per-head parts of the dot that the c_proj rank-1 term needs (eggroll.py:58, 92), and (b) the
// per-(member, head) first and second moments of y over tokens ("credit moments").
//
// gfx950 mapping: one workgroup = 4 waves = 256 queries of one (member, head); each wave owns 64
// queries as two 32-query MFMA blocks. Scores are formed transposed, S^T = K Q^T with
// v_mfma_f32_32x32x16_bf16, so a lane holds one query and 16 keys of every 32-key block and the
// softmax sum needs no cross-lane traffic until the end. The probabilities are reused in-register
// as the B operand of O^T = V^T P^T (the key order inside an MFMA's K dimension only has to agree
// between the operands); V is staged transposed in LDS with its keys permuted so that each lane's
// 8 keys are one 16-byte read.
//
// Softmax shift: the exponent is shifted by the constant 64 * scale (in log2 units), the largest
// score unit-rms q and k can reach, instead of by a running maximum: probabilities are then final
// when computed, so there is no rescaling of the output accumulators and no max reduction. Softmax
// is invariant to the shift; the constant keeps exp2 in range for every score with
// -80 < q.k * scale < 96 (unit-rms rows give |q.k * scale| <= 64 * scale = 8), which covers
// normalised and N(0, 1) rows alike. Probabilities are rounded to bf16 for the P V product; the
// normaliser sums them unrounded.
//
// Pipeline: K and V of key block b + 1 are in flight into registers while block b is computed,
// and are stored into the other of two LDS buffers after it: one barrier per 64-key block. Only blocks
// that cross the causal diagonal, the window edge or the end of the sequence evaluate the mask.
// Workgroups are numbered so that all query blocks of one (member, head) run on one XCD (the
// hardware deals consecutive workgroup ids round-robin over the 8 XCDs), longest first: that
// head's K and V are then read from HBM once into that XCD's L2.
#include "common.h"

namespace {

constexpr int BQ = 256, BKEY = 64, LDK = 64, NTH = 256;  // 128-byte LDS rows, chunk-swizzled
constexpr float LOG2E = 1.4426950408889634f;

// Every LDS tile here has 128-byte rows of eight 16-byte chunks, chunk c of row r stored at
// c ^ ((r >> 1) & 7): 16 lanes reading one chunk of 16 consecutive rows, or 16 lanes writing two
// whole rows, touch all 64 banks once (padded rows instead conflict on 16-byte stores).
NOISE_DEV int swz(int row, int elem) {  // element offset of (row, elem) within a 64-element row
  return row * LDK + ((((elem >> 3) ^ (row >> 1)) & 7) << 3) + (elem & 7);
}

struct AttnSmem {
  uint16_t kv[2][2][BKEY * LDK];  // [buffer][K | V^T] swizzled [key | dim][dim | permuted key], 32 KB
  float mom[4][2][64];           // per-wave moment partials
};

// LDS column of key k (0..63) in the transposed V tile: within each 32-key half, the keys a lane
// half `h` needs for k-step `ks` (accumulator rows 8a + 4h + b, a in {2ks', 2ks'+1}, b < 4) are
// 8 consecutive columns starting at 16 ks' + 8 h.
NOISE_DEV int vt_pos(int k) {
  const int kb2 = k >> 5, a = (k >> 3) & 3, hh = (k >> 2) & 1, b = k & 3;
  return kb2 * 32 + 16 * (a >> 1) + 8 * hh + 4 * (a & 1) + b;
}

__global__ __launch_bounds__(NTH) __attribute__((amdgpu_waves_per_eu(2, 2)))
void window_attention_kernel(const noise_attention_t g) {
  __shared__ __attribute__((aligned(16))) AttnSmem sm;

  const int T = g.T, window = g.window;
  const int nqb = (T + BQ - 1) / BQ;
  // XCD-aware numbering: xcd = blockIdx.x & 7 is the head; the rest enumerates (member, query
  // block), query blocks of one member consecutive and the longest (last) first.
  const int bid = blockIdx.x;
  const int h = bid & 7;
  const int loc = bid >> 3;
  const int qblk = nqb - 1 - loc % nqb;
  const int p = loc / nqb;
  // The wave index through readfirstlane: the compiler then knows every per-wave quantity below
  // (which blocks a wave needs, which are fully inside the window) is uniform, and branches on it.
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, q32 = lane & 31;
  const int q0 = qblk * BQ;
  const int64_t rowbase = (int64_t)p * T;
  const int64_t ld = g.ldqkv;
  const uint16_t* Qg = g.qkv + h * 64;
  const uint16_t* Kg = g.qkv + 512 + h * 64;
  const uint16_t* Vg = g.qkv + 1024 + h * 64;

  const int wq0 = q0 + w * 64;
  const bool wave_live = wq0 < T;
  const int wq1 = wq0 + 63 < T ? wq0 + 63 : T - 1;

  bf16x8 qf[2][4];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    int qi = wq0 + qb * 32 + q32;
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
  float lsum[2] = {0.f, 0.f};

  const float sl2 = g.scale * LOG2E;
  const float shift = 64.f * g.scale * LOG2E;
  int kfirst = q0 - window;
  kfirst = kfirst < 0 ? 0 : (kfirst & ~(BKEY - 1));
  const int qlast = q0 + BQ - 1 < T ? q0 + BQ - 1 : T - 1;
  const int nblk = (qlast - kfirst) / BKEY + 1;

  // Staging: K as 2 x 16 B (key c >> 3, dims (c & 7) * 8 for c = tid, tid + 256); V as a 4-key x
  // 4-dim patch (keys 4 kg.., dims 4 dg..; the 16 lanes sharing kg read one 128-byte row).
  const int kg = tid >> 4, dg = tid & 15;
  const int kpos = vt_pos(4 * kg);
  u32x4 sk[2];
  u32x2 sv[4];
#define NOISE_ATT_GLOAD(KB)                                                                     \
  {                                                                                           \
    _Pragma("unroll") for (int i = 0; i < 2; ++i) {                                           \
      const int c_ = tid + i * NTH;                                                           \
      int kj_ = (KB) + (c_ >> 3);                                                             \
      kj_ = kj_ < T ? kj_ : T - 1;                                                            \
      sk[i] = *reinterpret_cast<const u32x4*>(Kg + (rowbase + kj_) * ld + (c_ & 7) * 8);      \
    }                                                                                         \
    _Pragma("unroll") for (int r = 0; r < 4; ++r) {                                           \
      int kj_ = (KB) + 4 * kg + r;                                                            \
      kj_ = kj_ < T ? kj_ : T - 1;                                                            \
      sv[r] = *reinterpret_cast<const u32x2*>(Vg + (rowbase + kj_) * ld + 4 * dg);            \
    }                                                                                         \
  }
#define NOISE_ATT_SSTORE(BUF)                                                                   \
  {                                                                                           \
    _Pragma("unroll") for (int i = 0; i < 2; ++i) {                                           \
      const int c_ = tid + i * NTH;                                                           \
      *reinterpret_cast<u32x4*>(&sm.kv[BUF][0][swz(c_ >> 3, (c_ & 7) * 8)]) = sk[i];          \
    }                                                                                         \
    _Pragma("unroll") for (int c = 0; c < 4; ++c) {                                           \
      const int e_ = c >> 1, sh_ = (c & 1) * 16;                                              \
      u32x2 t_;                                                                               \
      t_[0] = ((sv[0][e_] >> sh_) & 0xffffu) | (((sv[1][e_] >> sh_) & 0xffffu) << 16);        \
      t_[1] = ((sv[2][e_] >> sh_) & 0xffffu) | (((sv[3][e_] >> sh_) & 0xffffu) << 16);        \
      *reinterpret_cast<u32x2*>(&sm.kv[BUF][1][swz(4 * dg + c, kpos)]) = t_;                  \
    }                                                                                         \
  }

  NOISE_ATT_GLOAD(kfirst)
  NOISE_ATT_SSTORE(0)
  __syncthreads();
  if (nblk > 1) NOISE_ATT_GLOAD(kfirst + BKEY)

  for (int b = 0; b < nblk; ++b) {
    const int cur = b & 1;
    const int kb = kfirst + b * BKEY;
    // Wave-uniform: does any (query, key) pair of this wave and block fall in the window, and
    // do all of them?
    const bool need = wave_live && kb <= wq1 && kb + BKEY - 1 >= wq0 - window;
    if (need) {
      const bool full = kb + BKEY - 1 <= wq0 && wq0 + 63 - kb <= window && kb + BKEY <= T;
      // One 32-key half at a time: scores, probabilities, then their P V product.
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2) {
        floatx16 s[2];  // [query block]
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int j = 0; j < 16; ++j) s[c][j] = 0.f;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const bf16x8 kf = __builtin_bit_cast(
              bf16x8, *reinterpret_cast<const u32x4*>(&sm.kv[cur][0][swz(kb2 * 32 + q32, ks * 16 + half * 8)]));
#pragma unroll
          for (int qb = 0; qb < 2; ++qb)
            s[qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[qb][ks], s[qb], 0, 0, 0);
        }
        if (full) {
#pragma unroll
          for (int qb = 0; qb < 2; ++qb)
#pragma unroll
            for (int j = 0; j < 16; ++j) {
              const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(s[qb][j], sl2, -shift));
              s[qb][j] = pv;
              lsum[qb] += pv;
            }
        } else {
#pragma unroll
          for (int qb = 0; qb < 2; ++qb) {
            // key kb + kb2*32 + 8(j/4) + 4 half + j%4 is visible iff 0 <= qi - key <= window
            const int base = wq0 + qb * 32 + q32 - kb - kb2 * 32 - 4 * half;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
              const int d = base - (8 * (j >> 2) + (j & 3));
              const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(s[qb][j], sl2, -shift));
              const float pm = (unsigned)d <= (unsigned)window ? pv : 0.f;
              s[qb][j] = pm;
              lsum[qb] += pm;
            }
          }
        }
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          bf16x8 pf[2];
#pragma unroll
          for (int qb = 0; qb < 2; ++qb) {
            u32x4 pk;
#pragma unroll
            for (int e = 0; e < 4; ++e) pk[e] = pack_bf2(s[qb][8 * kk + 2 * e], s[qb][8 * kk + 2 * e + 1]);
            pf[qb] = __builtin_bit_cast(bf16x8, pk);
          }
#pragma unroll
          for (int db = 0; db < 2; ++db) {
            const bf16x8 vf = __builtin_bit_cast(
                bf16x8,
                *reinterpret_cast<const u32x4*>(&sm.kv[cur][1][swz(db * 32 + q32, (kb2 * 2 + kk) * 16 + half * 8)]));
#pragma unroll
            for (int qb = 0; qb < 2; ++qb)
              o[qb][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[qb], o[qb][db], 0, 0, 0);
          }
        }
      }
    }
    if (b + 1 < nblk) NOISE_ATT_SSTORE(cur ^ 1)
    __syncthreads();
    if (b + 2 < nblk) NOISE_ATT_GLOAD(kb + 2 * BKEY)
  }
#undef NOISE_ATT_SSTORE
#undef NOISE_ATT_GLOAD

  // ---- epilogue: normalise, stage bf16 y through LDS for whole-row stores, dot with b_proj,
  // moments. The loop's last barrier has released both K/V buffers: wave w stages its 64 x 64
  // tile in buffer (w >> 1), half (w & 1).
  uint16_t* ys = sm.kv[w >> 1][w & 1];  // swizzled [64 queries][64 dims]
  float mom[64];
#pragma unroll
  for (int i = 0; i < 64; ++i) mom[i] = 0.f;
  const int64_t pn = p >> g.member_shift;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int qi = wq0 + qb * 32 + q32;
    const float lt = lsum[qb] + __shfl_xor(lsum[qb], 32, 64);
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
    const bool valid = qi < T;
    float dot = 0.f;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int jg = 0; jg < 4; ++jg) {
        const int dim = db * 32 + 8 * jg + 4 * half;
        float y[4];
        u32x2 pk;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          pk[e] = pack_bf2(o[qb][db][jg * 4 + 2 * e] * inv, o[qb][db][jg * 4 + 2 * e + 1] * inv);
          y[2 * e] = bf_lo(pk[e]);
          y[2 * e + 1] = bf_hi(pk[e]);
        }
        *reinterpret_cast<u32x2*>(&ys[swz(qb * 32 + q32, dim)]) = pk;
        if (valid) {
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
  __syncthreads();
  // 64 rows x 8 chunks of 16 B: 8 consecutive lanes store one 128-byte row of head h.
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int c = lane + 64 * i, row = c >> 3, c8 = (c & 7) * 8;
    if (wq0 + row < T)
      *reinterpret_cast<u32x4*>(g.y + (rowbase + wq0 + row) * 512 + h * 64 + c8) =
          *reinterpret_cast<const u32x4*>(&ys[swz(row, c8)]);
  }
  if (g.moments) {
    halfwave_transpose_sum(mom, lane);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int i = 2 * q32 + e;
      const int which = i >> 5, r = i & 31;
      const int dim = (r >> 4) * 32 + 8 * ((r & 15) >> 2) + 4 * half + (r & 3);
      sm.mom[w][which][dim] = mom[e];
    }
    __syncthreads();
    if (tid < 128) {
      float* dst = g.scratch + (((int64_t)p * g.heads + h) * nqb + qblk) * 128;
      const int which = tid >> 6, dim = tid & 63;
      dst[tid] = (sm.mom[0][which][dim] + sm.mom[1][which][dim]) + (sm.mom[2][which][dim] + sm.mom[3][which][dim]);
    }
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
  NOISE_REQUIRE(g.scale > 0.f && g.scale <= 0.25f, "window_attention: scale must be in (0, 0.25] (got %g)",
                (double)g.scale);
  NOISE_REQUIRE(g.ldqkv >= 1536 && g.ldqkv % 8 == 0, "window_attention: ldqkv must be >= 1536, multiple of 8");
  NOISE_REQUIRE(!g.b_proj || (g.u_proj && g.ld_b_proj >= 512 && g.ld_b_proj % 4 == 0),
                "window_attention: b_proj needs u_proj and a 4-float aligned row stride >= 512");
  NOISE_REQUIRE(!g.moments || g.scratch, "window_attention: moments need scratch");
  const int nqb = (g.T + BQ - 1) / BQ;
  const int64_t blocks = (int64_t)g.members * g.heads * nqb;
  NOISE_REQUIRE(blocks < (1ll << 31), "window_attention: too many workgroups");
  if (blocks == 0) return NOISE_OK;
  hipStream_t st = (hipStream_t)stream;
  window_attention_kernel<<<(int)blocks, NTH, 0, st>>>(g);
  int rc = noise::check_launch("window_attention");
  if (rc || !g.moments) return rc;
  moments_finalize_kernel<<<g.members * g.heads, 128, 0, st>>>(g.scratch, nqb, g.T, g.moments);
  return noise::check_launch("window_attention moments");
}
