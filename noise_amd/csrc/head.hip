// Perturbed fp32-accurate head + soft-cap + cross-entropy; the logits leave the chip only when the
// caller asks for them (the scoring forward without targets).
//
// Reference semantics (train/val/eggroll.py:94-102; utils/model.py:203-209): for every member
// row r, z = h_r (W + s a b^T)^T over the whole vocabulary, z' = 15 tanh(z / 15), and
// ce_r = logsumexp(z') - z'[target], or 0 when the target is the ignore_index. The reference materialises [32, T, V] fp32 logits per slice;
// here a workgroup (8 waves) owns 256 rows and sweeps the vocabulary in 256-column tiles of
// mma_tile<256> (measured 5% faster than two 4-wave workgroups on 128-column tiles), keeping only
// per-row running sums of exp(z') (the soft-cap bounds z' to [-15, 15], so no running max is
// needed in fp32) and the target's z'.
//
// Weight precision: w_hi = bf16(W) alone is the bf16 product the reference's trainer runs under
// autocast (train/val/eggroll.py:144-145). With w_lo = bf16(W - w_hi) as well, every tile
// accumulates h w_hi^T + h w_lo^T, which reproduces h W^T to about 2^-17 relative (fp32 weight
// accuracy at twice the MFMA work; h itself is the bf16 GEMM input either way).
#include <utility>

#include "mma_tile.h"

namespace {

constexpr int HBN = 256, HWN = HBN / 64;
constexpr int HNS = 2, HKB = 64;  // two 64-deep stages
using HCfg = noise::TileCfg<HBN, HNS, HKB>;
constexpr int HT = HCfg::THREADS;

// ALIGNED: every 256-row tile lies inside one member (T % 256 == 0), so the rank-1 vector a is one
// row per tile; the general instantiation reads a per row (and is only used for ragged T).
// LOGITS: also store every capped logit (the scoring forward without targets); the loss-only
// instantiation keeps no trace of the store.
constexpr int TGT_IGNORED = -2, TGT_INVALID = -1;

template <bool ALIGNED, bool LOGITS>
__global__ void __attribute__((amdgpu_flat_work_group_size(HT, HT), amdgpu_waves_per_eu(2, 2)))
head_ce_kernel(const noise_head_t g) {
  // One LDS object (per-row data first, where every access is an immediate offset, then the tile
  // buffers): the tile's direct global -> LDS loads are synchronised by explicit waits, and a
  // single object keeps the compiler from adding conservative waits for them before unrelated
  // LDS reads.
  constexpr int ROWS_BYTES = (3 + HWN) * 256 * 4;
  __shared__ __attribute__((aligned(16))) unsigned char lds[ROWS_BYTES + 2 * HCfg::SMEM_ELEMS];
  float* su_s = reinterpret_cast<float*>(lds);
  int* tgt_s = reinterpret_cast<int*>(lds + 1024);
  float* tz_s = reinterpret_cast<float*>(lds + 2048);
  float(*sum_s)[256] = reinterpret_cast<float(*)[256]>(lds + 3072);
  uint16_t* smem = reinterpret_cast<uint16_t*>(lds + ROWS_BYTES);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / HWN, wn = wave % HWN;
  const int m0 = blockIdx.x * 256;
  const int T = g.T;
  const bool perturbed = g.sign != nullptr;
  if (tid < 256) {
    const int row = m0 + tid;
    float su = 0.f;
    int tg = TGT_INVALID;
    if (row < g.M) {
      if (perturbed) su = g.sign[row / T] * g.u[row];
      const int64_t t = g.targets[(int64_t)(row / T) * g.targets_stride + row % T];
      tg = (t >= 0 && t < g.V) ? (int)t : (t == g.ignore_index ? TGT_IGNORED : TGT_INVALID);
    }
    su_s[tid] = su;
    tgt_s[tid] = tg;
    tz_s[tid] = __builtin_nanf("");  // stays NaN for a row whose target is out of range
  }
  const int last_row = (m0 + 256 < g.M ? m0 + 256 : g.M) - 1;
  const bool uniform = ALIGNED || (m0 / T) == (last_row / T);
  const int64_t pn0 = (int64_t)(m0 / T) >> g.member_shift;

  float rsum[4] = {0.f, 0.f, 0.f, 0.f};
  const uint16_t* A = g.h + (int64_t)m0 * 512;
  for (int n0 = 0; n0 < g.V; n0 += HBN) {
    floatx16 acc[4][2];
    noise::zero_acc(acc);
    noise::mma_tile<HBN, HNS, HKB>(A, 512, g.M - m0, g.w_hi + (int64_t)n0 * 512, 512, 512, smem, acc,
                         g.w_lo ? g.w_lo + (int64_t)n0 * 512 : nullptr);
    const int colbase = n0 + wn * 64 + (lane & 31);
    float a_val[2] = {0.f, 0.f};
    if (perturbed && uniform) {
#pragma unroll
      for (int ni = 0; ni < 2; ++ni) a_val[ni] = g.a[pn0 * g.lda + colbase + ni * 32];
    }
// One logit: rank-1 term, soft-cap 15 tanh(z / 15) = 15 - 30 / (exp(2z / 15) + 1) (exact at both
// saturations, absolute error a few 1e-7 near z = 0), exp(c) = exp2(c log2 e) into the row sum,
// and the target's capped logit.
#define NOISE_HEAD_LOGIT(AV)                                                                   \
  {                                                                                          \
    const float z = acc[mi][ni][j] + su * (AV);                                              \
    const float t = __builtin_amdgcn_exp2f(z * (2.0f / 15.0f * 1.4426950408889634f));        \
    const float c = __builtin_fmaf(-30.0f, __builtin_amdgcn_rcpf(t + 1.0f), 15.0f);          \
    e += __builtin_amdgcn_exp2f(c * 1.4426950408889634f);                                    \
    if (colbase + ni * 32 == tg) tz_s[rl] = c;                                               \
    if (LOGITS && m0 + rl < g.M) g.logits[(int64_t)(m0 + rl) * g.ld_logits + colbase + ni * 32] = c; \
  }
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      float es[16];
      if (uniform) {  // every row of the tile is one member: a is per column
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int rl = wm * 128 + mi * 32 + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
          const float su = su_s[rl];
          const int tg = tgt_s[rl];
          float e = 0.f;
#pragma unroll
          for (int ni = 0; ni < 2; ++ni) NOISE_HEAD_LOGIT(a_val[ni])
          es[j] = e;
        }
      } else if (!ALIGNED) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int rl = wm * 128 + mi * 32 + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
          const float su = su_s[rl];
          const int tg = tgt_s[rl];
          const int row = m0 + rl < g.M ? m0 + rl : g.M - 1;
          const float* arow = perturbed ? g.a + ((int64_t)(row / T) >> g.member_shift) * g.lda : nullptr;
          float e = 0.f;
#pragma unroll
          for (int ni = 0; ni < 2; ++ni) NOISE_HEAD_LOGIT(perturbed ? arow[colbase + ni * 32] : 0.f)
          es[j] = e;
        }
      }
      rsum[mi] += noise::halfwave_transpose_sum16(es, lane);
    }
#undef NOISE_HEAD_LOGIT
  }
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
    const int jj = (lane & 31) >> 1;
    const int rl = wm * 128 + mi * 32 + 8 * (jj >> 2) + 4 * (lane >> 5) + (jj & 3);
    if ((lane & 1) == 0) sum_s[wn][rl] = rsum[mi];
  }
  __syncthreads();
  if (tid < 256) {
    const int row = m0 + tid;
    float tot = 0.f;
#pragma unroll
    for (int c = 0; c < HWN; ++c) tot += sum_s[c][tid];
    if (row < g.M) g.ce[row] = tgt_s[tid] == TGT_IGNORED ? 0.f : logf(tot) - tz_s[tid];
  }
}

// ---- Row-resident head (the population step's shape) ----
//
// A workgroup owns 256 rows of one member: eight waves, two per SIMD, 32 rows each. A wave's rows
// are loaded once into 128 AGPRs as the B operand of v_mfma_f32_32x32x16_bf16 (lane l: row l % 32,
// k = 16 ks + 8 (l / 32) .. + 7 of k-step ks), and the weight streams past them in chunks of 32
// vocabulary rows through two LDS stages (rows padded to 1040 bytes: the fragment reads hit 16
// distinct bank groups), fetched a chunk ahead by direct global -> LDS loads spread over the
// chunk's MFMAs: logits^T[32 entries, 32 rows] = W[chunk] h^T, so lane l holds row l % 32 at the
// entries 8 (j / 4) + 4 (l / 32) + j % 4 of the chunk. h is read from HBM once per row (the tile
// kernel above re-reads it for every 256-column vocabulary tile) and every workgroup reads the
// weight once. Chunks alternate between two accumulator sets; the epilogue of chunk c - 1 runs in
// pieces between the MFMAs of chunk c, under the other wave's MFMAs on the SIMD: per value the
// rank-1 term, t = e^(2 z / 15), q = -30 log2(e) / (1 + t) and e^(cap(z) - 15) = 2^q into the row's
// sum (cap(z) = 15 tanh(z / 15) = 15 - 30 / (1 + t); the cap bounds every term to [e^-30, 1]); the
// target's q is picked out after the chunk's values when a lane of the wave has its target there.
// ce = log(sum) + 15 - cap(z_target) = log(sum) - q_target ln 2.
// SPLIT: w_lo as well, each chunk accumulating h w_hi^T then h w_lo^T (64 MFMAs per chunk).
constexpr int RR_ROWS = 256, RR_THREADS = 512, RR_CH = 32, RR_ROW = 1040;
constexpr int RR_AHEAD = 3;  // MFMAs of fragment-read lookahead
constexpr float RR_K1 = 0.19235933878519514f;       // 2 log2(e) / 15
constexpr float RR_K2INV = -0.023104906018664842f;  // 1 / (-30 log2(e))
constexpr float RR_LN2 = 0.69314718055994531f;

template <bool SPLIT>
struct RRCfg {
  static constexpr int STAGE = (SPLIT ? 2 : 1) * RR_CH * RR_ROW;  // 33280 | 66560
  static constexpr int A_OFS = 2 * STAGE;                           // the member's a [V] fp32
  static constexpr int VMAX = 4096;
  static constexpr int LDS = A_OFS + VMAX * 4;                      // 82944 | 149504
  static constexpr int NM = (SPLIT ? 2 : 1) * 32;                   // MFMAs per chunk
  static constexpr int NL = (SPLIT ? 2 : 1) * RR_CH / 8;            // 1-KB loads per wave per chunk
  static constexpr int LS = NM / 2 / NL;                            // MFMAs between two loads
  static constexpr int ES = NM / 16;                                // MFMAs per epilogue value
  static_assert(LDS <= 160 * 1024, "LDS budget");
};

#define RR_DSREAD(DST, ADDR, OFS) __asm__ volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(DST) : "v"(ADDR), "n"(OFS))
#define RR_LGKM(N) __asm__ volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N))

struct RRLane {
  float su;      // sign * u of the lane's row
  int tsel;      // 16 * chunk + value index of the row's target if this lane holds it, else -1
  float esum;    // sum of e^(cap(z) - 15) over this lane's entries
  float tq;      // q of the target (0 unless this lane holds it)
};

// One chunk: its MFMAs into acc[PAR] (FCP), the next chunk's loads (LOAD), and the epilogue of
// chunk cp = c - 1 from acc[1 - PAR] (EPI).
template <bool SPLIT, bool FCP, int PAR, bool EPI>
NOISE_DEV void rr_step(const noise_head_t& g, RRLane& ln, const bf16x8 (&hB)[32], floatx16 (&acc)[2],
                       uint32_t lds_base, unsigned char* lds, int lane, int wave, int c, bool load) {
  using Cf = RRCfg<SPLIT>;
  constexpr int NA = RR_AHEAD + 1, NM = Cf::NM;
  const int half = lane >> 5, cp = c - 1;
  // the previous chunk's a values (entries 8 g + 4 half .. + 3), read before every fragment so that
  // the first fragment wait covers them
  floatx4 av[4];
  if constexpr (EPI) {
    const uint32_t ab = lds_base + Cf::A_OFS + (uint32_t)(cp * RR_CH + 4 * half) * 4;
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) RR_DSREAD(av[gi], ab, 32 * gi);
  }
  const uint32_t fb = lds_base + (uint32_t)(PAR * Cf::STAGE + (lane & 31) * RR_ROW + 16 * half);
  bf16x8 fr[NA];
  // fragment of MFMA S: k-step S % 32 of the hi rows, then (SPLIT) of the lo rows
  auto read = [&fr, fb]<int S>() __attribute__((always_inline)) {
    RR_DSREAD(fr[S % NA], fb, (S >> 5) * RR_CH * RR_ROW + 32 * (S & 31));
  };
  if constexpr (FCP) {
    [&]<int... S>(std::integer_sequence<int, S...>) __attribute__((always_inline)) {
      (read.template operator()<S>(), ...);
    }(std::make_integer_sequence<int, RR_AHEAD>{});
  }
  // next chunk: wave w loads rows 4 w .. 4 w + 3 of the 32 (hi, then lo), 1 KB each
  const int cn = c + 1;
  auto src_row = [&](int k) {
    const int r = (k & 3) + 4 * wave;
    const uint16_t* w = (SPLIT && k >= 4) ? g.w_lo : g.w_hi;
    return w + (int64_t)(cn * RR_CH + r) * 512 + 8 * lane;
  };
  unsigned char* dst0 = lds + (1 - PAR) * Cf::STAGE + 4 * wave * RR_ROW;

  float qv[16];
  auto value = [&]<int J>() __attribute__((always_inline)) {
    constexpr int gi = J >> 2, q = J & 3;
    const float z = acc[1 - PAR][J] + ln.su * av[gi][q];
    const float t = __builtin_amdgcn_exp2f(z * RR_K1);
    const float qq = __builtin_amdgcn_rcpf(__builtin_fmaf(t, RR_K2INV, RR_K2INV));
    ln.esum += __builtin_amdgcn_exp2f(qq);
    qv[J] = qq;
  };
  auto pick = [&]() __attribute__((always_inline)) {
    const int key = 16 * cp;
    if (__builtin_amdgcn_ballot_w64(ln.tsel >= key && ln.tsel < key + 16) != 0) {
#pragma unroll
      for (int j = 0; j < 16; ++j) ln.tq = ln.tsel == key + j ? qv[j] : ln.tq;
    }
  };
  if constexpr (!FCP) {  // the last chunk's epilogue on its own
    RR_LGKM(0);
    __asm__ volatile("" : "+v"(av[0]), "+v"(av[1]), "+v"(av[2]), "+v"(av[3]));
    [&]<int... J>(std::integer_sequence<int, J...>) __attribute__((always_inline)) {
      (value.template operator()<J>(), ...);
    }(std::make_integer_sequence<int, 16>{});
    pick();
    return;
  }
  auto op = [&]<int S>() __attribute__((always_inline)) {
    if constexpr (S % Cf::LS == 0 && S / Cf::LS < Cf::NL) {  // over the chunk's first half
      if (load)
        __builtin_amdgcn_global_load_lds((const void*)src_row(S / Cf::LS),
                                         (void*)(dst0 + ((S / Cf::LS) >> 2) * RR_CH * RR_ROW +
                                                 ((S / Cf::LS) & 3) * RR_ROW),
                                         16, 0, 0);
    }
    if constexpr (S + RR_AHEAD < NM) read.template operator()<S + RR_AHEAD>();
    RR_LGKM(NM - 1 - S < RR_AHEAD ? NM - 1 - S : RR_AHEAD);
    const bf16x8 f = fr[S % NA];
    constexpr int ks = S & 31;
    if constexpr (S == 0)
      __asm__ volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(acc[PAR]) : "v"(f), "a"(hB[ks]));
    else if constexpr (S < NM - 1)
      __asm__ volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(acc[PAR]) : "v"(f), "a"(hB[ks]));
    else
      __asm__ volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
                       : "+v"(acc[PAR]) : "v"(f), "a"(hB[ks]));
    if constexpr (EPI) {
      // value J after MFMA ES J + ES - 1 (the a values were waited for with fragment 0), the
      // target pick after the last value
      if constexpr (S == 0) __asm__ volatile("" : "+v"(av[0]), "+v"(av[1]), "+v"(av[2]), "+v"(av[3]));
      if constexpr (S % Cf::ES == Cf::ES - 1) {
        __builtin_amdgcn_sched_barrier(0);
        value.template operator()<S / Cf::ES>();
        if constexpr (S / Cf::ES == 15) pick();
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  [&]<int... S>(std::integer_sequence<int, S...>) __attribute__((always_inline)) {
    (op.template operator()<S>(), ...);
  }(std::make_integer_sequence<int, NM>{});
}

// Opening of a chunk: its weight rows have landed for this wave, then for every wave; every wave
// is done reading the stage the next chunk goes to.
#define RR_STEP_WAIT() __asm__ volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory")

template <bool SPLIT>
__global__ void __launch_bounds__(RR_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
head_rr_kernel(const noise_head_t g) {
  using Cf = RRCfg<SPLIT>;
  __shared__ __attribute__((aligned(16))) unsigned char lds[Cf::LDS];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int64_t r0 = (int64_t)blockIdx.x * RR_ROWS;
  const int p = (int)(r0 / g.T);  // every row of the workgroup belongs to member p (T % 256 == 0)
  const bool pert = g.sign != nullptr;
  const int64_t pn = (int64_t)(p >> g.member_shift);
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)lds;
  const int nch = g.V / RR_CH;

  // chunk 0's rows into stage 0
  {
#pragma unroll
    for (int k = 0; k < Cf::NL; ++k) {
      const int r = (k & 3) + 4 * wave;
      const uint16_t* w = (SPLIT && k >= 4) ? g.w_lo : g.w_hi;
      __builtin_amdgcn_global_load_lds((const void*)(w + (int64_t)r * 512 + 8 * lane),
                                       (void*)(lds + (k >> 2) * RR_CH * RR_ROW + r * RR_ROW), 16, 0, 0);
    }
  }
  // the wave's 32 rows as B operands, straight into AGPRs
  const int64_t row = r0 + 32 * wave + (lane & 31);
  bf16x8 hB[32];
  {
    const uint16_t* hrow = g.h + row * 512 + 8 * half;
#pragma unroll
    for (int ks = 0; ks < 32; ++ks)
      __asm__ volatile("global_load_dwordx4 %0, %1, off offset:%2" : "=a"(hB[ks]) : "v"(hrow), "n"(32 * ks));
  }
  // the member's a into LDS (zeros unperturbed)
  float* a_s = reinterpret_cast<float*>(lds + Cf::A_OFS);
  for (int i = tid * 4; i < g.V; i += RR_THREADS * 4) {
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (pert) v = *reinterpret_cast<const float4*>(g.a + pn * g.lda + i);
    *reinterpret_cast<float4*>(a_s + i) = v;
  }
  RRLane ln;
  ln.su = pert ? g.sign[p] * g.u[row] : 0.f;
  const int64_t t = g.targets[(int64_t)p * g.targets_stride + (int)(row - (int64_t)p * g.T)];
  const bool t_ok = t >= 0 && t < g.V, t_ign = !t_ok && t == g.ignore_index;
  {
    const int o = (int)(t & (RR_CH - 1));
    const bool mine = t_ok && ((o >> 2) & 1) == half;
    ln.tsel = mine ? 16 * (int)(t >> 5) + 4 * (o >> 3) + (o & 3) : -1;
  }
  ln.esum = 0.f;
  ln.tq = 0.f;
  // the h loads have landed (vector memory retires in order: the stage's direct loads first)
  __asm__ volatile("s_waitcnt vmcnt(0)"
                   : "+a"(hB[0]), "+a"(hB[1]), "+a"(hB[2]), "+a"(hB[3]), "+a"(hB[4]), "+a"(hB[5]), "+a"(hB[6]),
                     "+a"(hB[7]), "+a"(hB[8]), "+a"(hB[9]), "+a"(hB[10]), "+a"(hB[11]), "+a"(hB[12]), "+a"(hB[13]),
                     "+a"(hB[14]), "+a"(hB[15]));
  __asm__ volatile("s_waitcnt vmcnt(0)"
                   : "+a"(hB[16]), "+a"(hB[17]), "+a"(hB[18]), "+a"(hB[19]), "+a"(hB[20]), "+a"(hB[21]),
                     "+a"(hB[22]), "+a"(hB[23]), "+a"(hB[24]), "+a"(hB[25]), "+a"(hB[26]), "+a"(hB[27]),
                     "+a"(hB[28]), "+a"(hB[29]), "+a"(hB[30]), "+a"(hB[31]));

  floatx16 acc[2];
  RR_STEP_WAIT();
  rr_step<SPLIT, true, 0, false>(g, ln, hB, acc, lds_base, lds, lane, wave, 0, nch > 1);
#pragma unroll 1
  for (int c = 1; c + 1 < nch; c += 2) {
    RR_STEP_WAIT();
    rr_step<SPLIT, true, 1, true>(g, ln, hB, acc, lds_base, lds, lane, wave, c, true);
    RR_STEP_WAIT();
    rr_step<SPLIT, true, 0, true>(g, ln, hB, acc, lds_base, lds, lane, wave, c + 1, c + 2 < nch);
  }
  // nch is even (V % 64 == 0): chunk nch - 1 sits in stage 1
  RR_STEP_WAIT();
  rr_step<SPLIT, true, 1, true>(g, ln, hB, acc, lds_base, lds, lane, wave, nch - 1, false);
  rr_step<SPLIT, false, 0, true>(g, ln, hB, acc, lds_base, lds, lane, wave, nch, false);

  const float tot = ln.esum + __shfl_xor(ln.esum, 32, 64);
  const float tq = ln.tq + __shfl_xor(ln.tq, 32, 64);
  if (half == 0 && row < g.M)
    g.ce[row] = t_ign ? 0.f : t_ok ? logf(tot) - tq * RR_LN2 : __builtin_nanf("");
}

}  // namespace

extern "C" int noise_head_ce(const noise_head_t* args, void* stream) {
  NOISE_REQUIRE(args && args->h && args->w_hi && args->targets && args->ce, "head_ce: null argument");
  const noise_head_t& g = *args;
  NOISE_REQUIRE(g.M >= 0 && g.T > 0 && g.V > 0 && g.V % 64 == 0, "head_ce: V=%d must be a positive multiple of 64", g.V);
  NOISE_REQUIRE(!g.sign || (g.a && g.u && g.lda >= g.V), "head_ce: perturbation needs a [*, V] and u");
  NOISE_REQUIRE(((uintptr_t)g.h % 16) == 0 && ((uintptr_t)g.w_hi % 16) == 0 && ((uintptr_t)g.w_lo % 16) == 0,
                "head_ce: h and weights must be 16-byte aligned");
  NOISE_REQUIRE(!g.logits || g.ld_logits >= g.V, "head_ce: ld_logits=%lld < V=%d", (long long)g.ld_logits, g.V);
  NOISE_REQUIRE(g.ignore_index < 0 || g.ignore_index >= g.V,
                "head_ce: ignore_index=%lld is a class index; only out-of-range values can be ignored",
                (long long)g.ignore_index);
  if (g.M == 0) return NOISE_OK;
  const dim3 grid((g.M + 255) / 256);
  hipStream_t s = (hipStream_t)stream;
  // The row-resident kernel where the shape allows it: whole 256-row workgroups inside one member,
  // the member's a in LDS (16-byte aligned rows), no logits out.
  if (g.T % RR_ROWS == 0 && g.M % RR_ROWS == 0 && g.V % 64 == 0 && g.V <= RRCfg<false>::VMAX && !g.logits &&
      (!g.sign || (g.lda % 4 == 0 && ((uintptr_t)g.a % 16) == 0))) {
    if (g.w_lo) head_rr_kernel<true><<<g.M / RR_ROWS, RR_THREADS, 0, s>>>(g);
    else head_rr_kernel<false><<<g.M / RR_ROWS, RR_THREADS, 0, s>>>(g);
    return noise::check_launch("head_ce (row-resident)");
  }
  NOISE_REQUIRE(g.V % 256 == 0, "head_ce: V=%d must be a multiple of 256 unless T and M are multiples of 256, "
                "V <= 4096 and no logits are asked for", g.V);
  if (g.T % 256 == 0) {
    if (g.logits) head_ce_kernel<true, true><<<grid, HT, 0, s>>>(g);
    else head_ce_kernel<true, false><<<grid, HT, 0, s>>>(g);
  } else {
    if (g.logits) head_ce_kernel<false, true><<<grid, HT, 0, s>>>(g);
    else head_ce_kernel<false, false><<<grid, HT, 0, s>>>(g);
  }
  return noise::check_launch("head_ce");
}
