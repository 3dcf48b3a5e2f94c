// Fused MLP block of the population forward, one launch per layer:
//   out = [in +] c_proj(relu(c_fc(norm in) + rank-1)^2) + rank-1
// Reference: train/val/eggroll.py:93 (x + lowrank(c_proj, relu(lowrank(c_fc, norm(x)))^2)),
// utils/model.py:100-107 (relu^2 MLP), `lowrank` eggroll.py:56-58 (x W^T + sign (x . b) a^T).
//
// The [rows, 2048] relu^2 hidden never leaves the chip. A workgroup owns 128 rows of one member
// (four waves, one per SIMD, 32 rows each) and all 512 output columns; the 2048 hidden features
// stream through in chunks of 32:
//   * the wave's rows arrive in one coalesced pass straight into the c_proj accumulators (where
//     they also start the residual sum); the row norms come from cross-lane sums, and h = bf16 of
//     the normalised rows is transposed into the c_fc operand layout by MFMAs against a permuted
//     identity (exact), ending in 128 VGPRs;
//   * c_fc is computed transposed, hid^T[32 features, 32 rows] = W_fc[chunk] h^T, with h as the B
//     operand of v_mfma_f32_32x32x16_bf16. The accumulator of that product gives lane l the hidden
//     values of row l % 32 -- exactly the row the A operand of the c_proj MFMA wants in lane l --
//     for the features 8 (j / 4) + 4 (l / 32) + j % 4 (j = 0..15). Both packed weight copies
//     (noise_mlp_pack) store their K dimension in that order, so the rank-1 term, relu^2 and the
//     bf16 rounding run on the accumulators in registers and their result is the next MFMA's
//     operand;
//   * c_proj accumulates out[32 rows, 512] per wave in 256 registers (16 32x32 blocks);
//   * the weights stream through two LDS stages of one chunk each (c_fc rows padded to 1040 bytes
//     so the fragment reads hit 16 distinct bank groups; the c_proj chunk pre-swizzled in HBM),
//     fetched one chunk ahead by direct global -> LDS loads. Step i runs the 32 c_fc MFMAs of
//     chunk i interleaved with the 32 c_proj MFMAs of chunk i - 1, whose hidden values come out of
//     the other c_fc accumulator set: the epilogue of one chunk overlaps the MFMAs of the next.
// Per row the kernel moves 2 KB in and 2 KB out (fp32), against 18 KB through HBM for the separate
// norm, c_fc and c_proj launches.
#include <stdlib.h>

#include <utility>

#include "mma_tile.h"

namespace noise {
// The two-wave (producer/consumer) form of the plain MLP (mlp_pc.hip): launched, and true, where it
// applies.
bool mlp_pc_launch(const noise_mlp_t& g, hipStream_t st);
}  // namespace noise

namespace {

constexpr int D = 512, F = 2048, FC = 32, NCH = F / FC;
constexpr int ROWS = 128;                        // rows per workgroup
constexpr int WFC_ROW = 1040;                    // bytes per c_fc row in LDS (1 KB + 16 pad)
constexpr int WFC_PART = FC * WFC_ROW;           // 33280
constexpr int WMP_PART = D * FC * 2;             // 32768: [512 rows][32 k] bf16, swizzled
constexpr int STAGE = WFC_PART + WMP_PART;       // 66048
constexpr int NOISE_OFS = 2 * STAGE;             // a_fc [2048] | b_proj [2048] | a_proj [512] | b_fc [512]
constexpr int LDS_BYTES = NOISE_OFS + (2 * F + 2 * D) * 4;  // 152576
// With the next layer's mix_norm in the epilogue: its dot vectors b[0..2] [3][512] | gate W [8][32]
// | gate b [32], staged in the prologue.
constexpr int NEXT_OFS = LDS_BYTES;
constexpr int NEXT_FLOATS = 3 * D + 8 * 32 + 32;  // 1824
constexpr int LDS_NEXT_BYTES = NEXT_OFS + NEXT_FLOATS * 4;  // 159872
constexpr float RMS_EPS = 1.1920928955078125e-07f;  // float32 machine epsilon (F.rms_norm default)
#ifndef MLP_AHEAD
#define MLP_AHEAD 3  // MFMAs of fragment-read lookahead
#endif
#ifndef MLP_NTSTORE
#define MLP_NTSTORE 0  // output rows stored past L2 (non-temporal)
#endif
#ifndef MLP_LSTRIDE
#define MLP_LSTRIDE 2  // MFMAs between two loads of the next stage (measured: 2 is 1.5% faster than 1)
#endif

static_assert(LDS_NEXT_BYTES <= 160 * 1024, "LDS budget");

// Position q (0..15) of a 16-deep k-step of the packed c_proj copy holds hidden feature
// perm16(q) of that step: lanes 0-31 supply k-slots 0-7 from accumulators j = 0..7 of the c_fc
// block (features 0-3, 8-11), lanes 32-63 slots 8-15 (features 4-7, 12-15).
__host__ __device__ constexpr int perm16(int q) { return 8 * ((q & 7) >> 2) + 4 * (q >> 3) + (q & 3); }

// Stage `buf` <- c_fc rows of the cf-th chunk (if cf >= 0) and the packed c_proj cm-th chunk (if
// cm >= 0) of the workgroup's chunk order.
// Each wave issues 8 + 8 direct loads of 1 KB (lane l's 16 bytes land at the base + 16 l).
NOISE_DEV void load_stage(const noise_mlp_t& g, unsigned char* lds, int wave, int lane, int buf, int cf, int cm,
                          int c0) {
  unsigned char* st = lds + buf * STAGE;
  if (cf >= 0) cf = (cf + c0) & (NCH - 1);  // the workgroup's chunk order starts at chunk c0
  if (cm >= 0) cm = (cm + c0) & (NCH - 1);
  if (cf >= 0) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int row = wave * 8 + k;
      __builtin_amdgcn_global_load_lds((const void*)(g.w_fc + (int64_t)(cf * FC + row) * D + lane * 8),
                                       (void*)(st + row * WFC_ROW), 16, 0, 0);
    }
  }
  if (cm >= 0) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int blk = wave * 8 + k;
      __builtin_amdgcn_global_load_lds((const void*)(g.w_proj + (int64_t)cm * (D * FC) + blk * 512 + lane * 8),
                                       (void*)(st + WFC_PART + blk * 1024), 16, 0, 0);
    }
  }
}

// Zero-initialised device memory: the source of the staged vectors a launch does not have
// (unperturbed members, absent dots or gate), so that every piece is one direct load.
__device__ __align__(16) float kZeroRow[256];

// A copy of an accumulator register the compiler cannot reuse: without it the prologue kept VGPR
// copies of all 256 input values alive between its two passes over them and spilled.
NOISE_DEV float agpr_read(float a) {
  float v;
  __asm__ volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(a));
  return v;
}

// The next stage's loads of one wave: 8 c_fc rows and 8 1-KB blocks of the packed c_proj chunk.
// mlp_step issues them one per MFMA pair through the first half of a step: issued back to back
// at the start of the step they stalled the wave's MFMA stream behind the memory pipeline
// (measured at the bench shape: 5.1 -> 4.7 ms per launch).
struct StageLoads {
  const uint16_t* fc_src;  // row wave * 8 of the c_fc chunk, this lane's 16 bytes
  const uint16_t* mp_src;  // block wave * 8 of the c_proj chunk, this lane's 16 bytes
  unsigned char* fc_dst;   // LDS: c_fc row wave * 8 of the stage
  unsigned char* mp_dst;   // LDS: c_proj block wave * 8 of the stage
};

NOISE_DEV StageLoads stage_loads(const noise_mlp_t& g, unsigned char* lds, int wave, int lane, int buf, int cf,
                                 int cm, int c0) {
  cf = (cf + c0) & (NCH - 1);
  cm = (cm + c0) & (NCH - 1);
  unsigned char* st = lds + buf * STAGE;
  return StageLoads{g.w_fc + (int64_t)(cf * FC + wave * 8) * D + lane * 8,
                    g.w_proj + (int64_t)cm * (D * FC) + wave * 8 * 512 + lane * 8, st + wave * 8 * WFC_ROW,
                    st + WFC_PART + wave * 8 * 1024};
}

NOISE_DEV bf16x8 as_bf16x8(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3) {
  return __builtin_bit_cast(bf16x8, (u32x4){w0, w1, w2, w3});
}

// ds_read_b128 at a byte address + immediate offset, invisible to the compiler's wait counting
// (every read is waited for explicitly with lgkm_wait).
#define MLP_DSREAD(DST, ADDR, OFS) __asm__ volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(DST) : "v"(ADDR), "n"(OFS))
#define MLP_LGKM(N) __asm__ volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N))

// The MFMA order of one step. With both halves: F0..F7 (c_fc k-steps 0-7) while the epilogue of
// the previous chunk produces the operand of the first 16 c_proj MFMAs, then P0 F8 P1 F9 ... P23
// F31, then P24..P31 (P t: c_proj block t & 15, k-step t >> 4); the epilogue's second half runs
// among the interleaved ones, before P16. With one half, its 32 MFMAs in order.
template <bool FCP, bool PRJ>
struct StepOps {
  static constexpr int N = (FCP ? 32 : 0) + (PRJ ? 32 : 0);
  static constexpr int NF0 = 8;  // leading c_fc MFMAs
  static constexpr bool is_fc(int s) {
    return !PRJ ? true : !FCP ? false : s < NF0 ? true : (s - NF0 >= 2 * (32 - NF0) ? false : ((s - NF0) & 1) != 0);
  }
  static constexpr int idx(int s) {
    return (!PRJ || !FCP || s < NF0) ? s
           : (s - NF0 >= 2 * (32 - NF0) ? (32 - NF0) + (s - NF0 - 2 * (32 - NF0))
                                         : (((s - NF0) & 1) ? NF0 + ((s - NF0) >> 1) : (s - NF0) >> 1));
  }
  // The epilogue piece that follows c_fc MFMA i, or -1: pieces 0-3 (the operand of P0..P15) after
  // F3..F6, pieces 4-7 (that of P16..P31) after F10, F14, F18, F22 -- all after F3, whose fragment
  // wait also covers the perturbation values (read after the first fragments).
  static constexpr int piece_after(int i) {
    return i >= 3 && i <= 6 ? i - 3 : i >= 10 && i <= 22 && (i - 10) % 4 == 0 ? 4 + (i - 10) / 4 : -1;
  }
  static constexpr int FIRST_PIECE = 3;
  // With both halves: every piece runs before the c_proj MFMAs that read its values (pieces 0-3
  // before P0, 4-7 before P16).
  static constexpr bool pieces_in_order() {
    int seen = 0;
    for (int s = 0; s < N; ++s) {
      if (is_fc(s) && piece_after(idx(s)) >= 0) ++seen;
      if (!is_fc(s) && ((idx(s) == 0 && seen < 4) || (idx(s) == 16 && seen < 8))) return false;
    }
    return seen == 8;
  }
};

// One step of the chunk pipeline. FCP: the c_fc MFMAs of chunk `cf` into fc[FB]; PRJ: turn
// fc[1 - FB] (chunk cf - 1) into the c_proj operand (rank-1 term, relu^2, bf16, u_proj dots) and
// run its 32 c_proj MFMAs. Stage buffer `buf` holds c_fc rows of chunk cf and c_proj chunk cf - 1;
// the 16 loads of the next stage (LFC, LMP) are issued one every MLP_LSTRIDE MFMAs from the
// step's first. Every MFMA is
// inline asm so that the c_fc accumulators stay in VGPRs and the c_proj ones in AGPRs; the hazards
// the compiler then cannot see are covered explicitly: 2 wait states between the VALU writing the
// c_proj operand and its first MFMA, and 24 after a chunk's last MFMA before VALU reads its result.
// Fragments are read MLP_AHEAD MFMAs ahead; the epilogue's perturbation values right after the
// first MLP_AHEAD fragments (before all of them in the last step), so the fragment wait before the
// first piece covers them too.
template <bool FCP, bool PRJ, int FB, bool LFC, bool LMP>
NOISE_DEV void mlp_step(const bf16x8 (&hB)[32], floatx16 (&fc)[2], floatx16 (&acc)[16], float& up,
                        uint32_t fcb, uint32_t mpb0, uint32_t mpb1, uint32_t ab_base, int chunk_prev, float su,
                        int c0, const StageLoads& ld) {
  using O = StepOps<FCP, PRJ>;
  constexpr int NA = MLP_AHEAD + 1;
  floatx4 av[4], bv[4];
  // Perturbation values of the previous chunk: this lane's features base + 8 g + 4 half + q. In a
  // step with both halves they are read after the first MLP_AHEAD fragments, so that the first
  // MFMA waits for its own fragment only (measured: 1.5-2.5% per launch); the last step, whose
  // epilogue runs before its MFMAs, reads them first.
  constexpr bool LATE = FCP && PRJ;
  const uint32_t ab = ab_base + (uint32_t)(((chunk_prev + c0) & (NCH - 1)) * FC * 4);
  auto read_ab = [&av, &bv, ab]() __attribute__((always_inline)) {
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
      MLP_DSREAD(av[gi], ab, 32 * gi);
      MLP_DSREAD(bv[gi], ab, 4 * F + 32 * gi);
    }
  };
  if (PRJ && !LATE) read_ab();
  bf16x8 fr[NA];
  // Fragment read for op S (S a compile-time constant, so the offsets are immediates).
  auto read = [&, fcb, mpb0, mpb1]<int S>() __attribute__((always_inline)) {
    constexpr int i = O::idx(S);
    if constexpr (O::is_fc(S)) MLP_DSREAD(fr[S % NA], fcb, 32 * i);
    else if constexpr (i < 16) MLP_DSREAD(fr[S % NA], mpb0, 2048 * (i & 15));
    else MLP_DSREAD(fr[S % NA], mpb1, 2048 * (i & 15));
  };
  [&]<int... S>(std::integer_sequence<int, S...>) __attribute__((always_inline)) {
    (read.template operator()<S>(), ...);
  }(std::make_integer_sequence<int, MLP_AHEAD>{});
  if (LATE) read_ab();
  static_assert(!LATE || O::FIRST_PIECE >= MLP_AHEAD, "the perturbation values must be in by the first piece");
  static_assert(!(FCP && PRJ) || O::pieces_in_order(), "an epilogue piece after the MFMA that reads it");
  uint32_t hw[8];
  bf16x8 hid[2];
  // Epilogue piece e (0..7): values 2 e, 2 e + 1 of the previous chunk's accumulators; pieces 0-3
  // make the operand of the first 16 c_proj MFMAs, pieces 4-7 that of the last 16.
  auto epi = [&]<int E>() __attribute__((always_inline)) {
    constexpr int gi = E >> 1, q = 2 * (E & 1);
    const float v0 = fmaxf(fc[1 - FB][2 * E] + su * av[gi][q], 0.f);
    const float v1 = fmaxf(fc[1 - FB][2 * E + 1] + su * av[gi][q + 1], 0.f);
    const uint32_t w = pack_bf2(v0 * v0, v1 * v1);
    hw[E] = w;
    up += bf_lo(w) * bv[gi][q] + bf_hi(w) * bv[gi][q + 1];
    if constexpr (E == 3) hid[0] = as_bf16x8(hw[0], hw[1], hw[2], hw[3]);
    if constexpr (E == 7) hid[1] = as_bf16x8(hw[4], hw[5], hw[6], hw[7]);
  };
  if constexpr (PRJ && !FCP) {  // last step: the epilogue runs first
    MLP_LGKM(MLP_AHEAD);
    __asm__ volatile("" : "+v"(av[0]), "+v"(av[1]), "+v"(av[2]), "+v"(av[3]), "+v"(bv[0]), "+v"(bv[1]), "+v"(bv[2]),
                     "+v"(bv[3]));
    [&]<int... E>(std::integer_sequence<int, E...>) __attribute__((always_inline)) {
      (epi.template operator()<E>(), ...);
    }(std::make_integer_sequence<int, 8>{});
  }
  auto op = [&]<int SX>() __attribute__((always_inline)) {
    // Load k of the next stage goes out with MFMA LS * k (all 16 within the step's MFMAs).
    constexpr int LS = O::N >= 16 * MLP_LSTRIDE ? MLP_LSTRIDE : O::N / 16;
    constexpr int LK = SX / LS;
    static_assert(16 * LS <= O::N, "every load of the next stage must be issued");
    if constexpr (SX % LS == 0 && LFC && LK < 8)
      __builtin_amdgcn_global_load_lds((const void*)(ld.fc_src + LK * D), (void*)(ld.fc_dst + LK * WFC_ROW), 16, 0, 0);
    if constexpr (SX % LS == 0 && LMP && LK >= 8 && LK < 16)
      __builtin_amdgcn_global_load_lds((const void*)(ld.mp_src + (LK - 8) * 512), (void*)(ld.mp_dst + (LK - 8) * 1024),
                                       16, 0, 0);
    if constexpr (SX + MLP_AHEAD < O::N) read.template operator()<SX + MLP_AHEAD>();
    // fragments read after this op's, plus the 8 perturbation reads while they are younger
    MLP_LGKM((O::N - 1 - SX < MLP_AHEAD ? O::N - 1 - SX : MLP_AHEAD) + (LATE && SX < MLP_AHEAD ? 8 : 0));
    const bf16x8 f = fr[SX % NA];
    constexpr int i = O::idx(SX);
    if constexpr (O::is_fc(SX)) {
      if constexpr (i == 0)
        __asm__ volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(fc[FB]) : "v"(f), "v"(hB[i]));
      else if constexpr (i < 31)
        __asm__ volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(fc[FB]) : "v"(f), "v"(hB[i]));
      else
        __asm__ volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
                         : "+v"(fc[FB]) : "v"(f), "v"(hB[i]));
      if constexpr (PRJ && i == O::FIRST_PIECE)  // the wait before this MFMA covered them
        __asm__ volatile("" : "+v"(av[0]), "+v"(av[1]), "+v"(av[2]), "+v"(av[3]), "+v"(bv[0]), "+v"(bv[1]),
                         "+v"(bv[2]), "+v"(bv[3]));
      if constexpr (PRJ && O::piece_after(i) >= 0) {  // held in place by the scheduling barriers
        __builtin_amdgcn_sched_barrier(0);
        epi.template operator()<O::piece_after(i)>();
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      if constexpr (i == 0 || i == 16)
        __asm__ volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0"
                         : "+a"(acc[i & 15]) : "v"(hid[i >> 4]), "v"(f));
      else if constexpr (i < 31 || FCP)
        __asm__ volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc[i & 15]) : "v"(hid[i >> 4]), "v"(f));
      else
        __asm__ volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
                         : "+a"(acc[i & 15]) : "v"(hid[i >> 4]), "v"(f));
    }
  };
  [&]<int... S>(std::integer_sequence<int, S...>) __attribute__((always_inline)) {
    (op.template operator()<S>(), ...);
  }(std::make_integer_sequence<int, O::N>{});
}

// The next layer's mix_norm on the wave's finished rows, straight from the c_proj accumulators
// (lane l: column 32 nb + l % 32 of rows tb + 8 (j / 4) + 4 (l / 32) + j % 4), in the arithmetic of
// noise_mix_norm (norm.hip): x = (lr + s er) (acc + rank-1) + (l0 + s e0) x0 (MIX: x0 given),
// written back to the stream; h = bf16(x rsqrt(mean x^2 + eps)) into the wave's 32 KB LDS tile,
// one row at a time (the norm is a half-wave sum); then from the tile: h as whole rows, the dots
// u_k = h . b_k (lane l: columns 8 l .. 8 l + 7 of every row, summed across the wave), and the gate
// 2 sigmoid(h[:32] (Wg + s a b^T)^T). The accumulators are only read; b, Wg and b_g were staged
// in LDS by the prologue.
template <bool MIX>
NOISE_DEV void mix_norm_epilogue(const noise_mlp_t& g, const noise_mixnorm_t& nx, const floatx16 (&acc)[16],
                                 const float (&am)[16], float sup, unsigned char* lds, int wave, int lane, int p,
                                 int tb) {
  // Opaque copies of the row coordinates: the addresses below are then formed here, not hoisted
  // above the main loop (where they would only wait in scratch memory).
  float* const out = g.out;
  const float* const x0p = nx.x0;
  uint16_t* const hp = nx.h;
  __asm__ volatile("" : "+s"(tb), "+v"(lane));
  const int r = lane & 31, half = lane >> 5;
  const int64_t pn = (int64_t)(p >> nx.member_shift);
  const float s = nx.sign ? nx.sign[p] : 0.f;
  const float* s_next = reinterpret_cast<const float*>(lds + NEXT_OFS);
  float lr = 1.f, l0 = 0.f;
  if constexpr (MIX) {
    lr = *nx.resid;
    l0 = *nx.mix;
    if (nx.sign) {
      lr += s * nx.eps_resid[pn * nx.ld_eps];
      l0 += s * nx.eps_mix[pn * nx.ld_eps];
    }
  }
  const int64_t mrow0 = (int64_t)p * g.T;  // the member's first row in nx's [M, 512] layout
  // x0 rows arrive XA rows ahead of their use, in a ring of XA x 16 registers
  constexpr int XA = 2;
  float x0v[XA][16];
  auto x0_load = [&](int j, float (&dst)[16]) {
    const int rj = tb + 8 * (j >> 2) + 4 * half + (j & 3);
    const float* src = x0p + (mrow0 + (rj < g.T ? rj : g.T - 1)) * D + r;
#pragma unroll
    for (int nb = 0; nb < 16; ++nb) dst[nb] = src[nb * 32];
  };
  if constexpr (MIX) {
#pragma unroll
    for (int j = 0; j < XA; ++j) x0_load(j, x0v[j]);
  }
  // The wave's LDS tile [32 rows][1 KB] of h: the four tiles cover both stage buffers, which
  // other waves may still be reading in their last step.
  static_assert(4 * 32 * 1024 <= NOISE_OFS, "h tiles must fit below the noise vectors");
  __syncthreads();
  uint16_t* tile = reinterpret_cast<uint16_t*>(lds + wave * 32 * 1024);
  float h0[16];  // h of column r (block 0) of each of the lane's rows: the gate's inputs
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int rl = 8 * (j >> 2) + 4 * half + (j & 3);
    const float sr = __shfl(sup, rl, 64);
    float v[16], ss = 0.f;
#pragma unroll
    for (int nb = 0; nb < 16; ++nb) {
      v[nb] = acc[nb][j] + sr * am[nb];
      if constexpr (MIX) v[nb] = lr * v[nb] + l0 * x0v[j % XA][nb];
      ss += v[nb] * v[nb];
    }
    if constexpr (MIX) {
      if (j + XA < 16) x0_load(j + XA, x0v[j % XA]);
    }
    if (tb + rl < g.T) {
      float* dst = out + (mrow0 + tb + rl) * D + r;
#pragma unroll
      for (int nb = 0; nb < 16; ++nb) dst[nb * 32] = v[nb];
    }
    const float rr = rsqrtf(noise::halfwave_sum(ss) * (1.0f / D) + RMS_EPS);
#pragma unroll
    for (int nb = 0; nb < 16; ++nb) {
      const uint16_t hb = f2bf(v[nb] * rr);
      tile[rl * 512 + nb * 32 + r] = hb;
      if (nb == 0) h0[j] = bf2f(hb);
    }
  }
  // From the tile (a wave's LDS operations run in order; the compiler barrier keeps the 16-byte
  // reads after the 2-byte writes): lane l holds bytes 16 l .. 16 l + 15 (columns 8 l .. 8 l + 7)
  // of each row. Pass k = 0 also writes the rows out.
  __asm__ volatile("" ::: "memory");
  const int nbv = nx.nb;
  // after the transpose sum, lane l (even) holds the total of row 16 (l / 32) + ((l % 32) >> 1)
  const int rw = tb + 16 * half + (r >> 1);
  const bool writer = (r & 1) == 0 && rw < g.T;
#pragma unroll 1
  for (int k = 0; k < (nbv > 1 ? nbv : 1); ++k) {
    float bk[8];
    {
      const float4 b0 = *reinterpret_cast<const float4*>(s_next + k * D + 8 * lane);
      const float4 b1 = *reinterpret_cast<const float4*>(s_next + k * D + 8 * lane + 4);
      bk[0] = b0.x; bk[1] = b0.y; bk[2] = b0.z; bk[3] = b0.w;
      bk[4] = b1.x; bk[5] = b1.y; bk[6] = b1.z; bk[7] = b1.w;
    }
    float part[32];
#pragma unroll
    for (int rl = 0; rl < 32; ++rl) {
      const u32x4 hv = *reinterpret_cast<const u32x4*>(tile + rl * 512 + 8 * lane);
      if (k == 0 && tb + rl < g.T) *reinterpret_cast<u32x4*>(hp + (mrow0 + tb + rl) * D + 8 * lane) = hv;
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) d += bf_lo(hv[e]) * bk[2 * e] + bf_hi(hv[e]) * bk[2 * e + 1];
      part[rl] = d;
    }
    if (k < nbv) {
      const float tot = noise::wave_transpose_sum32(part, lane);
      if (writer) nx.u[(mrow0 + rw) * nx.ldu + k] = tot;
    }
  }
  if (nx.gate_w) {
    // gate logit q of a row: its 32 columns of h . Wg[q], plus s (h[:32] . b_g) a_g[q]; rows in the
    // accumulator layout, lane q (even) of a half ends with row 8 (jj / 4) + 4 half + jj % 4,
    // jj = (q >> 1) & 15
    const int jj = (r >> 1) & 15;
    const int rg = tb + 8 * (jj >> 2) + 4 * half + (jj & 3);
    const bool gw = (r & 1) == 0 && rg < g.T;
    float t[16];
    const float bg = s_next[3 * D + 256 + r];
#pragma unroll
    for (int j = 0; j < 16; ++j) t[j] = h0[j] * bg;
    const float nd = noise::halfwave_transpose_sum16(t, lane);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float wq = s_next[3 * D + q * 32 + r];
#pragma unroll
      for (int j = 0; j < 16; ++j) t[j] = h0[j] * wq;
      float z = noise::halfwave_transpose_sum16(t, lane);
      if (nx.sign) z += s * nd * nx.gate_a[pn * nx.ld_gate_a + q];
      if (gw) nx.gate[(mrow0 + rg) * 8 + q] = 2.0f / (1.0f + expf(-z));
    }
  }
}

// NEXT 1 | 2: the next layer's mix_norm (noise_mixnorm_t `nx`; 2: with x0 mixing) runs in the
// epilogue on the finished rows.
// Chunk Q of the attention c_proj in the prologue (ATTN): wait for it, start chunk Q + 2 (and at
// Q = 15 the first c_fc chunk), then its 32 MFMAs acc[8 hh + nbb] += y[k-step 4 kc + ks4] Wo^T,
// the fragments of k-step ks4 + 1 read while those of ks4 run.
template <int Q, class WoLoad>
NOISE_DEV void attn_chunk(const noise_mlp_t& g, unsigned char* lds, floatx16 (&acc)[16], const bf16x8 (&yA)[32],
                          const uint32_t (&fk)[4], uint32_t lds0a, int wave, int lane, int c0, WoLoad& wo_load) {
  constexpr int kc = Q >> 1, hh = Q & 1, sl = Q & 3;
  constexpr uint32_t sbase = (sl >> 1) * STAGE + (sl & 1) * 32768;
  // chunk Q has landed for every wave, and every wave is done with chunk Q - 1
  if constexpr (Q < 15)
    __asm__ volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
  else
    __asm__ volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  if constexpr (Q + 2 < 16) wo_load(Q + 2);  // into slot (Q + 2) % 4, last read at chunk Q - 2
  if constexpr (Q == 15) load_stage(g, lds, wave, lane, 0, 0, -1, c0);  // slots 0 and 1 are free
  // 8 groups of 4 MFMAs (k-step ks4 = G / 2, blocks 4 (G % 2) .. + 3); the fragments of group
  // G + 1 are read while those of G run (two buffers of 4: fewer live registers than a whole
  // k-step ahead, which made the compiler move accumulators through VGPRs).
  bf16x8 fb[2][4];
  auto rd = [&](int G, bf16x8 (&dst)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __asm__ volatile("ds_read_b128 %0, %1 offset:%2"
                       : "=v"(dst[i]) : "v"(lds0a + sbase + fk[(G >> 1) & 3]), "i"(((G & 1) * 4 + i) * 4096));
  };
  rd(0, fb[0]);
#pragma unroll
  for (int G = 0; G < 8; ++G) {
    if (G + 1 < 8) {
      rd(G + 1, fb[(G + 1) & 1]);
      MLP_LGKM(4);
    } else {
      MLP_LGKM(0);
    }
    __asm__ volatile("" : "+v"(fb[G & 1][0]), "+v"(fb[G & 1][1]), "+v"(fb[G & 1][2]), "+v"(fb[G & 1][3]));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (kc == 0)  // an accumulator's first MFMA: the compiler may have just copied it into place
        __asm__ volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0"
                         : "+a"(acc[8 * hh + (G & 1) * 4 + i]) : "v"(yA[4 * kc + (G >> 1)]), "v"(fb[G & 1][i]));
      else if constexpr (kc == 7)  // its last: the compiler may spill or copy it right after the asm
        __asm__ volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 4"
                         : "+a"(acc[8 * hh + (G & 1) * 4 + i]) : "v"(yA[4 * kc + (G >> 1)]), "v"(fb[G & 1][i]));
      else
        __asm__ volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0"
                         : "+a"(acc[8 * hh + (G & 1) * 4 + i]) : "v"(yA[4 * kc + (G >> 1)]), "v"(fb[G & 1][i]));
    }
  }
}

template <class WoLoad, int... Q>
NOISE_DEV void attn_chunks(const noise_mlp_t& g, unsigned char* lds, floatx16 (&acc)[16], const bf16x8 (&yA)[32],
                           const uint32_t (&fk)[4], uint32_t lds0a, int wave, int lane, int c0, WoLoad& wo_load,
                           std::integer_sequence<int, Q...>) {
  (attn_chunk<Q>(g, lds, acc, yA, fk, lds0a, wave, lane, c0, wo_load), ...);
}

// ATTN: the attention c_proj (x += y Wo^T + s u_o a_o^T) runs on the rows in the prologue, before
// the norm.
template <bool NORM, bool RESID, int NEXT, bool ATTN>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
mlp_fused_kernel(const noise_mlp_t g, const noise_mixnorm_t nx) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[NEXT ? LDS_NEXT_BYTES : LDS_BYTES];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 31, half = lane >> 5;
  // Workgroup -> (member p, row block b). Workgroups go to the XCDs round-robin; numbering the
  // blocks of groups of 8 members so that XCD x runs b = 0, 1, 2, ... in turn lets each XCD walk
  // the feature chunks from bpm different starting points (c0 below) instead of every CU asking
  // L2 for the same weight lines at the same moment (measured on MI355X: 5.8 -> 5.2 ms at the
  // bench shape). c0 depends only on b, so a member's result does not depend on which other
  // members share the launch.
  const int bpm = (g.T + ROWS - 1) / ROWS;
  int p, b;
  {
    const int i = blockIdx.x, full = (g.members & ~7) * bpm;
    if (i < full) {
      const int q = i >> 3;
      b = q % bpm;
      p = (q / bpm) * 8 + (i & 7);
    } else {
      const int j = i - full;
      p = (g.members & ~7) + j / bpm;
      b = j % bpm;
    }
  }
  const int c0 = (b * (bpm >= NCH ? 1 : NCH / bpm)) & (NCH - 1);
  const int tb = b * ROWS + wave * 32;  // first row of this wave
  const bool pert = g.sign != nullptr;
  const int64_t pn = (int64_t)(p >> g.member_shift);
  const float s = pert ? g.sign[p] : 0.f;
  float* s_afc = reinterpret_cast<float*>(lds + NOISE_OFS);
  float* s_bmp = s_afc + F;
  float* s_amp = s_bmp + F;
  float* s_bfc = s_amp + D;

  // The first c_fc chunk starts streaming into stage 0 while the rows are normalised (with ATTN
  // the stage buffers first carry the attention c_proj weight; the chunk follows it).
  // With ATTN: Wo streams through the two stage buffers as 16 chunks of 256 output rows x 64 K
  // (32 KB of 128-byte rows, chunk c of row n at c ^ ((n >> 1) & 7)); chunk q sits in the 32 KB
  // slot q % 4 and is loaded two chunks ahead, 8 loads of 1 KB per wave.
  auto wo_load = [&](int q) {
    const int kc = q >> 1, hh = q & 1, sl = q & 3;
    unsigned char* st = lds + (sl >> 1) * STAGE + (sl & 1) * 32768;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int blk = 8 * wave + i, rl = 8 * blk + (lane >> 3);
      const int lc = (lane & 7) ^ ((rl >> 1) & 7);
      __builtin_amdgcn_global_load_lds((const void*)(g.attn_w + (int64_t)(256 * hh + rl) * D + 64 * kc + 8 * lc),
                                       (void*)(st + blk * 1024), 16, 0, 0);
    }
  };
  bf16x8 yA[ATTN ? 32 : 1];  // the wave's 32 rows of y as the A operand (lane l: row l % 32)
  if constexpr (ATTN) {
    wo_load(0);
    wo_load(1);
    const int ry = tb + r < g.T ? tb + r : g.T - 1;
    const uint16_t* ysrc = g.attn_y + ((int64_t)p * g.T + ry) * g.ld_attn_y + 8 * half;
#pragma unroll
    for (int ks = 0; ks < 32; ++ks) yA[ks] = *reinterpret_cast<const bf16x8*>(ysrc + 16 * ks);
  } else {
    load_stage(g, lds, wave, lane, 0, 0, -1, c0);
  }

  // The member's perturbation rows (a_fc | b_proj | a_proj | b_fc, 20 pieces of 256 floats, five
  // a wave; zeros when unperturbed, so the rank-1 terms vanish without a branch in the main loop)
  // and, with NEXT, the next norm's vectors (b[0..2], gate W, gate b) go straight into LDS by
  // direct loads issued before anything else: they land under the row loads and the attention
  // c_proj, and the waits that complete those cover them (vector memory loads retire in order);
  // the barriers that follow (the attention chunks' or the one after the norm) publish them.
#pragma unroll
  for (int k = 0; k < 5; ++k) {
    const int pc = 5 * wave + k;
    const float* src = !pert   ? kZeroRow
                       : pc < 8  ? g.a_fc + pn * g.ld_a_fc + 256 * pc
                       : pc < 16 ? g.b_proj + pn * g.ld_b_proj + 256 * (pc - 8)
                       : pc < 18 ? g.a_proj + pn * g.ld_a_proj + 256 * (pc - 16)
                                 : g.b_fc + pn * g.ld_b_fc + 256 * (pc - 18);
    __builtin_amdgcn_global_load_lds((const void*)(src + 4 * lane), (void*)(lds + NOISE_OFS + pc * 1024), 16, 0, 0);
  }
  if constexpr (NEXT != 0) {
    const int64_t pnx = (int64_t)(p >> nx.member_shift);
    for (int k = wave; k < 7; k += 4) {  // pieces 0-5: b[k / 2], piece 6: gate W
      const float* src = k < 6 ? (k / 2 < nx.nb ? nx.b[k / 2] + pnx * nx.ldb + 256 * (k & 1) : kZeroRow)
                               : (nx.gate_w ? nx.gate_w : kZeroRow);
      __builtin_amdgcn_global_load_lds((const void*)(src + 4 * lane), (void*)(lds + NEXT_OFS + k * 1024), 16, 0, 0);
    }
    if (wave == 3 && lane < 8) {  // gate b: 32 floats
      const float* src = nx.gate_w && nx.sign ? nx.gate_b + pnx * nx.ld_gate_b : kZeroRow;
      __builtin_amdgcn_global_load_lds((const void*)(src + 4 * lane), (void*)(lds + NEXT_OFS + (3 * D + 256) * 4), 16,
                                       0, 0);
    }
  }
  // ---- prologue, one pass over the input: the wave's 32 rows land in the c_proj accumulator
  // layout (lane l holds column 32 nb + l % 32 of rows 8 (j / 4) + 4 (l / 32) + j % 4), where they
  // also start the residual sum.
  // The 256 loads go straight into the accumulator AGPRs by inline asm, three rows of 16 ahead of
  // their use (left to itself the compiler waited for each load before issuing the next). Vector
  // loads complete in issue order, so once at most the later rows' loads are in flight a row has
  // landed; the wait is tied to that row's registers.
  floatx16 acc[16];
  const float* xrow = g.in + (int64_t)p * g.member_stride_in + r;
#define MLP_XLOAD(J_)                                                                                      \
  {                                                                                                      \
    const int rj_ = tb + 8 * ((J_) >> 2) + 4 * half + ((J_) & 3);                                         \
    const float* src_ = xrow + (int64_t)(rj_ < g.T ? rj_ : g.T - 1) * g.ld_in;                            \
    _Pragma("unroll") for (int nb = 0; nb < 16; ++nb)                                                     \
      __asm__ volatile("global_load_dword %0, %1, off offset:%2" : "=a"(acc[nb][J_]) : "v"(src_), "n"(nb * 128)); \
  }
#define MLP_XWAIT(J_, N_)                                                                                 \
  __asm__ volatile("s_waitcnt vmcnt(%16)"                                                                \
                   : "+a"(acc[0][J_]), "+a"(acc[1][J_]), "+a"(acc[2][J_]), "+a"(acc[3][J_]),               \
                     "+a"(acc[4][J_]), "+a"(acc[5][J_]), "+a"(acc[6][J_]), "+a"(acc[7][J_]),               \
                     "+a"(acc[8][J_]), "+a"(acc[9][J_]), "+a"(acc[10][J_]), "+a"(acc[11][J_]),             \
                     "+a"(acc[12][J_]), "+a"(acc[13][J_]), "+a"(acc[14][J_]), "+a"(acc[15][J_])            \
                   : "n"(N_))
  MLP_XLOAD(0)
  MLP_XLOAD(1)
  MLP_XLOAD(2)
  float ps[16];  // per-lane sums of squares of each accumulator row
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    if (j + 3 < 16) MLP_XLOAD(j + 3)
    MLP_XWAIT(j, 16 * (15 - j < 3 ? 15 - j : 3));
    if constexpr (!ATTN) {
      ps[j] = 0.f;
#pragma unroll
      for (int nb = 0; nb < 16; ++nb) {
        const float v = agpr_read(acc[nb][j]);
        ps[j] += v * v;
      }
    }
  }
#undef MLP_XWAIT
#undef MLP_XLOAD
  if constexpr (ATTN) {
    // ---- the attention c_proj into the accumulators: 16 chunks x (4 k-steps x 8 column blocks).
    // Fragment (k-step ks4, block nbb) of a chunk: row 32 nbb + r, logical 16-byte piece
    // 2 ks4 + half.
    const uint32_t lds0a = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)lds;
    uint32_t fk[4];
#pragma unroll
    for (int ks4 = 0; ks4 < 4; ++ks4) fk[ks4] = (uint32_t)(r * 128 + (((2 * ks4 + half) ^ ((r >> 1) & 7)) * 16));
    attn_chunks(g, lds, acc, yA, fk, lds0a, wave, lane, c0, wo_load, std::make_integer_sequence<int, 16>{});
    __asm__ volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");  // last MFMAs before VALU reads
    // the rank-1 term s (sum over the per-head parts of y . b_o) a_o of the rows' member
    if (pert) {
      const int ry = tb + r < g.T ? tb + r : g.T - 1;
      const float* up = g.attn_u + ((int64_t)p * g.T + ry) * g.ld_attn_u;
      float u = 0.f;
      for (int k = 0; k < g.attn_parts; ++k) u += up[k];
      const float su_r = s * u;
      float ao[16];
#pragma unroll
      for (int nb = 0; nb < 16; ++nb) ao[nb] = g.attn_a[pn * g.ld_attn_a + nb * 32 + r];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float suj = __shfl(su_r, 8 * (j >> 2) + 4 * half + (j & 3), 64);
#pragma unroll
        for (int nb = 0; nb < 16; ++nb) acc[nb][j] = agpr_read(acc[nb][j]) + suj * ao[nb];
      }
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      ps[j] = 0.f;
#pragma unroll
      for (int nb = 0; nb < 16; ++nb) {
        const float v = agpr_read(acc[nb][j]);
        ps[j] += v * v;
      }
    }
  }

  // Row norms: per-lane partial sums over the 16 column blocks, then across the half-wave
  // (lane q of a half ends with row value (q >> 1) & 15), broadcast back per accumulator row.
  float rrj[16];
  if (NORM) {
    const float rr = rsqrtf(noise::halfwave_transpose_sum16(ps, lane) * (1.0f / D) + RMS_EPS);
#pragma unroll
    for (int j = 0; j < 16; ++j) rrj[j] = __shfl(rr, (lane & 32) + 2 * j, 64);
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) rrj[j] = 1.f;
  }
  __syncthreads();  // the perturbation rows are in LDS

  // h = bf16(row * rr), turned into the c_fc B operand (lane l: row l % 32) by MFMAs against a
  // permuted identity: with A = h block nb (lane: column 32 nb + l % 32, k-slots = the lane's
  // accumulator rows 16 s + 8 (q / 4) + 4 (l / 32) + q % 4) and B[k][j] = 1 where row(k) = j, the
  // product is h^T exactly (every sum has one non-zero term), and its accumulators hold row l % 32
  // at the columns 32 nb + 8 (v / 4) + 4 (l / 32) + v % 4 -- the perm16 order in which the packed
  // c_fc copy stores its K dimension.
  bf16x8 ident[2];
#pragma unroll
  for (int sx = 0; sx < 2; ++sx) {
    const bool mine = (r >> 4) == sx && ((r >> 2) & 1) == half;
    const int q = 4 * ((r >> 3) & 1) + (r & 3);
    uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int k = 0; k < 4; ++k) w[k] = (mine && (q >> 1) == k) ? (0x3F80u << (16 * (q & 1))) : 0u;
    ident[sx] = as_bf16x8(w[0], w[1], w[2], w[3]);
  }
  bf16x8 hB[32];
#pragma unroll
  for (int nb = 0; nb < 16; ++nb) {
    uint32_t hw[8];
#pragma unroll
    for (int k = 0; k < 8; ++k)
      hw[k] = pack_bf2(agpr_read(acc[nb][2 * k]) * rrj[2 * k], agpr_read(acc[nb][2 * k + 1]) * rrj[2 * k + 1]);
    floatx16 tr = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(hw[0], hw[1], hw[2], hw[3]), ident[0],
                                                           (floatx16){}, 0, 0, 0);
    tr = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(hw[4], hw[5], hw[6], hw[7]), ident[1], tr, 0, 0, 0);
    hB[2 * nb] = as_bf16x8(pack_bf2(tr[0], tr[1]), pack_bf2(tr[2], tr[3]), pack_bf2(tr[4], tr[5]),
                           pack_bf2(tr[6], tr[7]));
    hB[2 * nb + 1] = as_bf16x8(pack_bf2(tr[8], tr[9]), pack_bf2(tr[10], tr[11]), pack_bf2(tr[12], tr[13]),
                               pack_bf2(tr[14], tr[15]));
  }
  // u_fc = bf16(h) . b_fc of row l % 32: this lane's 256 columns (k-step ks, slot q: column
  // 16 ks + 8 (q / 4) + 4 (l / 32) + q % 4), then the other half-row from lane l ^ 32.
  float uf = 0.f;
#pragma unroll
  for (int ks = 0; ks < 32; ++ks) {
    const float4 b0 = *reinterpret_cast<const float4*>(s_bfc + 16 * ks + 4 * half);
    const float4 b1 = *reinterpret_cast<const float4*>(s_bfc + 16 * ks + 8 + 4 * half);
    const u32x4 w = __builtin_bit_cast(u32x4, hB[ks]);
    uf += bf_lo(w[0]) * b0.x + bf_hi(w[0]) * b0.y + bf_lo(w[1]) * b0.z + bf_hi(w[1]) * b0.w;
    uf += bf_lo(w[2]) * b1.x + bf_hi(w[2]) * b1.y + bf_lo(w[3]) * b1.z + bf_hi(w[3]) * b1.w;
  }
  uf += __shfl_xor(uf, 32, 64);
  const float su = s * uf;
  if (!RESID) {
#pragma unroll
    for (int nb = 0; nb < 16; ++nb)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[nb][j] = 0.f;
  }

  // LDS byte addresses of this lane's fragment rows: c_fc row r (k-step ks at + 32 ks), c_proj
  // row 32 nb + r of k-step kk at chunk (2 kk + half) ^ ((r >> 2) & 3) (+ 2048 nb).
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)lds;
  const uint32_t ab_base = lds0 + NOISE_OFS + 16 * half;  // a_fc at + 0, b_proj at + 4 F floats
  const uint32_t fcb[2] = {lds0 + r * WFC_ROW + 16 * half, lds0 + STAGE + r * WFC_ROW + 16 * half};
  const int sw = (r >> 2) & 3;
  const uint32_t mpr = lds0 + WFC_PART + r * 64;
  const uint32_t mpb[2][2] = {{mpr + 16 * ((0 + half) ^ sw), mpr + 16 * ((2 + half) ^ sw)},
                              {mpr + STAGE + 16 * ((0 + half) ^ sw), mpr + STAGE + 16 * ((2 + half) ^ sw)}};

  floatx16 fc[2];
  float up = 0.f;  // bf16(hidden) . b_proj over this lane's features

  // Step i: stage i % 2 holds c_fc chunk i and c_proj chunk i - 1; stage (i + 1) % 2 is refilled.
#define MLP_BARRIER() __asm__ volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory")
  MLP_BARRIER();
  mlp_step<true, false, 0, true, true>(hB, fc, acc, up, fcb[0], mpb[0][0], mpb[0][1], ab_base, 0, su, c0,
                                       stage_loads(g, lds, wave, lane, 1, 1, 0, c0));
#pragma unroll 1
  for (int i = 1; i < NCH - 1; i += 2) {
    MLP_BARRIER();
    mlp_step<true, true, 1, true, true>(hB, fc, acc, up, fcb[1], mpb[1][0], mpb[1][1], ab_base, i - 1, su, c0,
                                        stage_loads(g, lds, wave, lane, 0, i + 1, i, c0));
    MLP_BARRIER();
    mlp_step<true, true, 0, true, true>(hB, fc, acc, up, fcb[0], mpb[0][0], mpb[0][1], ab_base, i, su, c0,
                                        stage_loads(g, lds, wave, lane, 1, i + 2, i + 1, c0));
  }
  // i = NCH - 1 (odd): stage 1 holds c_fc chunk 63 and c_proj chunk 62; stage 0 receives c_proj 63.
  MLP_BARRIER();
  mlp_step<true, true, 1, false, true>(hB, fc, acc, up, fcb[1], mpb[1][0], mpb[1][1], ab_base, NCH - 2, su, c0,
                                       stage_loads(g, lds, wave, lane, 0, 0, NCH - 1, c0));
  MLP_BARRIER();
  mlp_step<false, true, 0, false, false>(hB, fc, acc, up, fcb[0], mpb[0][0], mpb[0][1], ab_base, NCH - 1, su, c0,
                                         stage_loads(g, lds, wave, lane, 1, 0, 0, c0));
#undef MLP_BARRIER

  // ---- epilogue: rank-1 term of c_proj, sign (hidden . b_proj) a_proj, and the store.
  up += __shfl_xor(up, 32, 64);  // lane l: row l % 32
  const float sup = s * up;
  float am[16];
#pragma unroll
  for (int nb = 0; nb < 16; ++nb) am[nb] = s_amp[nb * 32 + r];
  if constexpr (NEXT != 0) {
    mix_norm_epilogue<NEXT == 2>(g, nx, acc, am, sup, lds, wave, lane, p, tb);
    return;
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int rl = 8 * (j >> 2) + 4 * half + (j & 3);
    const float sr = __shfl(sup, rl, 64);
    const int rj = tb + rl;
    if (rj < g.T) {
      float* dst = g.out + (int64_t)p * g.member_stride_out + (int64_t)rj * g.ld_out + r;
#pragma unroll
      for (int nb = 0; nb < 16; ++nb) {
#if MLP_NTSTORE
        __builtin_nontemporal_store(acc[nb][j] + sr * am[nb], dst + nb * 32);
#else
        dst[nb * 32] = acc[nb][j] + sr * am[nb];
#endif
      }
    }
  }
}

// One thread per 16-byte piece of the packed copies. c_fc: row f, piece c holds K positions
// 8 c .. 8 c + 7 with position 16 g + q reading column 16 g + perm16(q). c_proj: chunk c, row n,
// physical piece phi holds logical piece phi ^ ((n >> 2) & 3) of the chunk's 32 positions, position
// 16 g + q reading feature 32 c + 16 g + perm16(q).
__global__ void __launch_bounds__(256) mlp_pack_kernel(const float* __restrict__ w_fc, int64_t ld_fc,
                                                       const float* __restrict__ w_proj, int64_t ld_proj,
                                                       uint16_t* __restrict__ fc_packed,
                                                       uint16_t* __restrict__ proj_packed) {
  const int id = blockIdx.x * 256 + threadIdx.x;  // < 2 * 131072
  uint32_t out[4];
  if (id < F * D / 8) {
    if (!fc_packed) return;
    const int f = id >> 6, c = id & 63;
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const int q0 = 8 * c + e, q1 = q0 + 1;
      const int k0 = 16 * (q0 >> 4) + perm16(q0 & 15), k1 = 16 * (q1 >> 4) + perm16(q1 & 15);
      out[e / 2] = pack_bf2(w_fc[(int64_t)f * ld_fc + k0], w_fc[(int64_t)f * ld_fc + k1]);
    }
    *reinterpret_cast<u32x4*>(fc_packed + (int64_t)id * 8) = (u32x4){out[0], out[1], out[2], out[3]};
    return;
  }
  if (!proj_packed) return;
  const int jd = id - F * D / 8;
  const int phi = jd & 3, n = (jd >> 2) & (D - 1), c = jd >> 11;
  const int kc = phi ^ ((n >> 2) & 3);  // logical piece: positions 8 kc .. 8 kc + 7
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const int q0 = 8 * kc + e, q1 = q0 + 1;
    const int f0 = c * FC + 16 * (q0 >> 4) + perm16(q0 & 15), f1 = c * FC + 16 * (q1 >> 4) + perm16(q1 & 15);
    out[e / 2] = pack_bf2(w_proj[(int64_t)n * ld_proj + f0], w_proj[(int64_t)n * ld_proj + f1]);
  }
  *reinterpret_cast<u32x4*>(proj_packed + (int64_t)jd * 8) = (u32x4){out[0], out[1], out[2], out[3]};
}

}  // namespace

extern "C" int noise_mlp_pack(const float* w_fc, int64_t ld_fc, const float* w_proj, int64_t ld_proj,
                              uint16_t* fc_packed, uint16_t* proj_packed, void* stream) {
  NOISE_REQUIRE(!fc_packed || (w_fc && ld_fc >= D), "mlp_pack: c_fc needs w_fc with ld_fc >= 512");
  NOISE_REQUIRE(!proj_packed || (w_proj && ld_proj >= F), "mlp_pack: c_proj needs w_proj with ld_proj >= 2048");
  NOISE_REQUIRE(((uintptr_t)fc_packed % 16) == 0 && ((uintptr_t)proj_packed % 16) == 0,
                "mlp_pack: packed copies must be 16-byte aligned");
  if (!fc_packed && !proj_packed) return NOISE_OK;
  mlp_pack_kernel<<<2 * F * D / 8 / 256, 256, 0, (hipStream_t)stream>>>(w_fc, ld_fc, w_proj, ld_proj, fc_packed,
                                                                       proj_packed);
  return noise::check_launch("mlp_pack");
}

extern "C" int noise_mlp_fused(const noise_mlp_t* args, void* stream) {
  NOISE_REQUIRE(args, "mlp_fused: null arguments");
  const noise_mlp_t& g = *args;
  NOISE_REQUIRE(g.in && g.out && g.w_fc && g.w_proj, "mlp_fused: null in, out or weights");
  NOISE_REQUIRE(g.T > 0 && g.members >= 0, "mlp_fused: T=%d members=%d", g.T, g.members);
  NOISE_REQUIRE((g.flags & ~(NOISE_MLP_NORM | NOISE_MLP_RESIDUAL)) == 0, "mlp_fused: unknown flags %d", g.flags);
  NOISE_REQUIRE(g.ld_in >= D && g.ld_out >= D && g.ld_in % 4 == 0 && g.member_stride_in % 4 == 0 &&
                    g.member_stride_in >= 0 && g.member_stride_out >= 0,
                "mlp_fused: rows need ld >= 512 with ld_in and member_stride_in multiples of 4");
  NOISE_REQUIRE(((uintptr_t)g.in % 16) == 0 && ((uintptr_t)g.w_fc % 16) == 0 && ((uintptr_t)g.w_proj % 16) == 0,
                "mlp_fused: in, w_fc and w_proj must be 16-byte aligned");
  // Every output row has one writer, and a launch that overwrites its input does so row for row
  // (each workgroup reads its rows before it writes them).
  NOISE_REQUIRE(g.members <= 1 || g.member_stride_out >= (int64_t)g.T * g.ld_out,
                "mlp_fused: members' output rows overlap (member_stride_out %lld < T * ld_out)",
                (long long)g.member_stride_out);
  NOISE_REQUIRE(g.in != g.out || (g.ld_in == g.ld_out && g.member_stride_in == g.member_stride_out),
                "mlp_fused: in-place (out == in) needs equal row and member strides");
  if (g.sign) {
    NOISE_REQUIRE(g.a_fc && g.b_fc && g.a_proj && g.b_proj, "mlp_fused: perturbation needs a/b of both matrices");
    NOISE_REQUIRE(g.member_shift >= 0 && g.member_shift < 31, "mlp_fused: bad member_shift");
    NOISE_REQUIRE(g.ld_a_fc >= F && g.ld_b_proj >= F && g.ld_a_proj >= D && g.ld_b_fc >= D &&
                      g.ld_a_fc % 4 == 0 && g.ld_b_proj % 4 == 0 && g.ld_a_proj % 4 == 0 && g.ld_b_fc % 4 == 0,
                  "mlp_fused: noise rows need lda >= out, ldb >= in, multiples of 4");
    NOISE_REQUIRE(((uintptr_t)g.a_fc % 16) == 0 && ((uintptr_t)g.b_fc % 16) == 0 &&
                      ((uintptr_t)g.a_proj % 16) == 0 && ((uintptr_t)g.b_proj % 16) == 0,
                  "mlp_fused: noise rows must be 16-byte aligned");
  }
  if (g.attn_y) {
    NOISE_REQUIRE(g.flags == (NOISE_MLP_NORM | NOISE_MLP_RESIDUAL),
                  "mlp_fused: the attention c_proj needs the normed residual MLP");
    NOISE_REQUIRE(g.attn_w && g.ld_attn_y >= D && g.ld_attn_y % 8 == 0 && ((uintptr_t)g.attn_y % 16) == 0 &&
                      ((uintptr_t)g.attn_w % 16) == 0,
                  "mlp_fused: attention y [members * T, >= 512] bf16 and Wo [512, 512] bf16, 16-byte aligned rows");
    NOISE_REQUIRE(!g.sign || (g.attn_u && g.attn_a && g.attn_parts >= 1 && g.ld_attn_u >= g.attn_parts &&
                              g.ld_attn_a >= D),
                  "mlp_fused: the perturbed attention c_proj needs u [rows, parts] and a [noise rows, 512]");
  }
  const int64_t blocks = (int64_t)g.members * ((g.T + ROWS - 1) / ROWS);
  NOISE_REQUIRE(blocks < (1ll << 31), "mlp_fused: too many rows");
  if (blocks == 0) return NOISE_OK;
  const dim3 grid((unsigned)blocks);
  hipStream_t st = (hipStream_t)stream;
  const noise_mixnorm_t none{};
  if (g.next) {
    const noise_mixnorm_t& nx = *g.next;
    NOISE_REQUIRE(g.flags == (NOISE_MLP_NORM | NOISE_MLP_RESIDUAL),
                  "mlp_fused: the next layer's mix_norm needs the normed residual MLP");
    NOISE_REQUIRE(nx.x == g.out && nx.h && nx.T == g.T && (int64_t)nx.M == (int64_t)g.members * g.T &&
                      g.ld_out == D && g.member_stride_out == (int64_t)g.T * D,
                  "mlp_fused: the next mix_norm must cover exactly the output rows, [members * T, 512] contiguous");
    NOISE_REQUIRE(nx.nb >= 0 && nx.nb <= 3 && (nx.nb == 0 || (nx.u && nx.ldu >= nx.nb && nx.ldb >= D)),
                  "mlp_fused: next mix_norm dots need u, ldu >= nb and ldb >= 512");
    for (int j = 0; j < nx.nb; ++j)
      NOISE_REQUIRE(nx.b[j] && ((uintptr_t)nx.b[j] % 16) == 0 && nx.ldb % 4 == 0,
                    "mlp_fused: next mix_norm b[%d] must be non-null with 16-byte aligned rows", j);
    NOISE_REQUIRE(((uintptr_t)nx.gate_w % 16) == 0 && (!nx.gate_w || !nx.sign ||
                                                      (((uintptr_t)nx.gate_b % 16) == 0 && nx.ld_gate_b % 4 == 0)),
                  "mlp_fused: next gate W and b must be 16-byte aligned");
    NOISE_REQUIRE(!nx.x0 || (nx.resid && nx.mix && (!nx.sign || (nx.eps_resid && nx.eps_mix))),
                  "mlp_fused: next mixing needs the lambda scalars (and eps when perturbed)");
    NOISE_REQUIRE(!nx.gate_w || (nx.gate && (!nx.sign || (nx.gate_a && nx.gate_b))),
                  "mlp_fused: next gate needs its output and perturbation vectors");
    NOISE_REQUIRE(((uintptr_t)nx.h % 16) == 0, "mlp_fused: next h must be 16-byte aligned");
    NOISE_REQUIRE(nx.member_shift >= 0 && nx.member_shift < 31, "mlp_fused: next mix_norm has a bad member_shift");
    NOISE_REQUIRE(!nx.gain, "mlp_fused: the next mix_norm's gain is not supported in the fused epilogue "
                  "(the reference's norm has none); run noise_mix_norm for it");
    if (g.attn_y) {
      if (nx.x0) mlp_fused_kernel<true, true, 2, true><<<grid, 256, 0, st>>>(g, nx);
      else mlp_fused_kernel<true, true, 1, true><<<grid, 256, 0, st>>>(g, nx);
    } else {
      if (nx.x0) mlp_fused_kernel<true, true, 2, false><<<grid, 256, 0, st>>>(g, nx);
      else mlp_fused_kernel<true, true, 1, false><<<grid, 256, 0, st>>>(g, nx);
    }
    return noise::check_launch("mlp_fused (with the next mix_norm)");
  }
  // NOISE_MLP_TWO_WAVE=1 in the environment runs the plain normed residual MLP in the two-wave
  // (producer/consumer) form: bit-identical rows, measured slower on MI355X (4.9 against 4.46 ms
  // at 512 members x 2048 tokens), so not the default.
  const char* two_wave = getenv("NOISE_MLP_TWO_WAVE");
  if (two_wave && two_wave[0] == '1' && noise::mlp_pc_launch(g, st)) return noise::check_launch("mlp_fused");
  switch (g.flags) {
    case NOISE_MLP_NORM | NOISE_MLP_RESIDUAL:
      if (g.attn_y) mlp_fused_kernel<true, true, 0, true><<<grid, 256, 0, st>>>(g, none);
      else mlp_fused_kernel<true, true, 0, false><<<grid, 256, 0, st>>>(g, none);
      break;
    case NOISE_MLP_NORM: mlp_fused_kernel<true, false, 0, false><<<grid, 256, 0, st>>>(g, none); break;
    case NOISE_MLP_RESIDUAL: mlp_fused_kernel<false, true, 0, false><<<grid, 256, 0, st>>>(g, none); break;
    default: mlp_fused_kernel<false, false, 0, false><<<grid, 256, 0, st>>>(g, none); break;
  }
  return noise::check_launch("mlp_fused");
}
