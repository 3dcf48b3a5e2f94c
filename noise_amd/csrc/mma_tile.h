// 256 x BN bf16 MFMA tile main loop shared by the perturbed GEMM and the head kernel.
//
// acc += A[0:256, 0:K] * B[0:BN, 0:K]^T for A, B row-major bf16 with K contiguous. The workgroup
// has 2 x (BN / 64) waves; wave (wm, wn) owns rows wm*128.. and columns wn*64.. as 4 x 2 blocks
// of v_mfma_f32_32x32x16_bf16 (128 fp32 accumulators per lane). Block (mi, ni), accumulator j of
// lane l holds
//   row = wm*128 + mi*32 + 8*(j/4) + 4*(l/32) + j%4,   col = wn*64 + ni*32 + l%32.
//
// Pipeline:
//   * K advances KB (32 or 64) per stage through NS LDS stage buffers of 64- or 128-byte rows
//     whose 16-byte chunks are swizzled (see tile_swizzle), so that the fragment reads (one row
//     per lane, 16 lanes per bank cycle) touch 16 distinct 16-byte bank groups;
//   * global -> LDS direct loads (global_load_lds_dwordx4: each lane's 16 bytes land at the
//     wave's LDS base + 16 * lane, no registers involved) fetch stage s + NS - 1 while stage s
//     computes; lane l of a load covers row l / LPR of a slab at physical chunk l % LPR and
//     therefore fetches the logical chunk the swizzle maps there;
//   * one s_waitcnt vmcnt + s_barrier per stage (inline asm with a memory clobber: the compiler's
//     own fence would wait for every load in flight, including the later stages).
//   * the fragments of k-step ks + 1 are read (inline-asm ds_read_b128, explicit lgkmcnt waits)
//     while the MFMAs of k-step ks run: left to itself the compiler folded the two fragment sets
//     into one and waited for every read right before its MFMAs (+3-4% on the step when fixed).
// Measured on MI355X against the register-staged two-buffer loop it replaces: +12-15% in the
// main loop. With 256-column tiles two 64-deep stages beat three 32-deep ones by 4-8% (whole
// 128-byte lines per row); 128-column tiles keep three 32-deep stages (two workgroups per CU).
// With B2 (a second [BN, K] operand) the loop continues over K again with B2 in place of B, so
// acc += A B^T + A B2^T in one pipeline (the head's hi + lo weight halves).
// Rows of A at or beyond `a_rows` are read from row a_rows - 1 (their results are discarded).
// K must be a multiple of 64. Every global load the caller issued before the call is complete
// when the loop's first wait returns (vector memory loads retire in order).
#pragma once
#include "common.h"

namespace noise {

constexpr int TILE_M = 256, TBK = 32, TLDK = TBK;  // default stage depth: 64-byte LDS rows

// KB: K depth per stage, 32 (64-byte LDS rows, chunk c of row r at c ^ ((r >> 2) & 3)) or 64
// (128-byte rows, c ^ ((r >> 1) & 7)). Both swizzles keep the fragment reads conflict-free; 64
// fetches whole 128-byte lines per row, which the direct loads move at about twice the rate of
// 64-byte row pieces (measured on MI355X from L2: 55 vs 31 B/clk per CU).
template <int BN, int NS = 3, int KB = TBK>
struct TileCfg {
  static constexpr int WAVES = 2 * (BN / 64);
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int RPI = 512 / KB;                                 // rows per 1-KB load
  static constexpr int ROWS_A = TILE_M / WAVES, ROWS_B = BN / WAVES;  // rows per wave per stage
  static constexpr int NIA = ROWS_A / RPI, NIB = ROWS_B / RPI;         // 1-KB loads per wave
  static constexpr int BOFS = TILE_M * KB;          // elements from the A to the B half
  static constexpr int BUF = (TILE_M + BN) * KB;    // elements per stage buffer
  static constexpr int SMEM_ELEMS = NS * BUF;
  static_assert(KB == 32 || KB == 64, "stage depth");
  static_assert(NIA * RPI == ROWS_A && NIB * RPI == ROWS_B, "rows per wave");
};

template <int KB>
NOISE_DEV int tile_swizzle(int row) {
  return KB == 32 ? ((row >> 2) & 3) : ((row >> 1) & 7);
}

template <int BN, int NS = 3, int KB = TBK>
NOISE_DEV void mma_tile(const uint16_t* __restrict__ A, int64_t lda, int a_rows,
                        const uint16_t* __restrict__ B, int64_t ldb, int K, uint16_t* smem,
                        floatx16 (&acc)[4][2], const uint16_t* __restrict__ B2 = nullptr) {
  using C = TileCfg<BN, NS, KB>;
  constexpr int NIA = C::NIA, NIB = C::NIB, BUF = C::BUF, BOFS = C::BOFS, RPI = C::RPI;
  constexpr int LPR = 64 / RPI;                 // lanes per row in a load
  constexpr int WAIT = (NS - 2) * (NIA + NIB);  // loads of the younger stages left in flight
  static_assert(NS >= 2 && WAIT < 64, "stage count");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / (BN / 64), wn = wave % (BN / 64);
  const int KT = K / KB, KTT = B2 ? 2 * KT : KT;
  // Direct-load sources: this wave's slabs of A (rows wave * ROWS_A + RPI i ..) and B. Lane l of
  // a load lands at row l / LPR, physical chunk l % LPR, so it fetches the logical chunk the
  // swizzle puts there.
  const uint16_t* ga[NIA];
  int64_t gb[NIB];  // element offsets into B (and B2)
#pragma unroll
  for (int i = 0; i < NIA; ++i) {
    const int row = wave * C::ROWS_A + i * RPI + lane / LPR;
    const int c = (lane % LPR) ^ tile_swizzle<KB>(row);
    ga[i] = A + (int64_t)(row < a_rows ? row : a_rows - 1) * lda + c * 8;
  }
#pragma unroll
  for (int i = 0; i < NIB; ++i) {
    const int row = wave * C::ROWS_B + i * RPI + lane / LPR;
    const int c = (lane % LPR) ^ tile_swizzle<KB>(row);
    gb[i] = (int64_t)row * ldb + c * 8;
  }
  uint16_t* la = smem + wave * C::ROWS_A * KB;
  uint16_t* lb = smem + BOFS + wave * C::ROWS_B * KB;
  // Fragment rows are lane % 32 plus multiples of 32, so their swizzle is that of lane % 32;
  // k-step ks reads logical chunk 2 ks + lane / 32.
  const int sw = tile_swizzle<KB>(lane & 31);
  const int far = wm * 128 + (lane & 31), fbr = wn * 64 + (lane & 31);
  int kofs[KB / 16];
#pragma unroll
  for (int ks = 0; ks < KB / 16; ++ks) kofs[ks] = ((2 * ks + (lane >> 5)) ^ sw) * 8;
  // LDS byte addresses of this lane's fragment rows per k-step in stage buffer 0; a buffer adds
  // BUF * 2 bytes and a 32-row block 32 * KB * 2 (an immediate offset).
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t*)smem;
  uint32_t fra[KB / 16], frb[KB / 16];
#pragma unroll
  for (int ks = 0; ks < KB / 16; ++ks) {
    fra[ks] = lds0 + (uint32_t)(far * KB + kofs[ks]) * 2;
    frb[ks] = lds0 + (uint32_t)(BOFS + fbr * KB + kofs[ks]) * 2;
  }
  bf16x8 a0[4], b0[2], a1[4], b1[2];

// Stage KT_ (clamped to the last one: the surplus loads keep the wait counts exact) into buffer BUF_.
#define NOISE_DLOAD(KT_, BUF_)                                                                \
  {                                                                                         \
    const int kk_ = (KT_) < KTT ? (KT_) : KTT - 1;                                          \
    const bool second_ = kk_ >= KT;                                                         \
    const int k0_ = (second_ ? kk_ - KT : kk_) * KB;                                        \
    const uint16_t* bsrc_ = second_ ? B2 : B;                                               \
    _Pragma("unroll") for (int i = 0; i < NIA; ++i)                                         \
      __builtin_amdgcn_global_load_lds((const void*)(ga[i] + k0_),                          \
                                       (void*)(la + (BUF_) * BUF + i * RPI * KB), 16, 0, 0); \
    _Pragma("unroll") for (int i = 0; i < NIB; ++i)                                         \
      __builtin_amdgcn_global_load_lds((const void*)(bsrc_ + gb[i] + k0_),                  \
                                       (void*)(lb + (BUF_) * BUF + i * RPI * KB), 16, 0, 0); \
  }
// Fragment reads of k-step KS_ from stage buffer BUF_, as inline asm: the compiler neither sinks
// them next to their use nor waits for them on its own (it cannot see that they are in flight),
// so the loop below waits for exactly the reads each MFMA group needs (NOISE_FWAIT).
#define NOISE_FLOAD(FA, FB, BUF_, KS_)                                                        \
  {                                                                                         \
    const uint32_t pa_ = fra[KS_] + (uint32_t)(BUF_) * (BUF * 2);                           \
    const uint32_t pb_ = frb[KS_] + (uint32_t)(BUF_) * (BUF * 2);                           \
    _Pragma("unroll") for (int i = 0; i < 4; ++i)                                           \
      __asm__ volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(FA[i]) : "v"(pa_), "n"(i * 64 * KB)); \
    _Pragma("unroll") for (int i = 0; i < 2; ++i)                                           \
      __asm__ volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(FB[i]) : "v"(pb_), "n"(i * 64 * KB)); \
  }
// Wait until at most N_ LDS reads are in flight, then tie the fragments to that point so that no
// MFMA reading them is scheduled before the wait.
#define NOISE_FWAIT(N_, FA, FB)                                                               \
  {                                                                                         \
    __asm__ volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N_));                                    \
    __asm__ volatile("" : "+v"(FA[0]), "+v"(FA[1]), "+v"(FA[2]), "+v"(FA[3]), "+v"(FB[0]), "+v"(FB[1])); \
  }
#define NOISE_MFMA8(FA, FB)                                                                   \
  _Pragma("unroll") for (int mi = 0; mi < 4; ++mi)                                          \
    _Pragma("unroll") for (int ni = 0; ni < 2; ++ni)                                        \
      acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(FA[mi], FB[ni], acc[mi][ni], 0, 0, 0);

  // The previous user of smem (an epilogue, or an earlier call) is done with it.
  __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
  for (int s = 0; s < NS - 1; ++s) NOISE_DLOAD(s, s)
  // Not unrolled: full unrolling makes the compiler precompute every stage's addresses.
#pragma unroll 1
  for (int kt = 0; kt < KTT; ++kt) {
    const int cur = kt % NS;
    // Stage kt has landed for this wave, then for every wave; all reads of stage kt - 1 are done,
    // so its buffer takes stage kt + NS - 1.
    __asm__ volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(WAIT) : "memory");
    NOISE_DLOAD(kt + NS - 1, (kt + NS - 1) % NS)
    // Fragments of k-step ks + 1 are read while the MFMAs of k-step ks run; the scheduling
    // barriers keep each MFMA group between the wait for its fragments and the next reads.
    NOISE_FLOAD(a0, b0, cur, 0)
#pragma unroll
    for (int kp = 0; kp < KB / 32; ++kp) {
      NOISE_FLOAD(a1, b1, cur, 2 * kp + 1)
      NOISE_FWAIT(6, a0, b0)
      NOISE_MFMA8(a0, b0)
      __builtin_amdgcn_sched_barrier(0);
      if (2 * kp + 2 < KB / 16) {
        NOISE_FLOAD(a0, b0, cur, 2 * kp + 2)
        NOISE_FWAIT(6, a1, b1)
      } else {
        NOISE_FWAIT(0, a1, b1)
      }
      NOISE_MFMA8(a1, b1)
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // Drain the surplus loads before the caller reuses smem.
  __asm__ volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
#undef NOISE_MFMA8
#undef NOISE_FWAIT
#undef NOISE_FLOAD
#undef NOISE_DLOAD
}

NOISE_DEV void zero_acc(floatx16 (&acc)[4][2]) {
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[mi][ni][j] = 0.f;
}

// Row-local DPP read: lane i gets v from lane i + s (row_shl:s, CTRL 0x100 + s) or i - s (row_shr:s,
// CTRL 0x110 + s) of its 16-lane row; lanes whose source leaves the row get 0 (never used below).
template <int CTRL>
NOISE_DEV float dpp_row(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over the 32 lanes of each half-wave of 16 per-lane values; lane q of a half ends with the
// total of value (q >> 1) & 15 (lanes q and q ^ 1 hold the same total). Each halving step pairs
// two values: v_permlane16_swap exchanges them across the two 16-lane rows of the half, DPP row
// shifts fetch the partner inside a row; no LDS round trips.
NOISE_DEV float halfwave_transpose_sum16(float (&v)[16], int lane) {
  const int q = lane & 31;
#pragma unroll
  for (int i = 0; i < 8; ++i) {  // rows 0 | 1: row 0 keeps value i, row 1 value i + 8
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[i]), __float_as_uint(v[i + 8]), false, false);
    v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float x = v[i] + dpp_row<0x108>(v[i]), y = v[i + 4] + dpp_row<0x118>(v[i + 4]);
    v[i] = (q & 8) ? y : x;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float x = v[i] + dpp_row<0x104>(v[i]), y = v[i + 2] + dpp_row<0x114>(v[i + 2]);
    v[i] = (q & 4) ? y : x;
  }
  {
    const float x = v[0] + dpp_row<0x102>(v[0]), y = v[1] + dpp_row<0x112>(v[1]);
    v[0] = (q & 2) ? y : x;
  }
  return v[0] + dpp_row<0xB1>(v[0]);  // quad_perm [1, 0, 3, 2]: the lane's neighbour q ^ 1
}

// Sum over the 64 lanes of 32 per-lane values; lane l ends with the total of value
// 16 (l / 32) + ((l % 32) >> 1) (lanes l and l ^ 1 hold the same total). v_permlane32_swap pairs
// value i with value i + 16 across the two halves, then each half sums its 16 values.
NOISE_DEV float wave_transpose_sum32(float (&v)[32], int lane) {
  float w[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {  // half 0 keeps value i, half 1 value i + 16
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[i + 16]), false, false);
    w[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  return halfwave_transpose_sum16(w, lane);
}

// Sum over the 32 lanes of each half-wave, in every lane of the half: 16-lane row sums by DPP
// (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror), then the two rows of
// the half added through v_permlane16_swap.
NOISE_DEV float halfwave_sum(float v) {
  v += dpp_row<0xB1>(v);
  v += dpp_row<0x4E>(v);
  v += dpp_row<0x141>(v);
  v += dpp_row<0x140>(v);
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

}  // namespace noise
