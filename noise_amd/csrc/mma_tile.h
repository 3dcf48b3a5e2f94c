// 256 x BN bf16 MFMA tile main loop shared by the perturbed GEMM (BN = 128) and the head kernel
// (BN = 256).
//
// acc += A[0:256, 0:K] * B[0:BN, 0:K]^T for A, B row-major bf16 with K contiguous. The workgroup
// has 2 x (BN / 64) waves; wave (wm, wn) owns rows wm*128.. and columns wn*64.. as 4 x 2 blocks
// of v_mfma_f32_32x32x16_bf16 (128 fp32 accumulators per lane). Block (mi, ni), accumulator j of
// lane l holds
//   row = wm*128 + mi*32 + 8*(j/4) + 4*(l/32) + j%4,   col = wn*64 + ni*32 + l%32.
//
// Pipeline (measured on MI355X: under load a stage's global loads take longer than its MFMAs,
// so loads run two stages ahead):
//   * K advances 32 per stage through two LDS buffers of 64-byte rows whose four 16-byte chunks
//     are swizzled, chunk c of row r stored at c ^ ((r >> 2) & 3): both the staging stores (four
//     lanes per row) and the fragment reads (one row per lane) then touch 16 distinct 16-byte
//     bank groups per 16 lanes. Measured on MI355X: zero LDS bank-conflict cycles, against 8 per
//     16-byte store with padded 80-byte rows (which read conflict-free);
//   * global loads for stage s+2 are issued at the start of stage s into one of two register
//     staging sets (the sets alternate by name, never copied: a copy would wait for the loads in
//     flight) while the other set (stage s+1) drains into LDS at the end of stage s;
//   * fragments for k-step 1 are read while the 8 MFMAs of k-step 0 issue.
// With BN = 128 (4 waves, 60 KB of LDS) two workgroups share a CU, so one workgroup's barrier and
// epilogue overlap the other's MFMAs (measured: +10% over one 8-wave 256 x 256 workgroup in the
// main loop alone, more with the epilogue).
// Rows of A at or beyond `a_rows` are read from row a_rows - 1 (their results are discarded).
// K must be a multiple of 64.
#pragma once
#include "common.h"

namespace noise {

constexpr int TILE_M = 256, TBK = 32, TLDK = TBK;  // 64-byte LDS rows, chunk-swizzled

template <int BN>
struct TileCfg {
  static constexpr int WAVES = 2 * (BN / 64);
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int RP = THREADS / 4;             // rows per global-load pass
  static constexpr int NA = TILE_M / RP, NB = BN / RP;
  static constexpr int BOFS = TILE_M * TLDK;         // elements from the A to the B half
  static constexpr int BUF = (TILE_M + BN) * TLDK;   // elements per stage buffer
  static constexpr int SMEM_ELEMS = 2 * BUF;
};

template <int BN>
NOISE_DEV void mma_tile(const uint16_t* __restrict__ A, int64_t lda, int a_rows,
                        const uint16_t* __restrict__ B, int64_t ldb, int K, uint16_t* smem,
                        floatx16 (&acc)[4][2]) {
  using C = TileCfg<BN>;
  constexpr int NA = C::NA, NB = C::NB, RP = C::RP, BUF = C::BUF, BOFS = C::BOFS;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / (BN / 64), wn = wave % (BN / 64);
  const int KT = K / TBK;
  const int lr = tid >> 2, lc = (tid & 3) * 8;  // RP rows x 4 chunks of 16 B per pass
  const uint16_t* arow[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    int r = lr + i * RP;
    r = r < a_rows ? r : a_rows - 1;
    arow[i] = A + (int64_t)r * lda + lc;
  }
  const uint16_t* brow = B + (int64_t)lr * ldb + lc;
  const int64_t bstep = (int64_t)RP * ldb;
  // Fragment rows are lane % 32 plus multiples of 32, so their swizzle is ((lane % 32) >> 2) & 3;
  // k-step 0 reads logical chunk lane / 32, k-step 1 chunk 2 + lane / 32 (= that ^ 2).
  const int sw = ((lane & 31) >> 2) & 3;
  const int kofs0 = (((lane >> 5)) ^ sw) * 8, kofs1 = kofs0 ^ 16;
  const int far = wm * 128 + (lane & 31), fbr = wn * 64 + (lane & 31);
  const uint16_t* fa_base0 = smem + far * TLDK + kofs0;
  const uint16_t* fb_base0 = smem + BOFS + fbr * TLDK + kofs0;
  const uint16_t* fa_base1 = smem + far * TLDK + kofs1;
  const uint16_t* fb_base1 = smem + BOFS + fbr * TLDK + kofs1;
  // Staging rows lr + i * RP share lr's swizzle (RP is a multiple of 16).
  uint16_t* st_base = smem + lr * TLDK + ((lc >> 3) ^ ((lr >> 2) & 3)) * 8;
  bf16x8 a0[4], b0[2], a1[4], b1[2];
  u32x4 s0[NA + NB], s1[NA + NB];  // staging sets: NA rows of A, then NB rows of B

// Unconditional (past the end it re-reads the last stage, in bounds): a guarded load would make
// the wait before the LDS store conservative on the merged path and drain the prefetch.
#define NOISE_GLOAD(S, KT_)                                                                   \
  {                                                                                         \
    const int k0_ = ((KT_) < KT ? (KT_) : KT - 1) * TBK;                                    \
    _Pragma("unroll") for (int i = 0; i < NA; ++i)                                          \
      S[i] = *reinterpret_cast<const u32x4*>(arow[i] + k0_);                                \
    _Pragma("unroll") for (int i = 0; i < NB; ++i)                                          \
      S[NA + i] = *reinterpret_cast<const u32x4*>(brow + i * bstep + k0_);                  \
  }
#define NOISE_SSTORE(S, BUF_)                                                                 \
  {                                                                                         \
    uint16_t* d_ = st_base + (BUF_) * BUF;                                                  \
    _Pragma("unroll") for (int i = 0; i < NA; ++i)                                          \
      *reinterpret_cast<u32x4*>(d_ + i * RP * TLDK) = S[i];                                 \
    _Pragma("unroll") for (int i = 0; i < NB; ++i)                                          \
      *reinterpret_cast<u32x4*>(d_ + BOFS + i * RP * TLDK) = S[NA + i];                     \
  }
#define NOISE_FLOAD(FA, FB, BUF_, KS_)                                                        \
  {                                                                                         \
    const uint16_t* pa_ = ((KS_) ? fa_base1 : fa_base0) + (BUF_) * BUF;                     \
    const uint16_t* pb_ = ((KS_) ? fb_base1 : fb_base0) + (BUF_) * BUF;                     \
    _Pragma("unroll") for (int i = 0; i < 4; ++i)                                           \
      FA[i] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(pa_ + i * 32 * TLDK)); \
    _Pragma("unroll") for (int i = 0; i < 2; ++i)                                           \
      FB[i] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(pb_ + i * 32 * TLDK)); \
  }
#define NOISE_MFMA8(FA, FB)                                                                   \
  _Pragma("unroll") for (int mi = 0; mi < 4; ++mi)                                          \
    _Pragma("unroll") for (int ni = 0; ni < 2; ++ni)                                        \
      acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(FA[mi], FB[ni], acc[mi][ni], 0, 0, 0);
// Stage KS from LDS buffer CUR (k-step-0 fragments already in a0/b0): stage KS + 2 loads into
// the free set L; the set S holding stage KS + 1 drains into buffer CUR ^ 1 after the MFMAs.
#define NOISE_STAGE(KS, CUR, L, S)                                                            \
  NOISE_GLOAD(L, (KS) + 2)                                                                  \
  __builtin_amdgcn_sched_barrier(0);                                                        \
  NOISE_FLOAD(a1, b1, CUR, 1)                                                               \
  NOISE_MFMA8(a0, b0)                                                                       \
  NOISE_MFMA8(a1, b1)                                                                       \
  if ((KS) + 1 < KT) NOISE_SSTORE(S, (CUR) ^ 1)                                             \
  __syncthreads();                                                                          \
  if ((KS) + 1 < KT) NOISE_FLOAD(a0, b0, (CUR) ^ 1, 0)

  NOISE_GLOAD(s0, 0)
  NOISE_GLOAD(s1, 1)
  __syncthreads();  // the previous user of smem is done
  NOISE_SSTORE(s0, 0)
  __syncthreads();
  NOISE_FLOAD(a0, b0, 0, 0)
  // Not unrolled further even for a constant K: full unrolling makes the compiler precompute
  // every stage's addresses and spill them.
#pragma unroll 1
  for (int kt = 0; kt < KT; kt += 2) {
    NOISE_STAGE(kt, 0, s0, s1)
    NOISE_STAGE(kt + 1, 1, s1, s0)
  }
#undef NOISE_STAGE
#undef NOISE_MFMA8
#undef NOISE_FLOAD
#undef NOISE_SSTORE
#undef NOISE_GLOAD
}

NOISE_DEV void zero_acc(floatx16 (&acc)[4][2]) {
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[mi][ni][j] = 0.f;
}

// Sum over the 32 lanes of each half-wave of 16 per-lane values; lane q of a half ends with the
// total of value (q >> 1) & 15 (lanes q and q ^ 1 hold the same total).
NOISE_DEV float halfwave_transpose_sum16(float (&v)[16], int lane) {
  const int q = lane & 31;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const bool up = q & 16;
    const float send = up ? v[i] : v[i + 8];
    const float keep = up ? v[i + 8] : v[i];
    v[i] = keep + __shfl_xor(send, 16, 64);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool up = q & 8;
    const float send = up ? v[i] : v[i + 4];
    const float keep = up ? v[i + 4] : v[i];
    v[i] = keep + __shfl_xor(send, 8, 64);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const bool up = q & 4;
    const float send = up ? v[i] : v[i + 2];
    const float keep = up ? v[i + 2] : v[i];
    v[i] = keep + __shfl_xor(send, 4, 64);
  }
  {
    const bool up = q & 2;
    const float send = up ? v[0] : v[1];
    const float keep = up ? v[1] : v[0];
    v[0] = keep + __shfl_xor(send, 2, 64);
  }
  return v[0] + __shfl_xor(v[0], 1, 64);
}

}  // namespace noise
