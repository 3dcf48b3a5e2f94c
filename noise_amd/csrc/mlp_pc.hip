// Fused MLP block, producer/consumer form: two waves per SIMD.
//   out = in + c_proj(relu(c_fc(norm in) + rank-1)^2) + rank-1
// Reference: train/val/eggroll.py:93 (x + lowrank(c_proj, relu(lowrank(c_fc, norm(x)))^2)),
// utils/model.py:100-107 (relu^2 MLP), `lowrank` eggroll.py:56-58 (x W^T + sign (x . b) a^T).
//
// The one-wave form (mlp.hip) keeps a wave's 32 rows x all 512 output columns in 256 accumulator
// registers, which leaves one 512-register wave per SIMD: the weight stream and the per-chunk
// epilogue add to the MFMA time instead of hiding under another wave's MFMAs. Here the same 128
// rows of a workgroup are split by role over eight waves, two per SIMD, 256 registers each:
//   * P (waves 0-3, one per 32 rows): h of its rows as the c_fc B operand (128 registers), the c_fc
//     MFMAs of every chunk, the chunk epilogue (rank-1 term, relu^2, bf16, the u_proj dots) and
//     the c_proj MFMAs of output columns 0-95 (3 accumulator blocks);
//   * C (waves 4-7, the same rows as P of wave - 4): the c_proj MFMAs of columns 96-511 (13
//     accumulator blocks, 208 registers) and every load of the weight stream.
// P hands each chunk's bf16 relu^2 operand (32 rows x 32 features, 2 KB) to its C through LDS.
// Step s (one barrier each, s = 0 .. 65) runs P's c_fc chunk s with the epilogue of chunk s - 1
// interleaved and P's c_proj of chunk s - 1, and C's c_proj of chunk s - 2 (its operand written by
// P in step s - 1); the stage buffer of step s holds c_fc chunk s, c_proj chunk s - 1 (blocks 0-2),
// c_proj chunk s - 2 (blocks 3-15) and the a_fc / b_proj slices of chunk s - 1, loaded by C during
// step s - 1. Every output value accumulates in the same order as in the one-wave form (the chunk
// order, k-step 0 then 1), and the norm, epilogue and rank-1 arithmetic is the same, so both
// forms give bit-identical rows.
// Measured on MI355X at 512 members x 2048 tokens: 4.9 ms against 4.46 ms for the one-wave form,
// so it runs only when asked for (NOISE_MLP_TWO_WAVE=1). Per workgroup the loop takes 129 us
// against about 131 us; a loop-only model of this layout is 27% faster on all-zero weights than on
// random ones (2.63 against 3.33 ms, the same instructions: the MFMA-bound kernels here run at the
// power limit, 1.9-2.0 GHz), and with random weights the model's loop is within 7% of the
// one-wave loop. The registers leave no room to close that: C at 256 with 13 blocks (14 spill
// inside the loop), P at 248.
#include <utility>

#include "mma_tile.h"

namespace {

constexpr int D = 512, F = 2048, FC = 32, NCH = F / FC;
constexpr int ROWS = 128;                          // rows per workgroup
constexpr int PB = 3, CB = 16 - PB;                // c_proj blocks of P and of C
constexpr int WFC_ROW = 1040;                      // bytes per c_fc row in LDS (1 KB + 16 pad)
constexpr int WFC_PART = FC * WFC_ROW;             // 33280
constexpr int WMP_PART = D * FC * 2;               // 32768: [16 blocks][32 rows][64 B], swizzled
// The two stage buffers, grouped by part so that one lane address serves both stages (the stage
// offset fits the 16-bit immediate of the LDS reads): c_fc parts, c_proj parts, the a_fc | b_proj
// slices of the stage's epilogue chunk, then the operand hand-over [2][4 pairs][64 lanes][32 B].
constexpr int FC_OFS = 0;
constexpr int MP_OFS = 2 * WFC_PART;               // 66560
constexpr int NZ_OFS = MP_OFS + 2 * WMP_PART;      // 132096
constexpr int NZ_PART = 2 * FC * 4;                // 256
constexpr int XB_OFS = NZ_OFS + 2 * NZ_PART;       // 132608
constexpr int XB_BYTES = 2 * 4 * 64 * 32;          // 16384
constexpr int LDS_BYTES = XB_OFS + XB_BYTES;       // 148992
// Prologue exchanges (before the stream starts; stage 0's c_fc part is loading meanwhile): the
// per-lane sums of squares [4 pairs][64 lanes][16] at PS_OFS (P's partial, then C's total); the
// row factors [4][32] at RR_OFS (the end of the hand-over buffer); after B3, h = bf16 of C's
// normalised columns 96-511, row-major [4 pairs][32 rows][832 B] at TILE_OFS (over the sums).
constexpr int TILE_ROW = 2 * (D - 32 * PB);        // 832
constexpr int TILE_OFS = WFC_PART;
constexpr int PS_OFS = TILE_OFS;
constexpr int RR_OFS = XB_OFS + XB_BYTES - 4 * 32 * 4;
constexpr int PC_AHEAD = 2;                        // MFMAs of fragment-read lookahead
constexpr float RMS_EPS = 1.1920928955078125e-07f;  // float32 machine epsilon (F.rms_norm default)

static_assert(TILE_OFS + 4 * 32 * TILE_ROW <= RR_OFS && PS_OFS + 4 * 64 * 64 <= RR_OFS, "prologue exchanges overlap");
static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
static_assert(WFC_PART + 32 * 31 + 16 < 65536 && WMP_PART + 2048 * 15 + 48 < 65536, "stage offsets as immediates");

#define PC_DSREAD(DST, ADDR, OFS) __asm__ volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(DST) : "v"(ADDR), "n"(OFS))
#define PC_LGKM(N) __asm__ volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N))
// Opening of a step: this wave's loads of the stage have landed and its LDS writes are done, then
// every wave's.
#define PC_STEP_WAIT() __asm__ volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory")

NOISE_DEV bf16x8 as_bf16x8(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3) {
  return __builtin_bit_cast(bf16x8, (u32x4){w0, w1, w2, w3});
}

// The permuted identities of the h transpose (as in the one-wave form): with A = h block nb (lane:
// column 32 nb + l % 32, k-slots = the lane's accumulator rows 16 sx + 8 (q / 4) + 4 (l / 32) +
// q % 4) and B[k][j] = 1 where row(k) = j, the two MFMAs give h^T exactly, its accumulators holding
// row l % 32 at the columns 32 nb + 8 (v / 4) + 4 (l / 32) + v % 4: the k order of the packed c_fc.
NOISE_DEV void identities(bf16x8 (&ident)[2], int r, int half) {
#pragma unroll
  for (int sx = 0; sx < 2; ++sx) {
    const bool mine = (r >> 4) == sx && ((r >> 2) & 1) == half;
    const int q = 4 * ((r >> 3) & 1) + (r & 3);
    uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int k = 0; k < 4; ++k) w[k] = (mine && (q >> 1) == k) ? (0x3F80u << (16 * (q & 1))) : 0u;
    ident[sx] = as_bf16x8(w[0], w[1], w[2], w[3]);
  }
}

// h operand pieces (k-steps 2 nb, 2 nb + 1) of one accumulator block of rows scaled by rrj.
NOISE_DEV void h_block(const floatx16& a, const float (&rrj)[16], const bf16x8 (&ident)[2], bf16x8& h0, bf16x8& h1) {
  uint32_t hw[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) hw[k] = pack_bf2(a[2 * k] * rrj[2 * k], a[2 * k + 1] * rrj[2 * k + 1]);
  floatx16 tr = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(hw[0], hw[1], hw[2], hw[3]), ident[0],
                                                         (floatx16){}, 0, 0, 0);
  tr = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(hw[4], hw[5], hw[6], hw[7]), ident[1], tr, 0, 0, 0);
  h0 = as_bf16x8(pack_bf2(tr[0], tr[1]), pack_bf2(tr[2], tr[3]), pack_bf2(tr[4], tr[5]), pack_bf2(tr[6], tr[7]));
  h1 = as_bf16x8(pack_bf2(tr[8], tr[9]), pack_bf2(tr[10], tr[11]), pack_bf2(tr[12], tr[13]), pack_bf2(tr[14], tr[15]));
}

// x rows of the pair into accumulator blocks NB0 .. NB0 + NBK - 1 (lane l: column 32 nb + l % 32 of
// rows tb + 8 (j / 4) + 4 (l / 32) + j % 4), the loads straight into the registers by inline asm,
// three rows of blocks ahead of the wait that ties them to their registers.
template <int NB0, int NBK, int J>
NOISE_DEV void row_issue(floatx16 (&acc)[NBK], const float* xrow, int64_t ld_in, int tb, int T, int half) {
  const int rj = tb + 8 * (J >> 2) + 4 * half + (J & 3);
  const float* src = xrow + (int64_t)(rj < T ? rj : T - 1) * ld_in;
#pragma unroll
  for (int nb = 0; nb < NBK; ++nb)
    __asm__ volatile("global_load_dword %0, %1, off offset:%2" : "=v"(acc[nb][J]) : "v"(src), "n"((NB0 + nb) * 128));
}

template <int NBK, int J, int N>
NOISE_DEV void row_wait(floatx16 (&acc)[NBK]) {
  __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(N));
#pragma unroll
  for (int nb = 0; nb < NBK; ++nb) __asm__ volatile("" : "+v"(acc[nb][J]));
}

template <int NB0, int NBK, int... J>
NOISE_DEV void load_rows_seq(floatx16 (&acc)[NBK], const float* xrow, int64_t ld_in, int tb, int T, int half,
                             std::integer_sequence<int, J...>) {
  row_issue<NB0, NBK, 0>(acc, xrow, ld_in, tb, T, half);
  row_issue<NB0, NBK, 1>(acc, xrow, ld_in, tb, T, half);
  row_issue<NB0, NBK, 2>(acc, xrow, ld_in, tb, T, half);
  (([&] {
     if constexpr (J + 3 < 16) row_issue<NB0, NBK, (J + 3 < 16 ? J + 3 : 0)>(acc, xrow, ld_in, tb, T, half);
     row_wait<NBK, J, NBK * (15 - J < 3 ? 15 - J : 3)>(acc);
   }()),
   ...);
}

// x rows of the pair into accumulator blocks NB0 .. NB0 + NBK - 1 (lane l: column 32 nb + l % 32 of
// rows tb + 8 (j / 4) + 4 (l / 32) + j % 4), the loads straight into the registers by inline asm,
// three rows of blocks ahead of the wait that ties them to their registers (vector loads retire in
// issue order).
template <int NB0, int NBK>
NOISE_DEV void load_rows(floatx16 (&acc)[NBK], const float* xrow, int64_t ld_in, int tb, int T, int half) {
  load_rows_seq<NB0, NBK>(acc, xrow, ld_in, tb, T, half, std::make_integer_sequence<int, 16>{});
}

// ---- P: one step. FCP: the c_fc MFMAs of this step's chunk into fc[FB]; EPI: the epilogue of the
// previous chunk from fc[1 - FB] (rank-1 term, relu^2, bf16, u_proj dots) in 8 pieces after c_fc
// MFMAs 0-7 (all of them first when !FCP), its operand handed to C, and P's 2 PB c_proj MFMAs of
// it (blocks 0 .. PB - 1, k-step 0 then 1), after c_fc MFMAs PRJ_AFTER[].
// With both halves, piece E's four perturbation values (a_fc and b_proj of its two features) are
// read two MFMAs ahead of it, next to the fragment reads; POps counts the LDS reads issued after
// each one so that every wait is exact.
constexpr int PRJ_AFTER[6] = {8, 13, 18, 23, 28, 32};  // k-step 1 needs pieces 4-7 (after MFMA 7)
static_assert(PB == 3, "PRJ_AFTER lists 2 PB positions");
template <bool FCP, bool EPI>
struct POps {
  static constexpr int N = (FCP ? 32 : 0) + (EPI ? 2 * PB : 0);
  // op s is c_proj MFMA pi when it directly follows c_fc MFMA PRJ_AFTER[pi] - 1
  static constexpr int prj(int s) {
    if (!EPI) return -1;
    if (!FCP) return s;
    for (int pi = 0; pi < 2 * PB; ++pi)
      if (s == PRJ_AFTER[pi] + pi) return pi;
    return -1;
  }
  static constexpr bool is_fc(int s) { return prj(s) < 0; }
  static constexpr int idx(int s) {
    if (prj(s) >= 0) return prj(s);
    int before = 0;
    for (int x = 0; x < s; ++x) before += prj(x) >= 0;
    return s - before;
  }
  static constexpr bool PIECES = FCP && EPI;  // pieces interleaved, their values read ahead
  // Issue order: fragments 0 .. PC_AHEAD - 1, piece reads 0 and 1 (two each); then before op x:
  // fragment x + PC_AHEAD, piece reads x + 2 (x + 2 < 8).
  static constexpr int wait_frag(int sx) {
    int pos = 0, fpos = -1;
    for (int f = 0; f < PC_AHEAD && f < N; ++f) {
      if (f == sx) fpos = pos;
      ++pos;
    }
    if (PIECES) pos += 4;
    for (int x = 0; x <= sx; ++x) {
      if (x + PC_AHEAD < N) {
        if (x + PC_AHEAD == sx) fpos = pos;
        ++pos;
      }
      if (PIECES && x + 2 < 8) pos += 2;
    }
    return pos - fpos - 1;
  }
  static constexpr int wait_piece(int e) {
    int pos = PC_AHEAD < N ? PC_AHEAD : N, ppos = -1;
    for (int k = 0; k < 2; ++k) {
      pos += 2;
      if (k == e) ppos = pos - 1;
    }
    for (int x = 0; x <= e; ++x) {
      if (x + PC_AHEAD < N) ++pos;
      if (x + 2 < 8) {
        pos += 2;
        if (x + 2 == e) ppos = pos - 1;
      }
    }
    return pos - ppos - 1;
  }
  static constexpr bool waits_fit() {
    for (int sx = 0; sx < N; ++sx)
      if (wait_frag(sx) < 0 || wait_frag(sx) > 15) return false;
    if (PIECES)
      for (int e = 0; e < 8; ++e)
        if (wait_piece(e) < 0 || wait_piece(e) > 15) return false;
    return true;
  }
};

template <bool FCP, bool EPI, int FB>
NOISE_DEV void p_step(const bf16x8 (&hB)[32], floatx16 (&fc)[2], floatx16 (&acc)[PB], float& up, uint32_t fcb,
                      uint32_t mpb0, uint32_t mpb1, uint32_t nzb, float su, uint32_t xo) {
  // FB is also the stage: step s uses fc[s % 2] and stage s % 2
  using O = POps<FCP, EPI>;
  static_assert(O::waits_fit(), "lgkmcnt out of range");
  constexpr int NA = PC_AHEAD + 1;
  // piece E's values: pa = a_fc, pb = b_proj of features 8 (E / 2) + 4 half + 2 (E % 2) + 0, 1
  floatx2 pa[8], pb[8];
  auto read_piece = [&pa, &pb, nzb]<int E>() __attribute__((always_inline)) {
    constexpr int ofs = FB * NZ_PART + 32 * (E >> 1) + 8 * (E & 1);
    __asm__ volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(pa[E]) : "v"(nzb), "n"(ofs));
    __asm__ volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(pb[E]) : "v"(nzb), "n"(128 + ofs));
  };
  bf16x8 fr[NA];
  auto read = [&fr, fcb, mpb0, mpb1]<int S>() __attribute__((always_inline)) {
    constexpr int i = O::idx(S);
    if constexpr (O::is_fc(S)) PC_DSREAD(fr[S % NA], fcb, FB * WFC_PART + 32 * i);
    else if constexpr (i < PB) PC_DSREAD(fr[S % NA], mpb0, FB * WMP_PART + 2048 * i);
    else PC_DSREAD(fr[S % NA], mpb1, FB * WMP_PART + 2048 * (i - PB));
  };
  [&]<int... S>(std::integer_sequence<int, S...>) __attribute__((always_inline)) {
    (read.template operator()<S>(), ...);
  }(std::make_integer_sequence<int, PC_AHEAD>{});
  if constexpr (EPI) {
    if constexpr (O::PIECES) {
      read_piece.template operator()<0>();
      read_piece.template operator()<1>();
    } else {  // the last step: every piece's values now
      [&]<int... E>(std::integer_sequence<int, E...>) __attribute__((always_inline)) {
        (read_piece.template operator()<E>(), ...);
      }(std::make_integer_sequence<int, 8>{});
    }
  }
  uint32_t hw[8];
  bf16x8 hid[2];
  auto epi = [&]<int E>() __attribute__((always_inline)) {
    const float v0 = fmaxf(fc[1 - FB][2 * E] + su * pa[E][0], 0.f);
    const float v1 = fmaxf(fc[1 - FB][2 * E + 1] + su * pa[E][1], 0.f);
    const uint32_t w = pack_bf2(v0 * v0, v1 * v1);
    hw[E] = w;
    up += bf_lo(w) * pb[E][0] + bf_hi(w) * pb[E][1];
    if constexpr (E == 3) hid[0] = as_bf16x8(hw[0], hw[1], hw[2], hw[3]);
    if constexpr (E == 7) {
      hid[1] = as_bf16x8(hw[4], hw[5], hw[6], hw[7]);
      // handed to C (read there after the next barrier); later than every read above
      const uint32_t xa = xo;
      __asm__ volatile("ds_write_b128 %0, %1 offset:%2\n\tds_write_b128 %0, %3 offset:%4"
                       :: "v"(xa), "v"(hid[0]), "n"(FB * 8192), "v"(hid[1]), "n"(FB * 8192 + 16));
    }
  };
  if constexpr (EPI && !FCP) {  // last step: the whole epilogue first
    PC_LGKM(0);
    [&]<int... E>(std::integer_sequence<int, E...>) __attribute__((always_inline)) {
      ([&] {
        floatx2& ra = pa[E];
        floatx2& rb = pb[E];
        __asm__ volatile("" : "+v"(ra), "+v"(rb));
      }(), ...);
      (epi.template operator()<E>(), ...);
    }(std::make_integer_sequence<int, 8>{});
  }
  auto op = [&]<int SX>() __attribute__((always_inline)) {
    if constexpr (SX + PC_AHEAD < O::N) read.template operator()<SX + PC_AHEAD>();
    if constexpr (O::PIECES && SX + 2 < 8) read_piece.template operator()<SX + 2>();
    PC_LGKM(O::wait_frag(SX));
    const bf16x8 f = fr[SX % NA];
    constexpr int i = O::idx(SX);
    if constexpr (O::is_fc(SX)) {
      if constexpr (i == 0)
        __asm__ volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(fc[FB]) : "v"(f), "v"(hB[i]));
      else if constexpr (i < 31)
        __asm__ volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(fc[FB]) : "v"(f), "v"(hB[i]));
      else  // read by VALU in the next step's epilogue
        __asm__ volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
                         : "+v"(fc[FB]) : "v"(f), "v"(hB[i]));
      if constexpr (O::PIECES && i < 8) {
        __builtin_amdgcn_sched_barrier(0);
        PC_LGKM(O::wait_piece(i));
        {
          floatx2& ra = pa[i];
          floatx2& rb = pb[i];
          __asm__ volatile("" : "+v"(ra), "+v"(rb));
        }
        epi.template operator()<i>();
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {  // c_proj block i % PB, k-step i / PB; its operand was written by VALU
      floatx16& a = acc[i % PB];
      const bf16x8 hx = hid[i / PB];
      if constexpr (i < 2 * PB - 1 || FCP)
        __asm__ volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(a) : "v"(hx), "v"(f));
      else  // the last c_proj MFMA: the epilogue's VALU reads the accumulators next
        __asm__ volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
                         : "+v"(a) : "v"(hx), "v"(f));
    }
  };
  [&]<int... S>(std::integer_sequence<int, S...>) __attribute__((always_inline)) {
    (op.template operator()<S>(), ...);
  }(std::make_integer_sequence<int, O::N>{});
}

// ---- C: the loads of the next stage during step s. Wave LW takes pieces t = 16 LW .. 16 LW + 15 of
// 64 1-KB pieces (this lane's 16 bytes at + 16 lane): t < 32 c_fc chunk s + 1 row t; 32 <= t < 38
// c_proj chunk s piece t - 32 (blocks 0-2); t >= 38 c_proj chunk s - 1 piece t - 32 (blocks 3-15);
// wave 3 also the 256-byte slice a_fc | b_proj of chunk s (zeros when unperturbed). Chunk indices
// wrap, so the pieces no later step reads (past the last chunk, before the first) are loaded from
// a valid chunk and never used.
__device__ __align__(16) float kZeroSlice[64];  // zero-initialised device memory

struct CLoadPtrs {
  const uint16_t* fc;   // c_fc chunk s + 1, row 16 LW (LW < 2)
  const uint16_t* mp0;  // c_proj chunk s, piece 0
  const uint16_t* mp1;  // c_proj chunk s - 1, piece 0
  const float* nz;      // this lane's float of the slice
};

template <int LW>
NOISE_DEV CLoadPtrs c_ptrs(const noise_mlp_t& g, int s, int c0, int64_t pn, bool pert, int lane) {
  CLoadPtrs P;
  const int cf = (s + 1 + c0) & (NCH - 1), cm = (s + c0) & (NCH - 1), cm1 = (s - 1 + c0) & (NCH - 1);
  P.fc = g.w_fc + (int64_t)(cf * FC + 16 * LW) * D + lane * 8;
  P.mp0 = g.w_proj + (int64_t)cm * (D * FC) + lane * 8;
  P.mp1 = g.w_proj + (int64_t)cm1 * (D * FC) + lane * 8;
  P.nz = !pert ? kZeroSlice + lane
         : lane < 32 ? g.a_fc + pn * g.ld_a_fc + cm * FC + lane
                     : g.b_proj + pn * g.ld_b_proj + cm * FC + (lane - 32);
  return P;
}

template <int LW, int K>
NOISE_DEV void c_load(const CLoadPtrs& P, unsigned char* lds, int st) {
  if constexpr (K < 16) {
    constexpr int t = 16 * LW + K;
    if constexpr (t < 32)
      __builtin_amdgcn_global_load_lds((const void*)(P.fc + K * D), (void*)(lds + FC_OFS + st * WFC_PART + t * WFC_ROW),
                                       16, 0, 0);
    else if constexpr (t < 32 + 2 * PB)
      __builtin_amdgcn_global_load_lds((const void*)(P.mp0 + (t - 32) * 512),
                                       (void*)(lds + MP_OFS + st * WMP_PART + (t - 32) * 1024), 16, 0, 0);
    else
      __builtin_amdgcn_global_load_lds((const void*)(P.mp1 + (t - 32) * 512),
                                       (void*)(lds + MP_OFS + st * WMP_PART + (t - 32) * 1024), 16, 0, 0);
  } else if constexpr (LW == 3) {
    __builtin_amdgcn_global_load_lds((const void*)P.nz, (void*)(lds + NZ_OFS + st * NZ_PART), 4, 0, 0);
  }
}

// C: one step in stage ST. PRJ: 2 CB c_proj MFMAs (k-step 0 over blocks PB-15, then k-step 1) of the
// operand P handed over in the previous step; LOAD: the next stage's loads (into stage 1 - ST),
// spread over the MFMAs; LAST: the accumulators are read by VALU after it.
template <int LW, int ST, bool PRJ, bool LOAD, bool LAST>
NOISE_DEV void c_step(floatx16 (&acc)[CB], uint32_t xa, uint32_t mpb0, uint32_t mpb1, const CLoadPtrs& L,
                      unsigned char* lds) {
  if constexpr (!PRJ) {
    [&]<int... K>(std::integer_sequence<int, K...>) __attribute__((always_inline)) {
      (c_load<LW, K>(L, lds, 1 - ST), ...);
    }(std::make_integer_sequence<int, 17>{});
    return;
  } else {
    constexpr int N = 2 * CB, NA = PC_AHEAD + 1;
    bf16x8 h0, h1;
    // the operand of the chunk before, handed over in the previous step (its parity 1 - ST)
    PC_DSREAD(h0, xa, (1 - ST) * 8192);
    PC_DSREAD(h1, xa, (1 - ST) * 8192 + 16);
    bf16x8 fr[NA];
    auto read = [&fr, mpb0, mpb1]<int S>() __attribute__((always_inline)) {
      if constexpr (S < CB) PC_DSREAD(fr[S % NA], mpb0, ST * WMP_PART + 2048 * (PB + S));
      else PC_DSREAD(fr[S % NA], mpb1, ST * WMP_PART + 2048 * (PB + S - CB));
    };
    [&]<int... S>(std::integer_sequence<int, S...>) __attribute__((always_inline)) {
      (read.template operator()<S>(), ...);
    }(std::make_integer_sequence<int, PC_AHEAD>{});
    auto op = [&]<int SX>() __attribute__((always_inline)) {
      // load k goes out with MFMA N k / 17 (integer), k = 0 .. 16
      if constexpr (LOAD) {
        [&]<int... K>(std::integer_sequence<int, K...>) __attribute__((always_inline)) {
          ([&] {
            if constexpr ((N * K) / 17 == SX) c_load<LW, K>(L, lds, 1 - ST);
          }(), ...);
        }(std::make_integer_sequence<int, 17>{});
      }
      if constexpr (SX + PC_AHEAD < N) read.template operator()<SX + PC_AHEAD>();
      PC_LGKM(N - 1 - SX < PC_AHEAD ? N - 1 - SX : PC_AHEAD);
      if constexpr (SX == 0) {  // the first wait covered the operand reads too
        bf16x8& r0 = h0;
        bf16x8& r1 = h1;
        __asm__ volatile("" : "+v"(r0), "+v"(r1));
      }
      const bf16x8 f = fr[SX % NA];
      const bf16x8 hx = SX < CB ? h0 : h1;
      floatx16& a = acc[SX % CB];
      if constexpr (LAST && SX == N - 1)
        __asm__ volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
                         : "+v"(a) : "v"(hx), "v"(f));
      else
        __asm__ volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(a) : "v"(hx), "v"(f));
    };
    [&]<int... S>(std::integer_sequence<int, S...>) __attribute__((always_inline)) {
      (op.template operator()<S>(), ...);
    }(std::make_integer_sequence<int, N>{});
  }
}

// LDS byte address of lane (r, half)'s c_proj fragment of k-step kk in stage 0 (stage 1 at
// + WMP_PART, block nb at + 2048 nb): row 32 nb + r at piece (2 kk + half) ^ ((r >> 2) & 3).
NOISE_DEV uint32_t mp_addr(uint32_t lds0, int kk, int r, int half) {
  return lds0 + MP_OFS + r * 64 + 16 * ((2 * kk + half) ^ ((r >> 2) & 3));
}

struct Work {
  int p, tb, c0;
  int64_t pn;
  float s;
  bool pert;
};

template <bool NORM, bool RESID>
NOISE_DEV void p_wave(const noise_mlp_t& g, const Work& w, unsigned char* lds, int q, int lane) {
  const int r = lane & 31, half = lane >> 5;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)lds;
  floatx16 acc[PB];
  load_rows<0, PB>(acc, g.in + (int64_t)w.p * g.member_stride_in + r, g.ld_in, w.tb, g.T, half);
  float4* psb = reinterpret_cast<float4*>(lds + PS_OFS + (q * 64 + lane) * 64);
  if (NORM) {  // this lane's partial sums of squares over blocks 0 .. PB - 1, continued by C
    float ps[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      ps[j] = 0.f;
#pragma unroll
      for (int nb = 0; nb < PB; ++nb) ps[j] += acc[nb][j] * acc[nb][j];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) psb[k] = make_float4(ps[4 * k], ps[4 * k + 1], ps[4 * k + 2], ps[4 * k + 3]);
  }
  __syncthreads();  // B1: P's partial sums are in
  __syncthreads();  // B2: C's totals are in
  float rrj[16];
  if (NORM) {
    // the row factors as the one-wave form forms them: the half-wave transpose sum leaves lane
    // 2 j + 32 half with row 8 (j / 4) + 4 half + j % 4
    float ps[16];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float4 v = psb[k];
      ps[4 * k] = v.x;
      ps[4 * k + 1] = v.y;
      ps[4 * k + 2] = v.z;
      ps[4 * k + 3] = v.w;
    }
    const float rr = rsqrtf(noise::halfwave_transpose_sum16(ps, lane) * (1.0f / D) + RMS_EPS);
    if ((lane & 1) == 0) {
      const int j = (lane & 31) >> 1;
      reinterpret_cast<float*>(lds + RR_OFS)[q * 32 + 8 * (j >> 2) + 4 * half + (j & 3)] = rr;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) rrj[j] = __shfl(rr, (lane & 32) + 2 * j, 64);
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) rrj[j] = 1.f;
  }
  bf16x8 ident[2];
  identities(ident, r, half);
  bf16x8 hB[32];
#pragma unroll
  for (int nb = 0; nb < PB; ++nb) h_block(acc[nb], rrj, ident, hB[2 * nb], hB[2 * nb + 1]);
  __syncthreads();  // B3: the row factors are in
  __syncthreads();  // B4: C's columns of h are in the tile
  {
    // k-step ks = 2 nb + t, slot e: column 32 nb + 16 t + 8 (e / 4) + 4 half + e % 4 of row r
    const unsigned char* row = lds + TILE_OFS + q * 32 * TILE_ROW + r * TILE_ROW + 8 * half - 64 * PB;
#pragma unroll
    for (int ks = 2 * PB; ks < 32; ++ks) {
      const u32x2 lo = *reinterpret_cast<const u32x2*>(row + 32 * ks);
      const u32x2 hi = *reinterpret_cast<const u32x2*>(row + 32 * ks + 16);
      hB[ks] = as_bf16x8(lo[0], lo[1], hi[0], hi[1]);
    }
  }
  // u_fc = bf16(h) . b_fc of row l % 32 (as the one-wave form: this lane's 256 columns, then the
  // other half-row from lane l ^ 32)
  float uf = 0.f;
  if (w.pert) {
    const float* bfc = g.b_fc + w.pn * g.ld_b_fc;
#pragma unroll
    for (int ks = 0; ks < 32; ++ks) {
      const float4 b0 = *reinterpret_cast<const float4*>(bfc + 16 * ks + 4 * half);
      const float4 b1 = *reinterpret_cast<const float4*>(bfc + 16 * ks + 8 + 4 * half);
      const u32x4 hv = __builtin_bit_cast(u32x4, hB[ks]);
      uf += bf_lo(hv[0]) * b0.x + bf_hi(hv[0]) * b0.y + bf_lo(hv[1]) * b0.z + bf_hi(hv[1]) * b0.w;
      uf += bf_lo(hv[2]) * b1.x + bf_hi(hv[2]) * b1.y + bf_lo(hv[3]) * b1.z + bf_hi(hv[3]) * b1.w;
    }
  }
  uf += __shfl_xor(uf, 32, 64);
  const float su = w.s * uf;
  if (!RESID) {
#pragma unroll
    for (int nb = 0; nb < PB; ++nb)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[nb][j] = 0.f;
  }

  const uint32_t fcb = lds0 + FC_OFS + r * WFC_ROW + 16 * half;
  const uint32_t mpb0 = mp_addr(lds0, 0, r, half), mpb1 = mp_addr(lds0, 1, r, half);
  const uint32_t nzb = lds0 + NZ_OFS + 16 * half;
  const uint32_t xo = lds0 + XB_OFS + (q * 64 + lane) * 32;
  floatx16 fc[2];
  float up = 0.f;
  PC_STEP_WAIT();  // step 0
  p_step<true, false, 0>(hB, fc, acc, up, fcb, mpb0, mpb1, nzb, su, xo);
#pragma unroll 1
  for (int s = 1; s < NCH - 1; s += 2) {
    PC_STEP_WAIT();
    p_step<true, true, 1>(hB, fc, acc, up, fcb, mpb0, mpb1, nzb, su, xo);
    PC_STEP_WAIT();
    p_step<true, true, 0>(hB, fc, acc, up, fcb, mpb0, mpb1, nzb, su, xo);
  }
  PC_STEP_WAIT();  // step 63
  p_step<true, true, 1>(hB, fc, acc, up, fcb, mpb0, mpb1, nzb, su, xo);
  PC_STEP_WAIT();  // step 64: the last chunk's epilogue and c_proj
  p_step<false, true, 0>(hB, fc, acc, up, fcb, mpb0, mpb1, nzb, su, xo);
  PC_STEP_WAIT();  // step 65: C's last c_proj

  up += __shfl_xor(up, 32, 64);  // lane l: row l % 32
  const float sup = w.s * up;
  // the u_proj factors for C: the hand-over slot of parity 1 was last read by C in step 64
  if (lane < 32) reinterpret_cast<float*>(lds + XB_OFS + 8192)[q * 32 + r] = sup;
  __syncthreads();  // B5
  float am[PB];
#pragma unroll
  for (int nb = 0; nb < PB; ++nb) am[nb] = w.pert ? g.a_proj[w.pn * g.ld_a_proj + nb * 32 + r] : 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int rl = 8 * (j >> 2) + 4 * half + (j & 3);
    const float sr = __shfl(sup, rl, 64);
    const int rj = w.tb + rl;
    if (rj < g.T) {
      float* dst = g.out + (int64_t)w.p * g.member_stride_out + (int64_t)rj * g.ld_out + r;
#pragma unroll
      for (int nb = 0; nb < PB; ++nb) dst[nb * 32] = acc[nb][j] + sr * am[nb];
    }
  }
}

template <bool NORM, bool RESID, int LW>
NOISE_DEV void c_wave(const noise_mlp_t& g, const Work& w, unsigned char* lds, int lane) {
  constexpr int q = LW;
  const int r = lane & 31, half = lane >> 5;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)lds;
  floatx16 acc[CB];
  load_rows<PB, CB>(acc, g.in + (int64_t)w.p * g.member_stride_in + r, g.ld_in, w.tb, g.T, half);
  __syncthreads();  // B1
  if (NORM) {  // P's partial sums continued over blocks PB-15, in the one-wave form's order
    float4* psb = reinterpret_cast<float4*>(lds + PS_OFS + (q * 64 + lane) * 64);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float4 v = psb[k];
#pragma unroll
      for (int nb = 0; nb < CB; ++nb) {
        v.x += acc[nb][4 * k] * acc[nb][4 * k];
        v.y += acc[nb][4 * k + 1] * acc[nb][4 * k + 1];
        v.z += acc[nb][4 * k + 2] * acc[nb][4 * k + 2];
        v.w += acc[nb][4 * k + 3] * acc[nb][4 * k + 3];
      }
      psb[k] = v;
    }
  }
  __syncthreads();  // B2
  __syncthreads();  // B3: P's row factors are in
  {
    const float* rrb = reinterpret_cast<const float*>(lds + RR_OFS) + q * 32;
    uint16_t* tile = reinterpret_cast<uint16_t*>(lds + TILE_OFS + q * 32 * TILE_ROW) + r;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int rl = 8 * (j >> 2) + 4 * half + (j & 3);
      const float rrj = NORM ? rrb[rl] : 1.f;
#pragma unroll
      for (int nb = 0; nb < CB; ++nb) tile[rl * (TILE_ROW / 2) + 32 * nb] = f2bf(acc[nb][j] * rrj);
    }
  }
  __syncthreads();  // B4
  if (!RESID) {
#pragma unroll
    for (int nb = 0; nb < CB; ++nb)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[nb][j] = 0.f;
  }

  const uint32_t mpb0 = mp_addr(lds0, 0, r, half), mpb1 = mp_addr(lds0, 1, r, half);
  const uint32_t xa = lds0 + XB_OFS + (q * 64 + lane) * 32;
  PC_STEP_WAIT();  // step 0 (P has read its h pieces)
  c_step<LW, 0, false, true, false>(acc, 0, 0, 0, c_ptrs<LW>(g, 0, w.c0, w.pn, w.pert, lane), lds);
  PC_STEP_WAIT();  // step 1
  c_step<LW, 1, false, true, false>(acc, 0, 0, 0, c_ptrs<LW>(g, 1, w.c0, w.pn, w.pert, lane), lds);
#pragma unroll 1
  for (int s = 2; s < NCH; s += 2) {
    PC_STEP_WAIT();
    c_step<LW, 0, true, true, false>(acc, xa, mpb0, mpb1, c_ptrs<LW>(g, s, w.c0, w.pn, w.pert, lane), lds);
    PC_STEP_WAIT();
    c_step<LW, 1, true, true, false>(acc, xa, mpb0, mpb1, c_ptrs<LW>(g, s + 1, w.c0, w.pn, w.pert, lane), lds);
  }
  PC_STEP_WAIT();  // step 64: loads c_proj chunk 63 (blocks PB-15) for the last step
  c_step<LW, 0, true, true, false>(acc, xa, mpb0, mpb1, c_ptrs<LW>(g, NCH, w.c0, w.pn, w.pert, lane), lds);
  PC_STEP_WAIT();  // step 65
  c_step<LW, 1, true, false, true>(acc, xa, mpb0, mpb1, c_ptrs<LW>(g, NCH + 1, w.c0, w.pn, w.pert, lane), lds);
  __syncthreads();  // B5: P's u_proj factors are in
  const float* supb = reinterpret_cast<const float*>(lds + XB_OFS + 8192) + q * 32;
  float am[CB];
#pragma unroll
  for (int nb = 0; nb < CB; ++nb) am[nb] = w.pert ? g.a_proj[w.pn * g.ld_a_proj + (nb + PB) * 32 + r] : 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int rl = 8 * (j >> 2) + 4 * half + (j & 3);
    const float sr = supb[rl];
    const int rj = w.tb + rl;
    if (rj < g.T) {
      float* dst = g.out + (int64_t)w.p * g.member_stride_out + (int64_t)rj * g.ld_out + r;
#pragma unroll
      for (int nb = 0; nb < CB; ++nb) dst[(nb + PB) * 32] = acc[nb][j] + sr * am[nb];
    }
  }
}

template <bool NORM, bool RESID>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
mlp_pc_kernel(const noise_mlp_t g) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[LDS_BYTES];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Workgroup -> (member p, row block b), and the chunk order's start c0, as in the one-wave form.
  const int bpm = (g.T + ROWS - 1) / ROWS;
  int p, b;
  {
    const int i = blockIdx.x, full = (g.members & ~7) * bpm;
    if (i < full) {
      const int qq = i >> 3;
      b = qq % bpm;
      p = (qq / bpm) * 8 + (i & 7);
    } else {
      const int j = i - full;
      p = (g.members & ~7) + j / bpm;
      b = j % bpm;
    }
  }
  Work w;
  w.p = p;
  w.c0 = (b * (bpm >= NCH ? 1 : NCH / bpm)) & (NCH - 1);
  w.tb = b * ROWS + (wave & 3) * 32;
  w.pert = g.sign != nullptr;
  w.pn = (int64_t)(p >> g.member_shift);
  w.s = w.pert ? g.sign[p] : 0.f;
  // stage 0: c_fc chunk c0, 4 rows per wave
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int row = 4 * wave + k;
    __builtin_amdgcn_global_load_lds((const void*)(g.w_fc + (int64_t)(w.c0 * FC + row) * D + lane * 8),
                                     (void*)(lds + FC_OFS + row * WFC_ROW), 16, 0, 0);
  }
  if (wave < 4) p_wave<NORM, RESID>(g, w, lds, wave, lane);
  else if (wave == 4) c_wave<NORM, RESID, 0>(g, w, lds, lane);
  else if (wave == 5) c_wave<NORM, RESID, 1>(g, w, lds, lane);
  else if (wave == 6) c_wave<NORM, RESID, 2>(g, w, lds, lane);
  else c_wave<NORM, RESID, 3>(g, w, lds, lane);
}

}  // namespace

namespace noise {

// Launches the producer/consumer form for the plain MLP (no attention c_proj, no next norm) and
// returns true, or returns false where it does not apply.
bool mlp_pc_launch(const noise_mlp_t& g, hipStream_t st) {
  if (g.attn_y || g.next || g.flags != (NOISE_MLP_NORM | NOISE_MLP_RESIDUAL)) return false;
  const int64_t blocks = (int64_t)g.members * ((g.T + ROWS - 1) / ROWS);
  mlp_pc_kernel<true, true><<<dim3((unsigned)blocks), 512, 0, st>>>(g);
  return true;
}

}  // namespace noise
