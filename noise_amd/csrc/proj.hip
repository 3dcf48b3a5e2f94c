// Row-resident q|k|v projection of the population forward (K = 512) with its rotary / q,k-norm /
// value-embedding epilogue:
//   out16 = rope_norm_ve(h [Wq; Wk; Wv]^T + sign (h . b) a^T)   (eggroll.py:82-90)
// Reference: `lowrank` (train/val/eggroll.py:56-58), apply_rotary_emb + norm (utils/model.py:55-58),
// the value-embedding gate (eggroll.py:85-89; utils/model.py:87-89).
//
// A workgroup owns 128 rows of one member (four waves, one per SIMD, 32 rows each) and every output
// column. The wave's rows are loaded once, straight into the B-operand registers of
// v_mfma_f32_32x32x16_bf16 (lane l: row l % 32, k = 16 ks + 8 (l / 32) .. + 8 of k-step ks; 128
// VGPRs for K = 512), and the weight streams past them in chunks of 64 output features (one head):
// out^T[64 features, 32 rows] = W[chunk] h^T, the chunk's rows read from LDS as the A operand. The
// accumulator gives lane l the features 8 (j / 4) + 4 (l / 32) + j % 4 (+ 32 in the second block)
// of row l % 32, so the rotary pairs (d, d + 32) of a head sit in one lane and a head's 64 values
// in lanes l and l ^ 32. Chunks alternate between two accumulator sets: the epilogue of chunk c - 1
// (rank-1 term, rotary, norm or value embedding, stores) runs between the MFMAs of chunk c, in
// small pieces. Weight chunks (64 rows x 1 KB, rows padded to 1040 bytes so that fragment reads hit
// 16 distinct bank groups) stream through two LDS stages by direct global -> LDS loads issued
// during the previous chunk's MFMAs; the chunk's bf16 output leaves through a per-wave LDS tile as
// whole 128-byte row segments.
// Per row the kernel reads 1 KB (bf16) and writes 3 KB (bf16); the 1.5 MB bf16 weight is read from
// L2 by every workgroup. Measured on MI355X at the bench shape (1,048,576 rows): 2.2 ms with the
// value embedding and 1.9 ms without, against 2.5 ms for the 256 x 256 tile GEMM with the same
// epilogue. Every wave reads the whole weight chunk from LDS (1 KB per MFMA), which with the MFMAs
// themselves bounds the kernel.
// qkv_rr_kernel (below) is the same product and epilogue at two waves per SIMD, with identical
// output bits; it runs where T and the row count are multiples of 256 (about 7% faster per launch
// at the bench shape: 1.92-1.96 against 2.10 ms without the value embedding, 2.03-2.04 against
// 2.17-2.24 with it).
#include <utility>

#include "mma_tile.h"

namespace {

constexpr int PK = 512;                    // K of every row-resident projection
constexpr int PROWS = 128;                 // rows per workgroup
constexpr int PCH = 64;                    // output features per chunk
constexpr int PW_ROW = 1040;               // LDS bytes per weight row (1 KB + 16 pad)
constexpr int PSTAGE = PCH * PW_ROW;       // 66560
constexpr int PVEC_OFS = 2 * PSTAGE;       // a vectors [N] | b_ve [512] | gate [128 rows][8] (fp32)
constexpr int PGATE_OFS = PVEC_OFS + (1536 + 512) * 4;
// Per-wave output staging of the q|k|v projection: 32 rows x 64 bf16 features, rows padded to 144
// bytes (conflict-free 8-byte writes by row, 16-byte reads along rows).
constexpr int POUT_ROW = 144;
constexpr int POUT_OFS = PGATE_OFS + PROWS * 8 * 4;
constexpr int PLDS = POUT_OFS + 4 * 32 * POUT_ROW;  // 163840
constexpr float PRMS_EPS = 1.1920928955078125e-07f;  // float32 machine epsilon (F.rms_norm default)
#ifndef PROJ_AHEAD
#define PROJ_AHEAD 5  // MFMAs of fragment-read lookahead (measured: 3 -> 5 is 4-6% faster, 7 no better)
#endif
static_assert(PLDS <= 160 * 1024, "LDS budget");

// Epilogue kinds of one chunk: q head, k head (rotary + norm), v head without / with the value
// embedding.
constexpr int EK_NONE = 0, EK_ROTQ = 1, EK_ROTK = 2, EK_V = 3, EK_VE = 4;

struct ProjArgs {
  const uint16_t* A;
  int64_t lda;
  const uint16_t* W;
  int64_t ldw;
  int M, T;
  noise_rank1_t r1;
  noise_rope_t rope;  // out [M, 1536] bf16, rotary tables, value embedding
};

#define PROJ_DSREAD(DST, ADDR, OFS) __asm__ volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(DST) : "v"(ADDR), "n"(OFS))
#define PROJ_LGKM(N) __asm__ volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N))

// Per-lane state that lives for the whole kernel.
struct Lane {
  int64_t row;           // this lane's row
  float su[3];           // sign * (row . b) per rank-1 segment
  floatx4 cs[4], sn[4];  // rotary cos / sin of the row's position for features 8 g + 4 half + q
  float sa;              // with the value embedding: sign * a_ve[token]
  int64_t ve_row;        // element offset of the token's table row (0 for an invalid token)
  bool tok_ok;
};

// Stores each step issues after its last weight load (four whole-row quarters of the chunk): the
// next step waits for everything older than them, the weight chunk and the prefetches included
// (vector memory operations retire in issue order), and lets the stores drain behind it.
constexpr int STEP_STORES = 4;

// One step: the 64 MFMAs of chunk `c` into acc[PAR] (FCP), the next chunk's weight loads (if
// `load_next`), the prefetch of chunk c's value-embedding table rows into pf[PAR] (PFK), and the
// epilogue of chunk c - 1 (kind EK) from acc[1 - PAR] and pf[1 - PAR]. Every kind is a template
// argument, so each step instance is straight-line code.
template <bool FCP, int PAR, int EK, int PFK>
NOISE_DEV void proj_step(const ProjArgs& g, const Lane& ln, const bf16x8 (&hB)[32], floatx16 (&acc)[2][2],
                         floatx4 (&pf)[2][8], unsigned char* lds, uint32_t lds_base, int lane, int wave, int c,
                         bool load_next) {
  constexpr int NA = PROJ_AHEAD + 1;
  const int half = lane >> 5;
  const int cp = c - 1;  // the chunk whose epilogue runs here
  // The previous step's prefetch has landed (this step's opening wait): hand it to the compiler.
  if constexpr (EK == EK_VE)
    __asm__ volatile("" : "+v"(pf[1 - PAR][0]), "+v"(pf[1 - PAR][1]), "+v"(pf[1 - PAR][2]), "+v"(pf[1 - PAR][3]),
                     "+v"(pf[1 - PAR][4]), "+v"(pf[1 - PAR][5]), "+v"(pf[1 - PAR][6]), "+v"(pf[1 - PAR][7]));
  // Epilogue operands from LDS, read before every fragment so that the first fragment wait covers
  // them: the chunk's rank-1 a values, for the value embedding b_ve and the row's gate.
  constexpr int SEG = EK == EK_ROTK ? 1 : (EK == EK_V || EK == EK_VE) ? 2 : 0;
  const float su = ln.su[SEG];
  floatx4 av[8], bv[8];
  float gt = 0.f;
  if constexpr (EK != EK_NONE) {
    const uint32_t ab = lds_base + PVEC_OFS + (uint32_t)(cp * PCH + 4 * half) * 4;
#pragma unroll
    for (int i = 0; i < 8; ++i) PROJ_DSREAD(av[i], ab, (i >> 2) * 128 + (i & 3) * 32);
    if constexpr (EK == EK_VE) {
      const uint32_t bb = lds_base + PVEC_OFS + 1536 * 4 + (uint32_t)(((cp & 7) * PCH + 4 * half) * 4);
#pragma unroll
      for (int i = 0; i < 8; ++i) PROJ_DSREAD(bv[i], bb, (i >> 2) * 128 + (i & 3) * 32);
      const uint32_t ga = lds_base + PGATE_OFS + (uint32_t)(((wave * 32 + (lane & 31)) * 8 + (cp & 7)) * 4);
      __asm__ volatile("ds_read_b32 %0, %1" : "=v"(gt) : "v"(ga));
    }
  }
  // Prefetch of chunk c's table rows: asm loads, so that the compiler neither waits for them nor for
  // anything issued after them; they are complete after the next step's opening wait, and they
  // stay live until the epilogue reads them (a destination register the compiler reused while the
  // load is in flight would be overwritten when it lands).
  if constexpr (FCP && PFK == EK_VE) {
    const float* src = g.rope.ve_table + ln.ve_row + (c & 7) * PCH + 4 * half;
    auto ld = [&pf, src]<int I>() __attribute__((always_inline)) {
      __asm__ volatile("global_load_dwordx4 %0, %1, off offset:%2"
                       : "=v"(pf[PAR][I]) : "v"(src), "n"((I >> 2) * 128 + (I & 3) * 32));
    };
    [&]<int... I>(std::integer_sequence<int, I...>) __attribute__((always_inline)) {
      (ld.template operator()<I>(), ...);
    }(std::make_integer_sequence<int, 8>{});
  }

  const uint32_t fb = lds_base + (uint32_t)(PAR * PSTAGE + (lane & 31) * PW_ROW + 16 * half);
  bf16x8 fr[NA];
  auto read = [&fr, fb]<int S>() __attribute__((always_inline)) {
    PROJ_DSREAD(fr[S % NA], fb, (S & 1) * 32 * PW_ROW + 32 * (S >> 1));
  };
  if constexpr (FCP) {
    [&]<int... S>(std::integer_sequence<int, S...>) __attribute__((always_inline)) {
      (read.template operator()<S>(), ...);
    }(std::make_integer_sequence<int, PROJ_AHEAD>{});
  }
  // Next chunk's weight rows: wave w loads rows 16 w .. 16 w + 15 of the chunk (1 KB each).
  const uint16_t* wsrc = g.W + (int64_t)((c + 1) * PCH + 16 * wave) * g.ldw + 8 * lane;
  unsigned char* wdst = lds + (1 - PAR) * PSTAGE + 16 * wave * PW_ROW;

  // ---- the epilogue of chunk cp, in NPIECE small pieces (one after every second MFMA) ----
  // pieces 0-15: value j = E of both blocks (rank-1 term, then rotary / value embedding / residual);
  // 16: the head's norm factor; 17-24: normalise and pack two values of each block; 25: into the
  // wave's LDS tile; 26-29: four whole-row quarters out.
  constexpr int NPIECE = 30;
  float o1[16], o2[16];
  uint32_t w1[8], w2[8];
  float ss = 0.f, rr = 1.f;
  auto epi = [&]<int E>() __attribute__((always_inline)) {
    if constexpr (EK == EK_NONE) {
    } else if constexpr (E < 16) {
      constexpr int j = E, gg = j >> 2, q = j & 3;
      float x1 = acc[1 - PAR][0][j] + su * av[gg][q];
      float x2 = acc[1 - PAR][1][j] + su * av[4 + gg][q];
      if constexpr (EK == EK_ROTQ || EK == EK_ROTK) {
        const float c_ = ln.cs[gg][q], s_ = ln.sn[gg][q];
        const float r1 = x1 * c_ + x2 * s_;
        const float r2 = x1 * -s_ + x2 * c_;
        ss += r1 * r1 + r2 * r2;
        x1 = r1;
        x2 = r2;
      } else if constexpr (EK == EK_VE) {
        const float e1 = ln.tok_ok ? pf[1 - PAR][gg][q] + ln.sa * bv[gg][q] : __builtin_nanf("");
        const float e2 = ln.tok_ok ? pf[1 - PAR][4 + gg][q] + ln.sa * bv[4 + gg][q] : __builtin_nanf("");
        x1 += gt * e1;
        x2 += gt * e2;
      }
      o1[j] = x1;
      o2[j] = x2;
    } else if constexpr (E == 16) {
      if constexpr (EK == EK_ROTQ || EK == EK_ROTK) {
        // the head's 64 squares: this lane's 32 plus those of lane l ^ 32 (same row)
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(ss), __float_as_uint(ss), false, false);
        rr = rsqrtf((__uint_as_float(r[0]) + __uint_as_float(r[1])) * (1.0f / 64) + PRMS_EPS);
      }
    } else if constexpr (E < 25) {
      constexpr int k = E - 17;  // values 2 k, 2 k + 1 of both blocks
      if constexpr (EK == EK_ROTQ || EK == EK_ROTK) {
        o1[2 * k] *= rr;
        o1[2 * k + 1] *= rr;
        o2[2 * k] *= rr;
        o2[2 * k + 1] *= rr;
      }
      w1[k] = pack_bf2(o1[2 * k], o1[2 * k + 1]);
      w2[k] = pack_bf2(o2[2 * k], o2[2 * k + 1]);
    } else if constexpr (E == 25) {
      // the chunk's bf16 values into the wave's staging tile (row lane % 32, this lane's features)
      unsigned char* st = lds + POUT_OFS + wave * 32 * POUT_ROW + (lane & 31) * POUT_ROW + 8 * half;
#pragma unroll
      for (int gg = 0; gg < 4; ++gg) {
        *reinterpret_cast<u32x2*>(st + 16 * gg) = u32x2{w1[2 * gg], w1[2 * gg + 1]};
        *reinterpret_cast<u32x2*>(st + 64 + 16 * gg) = u32x2{w2[2 * gg], w2[2 * gg + 1]};
      }
    } else if constexpr (E < 30) {
      // one quarter of the tile out as whole rows: lane l copies 16 bytes of row 8 (E - 26) + l / 8
      // (the wave's writes above are complete for its own reads: LDS operations of a wave run in order)
      const int rr_ = 8 * (E - 26) + (lane >> 3);
      const u32x4 v = *reinterpret_cast<const u32x4*>(lds + POUT_OFS + wave * 32 * POUT_ROW + rr_ * POUT_ROW + 16 * (lane & 7));
      __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(g.rope.out + (ln.row - (lane & 31) + rr_) * 1536 + cp * PCH +
                                                              8 * (lane & 7)));
    }
  };
  auto tie_epi_inputs = [&]() __attribute__((always_inline)) {
    __asm__ volatile("" : "+v"(av[0]), "+v"(av[1]), "+v"(av[2]), "+v"(av[3]), "+v"(av[4]), "+v"(av[5]), "+v"(av[6]),
                     "+v"(av[7]));
    if constexpr (EK == EK_VE)
      __asm__ volatile("" : "+v"(bv[0]), "+v"(bv[1]), "+v"(bv[2]), "+v"(bv[3]), "+v"(bv[4]), "+v"(bv[5]), "+v"(bv[6]),
                       "+v"(bv[7]), "+v"(gt));
  };

  if constexpr (!FCP) {  // the last chunk's epilogue on its own
    PROJ_LGKM(0);
    tie_epi_inputs();
    [&]<int... E>(std::integer_sequence<int, E...>) __attribute__((always_inline)) {
      (epi.template operator()<E>(), ...);
    }(std::make_integer_sequence<int, NPIECE>{});
    return;
  }

  auto op = [&]<int S>() __attribute__((always_inline)) {
    // next chunk's loads: one per two MFMAs over the first 32
    if constexpr ((S & 1) == 0 && S < 32) {
      if (load_next)
        __builtin_amdgcn_global_load_lds((const void*)(wsrc + (int64_t)(S >> 1) * g.ldw),
                                         (void*)(wdst + (S >> 1) * PW_ROW), 16, 0, 0);
    }
    if constexpr (S + PROJ_AHEAD < 64) read.template operator()<S + PROJ_AHEAD>();
    PROJ_LGKM(63 - S < PROJ_AHEAD ? 63 - S : PROJ_AHEAD);
    const bf16x8 f = fr[S % NA];
    constexpr int b = S & 1, ks = S >> 1;
    if constexpr (ks == 0)
      __asm__ volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&a"(acc[PAR][b]) : "v"(f), "a"(hB[ks]));
    else if constexpr (S < 63)
      __asm__ volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc[PAR][b]) : "v"(f), "a"(hB[ks]));
    else
      __asm__ volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
                       : "+a"(acc[PAR][b]) : "v"(f), "a"(hB[ks]));
    // epilogue piece E after MFMA 2 E + 1 (the LDS values it reads were waited for with fragment 0)
    if constexpr (EK != EK_NONE && (S & 1) == 1 && (S >> 1) < NPIECE) {
      if constexpr (S == 1) tie_epi_inputs();
      __builtin_amdgcn_sched_barrier(0);
      epi.template operator()<(S >> 1)>();
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  [&]<int... S>(std::integer_sequence<int, S...>) __attribute__((always_inline)) {
    (op.template operator()<S>(), ...);
  }(std::make_integer_sequence<int, 64>{});
}

// Opening of a step: the previous step's weight chunk and prefetches have landed for this wave
// (only its last N vector memory operations, its stores, may still be in flight), then for every
// wave; every wave is done reading the stage the next chunk goes to.
template <int N>
NOISE_DEV void step_wait() {
  __asm__ volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

template <bool HAS_VE>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
qkv_proj_kernel(const ProjArgs g) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[PLDS];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int64_t r0 = (int64_t)blockIdx.x * PROWS;
  const int p = (int)(r0 / g.T);  // every row of the workgroup belongs to member p (T % 128 == 0)
  const bool pert = g.r1.sign != nullptr;
  const int64_t pn = (int64_t)(p >> g.r1.member_shift);
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)lds;

  // Chunk 0's weight rows start streaming into stage 0.
  {
    const uint16_t* wsrc = g.W + (int64_t)(16 * wave) * g.ldw + 8 * lane;
#pragma unroll
    for (int k = 0; k < 16; ++k)
      __builtin_amdgcn_global_load_lds((const void*)(wsrc + (int64_t)k * g.ldw), (void*)(lds + (16 * wave + k) * PW_ROW),
                                       16, 0, 0);
  }
  // ---- prologue: every independent load first, then one wait ----
  Lane ln;
  ln.row = r0 + 32 * wave + (lane & 31);
  // The wave's 32 rows as B operands: lane l holds row l % 32, k = 16 ks + 8 (l / 32) .. + 8. They
  // are loaded straight into AGPRs (which MFMAs read as operands) and stay there: in VGPRs they
  // crowded the epilogue, and the compiler's copies of them back into VGPRs right before an
  // inline-asm MFMA are writes it does not guard with the wait states the MFMA needs.
  bf16x8 hB[32];
  {
    const uint16_t* arow = g.A + ln.row * g.lda + 8 * half;
#pragma unroll
    for (int ks = 0; ks < 32; ++ks)
      __asm__ volatile("global_load_dwordx4 %0, %1, off offset:%2" : "=a"(hB[ks]) : "v"(arow), "n"(32 * ks));
  }
  // The member's rank-1 a vectors (zeros when unperturbed): 1536 floats, 6 per thread.
  float av_ld[6];
  [&]<int... K>(std::integer_sequence<int, K...>) __attribute__((always_inline)) {
    auto one = [&]<int k>() __attribute__((always_inline)) {
      const int i = tid + 256 * k;
      av_ld[k] = 0.f;
      if (pert) {
        // segment of element i: 512 columns each for q | k | v (slots 2 s, 2 s + 1)
        constexpr int sg = k >> 1;
        av_ld[k] = g.r1.a[sg][pn * g.r1.lda + (i - sg * 512)];
      }
    };
    (one.template operator()<K>(), ...);
  }(std::make_integer_sequence<int, 6>{});
  // sign * (row . b) per segment: u of a row is the sum of u_parts consecutive floats.
  float us[3][8];
#pragma unroll
  for (int sg = 0; sg < 3; ++sg)
#pragma unroll
    for (int j = 0; j < 8; ++j) us[sg][j] = 0.f;
  if (pert) {
#pragma unroll
    for (int sg = 0; sg < 3; ++sg) {
      if (sg < g.r1.nseg) {
        const float* up = g.r1.u[sg] + ln.row * g.r1.ldu;
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (j < g.r1.u_parts) us[sg][j] = up[j];
      }
    }
  }
  float bve_ld[2] = {0.f, 0.f};
  floatx4 gate_ld = {0.f, 0.f, 0.f, 0.f};
  int64_t tok = 0;
  {
    const noise_rope_t& rp = g.rope;
    const int t = (int)(ln.row - (int64_t)p * g.T);
#pragma unroll
    for (int gg = 0; gg < 4; ++gg) {
      ln.cs[gg] = *reinterpret_cast<const floatx4*>(rp.cos + t * 32 + 8 * gg + 4 * half);
      ln.sn[gg] = *reinterpret_cast<const floatx4*>(rp.sin + t * 32 + 8 * gg + 4 * half);
    }
    if constexpr (HAS_VE) {
      const int64_t pv = (int64_t)(p >> rp.member_shift);
      if (rp.sign) {
        bve_ld[0] = rp.ve_b[pv * rp.ld_ve_b + tid];
        bve_ld[1] = rp.ve_b[pv * rp.ld_ve_b + tid + 256];
      }
      gate_ld = *reinterpret_cast<const floatx4*>(rp.gate + r0 * 8 + 4 * tid);
      tok = rp.idx[(int64_t)p * rp.idx_stride + t];
    }
  }
  // (the second round trip: the token's a_ve value)
  ln.sa = 0.f;
  ln.ve_row = 0;
  ln.tok_ok = true;
  if constexpr (HAS_VE) {
    const noise_rope_t& rp = g.rope;
    ln.tok_ok = tok >= 0 && tok < rp.vocab;
    ln.ve_row = ln.tok_ok ? tok * 512 : 0;
    const int64_t pv = (int64_t)(p >> rp.member_shift);
    ln.sa = (ln.tok_ok && rp.sign) ? rp.sign[p] * rp.ve_a[pv * rp.ld_ve_a + tok] : 0.f;
  }
  const float s = pert ? g.r1.sign[p] : 0.f;
#pragma unroll
  for (int sg = 0; sg < 3; ++sg) {
    float u = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) u += us[sg][j];
    ln.su[sg] = s * u;
  }
  float* s_a = reinterpret_cast<float*>(lds + PVEC_OFS);
#pragma unroll
  for (int k = 0; k < 6; ++k) s_a[tid + 256 * k] = av_ld[k];
  if constexpr (HAS_VE) {
    float* s_b = s_a + 1536;
    s_b[tid] = bve_ld[0];
    s_b[tid + 256] = bve_ld[1];
    *reinterpret_cast<floatx4*>(lds + PGATE_OFS + 16 * tid) = gate_ld;
  }

  floatx16 acc[2][2];
  floatx4 pf[2][8];
  // The per-lane values are computed here, not where the steps first use them (the compiler would
  // wait there for their loads, and with them for the weight loads issued by then).
  __asm__ volatile("" ::"v"(ln.su[0]), "v"(ln.su[1]), "v"(ln.su[2]), "v"(ln.sa), "v"(ln.ve_row));
  __asm__ volatile("" ::"v"(ln.cs[0]), "v"(ln.cs[1]), "v"(ln.cs[2]), "v"(ln.cs[3]), "v"(ln.sn[0]), "v"(ln.sn[1]),
                   "v"(ln.sn[2]), "v"(ln.sn[3]));
  // Every load so far (weight chunk 0, the rows, the per-row data) has landed.
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  step_wait<0>();
#define PROJ_S(FCP_, PAR_, EK_, PFK_, C_, NEXT_) \
  proj_step<FCP_, PAR_, EK_, PFK_>(g, ln, hB, acc, pf, lds, lds_base, lane, wave, C_, NEXT_)
  {
    // chunks 0-7: q heads, 8-15: k heads, 16-23: v heads; step c runs chunk c and the epilogue of c - 1
    constexpr int VK = HAS_VE ? EK_VE : EK_V, VPF = HAS_VE ? EK_VE : EK_NONE;
    PROJ_S(true, 0, EK_NONE, EK_NONE, 0, true);
    step_wait<0>();
    PROJ_S(true, 1, EK_ROTQ, EK_NONE, 1, true);
    for (int c = 2; c < 8; c += 2) {
      step_wait<STEP_STORES>();
      PROJ_S(true, 0, EK_ROTQ, EK_NONE, c, true);
      step_wait<STEP_STORES>();
      PROJ_S(true, 1, EK_ROTQ, EK_NONE, c + 1, true);
    }
    step_wait<STEP_STORES>();
    PROJ_S(true, 0, EK_ROTQ, EK_NONE, 8, true);
    for (int c = 9; c < 15; c += 2) {
      step_wait<STEP_STORES>();
      PROJ_S(true, 1, EK_ROTK, EK_NONE, c, true);
      step_wait<STEP_STORES>();
      PROJ_S(true, 0, EK_ROTK, EK_NONE, c + 1, true);
    }
    step_wait<STEP_STORES>();
    PROJ_S(true, 1, EK_ROTK, EK_NONE, 15, true);
    step_wait<STEP_STORES>();
    PROJ_S(true, 0, EK_ROTK, VPF, 16, true);
    for (int c = 17; c < 23; c += 2) {
      step_wait<STEP_STORES>();
      PROJ_S(true, 1, VK, VPF, c, true);
      step_wait<STEP_STORES>();
      PROJ_S(true, 0, VK, VPF, c + 1, true);
    }
    step_wait<STEP_STORES>();
    PROJ_S(true, 1, VK, VPF, 23, false);
    step_wait<STEP_STORES>();
    PROJ_S(false, 0, VK, EK_NONE, 24, false);
  }
#undef PROJ_S
}

// ---- the same product at two waves per SIMD: 32-feature chunks ----
// A workgroup owns 256 rows of one member (eight waves, two per SIMD, 32 rows each, the rows in 128
// AGPRs as above). The weight streams in 48 chunks of 32 features: chunk c holds features
// 16 (c & 1) + (r & 15) + 32 (r >> 4) (r = 0..31) of head c / 2, so the accumulator gives lane l the
// rotary pairs (d, d + 32) of row l % 32 for d = 16 (c & 1) + 8 j + 4 (l / 32) + i (j = 0, 1), as
// values 4 j + i and 4 j + i + 8. A head's two chunks follow each other: the first one's rotated
// values wait in a per-wave LDS hold (fp32) until the second one's squares complete the head's
// norm; then both leave through the staging tile as whole 128-byte row segments. Each output
// value sees the same MFMAs in the same order and the same epilogue operations as in
// qkv_proj_kernel, and the norm's sum of squares runs in the same order, so the two kernels give
// identical bits. Chunks alternate between two accumulator sets; the epilogue of chunk c - 1 runs
// in small pieces between the MFMAs of chunk c and, with a second wave on the SIMD, under the
// other wave's MFMAs.
constexpr int QR_ROWS = 256, QR_THREADS = 512, QR_CH = 32;  // 48 chunks: 1536 / QR_CH
constexpr int QR_STAGE = QR_CH * PW_ROW;                    // 33280
constexpr int QR_A_OFS = 2 * QR_STAGE;                      // a [1536] fp32
constexpr int QR_BVE_OFS = QR_A_OFS + 1536 * 4;             // b_ve [512] fp32
constexpr int QR_GATE_OFS = QR_BVE_OFS + 512 * 4;           // gate [256 rows][8] fp32
constexpr int QR_HOLD_OFS = QR_GATE_OFS + QR_ROWS * 8 * 4;  // per wave: 16 floats per lane
constexpr int QR_OUT_OFS = QR_HOLD_OFS + 8 * 4096;          // per wave: 32 rows x POUT_ROW
constexpr int QR_LDS = QR_OUT_OFS + 8 * 32 * POUT_ROW;      // 152576
#ifndef QR_AHEAD_N
#define QR_AHEAD_N 3
#endif
constexpr int QR_AHEAD = QR_AHEAD_N;  // MFMAs of fragment-read lookahead
constexpr int QR_LS = 4;                                    // MFMAs between two weight-row loads
constexpr int QR_PF_AFTER = 10;  // MFMA after which the value-embedding prefetch issues (past the
                                 // epilogue's reads of the previous values, before the stores)
static_assert(QR_LDS <= 160 * 1024, "LDS budget");
static_assert(3 * QR_LS < 26 && QR_PF_AFTER > 9 && QR_PF_AFTER < 26, "the loads precede the stores");
static_assert(QR_AHEAD <= 3, "an LDS read issued after MFMA S is used after MFMA S + 3");

struct QRLane {
  int64_t row;
  float su[3];     // sign * (row . b) per rank-1 segment
  uint32_t cs[16]; // rotary cos (high half) and sin (low half) as bf16 of the row's position for
                   // pair 8 (k / 4) + 4 half + k % 4 (the tables hold bf16 values)
  float sa;              // with the value embedding: sign * a_ve[token]; NaN for an invalid token,
                         // which makes every value-embedding term of the row NaN
  int64_t ve_row;        // element offset of the token's table row (0 for an invalid token)
};

// Weight row of chunk-row r of chunk c (see above).
NOISE_DEV int qr_wrow(int c, int r) { return 64 * (c >> 1) + 16 * (c & 1) + (r & 15) + 32 * (r >> 4); }

// One step: the 32 MFMAs of chunk c into acc[PAR] (FCP), the next chunk's weight rows (load_next),
// the epilogue of chunk c - 1 (kind EK; its parity is 1 - PAR) from acc[1 - PAR] and pf, and then
// the prefetch of chunk c's value-embedding table values into pf (VEPF).
template <bool FCP, int PAR, int EK, bool VEPF>
NOISE_DEV void qr_step(const ProjArgs& g, const QRLane& ln, const bf16x8 (&hB)[32], floatx16 (&acc)[2],
                       floatx4 (&pf)[4], float& ss0, unsigned char* lds, uint32_t lds_base, int lane, int wave,
                       int c, bool load_next) {
  // the value-embedding epilogue holds 16 more values; its steps read one fragment less ahead
  constexpr int AH = EK == EK_VE ? QR_AHEAD - 1 : QR_AHEAD;
  constexpr int NA = AH + 1, NM = 32;
  constexpr int SP = 1 - PAR;  // parity of chunk cp: 0 = a head's first chunk, 1 = its second
  constexpr bool ROT = EK == EK_ROTQ || EK == EK_ROTK;
  const int half = lane >> 5;
  const int cp = c - 1, hd = cp >> 1;
  if constexpr (EK == EK_VE) __asm__ volatile("" : "+v"(pf[0]), "+v"(pf[1]), "+v"(pf[2]), "+v"(pf[3]));
  // Epilogue operands from LDS, read before every fragment so that the first fragment wait covers
  // them: group j of the chunk's values is features 16 SP + 8 (j & 1) + 4 half + 32 (j >> 1) + 0..3.
  constexpr int SEG = EK == EK_ROTK ? 1 : (EK == EK_V || EK == EK_VE) ? 2 : 0;
  const float su = ln.su[SEG];
  floatx4 av[4], bv[4];
  float gt = 0.f;
  // The v kinds use groups 2 and 3 only from piece 4 on: they are read after MFMA 2 (SPLIT_READ),
  // so that fewer values are live at once.
  constexpr bool SPLIT_READ = !ROT && EK != EK_NONE;
  const uint32_t ab = lds_base + QR_A_OFS + (uint32_t)(64 * hd + 16 * SP + 4 * half) * 4;
  const uint32_t bb = lds_base + QR_BVE_OFS + (uint32_t)(64 * (hd & 7) + 16 * SP + 4 * half) * 4;
  auto read_groups = [&av, &bv, ab, bb]<int J0, int J1>() __attribute__((always_inline)) {
#pragma unroll
    for (int j = J0; j < J1; ++j) PROJ_DSREAD(av[j], ab, 32 * (j & 1) + 128 * (j >> 1));
    if constexpr (EK == EK_VE) {
#pragma unroll
      for (int j = J0; j < J1; ++j) PROJ_DSREAD(bv[j], bb, 32 * (j & 1) + 128 * (j >> 1));
    }
  };
  if constexpr (EK != EK_NONE) {
    if constexpr (SPLIT_READ) read_groups.template operator()<0, 2>();
    else read_groups.template operator()<0, 4>();
    if constexpr (EK == EK_VE) {
      const uint32_t ga = lds_base + QR_GATE_OFS + (uint32_t)(((wave * 32 + (lane & 31)) * 8 + (hd & 7)) * 4);
      __asm__ volatile("ds_read_b32 %0, %1" : "=v"(gt) : "v"(ga));
    }
  }
  // Prefetch of chunk c's table values into pf, once the epilogue has read the previous ones (asm
  // loads: complete after the next step's opening wait; issued before the step's stores).
  auto prefetch = [&]() __attribute__((always_inline)) {
    const float* src = g.rope.ve_table + ln.ve_row + 64 * ((c >> 1) & 7) + 16 * (c & 1) + 4 * half;
    auto ld = [&pf, src]<int J>() __attribute__((always_inline)) {
      __asm__ volatile("global_load_dwordx4 %0, %1, off offset:%2"
                       : "=v"(pf[J]) : "v"(src), "n"(32 * (J & 1) + 128 * (J >> 1)));
    };
    [&]<int... J>(std::integer_sequence<int, J...>) __attribute__((always_inline)) {
      (ld.template operator()<J>(), ...);
    }(std::make_integer_sequence<int, 4>{});
  };

  const uint32_t fb = lds_base + (uint32_t)(PAR * QR_STAGE + (lane & 31) * PW_ROW + 16 * half);
  bf16x8 fr[NA];
  auto read = [&fr, fb]<int S>() __attribute__((always_inline)) {
    PROJ_DSREAD(fr[S % NA], fb, 32 * S);
  };
  if constexpr (FCP) {
    [&]<int... S>(std::integer_sequence<int, S...>) __attribute__((always_inline)) {
      (read.template operator()<S>(), ...);
    }(std::make_integer_sequence<int, AH>{});
  }
  // next chunk: wave w loads its chunk-rows 4 w .. 4 w + 3 (1 KB each)
  unsigned char* wdst = lds + (1 - PAR) * QR_STAGE + 4 * wave * PW_ROW;

  // ---- the epilogue of chunk cp ----
  // rotary kinds: pieces 0-7 pair j (rank-1 term, rotation, squares); SP 0: 8 into the hold;
  // SP 1: 8 the head's norm factor and the hold's reads, 9-10 this chunk normalised into the tile,
  // 11-12 the held chunk likewise, two groups each. v kinds: pieces 0-7 values 2 k, 2 k + 1, 8 into
  // the tile. SP 1 then reads four whole-row quarters of the tile (pieces NBODY .. + 3) and stores
  // them (NBODY + 4 .. + 7). The hold's and the quarters' LDS reads are asm, issued three MFMAs
  // before their use: the fragment waits in between cover them, so no wait drains the fragment
  // reads in flight.
  constexpr int NBODY = EK == EK_NONE ? 0 : ROT ? (SP == 0 ? 9 : 13) : 9;
  constexpr int NPIECE = SP == 1 && EK != EK_NONE ? NBODY + 8 : NBODY;
  floatx16& ea = acc[1 - PAR];
  floatx4 hv[4];  // the held chunk (SP 1 rotary kinds)
  u32x4 qd[4];    // the quarters
  const uint32_t hold_a = lds_base + QR_HOLD_OFS + wave * 4096 + 16 * lane;
  const uint32_t quarter_a = lds_base + QR_OUT_OFS + wave * 32 * POUT_ROW + (lane >> 3) * POUT_ROW + 16 * (lane & 7);
  float ss = SP == 0 ? 0.f : ss0, rr = 1.f;
  uint32_t w[8];
  unsigned char* tile = lds + QR_OUT_OFS + wave * 32 * POUT_ROW + (lane & 31) * POUT_ROW + 8 * half;
  auto to_tile = [&](int s) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<u32x2*>(tile + 32 * s + 16 * (j & 1) + 64 * (j >> 1)) = u32x2{w[2 * j], w[2 * j + 1]};
  };
  auto hold_reads = [&hv, hold_a]() __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __asm__ volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(hv[j]) : "v"(hold_a), "n"(1024 * j) : "memory");
  };
  auto epi = [&]<int E>() __attribute__((always_inline)) {
    if constexpr (ROT && E < 8) {
      constexpr int j = E >> 2, q = E & 3;
      const float x1 = ea[E] + su * av[j][q];
      const float x2 = ea[E + 8] + su * av[2 + j][q];
      const uint32_t cw = ln.cs[4 * (2 * SP + j) + q];
      const float c_ = bf_hi(cw), s_ = bf_lo(cw);
      const float r1 = x1 * c_ + x2 * s_;
      const float r2 = x1 * -s_ + x2 * c_;
      ss += r1 * r1 + r2 * r2;
      ea[E] = r1;
      ea[E + 8] = r2;
    } else if constexpr (ROT && SP == 0 && E == 8) {
      ss0 = ss;
      float* hold = reinterpret_cast<float*>(lds + QR_HOLD_OFS + wave * 4096) + 4 * lane;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        *reinterpret_cast<floatx4*>(hold + 256 * j) = floatx4{ea[4 * j], ea[4 * j + 1], ea[4 * j + 2], ea[4 * j + 3]};
    } else if constexpr (ROT && E == 8) {
      // the head's 64 squares: both chunks of this lane plus those of lane l ^ 32 (same row)
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(ss), __float_as_uint(ss), false, false);
      rr = rsqrtf((__uint_as_float(r[0]) + __uint_as_float(r[1])) * (1.0f / 64) + PRMS_EPS);
      hold_reads();
    } else if constexpr (ROT && E == 9) {
#pragma unroll
      for (int k = 0; k < 8; ++k) w[k] = pack_bf2(ea[2 * k] * rr, ea[2 * k + 1] * rr);
    } else if constexpr (ROT && E == 10) {
      to_tile(1);
    } else if constexpr (ROT && (E == 11 || E == 12)) {
      // groups 2 (E - 11) and 2 (E - 11) + 1 of the held chunk
      constexpr int j0 = 2 * (E - 11);
      __asm__ volatile("" : "+v"(hv[j0]), "+v"(hv[j0 + 1]));
#pragma unroll
      for (int j = j0; j < j0 + 2; ++j) {
        const floatx4 h = hv[j];
        const u32x2 pw{pack_bf2(h[0] * rr, h[1] * rr), pack_bf2(h[2] * rr, h[3] * rr)};
        *reinterpret_cast<u32x2*>(tile + 16 * (j & 1) + 64 * (j >> 1)) = pw;
      }
    } else if constexpr (!ROT && E < 8) {
#pragma unroll
      for (int v = 2 * E; v < 2 * E + 2; ++v) {
        const int j = v >> 2, q = v & 3;
        float x = ea[v] + su * av[j][q];
        if constexpr (EK == EK_VE) {
          const float e = pf[j][q] + ln.sa * bv[j][q];
          x += gt * e;
        }
        ea[v] = x;
      }
    } else if constexpr (!ROT && E == 8) {
#pragma unroll
      for (int k = 0; k < 8; ++k) w[k] = pack_bf2(ea[2 * k], ea[2 * k + 1]);
      to_tile(SP);
    } else if constexpr (SP == 1 && E >= NBODY && E < NBODY + 4) {
      // quarter q of the tile: lane l reads 16 bytes of row 8 q + l / 8 (the wave's tile writes are
      // complete for its own reads: LDS operations of a wave run in order)
      constexpr int q = E - NBODY;
      __asm__ volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(qd[q]) : "v"(quarter_a), "n"(8 * q * POUT_ROW) : "memory");
    } else if constexpr (SP == 1 && E >= NBODY + 4 && E < NBODY + 8) {
      // ... and out as whole rows
      constexpr int q = E - NBODY - 4;
      __asm__ volatile("" : "+v"(qd[q]));
      const int r_ = 8 * q + (lane >> 3);
      __builtin_nontemporal_store(qd[q], reinterpret_cast<u32x4*>(g.rope.out + (ln.row - (lane & 31) + r_) * 1536 +
                                                                  hd * 64 + 8 * (lane & 7)));
    }
  };
  auto tie_epi_inputs = [&]() __attribute__((always_inline)) {
    if constexpr (SPLIT_READ) {
      __asm__ volatile("" : "+v"(av[0]), "+v"(av[1]));
      if constexpr (EK == EK_VE) __asm__ volatile("" : "+v"(bv[0]), "+v"(bv[1]), "+v"(gt));
    } else {
      __asm__ volatile("" : "+v"(av[0]), "+v"(av[1]), "+v"(av[2]), "+v"(av[3]));
    }
  };

  if constexpr (!FCP) {  // the last chunk's epilogue on its own
    if constexpr (SPLIT_READ) read_groups.template operator()<2, 4>();
    PROJ_LGKM(0);
    tie_epi_inputs();
    if constexpr (SPLIT_READ) {
      __asm__ volatile("" : "+v"(av[2]), "+v"(av[3]));
      if constexpr (EK == EK_VE) __asm__ volatile("" : "+v"(bv[2]), "+v"(bv[3]));
    }
    // (no fragment waits here: every piece waits for all LDS reads before it)
    auto one = [&]<int E>() __attribute__((always_inline)) {
      PROJ_LGKM(0);
      epi.template operator()<E>();
    };
    [&]<int... E>(std::integer_sequence<int, E...>) __attribute__((always_inline)) {
      (one.template operator()<E>(), ...);
    }(std::make_integer_sequence<int, NPIECE>{});
    return;
  }

  // MFMA after which piece E runs. Rotary kinds: the pairs after every second MFMA, the norm
  // factor (with the hold's reads) after MFMA 16 and the held chunk from MFMA 20 on (three MFMAs
  // later). v kinds: one piece after every MFMA from the first, so that the value-embedding values
  // are free for the next prefetch early. The tile reads after 22-25, the stores after 26-29.
  auto slot = [](int E) constexpr {
    if (!ROT) return E < 9 ? E + 1 : E < 13 ? 22 + (E - 9) : 26 + (E - 13);
    if (E < 8) return 2 * E + 1;
    if (SP == 0) return 17;
    constexpr int tail[5] = {16, 17, 18, 20, 21};
    return E < 13 ? tail[E - 8] : E < 17 ? 22 + (E - 13) : 26 + (E - 17);
  };
  auto run_at = [&]<int E, int S>() __attribute__((always_inline)) {
    if constexpr (slot(E) == S) {
      __builtin_amdgcn_sched_barrier(0);
      epi.template operator()<E>();
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto op = [&]<int S>() __attribute__((always_inline)) {
    if constexpr (S % QR_LS == 0 && S / QR_LS < 4) {
      if (load_next) {
        constexpr int k = S / QR_LS;
        const int r = 4 * wave + k;
        __builtin_amdgcn_global_load_lds((const void*)(g.W + (int64_t)qr_wrow(c + 1, r) * g.ldw + 8 * lane),
                                         (void*)(wdst + k * PW_ROW), 16, 0, 0);
      }
    }
    if constexpr (S + AH < NM) read.template operator()<S + AH>();
    PROJ_LGKM(NM - 1 - S < AH ? NM - 1 - S : AH);
    const bf16x8 f = fr[S % NA];
    if constexpr (S == 0)
      __asm__ volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(acc[PAR]) : "v"(f), "a"(hB[S]));
    else if constexpr (S < NM - 1)
      __asm__ volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(acc[PAR]) : "v"(f), "a"(hB[S]));
    else
      __asm__ volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
                       : "+v"(acc[PAR]) : "v"(f), "a"(hB[S]));
    // epilogue piece E after MFMA slot(E) (the LDS values it reads were waited for with fragment
    // 0); quarter q read after MFMA 22 + q and stored after MFMA 26 + q, behind the step's last
    // weight load, so that the next step's opening wait can leave exactly the stores in flight
    if constexpr (SPLIT_READ && S == 2) read_groups.template operator()<2, 4>();
    if constexpr (SPLIT_READ && S == 5) {
      __asm__ volatile("" : "+v"(av[2]), "+v"(av[3]));
      if constexpr (EK == EK_VE) __asm__ volatile("" : "+v"(bv[2]), "+v"(bv[3]));
    }
    if constexpr (VEPF && S == QR_PF_AFTER) {
      __builtin_amdgcn_sched_barrier(0);
      prefetch();
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (EK != EK_NONE) {
      if constexpr (S == 1) tie_epi_inputs();
      [&]<int... E>(std::integer_sequence<int, E...>) __attribute__((always_inline)) {
        (run_at.template operator()<E, S>(), ...);
      }(std::make_integer_sequence<int, NPIECE>{});
    }
  };
  [&]<int... S>(std::integer_sequence<int, S...>) __attribute__((always_inline)) {
    (op.template operator()<S>(), ...);
  }(std::make_integer_sequence<int, NM>{});
}

template <bool HAS_VE>
__global__ void __launch_bounds__(QR_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
qkv_rr_kernel(const ProjArgs g) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[QR_LDS];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int64_t r0 = (int64_t)blockIdx.x * QR_ROWS;
  const int p = (int)(r0 / g.T);  // every row of the workgroup belongs to member p (T % 256 == 0)
  const bool pert = g.r1.sign != nullptr;
  const int64_t pn = (int64_t)(p >> g.r1.member_shift);
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)lds;

  // chunk 0's weight rows into stage 0
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int r = 4 * wave + k;
    __builtin_amdgcn_global_load_lds((const void*)(g.W + (int64_t)qr_wrow(0, r) * g.ldw + 8 * lane),
                                     (void*)(lds + r * PW_ROW), 16, 0, 0);
  }
  QRLane ln;
  ln.row = r0 + 32 * wave + (lane & 31);
  // the wave's 32 rows as B operands, straight into AGPRs
  bf16x8 hB[32];
  {
    const uint16_t* arow = g.A + ln.row * g.lda + 8 * half;
#pragma unroll
    for (int ks = 0; ks < 32; ++ks)
      __asm__ volatile("global_load_dwordx4 %0, %1, off offset:%2" : "=a"(hB[ks]) : "v"(arow), "n"(32 * ks));
  }
  // the member's rank-1 a vectors (zeros when unperturbed): 1536 floats, 3 per thread
  float av_ld[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const int i = tid + 512 * k;  // segment k
    av_ld[k] = pert ? g.r1.a[k][pn * g.r1.lda + (i - 512 * k)] : 0.f;
  }
  float us[3][8];
#pragma unroll
  for (int sg = 0; sg < 3; ++sg)
#pragma unroll
    for (int j = 0; j < 8; ++j) us[sg][j] = 0.f;
  if (pert) {
#pragma unroll
    for (int sg = 0; sg < 3; ++sg) {
      if (sg < g.r1.nseg) {
        const float* up = g.r1.u[sg] + ln.row * g.r1.ldu;
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (j < g.r1.u_parts) us[sg][j] = up[j];
      }
    }
  }
  float bve_ld = 0.f;
  floatx4 gate_ld = {0.f, 0.f, 0.f, 0.f};
  int64_t tok = 0;
  {
    const noise_rope_t& rp = g.rope;
    const int t = (int)(ln.row - (int64_t)p * g.T);
#pragma unroll
    for (int gg = 0; gg < 4; ++gg) {
      const floatx4 cv = *reinterpret_cast<const floatx4*>(rp.cos + t * 32 + 8 * gg + 4 * half);
      const floatx4 sv = *reinterpret_cast<const floatx4*>(rp.sin + t * 32 + 8 * gg + 4 * half);
#pragma unroll
      for (int q = 0; q < 4; ++q) ln.cs[4 * gg + q] = pack_bf2(sv[q], cv[q]);
    }
    if constexpr (HAS_VE) {
      const int64_t pv = (int64_t)(p >> rp.member_shift);
      if (rp.sign) bve_ld = rp.ve_b[pv * rp.ld_ve_b + tid];
      gate_ld = *reinterpret_cast<const floatx4*>(rp.gate + r0 * 8 + 4 * tid);
      tok = rp.idx[(int64_t)p * rp.idx_stride + t];
    }
  }
  ln.sa = 0.f;
  ln.ve_row = 0;
  if constexpr (HAS_VE) {
    const noise_rope_t& rp = g.rope;
    const bool tok_ok = tok >= 0 && tok < rp.vocab;
    ln.ve_row = tok_ok ? tok * 512 : 0;
    const int64_t pv = (int64_t)(p >> rp.member_shift);
    ln.sa = !tok_ok ? __builtin_nanf("") : rp.sign ? rp.sign[p] * rp.ve_a[pv * rp.ld_ve_a + tok] : 0.f;
  }
  const float s = pert ? g.r1.sign[p] : 0.f;
#pragma unroll
  for (int sg = 0; sg < 3; ++sg) {
    float u = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) u += us[sg][j];
    ln.su[sg] = s * u;
  }
  float* s_a = reinterpret_cast<float*>(lds + QR_A_OFS);
#pragma unroll
  for (int k = 0; k < 3; ++k) s_a[tid + 512 * k] = av_ld[k];
  if constexpr (HAS_VE) {
    reinterpret_cast<float*>(lds + QR_BVE_OFS)[tid] = bve_ld;
    *reinterpret_cast<floatx4*>(lds + QR_GATE_OFS + 16 * tid) = gate_ld;
  }

  floatx16 acc[2];
  floatx4 pf[4];
  float ss0 = 0.f;
  __asm__ volatile("" ::"v"(ln.su[0]), "v"(ln.su[1]), "v"(ln.su[2]), "v"(ln.sa), "v"(ln.ve_row));
  __asm__ volatile("" ::"v"(ln.cs[0]), "v"(ln.cs[1]), "v"(ln.cs[2]), "v"(ln.cs[3]), "v"(ln.cs[4]), "v"(ln.cs[5]),
                   "v"(ln.cs[6]), "v"(ln.cs[7]), "v"(ln.cs[8]), "v"(ln.cs[9]), "v"(ln.cs[10]), "v"(ln.cs[11]),
                   "v"(ln.cs[12]), "v"(ln.cs[13]), "v"(ln.cs[14]), "v"(ln.cs[15]));
  // every load so far (weight chunk 0, the rows, the per-row data) has landed
  __asm__ volatile("s_waitcnt vmcnt(0)"
                   : "+a"(hB[0]), "+a"(hB[1]), "+a"(hB[2]), "+a"(hB[3]), "+a"(hB[4]), "+a"(hB[5]), "+a"(hB[6]),
                     "+a"(hB[7]), "+a"(hB[8]), "+a"(hB[9]), "+a"(hB[10]), "+a"(hB[11]), "+a"(hB[12]), "+a"(hB[13]),
                     "+a"(hB[14]), "+a"(hB[15]));
  __asm__ volatile("s_waitcnt vmcnt(0)"
                   : "+a"(hB[16]), "+a"(hB[17]), "+a"(hB[18]), "+a"(hB[19]), "+a"(hB[20]), "+a"(hB[21]),
                     "+a"(hB[22]), "+a"(hB[23]), "+a"(hB[24]), "+a"(hB[25]), "+a"(hB[26]), "+a"(hB[27]),
                     "+a"(hB[28]), "+a"(hB[29]), "+a"(hB[30]), "+a"(hB[31]));
  step_wait<0>();
#define QR_S(FCP_, PAR_, EK_, PF_, C_, NEXT_) \
  qr_step<FCP_, PAR_, EK_, PF_>(g, ln, hB, acc, pf, ss0, lds, lds_base, lane, wave, C_, NEXT_)
  {
    // chunks 0-15: q heads, 16-31: k heads, 32-47: v heads; step c runs chunk c and the epilogue of
    // c - 1. A step whose epilogue closes a head (c even) ends with four stores, which the next
    // step's opening wait leaves in flight.
    constexpr int VK = HAS_VE ? EK_VE : EK_V;
    QR_S(true, 0, EK_NONE, false, 0, true);
    step_wait<0>();
    QR_S(true, 1, EK_ROTQ, false, 1, true);
    for (int c = 2; c < 16; c += 2) {
      step_wait<0>();
      QR_S(true, 0, EK_ROTQ, false, c, true);
      step_wait<STEP_STORES>();
      QR_S(true, 1, EK_ROTQ, false, c + 1, true);
    }
    step_wait<0>();
    QR_S(true, 0, EK_ROTQ, false, 16, true);
    for (int c = 17; c < 31; c += 2) {
      step_wait<STEP_STORES>();
      QR_S(true, 1, EK_ROTK, false, c, true);
      step_wait<0>();
      QR_S(true, 0, EK_ROTK, false, c + 1, true);
    }
    step_wait<STEP_STORES>();
    QR_S(true, 1, EK_ROTK, false, 31, true);
    step_wait<0>();
    QR_S(true, 0, EK_ROTK, HAS_VE, 32, true);
    for (int c = 33; c < 47; c += 2) {
      step_wait<STEP_STORES>();
      QR_S(true, 1, VK, HAS_VE, c, true);
      step_wait<0>();
      QR_S(true, 0, VK, HAS_VE, c + 1, true);
    }
    step_wait<STEP_STORES>();
    QR_S(true, 1, VK, HAS_VE, 47, false);
    step_wait<0>();
    QR_S(false, 0, VK, false, 48, false);
  }
#undef QR_S
}

}  // namespace

namespace noise {

// The row-resident q|k|v projection when the shapes allow it (K = 512, every 128-row block inside
// one member; the two-waves-per-SIMD form when every 256-row block is); returns false (nothing
// launched) otherwise.
bool proj_qkv_launch(const uint16_t* A, int64_t lda, const uint16_t* W, int64_t ldw, int M, int K,
                     const noise_rank1_t& r1, const noise_rope_t& rope, hipStream_t stream) {
  if (K != PK || M % PROWS != 0 || rope.T % PROWS != 0 || lda % 8 != 0 || ldw % 8 != 0) return false;
  if (r1.sign && (r1.nseg != 3 || r1.seg_cols != 512 || r1.rows_per_member != rope.T || r1.u_parts > 8)) return false;
  if (rope.gate && ((uintptr_t)rope.gate % 16) != 0) return false;
  ProjArgs g{};
  g.A = A; g.lda = lda; g.W = W; g.ldw = ldw; g.M = M; g.T = rope.T;
  g.r1 = r1;
  if (!r1.sign) { g.r1.nseg = 3; g.r1.seg_cols = 512; g.r1.u_parts = 0; }
  g.rope = rope;
  if (M % QR_ROWS == 0 && rope.T % QR_ROWS == 0) {
    if (rope.gate) qkv_rr_kernel<true><<<M / QR_ROWS, QR_THREADS, 0, stream>>>(g);
    else qkv_rr_kernel<false><<<M / QR_ROWS, QR_THREADS, 0, stream>>>(g);
  } else if (rope.gate) {
    qkv_proj_kernel<true><<<M / PROWS, 256, 0, stream>>>(g);
  } else {
    qkv_proj_kernel<false><<<M / PROWS, 256, 0, stream>>>(g);
  }
  return true;
}

}  // namespace noise
