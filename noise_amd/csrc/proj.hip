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

}  // namespace

namespace noise {

// The row-resident q|k|v projection when the shapes allow it (K = 512, every 128-row block inside
// one member); returns false (nothing launched) otherwise.
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
  if (rope.gate) qkv_proj_kernel<true><<<M / PROWS, 256, 0, stream>>>(g);
  else qkv_proj_kernel<false><<<M / PROWS, 256, 0, stream>>>(g);
  return true;
}

}  // namespace noise
