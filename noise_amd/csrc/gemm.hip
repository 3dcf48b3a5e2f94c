// Perturbed GEMM of the population forward: C = A W^T + sign (A . b) a^T with fused epilogues.
//
// Reference semantics: `lowrank` (train/val/eggroll.py:56-58) for every block matrix, with the
// residual adds (eggroll.py:92-93) and relu^2 (eggroll.py:93; utils/model.py:107) folded into the
// epilogue. The dot products u = A . b arrive precomputed per row (written by the producer of A),
// so the rank-1 term costs one FMA per output element.
//
// Tiling for gfx950: a 256 x BN output tile per workgroup of 2 x (BN / 64) waves, each wave
// owning a 128x64 sub-tile as 4 x 2 blocks of v_mfma_f32_32x32x16_bf16 (128 fp32 accumulators
// per lane); the K loop is mma_tile. BN = 256 (8 waves, one workgroup per CU, two 64-deep stages
// of whole 128-byte rows) serves every shape in the step; BN = 128 (4 waves, three 32-deep stages,
// two workgroups per CU) remains for N or rank-1 segments that are not multiples of 256. Measured
// on MI355X: 256-column tiles with 64-deep stages beat 128-column ones by 4-6% on the relu^2 and
// q|k|v projections and by 3-8% on the fp32-output shapes.
// The epilogue runs in four rounds of 32 rows per wave: the rank-1 term and the mode's transform
// are applied to one accumulator block, the block is staged through LDS as fp32 and written out
// with 16-byte coalesced accesses. Workgroups are renumbered so that each XCD walks a contiguous
// run of tiles (neighbouring N tiles share the A rows in that XCD's L2).
#include "mma_tile.h"

namespace {

constexpr int BM = noise::TILE_M, BK = 2 * noise::TBK;
// Epilogue of the fused q|k|v projection (noise_qkv_rope_gemm only): rotary + RMSNorm on the q
// and k heads, v + gate * value embedding on the v heads, bf16 out.
constexpr int EPI_QKV_ROPE = 4;
constexpr float RMS_EPS = 1.1920928955078125e-07f;  // float32 machine epsilon (F.rms_norm default)
constexpr int SLD = 72;  // epilogue staging row stride (floats): the two half-waves of a store
                         // are 4 rows apart = 288 floats = 32 banks apart

struct GemmArgs {
  const uint16_t* A;
  int64_t lda;
  const uint16_t* W;
  int64_t ldw;
  int M, N, K;
  noise_rank1_t r1;
  void* C;
  int64_t ldc;
  const float* b_next;
  int64_t ld_bnext;
  float* u_next;
  int64_t ld_unext;
  noise_rope_t rope;  // EPI_QKV_ROPE only (rope.qkv unused: the input is this GEMM's accumulator)
};

// LONGK marks the K >= 1024 instantiation (the MLP down-projection, K = 2048) so that it is a
// kernel of its own in profiles; the code is the same.
template <int MODE, int BN, bool LONGK>
__global__ void __attribute__((amdgpu_flat_work_group_size(2 * BN, 2 * BN), amdgpu_waves_per_eu(2, 2)))
lowrank_gemm_kernel(const GemmArgs g) {
  // 256-column tiles run 64-deep stages (two stage buffers of 64 KB), 128-column tiles 32-deep
  // stages (three of 24 KB, so that two workgroups fit in a CU).
  constexpr int NSTG = BN == 256 ? 2 : 3, KDEPTH = BN == 256 ? 64 : 32;
  using Cfg = noise::TileCfg<BN, NSTG, KDEPTH>;
  constexpr int NT = Cfg::THREADS, WN = BN / 64;
  // The main loop's stage buffers, reused by the epilogue's fp32 staging (whichever is larger).
  constexpr int STAGE_ELEMS = Cfg::WAVES * 32 * SLD * 2;
  // All of the kernel's LDS is one array: the tile's direct global -> LDS loads are synchronised
  // by explicit waits, and a single LDS object keeps the compiler from adding conservative waits
  // for them before unrelated LDS reads. Per-row data first (immediate-offset addressing), then
  // the tile buffers / epilogue staging.
  constexpr int TILE_BYTES = 2 * (Cfg::SMEM_ELEMS > STAGE_ELEMS ? Cfg::SMEM_ELEMS : STAGE_ELEMS);
  constexpr int ROW_BYTES = BM * 4;
  constexpr int ROW_ARRAYS = MODE == EPI_QKV_ROPE ? 5 + BN / 64 : 2;
  __shared__ __attribute__((aligned(16))) unsigned char lds[ROW_ARRAYS * ROW_BYTES + TILE_BYTES];
  float* su_s = reinterpret_cast<float*>(lds);
  int* pn_s = reinterpret_cast<int*>(lds + ROW_BYTES);  // noise row of each tile row
  // EPI_QKV_ROPE per-row data: token position, token id (-1 if out of range), sign * a_ve[token],
  // and the VE gate of the tile's BN / 64 heads.
  int* t_s = reinterpret_cast<int*>(lds + 2 * ROW_BYTES);
  int* tok_s = reinterpret_cast<int*>(lds + 3 * ROW_BYTES);
  float* sa_s = reinterpret_cast<float*>(lds + 4 * ROW_BYTES);
  float(*gate_s)[BN / 64] = reinterpret_cast<float(*)[BN / 64]>(lds + 5 * ROW_BYTES);
  uint16_t* smem = reinterpret_cast<uint16_t*>(lds + ROW_ARRAYS * ROW_BYTES);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int ntn = g.N / BN;
  const int ntiles = gridDim.x;
  int bid = blockIdx.x;
  if ((ntiles & 7) == 0) bid = (bid & 7) * (ntiles >> 3) + (bid >> 3);  // XCD-contiguous runs
  const int m0 = (bid / ntn) * BM, n0 = (bid % ntn) * BN;
  const int T = g.r1.rows_per_member;
  const bool perturbed = g.r1.sign != nullptr;

  // Per-row sign * u, staged once per tile (visible after the main loop's first barrier).
  const int seg = perturbed ? n0 / g.r1.seg_cols : 0;
  if (tid < BM) {
    const int row = m0 + tid;
    float su = 0.f;
    if (perturbed && row < g.M) {
      const float* up = g.r1.u[seg] + (int64_t)row * g.r1.ldu;
      float u = 0.f;
      for (int j = 0; j < g.r1.u_parts; ++j) u += up[j];
      su = g.r1.sign[row / T] * u;
    }
    su_s[tid] = su;
    pn_s[tid] = ((row < g.M ? row : g.M - 1) / T) >> g.r1.member_shift;
    if (MODE == EPI_QKV_ROPE) {
      const int r = row < g.M ? row : g.M - 1;
      const int p = r / T, t = r - p * T;
      t_s[tid] = t;
      if (n0 >= 1024 && g.rope.gate) {
        const int64_t tok = g.rope.idx[(int64_t)p * g.rope.idx_stride + t];
        const bool ok = tok >= 0 && tok < g.rope.vocab;
        tok_s[tid] = ok ? (int)tok : -1;
        sa_s[tid] = (ok && g.rope.sign)
                        ? g.rope.sign[p] * g.rope.ve_a[((int64_t)p >> g.rope.member_shift) * g.rope.ld_ve_a + tok]
                        : 0.f;
#pragma unroll
        for (int hh = 0; hh < WN; ++hh) gate_s[tid][hh] = g.rope.gate[(int64_t)r * 8 + (n0 - 1024) / 64 + hh];
      }
    }
  }

  floatx16 acc[4][2];
  noise::zero_acc(acc);
  noise::mma_tile<BN, NSTG, KDEPTH>(g.A + (int64_t)m0 * g.lda, g.lda, g.M - m0, g.W + (int64_t)n0 * g.ldw, g.ldw, g.K,
                      smem, acc);

  // ---- epilogue ----
  const int last_row = (m0 + BM < g.M ? m0 + BM : g.M) - 1;
  const bool uniform = (m0 / T) == (last_row / T);  // one member (one noise row) per tile
  const float* aseg = perturbed ? g.r1.a[seg] : nullptr;
  const int seg_base = perturbed ? seg * g.r1.seg_cols : 0;
  const int colbase = n0 + wn * 64 + (lane & 31);
  const bool want_u = MODE == NOISE_EPI_RELU2_BF16 && g.u_next != nullptr;

  // Uniform tiles: a and b_next are one value per column for the whole tile.
  float a_val[2] = {0.f, 0.f}, bn_val[2] = {0.f, 0.f};
  if (uniform) {
    const int64_t pn = pn_s[0];
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
      const int col = colbase + ni * 32;
      if (perturbed) a_val[ni] = aseg[pn * g.r1.lda + (col - seg_base)];
      if (want_u) bn_val[ni] = g.b_next[pn * g.ld_bnext + col];
    }
  }

  float* stage = reinterpret_cast<float*>(smem);  // [waves][32 rows][SLD] fp32
  float* wstage = stage + wave * 32 * SLD + 4 * (lane >> 5) * SLD + (lane & 31);
  constexpr bool OUT_BF16 = MODE == NOISE_EPI_BF16 || MODE == NOISE_EPI_RELU2_BF16 || MODE == EPI_QKV_ROPE;

// Tile row of accumulator j in block row mi, and its rank-1 value x = acc + sign u a.
#define NOISE_RL(J) (wm * 128 + mi * 32 + 8 * ((J) >> 2) + 4 * (lane >> 5) + ((J) & 3))
#define NOISE_RANK1(X)                                                                          \
  if (uniform) {                                                                              \
    _Pragma("unroll") for (int j = 0; j < 16; ++j) {                                          \
      const float su = su_s[NOISE_RL(j)];                                                     \
      _Pragma("unroll") for (int ni = 0; ni < 2; ++ni) X[ni][j] = acc[mi][ni][j] + su * a_val[ni]; \
    }                                                                                         \
  } else {                                                                                    \
    _Pragma("unroll") for (int j = 0; j < 16; ++j) {                                          \
      const float su = su_s[NOISE_RL(j)];                                                     \
      const float* ar = perturbed ? aseg + (int64_t)pn_s[NOISE_RL(j)] * g.r1.lda - seg_base : nullptr; \
      _Pragma("unroll") for (int ni = 0; ni < 2; ++ni)                                        \
        X[ni][j] = acc[mi][ni][j] + (perturbed ? su * ar[colbase + ni * 32] : 0.f);           \
    }                                                                                         \
  }

#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
    // (1) rank-1 term + transform of block row mi, staged as fp32 in this wave's LDS slice.
    float x[2][16];
    float pd[16];
    NOISE_RANK1(x)
    if (MODE == EPI_QKV_ROPE) {
      // Lane holds dims d = lane % 32 (ni = 0) and d + 32 (ni = 1) of one head for 16 rows: the
      // rotary pairs (x1, x2) of apply_rotary_emb are the lane's two values.
      if (n0 < 1024) {  // q or k: rotate, then RMS-normalise over the head's 64 dims
        const int d = lane & 31;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int t = t_s[NOISE_RL(j)];
          const float cs = g.rope.cos[t * 32 + d], sn = g.rope.sin[t * 32 + d];
          const float o1 = x[0][j] * cs + x[1][j] * sn;
          const float o2 = x[0][j] * -sn + x[1][j] * cs;
          x[0][j] = o1;
          x[1][j] = o2;
          pd[j] = o1 * o1 + o2 * o2;
        }
        const float tot = noise::halfwave_transpose_sum16(pd, lane);  // row (lane/2) % 16 of the half
        const float rr = rsqrtf(tot * (1.0f / 64) + RMS_EPS);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const float r = __shfl(rr, (lane & 32) + 2 * j, 64);
          x[0][j] *= r;
          x[1][j] *= r;
        }
      }  // v + gate * value embedding: added in the copy-out below, from full table-row chunks
    } else if (MODE == NOISE_EPI_RELU2_BF16) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        pd[j] = 0.f;
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) x[ni][j] = bf2f(f2bf(x[ni][j] > 0.f ? x[ni][j] * x[ni][j] : 0.f));
      }
      if (want_u) {
        if (uniform) {
#pragma unroll
          for (int j = 0; j < 16; ++j) pd[j] = x[0][j] * bn_val[0] + x[1][j] * bn_val[1];
        } else {
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const float* br = g.b_next + (int64_t)pn_s[NOISE_RL(j)] * g.ld_bnext + colbase;
            pd[j] = x[0][j] * br[0] + x[1][j] * br[32];
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 16; ++j)
#pragma unroll
      for (int ni = 0; ni < 2; ++ni) wstage[(8 * (j >> 2) + (j & 3)) * SLD + ni * 32] = x[ni][j];
    if (want_u) {
      const float tot = noise::halfwave_transpose_sum16(pd, lane);
      const int jj = (lane & 31) >> 1;
      const int row = m0 + wm * 128 + mi * 32 + 8 * (jj >> 2) + 4 * (lane >> 5) + (jj & 3);
      if ((lane & 1) == 0 && row < g.M) g.u_next[(int64_t)row * g.ld_unext + (n0 + wn * 64) / 64] = tot;
    }
    __syncthreads();
    // (2) copy-out: this round covers rows wm*128 + mi*32 .. +32 of both row halves, all BN
    // columns. Chunk id -> (row half h, row r, column c); wave (h, c / 64) staged it.
    if (OUT_BF16) {
      uint16_t* C16 = reinterpret_cast<uint16_t*>(g.C);
#pragma unroll
      for (int q = 0; q < 4; ++q) {  // 64 rows x BN/8 chunks of 8 columns
        const int id = q * NT + tid, rr = id / (BN / 8), c8 = (id % (BN / 8)) * 8;
        const int h = rr >> 5, r = rr & 31;
        const int row = m0 + h * 128 + mi * 32 + r;
        const float* src = stage + ((h * WN + (c8 >> 6)) * 32 + r) * SLD + (c8 & 63);
        float4 lo = *reinterpret_cast<const float4*>(src);
        float4 hi = *reinterpret_cast<const float4*>(src + 4);
        if (MODE == EPI_QKV_ROPE && n0 >= 1024 && g.rope.gate) {
          // v + gate * (table[token] + sign a_ve[token] b_ve) on 8 consecutive columns of the row.
          const int tl = h * 128 + mi * 32 + r, vc = n0 - 1024 + c8;
          const int tok = tok_s[tl];
          const float gt = gate_s[tl][c8 >> 6], sa = sa_s[tl];
          float ve[8];
          if (tok >= 0) {
            const float* tv = g.rope.ve_table + (int64_t)tok * 512 + vc;
            const float4 t0 = *reinterpret_cast<const float4*>(tv), t1 = *reinterpret_cast<const float4*>(tv + 4);
            ve[0] = t0.x; ve[1] = t0.y; ve[2] = t0.z; ve[3] = t0.w;
            ve[4] = t1.x; ve[5] = t1.y; ve[6] = t1.z; ve[7] = t1.w;
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) ve[e] = __builtin_nanf("");
          }
          if (g.rope.sign) {
            const float* bv = g.rope.ve_b + (int64_t)pn_s[tl] * g.rope.ld_ve_b + vc;
            const float4 b0 = *reinterpret_cast<const float4*>(bv), b1 = *reinterpret_cast<const float4*>(bv + 4);
            ve[0] += sa * b0.x; ve[1] += sa * b0.y; ve[2] += sa * b0.z; ve[3] += sa * b0.w;
            ve[4] += sa * b1.x; ve[5] += sa * b1.y; ve[6] += sa * b1.z; ve[7] += sa * b1.w;
          }
          lo.x += gt * ve[0]; lo.y += gt * ve[1]; lo.z += gt * ve[2]; lo.w += gt * ve[3];
          hi.x += gt * ve[4]; hi.y += gt * ve[5]; hi.z += gt * ve[6]; hi.w += gt * ve[7];
        }
        // Non-temporal: the output streams past L2 instead of evicting the tile operands there
        // (measured 2-4% faster on the relu^2 and bf16 outputs; the fp32 residual stream, which
        // the next kernel reads straight back, is better kept on the normal path).
        if (row < g.M)
          __builtin_nontemporal_store(
              u32x4{pack_bf2(lo.x, lo.y), pack_bf2(lo.z, lo.w), pack_bf2(hi.x, hi.y), pack_bf2(hi.z, hi.w)},
              reinterpret_cast<u32x4*>(C16 + (int64_t)row * g.ldc + n0 + c8));
      }
    } else {
      float* C32 = reinterpret_cast<float*>(g.C);
      float4 prev[8];
      if (MODE == NOISE_EPI_ADD_F32) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {  // 64 rows x BN/4 chunks of 4 columns
          const int id = q * NT + tid, rr = id / (BN / 4), c4 = (id % (BN / 4)) * 4;
          const int row = m0 + (rr >> 5) * 128 + mi * 32 + (rr & 31);
          prev[q] = *reinterpret_cast<const float4*>(C32 + (int64_t)(row < g.M ? row : g.M - 1) * g.ldc + n0 + c4);
        }
      }
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int id = q * NT + tid, rr = id / (BN / 4), c4 = (id % (BN / 4)) * 4;
        const int h = rr >> 5, r = rr & 31;
        const int row = m0 + h * 128 + mi * 32 + r;
        float4 v = *reinterpret_cast<const float4*>(stage + ((h * WN + (c4 >> 6)) * 32 + r) * SLD + (c4 & 63));
        if (MODE == NOISE_EPI_ADD_F32) {
          v.x += prev[q].x; v.y += prev[q].y; v.z += prev[q].z; v.w += prev[q].w;
        }
        if (row < g.M) *reinterpret_cast<float4*>(C32 + (int64_t)row * g.ldc + n0 + c4) = v;
      }
    }
    if (mi < 3) __syncthreads();  // the copy-out reads are done before the next round writes
  }
#undef NOISE_RANK1
#undef NOISE_RL
}

// Validates the arguments shared by both entry points and fills g (everything but the rope part).
int prepare_gemm(GemmArgs& g, const uint16_t* A, int64_t lda, const uint16_t* W, int64_t ldw, int M,
                 int N, int K, const noise_rank1_t* r1, void* C, int64_t ldc, int T_unperturbed) {
  NOISE_REQUIRE(A && W && C, "lowrank_gemm: null A, W or C");
  NOISE_REQUIRE(M >= 0 && N > 0 && K > 0, "lowrank_gemm: bad sizes M=%d N=%d K=%d", M, N, K);
  NOISE_REQUIRE(N % 128 == 0, "lowrank_gemm: N=%d must be a multiple of 128", N);
  NOISE_REQUIRE(K % BK == 0, "lowrank_gemm: K=%d must be a multiple of %d", K, BK);
  NOISE_REQUIRE(lda >= K && ldw >= K && lda % 8 == 0 && ldw % 8 == 0,
                "lowrank_gemm: lda=%lld ldw=%lld must be >= K and multiples of 8", (long long)lda,
                (long long)ldw);
  NOISE_REQUIRE(ldc >= N, "lowrank_gemm: ldc=%lld < N=%d", (long long)ldc, N);
  NOISE_REQUIRE(ldc % 8 == 0 && ((uintptr_t)C % 16) == 0,
                "lowrank_gemm: C must be 16-byte aligned with ldc a multiple of 8");
  NOISE_REQUIRE(((uintptr_t)A % 16) == 0 && ((uintptr_t)W % 16) == 0,
                "lowrank_gemm: A and W must be 16-byte aligned");
  g = GemmArgs{};
  g.A = A; g.lda = lda; g.W = W; g.ldw = ldw; g.M = M; g.N = N; g.K = K;
  g.C = C; g.ldc = ldc;
  noise_rank1_t none = {};
  none.seg_cols = N;
  none.nseg = 1;
  none.u_parts = 1;
  g.r1 = r1 ? *r1 : none;
  if (g.r1.sign) {
    NOISE_REQUIRE(g.r1.rows_per_member > 0, "lowrank_gemm: rows_per_member must be > 0");
    NOISE_REQUIRE(g.r1.nseg >= 1 && g.r1.nseg <= 3 && g.r1.seg_cols % 128 == 0 &&
                      g.r1.seg_cols * g.r1.nseg == N,
                  "lowrank_gemm: segments (%d x %d) must tile N=%d in multiples of %d", g.r1.nseg,
                  g.r1.seg_cols, N, 128);
    NOISE_REQUIRE(g.r1.u_parts >= 1 && g.r1.ldu >= g.r1.u_parts, "lowrank_gemm: bad u_parts/ldu");
    NOISE_REQUIRE(g.r1.member_shift >= 0 && g.r1.member_shift < 31, "lowrank_gemm: bad member_shift");
    for (int s = 0; s < g.r1.nseg; ++s)
      NOISE_REQUIRE(g.r1.a[s] && g.r1.u[s], "lowrank_gemm: null a/u for segment %d", s);
    NOISE_REQUIRE(g.r1.lda >= g.r1.seg_cols, "lowrank_gemm: r1.lda < seg_cols");
  } else {
    g.r1.rows_per_member = T_unperturbed;
  }
  const int64_t tiles = (int64_t)((M + BM - 1) / BM) * (N / 128);
  NOISE_REQUIRE(tiles < (1ll << 31), "lowrank_gemm: too many tiles");
  return NOISE_OK;
}

}  // namespace

extern "C" int noise_lowrank_gemm(const uint16_t* A, int64_t lda, const uint16_t* W, int64_t ldw,
                                  int M, int N, int K, const noise_rank1_t* r1, int mode, void* C,
                                  int64_t ldc, const float* b_next, int64_t ld_bnext, float* u_next,
                                  int64_t ld_unext, void* stream) {
  NOISE_REQUIRE(mode >= NOISE_EPI_BF16 && mode <= NOISE_EPI_RELU2_BF16, "lowrank_gemm: bad mode %d", mode);
  GemmArgs g;
  int rc = prepare_gemm(g, A, lda, W, ldw, M, N, K, r1, C, ldc, M > 0 ? M : 1);
  if (rc) return rc;
  NOISE_REQUIRE(!b_next == !u_next, "lowrank_gemm: b_next and u_next go together");
  if (b_next) {
    NOISE_REQUIRE(mode == NOISE_EPI_RELU2_BF16, "lowrank_gemm: b_next/u_next only apply to the relu2 epilogue");
    NOISE_REQUIRE(ld_unext >= N / 64 && ld_bnext >= N, "lowrank_gemm: ld_unext/ld_bnext too small");
  }
  g.b_next = b_next; g.ld_bnext = ld_bnext; g.u_next = u_next; g.ld_unext = ld_unext;
  if (M == 0) return NOISE_OK;
  // 256-column tiles unless N or a rank-1 segment asks for 128.
  const bool wide = N % 256 == 0 && (!g.r1.sign || g.r1.seg_cols % 256 == 0);
  const int bn = wide ? 256 : 128;
  const dim3 grid((unsigned)((int64_t)((M + BM - 1) / BM) * (N / bn)));
  hipStream_t st = (hipStream_t)stream;
  const bool longk = K >= 1024;
#define NOISE_GEMM_LAUNCH(MODE_, BN_, LK_) lowrank_gemm_kernel<MODE_, BN_, LK_><<<grid, 2 * (BN_), 0, st>>>(g)
  switch (mode) {
    case NOISE_EPI_BF16:
      if (wide) NOISE_GEMM_LAUNCH(NOISE_EPI_BF16, 256, false); else NOISE_GEMM_LAUNCH(NOISE_EPI_BF16, 128, false);
      break;
    case NOISE_EPI_F32:
      if (wide) NOISE_GEMM_LAUNCH(NOISE_EPI_F32, 256, false); else NOISE_GEMM_LAUNCH(NOISE_EPI_F32, 128, false);
      break;
    case NOISE_EPI_ADD_F32:
      if (wide && longk) NOISE_GEMM_LAUNCH(NOISE_EPI_ADD_F32, 256, true);
      else if (wide) NOISE_GEMM_LAUNCH(NOISE_EPI_ADD_F32, 256, false);
      else NOISE_GEMM_LAUNCH(NOISE_EPI_ADD_F32, 128, false);
      break;
    default:
      if (wide) NOISE_GEMM_LAUNCH(NOISE_EPI_RELU2_BF16, 256, false); else NOISE_GEMM_LAUNCH(NOISE_EPI_RELU2_BF16, 128, false);
      break;
  }
#undef NOISE_GEMM_LAUNCH
  return noise::check_launch("lowrank_gemm");
}

extern "C" int noise_qkv_rope_gemm(const uint16_t* A, int64_t lda, const uint16_t* W, int64_t ldw, int M,
                                   int K, const noise_rank1_t* r1, const noise_rope_t* rope, void* stream) {
  NOISE_REQUIRE(rope && rope->out && rope->cos && rope->sin, "qkv_rope_gemm: null rope, out or tables");
  const noise_rope_t& rp = *rope;
  NOISE_REQUIRE(rp.M == M && rp.T > 0, "qkv_rope_gemm: rope.M=%d must equal M=%d, T=%d > 0", rp.M, M, rp.T);
  NOISE_REQUIRE(!r1 || !r1->sign || r1->rows_per_member == rp.T,
                "qkv_rope_gemm: rank-1 rows_per_member must equal rope.T");
  NOISE_REQUIRE(!rp.gate || (rp.ve_table && rp.idx && rp.vocab > 0 && rp.member_shift >= 0 &&
                             (!rp.sign || (rp.ve_a && rp.ve_b && rp.ld_ve_a >= rp.vocab && rp.ld_ve_b >= 512))),
                "qkv_rope_gemm: value embedding needs table, idx, vocab and (perturbed) ve_a/ve_b");
  NOISE_REQUIRE(!rp.gate || (((uintptr_t)rp.ve_table % 16) == 0 &&
                             (!rp.sign || (((uintptr_t)rp.ve_b % 16) == 0 && rp.ld_ve_b % 4 == 0))),
                "qkv_rope_gemm: ve_table and ve_b must be 16-byte aligned, ld_ve_b a multiple of 4");
  GemmArgs g;
  int rc = prepare_gemm(g, A, lda, W, ldw, M, 1536, K, r1, rp.out, 1536, rp.T);
  if (rc) return rc;
  g.rope = rp;
  if (M == 0) return NOISE_OK;
  if (noise::proj_qkv_launch(A, lda, W, ldw, M, K, g.r1, rp, (hipStream_t)stream))
    return noise::check_launch("qkv_rope_gemm (row-resident)");
  const dim3 grid((unsigned)((int64_t)((M + BM - 1) / BM) * (1536 / 256)));
  lowrank_gemm_kernel<EPI_QKV_ROPE, 256, false><<<grid, 512, 0, (hipStream_t)stream>>>(g);
  return noise::check_launch("qkv_rope_gemm");
}
