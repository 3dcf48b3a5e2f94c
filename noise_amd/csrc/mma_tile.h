// 256 x 256 bf16 MFMA tile main loop shared by the perturbed GEMM and the head kernel.
//
// acc += A[0:256, 0:K] * B[0:256, 0:K]^T for A, B row-major bf16 with K contiguous. 256 threads
// (4 waves, 2 x 2); wave (wm, wn) owns rows wm*128.. and columns wn*128.. as 4 x 4 blocks of
// v_mfma_f32_32x32x16_bf16. Block (mi, ni), accumulator j of lane l holds
//   row = wm*128 + mi*32 + 8*(j/4) + 4*(l/32) + j%4,   col = wn*128 + ni*32 + l%32.
// K steps by 64 through two LDS stages with rows padded to 144 B; the next stage's global loads
// are in flight while the current stage feeds the MFMAs. Rows of A at or beyond `a_rows` are read
// from row a_rows - 1 (their results are discarded by the caller).
#pragma once
#include "common.h"

namespace noise {

constexpr int TILE = 256, TBK = 64, TLDK = TBK + 8;
typedef uint16_t TileSmem[2][2][TILE][TLDK];  // [stage][A|B][row][k]

NOISE_DEV void mma_tile_256(const uint16_t* __restrict__ A, int64_t lda, int a_rows,
                            const uint16_t* __restrict__ B, int64_t ldb, int K, TileSmem& smem,
                            floatx16 (&acc)[4][4]) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int KT = K / TBK;
  const int lr = tid >> 3, lc = (tid & 7) * 8;
  u32x4 ra[8], rb[8];
  const uint16_t* arow_ptr[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    int r = i * 32 + lr;
    r = r < a_rows ? r : a_rows - 1;
    arow_ptr[i] = A + (int64_t)r * lda + lc;
  }
  auto gload = [&](int kt) {
    const int k0 = kt * TBK;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      ra[i] = *reinterpret_cast<const u32x4*>(arow_ptr[i] + k0);
      rb[i] = *reinterpret_cast<const u32x4*>(B + (int64_t)(i * 32 + lr) * ldb + lc + k0);
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      *reinterpret_cast<u32x4*>(&smem[buf][0][i * 32 + lr][lc]) = ra[i];
      *reinterpret_cast<u32x4*>(&smem[buf][1][i * 32 + lr][lc]) = rb[i];
    }
  };
  gload(0);
  __syncthreads();  // the previous user of smem is done
  sstore(0);
  __syncthreads();
  const int arow = wm * 128 + (lane & 31), brow = wn * 128 + (lane & 31), kofs = (lane >> 5) * 8;
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) gload(kt + 1);
#pragma unroll
    for (int kk = 0; kk < TBK / 16; ++kk) {
      bf16x8 fa[4], fb[4];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
        fa[mi] = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const u32x4*>(&smem[cur][0][arow + mi * 32][kk * 16 + kofs]));
#pragma unroll
      for (int ni = 0; ni < 4; ++ni)
        fb[ni] = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const u32x4*>(&smem[cur][1][brow + ni * 32][kk * 16 + kofs]));
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
          acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[mi], fb[ni], acc[mi][ni], 0, 0, 0);
    }
    if (kt + 1 < KT) sstore(cur ^ 1);
    __syncthreads();
  }
}

NOISE_DEV void zero_acc(floatx16 (&acc)[4][4]) {
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[mi][ni][j] = 0.f;
}

}  // namespace noise
