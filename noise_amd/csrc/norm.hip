// Row kernels over the d = 512 residual stream: one wavefront per row, 8 floats per lane.
//
// * embed_norm: x0 = norm(W[idx] + s a[idx] b) -- `lowrank_embed` + `norm`
//   (train/val/eggroll.py:61-63, 74; utils/model.py:46-47).
// * mix_norm: x = (lr + s er) x + (l0 + s e0) x0 (eggroll.py:77-79), h = bf16(norm(x))
//   (eggroll.py:81, 93, 94), the dots u_j = h . b_j that the rank-1 terms of the GEMMs reading h
//   need (eggroll.py:58), and the value-embedding gate 2 sigmoid(lowrank(h[:32], ve_gate))
//   (eggroll.py:88; utils/model.py:89).
// * rope_norm_ve: q, k -> norm(rotary(.)) (utils/model.py:55-58; eggroll.py:90) and
//   v + gate * (VE[idx] + s a[idx] b) (eggroll.py:85-89), written as the bf16 attention inputs.
#include "common.h"

namespace {

constexpr int D = 512;

// Sum over a fully active wave: 16-lane row sums by DPP (quad_perm [1,0,3,2], quad_perm
// [2,3,0,1], row_half_mirror, row_mirror), then the four rows' totals through readlane. No LDS
// traffic, unlike the shuffle-based sum.
template <int CTRL>
NOISE_DEV float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
NOISE_DEV float wave_sum_dpp(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  v += dpp_f<0x140>(v);
  return (__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)) +
          __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16))) +
         (__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)) +
          __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48)));
}


NOISE_DEV void load8(const float* p, float (&v)[8]) {
  float4 a = *reinterpret_cast<const float4*>(p);
  float4 b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
NOISE_DEV void store8(float* p, const float (&v)[8]) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
}

// The values mix_norm needs besides the row itself, all of them the same for every row of a member
// (or of the launch): loaded at the start of a row's wave, next to the row's own loads, so that
// their latency overlaps instead of following the row's stores.
struct MixPre {
  float s, lr, l0;     // sign; the mixing factors (lr + s er), (l0 + s e0)
  float bv[3][8];      // the dot vectors' columns 8 lane .. + 7
  float gn[8];         // the gain's columns (1 without a gain)
  float wv[8];         // gate: W row lane / 4, block lane % 4 (lanes < 32), or b_gate (lanes >= 32)
  float ga;            // gate: a_gate[q] of lane q * 4 (lanes < 32)
};

NOISE_DEV MixPre mix_pre(const noise_mixnorm_t& g, int row, int lane) {
  MixPre m;
  const int p = row / g.T;
  const int64_t pn = p >> g.member_shift;
  const int c = lane * 8;
  m.s = g.sign ? g.sign[p] : 0.f;
  m.lr = 1.f;
  m.l0 = 0.f;
  if (g.x0) {
    m.lr = *g.resid;
    m.l0 = *g.mix;
    if (g.sign) {
      m.lr += m.s * g.eps_resid[pn * g.ld_eps];
      m.l0 += m.s * g.eps_mix[pn * g.ld_eps];
    }
  }
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    if (j < g.nb) {
      load8(g.b[j] + pn * g.ldb + c, m.bv[j]);
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) m.bv[j][k] = 0.f;
    }
  }
  if (g.gain) {
    load8(g.gain + c, m.gn);
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) m.gn[k] = 1.f;
  }
  m.ga = 0.f;
  if (g.gate_w) {
    const int blk = lane & 3;
    if (lane < 32) {
      load8(g.gate_w + (lane >> 2) * 32 + blk * 8, m.wv);
      if (g.sign) m.ga = g.gate_a[pn * g.ld_gate_a + (lane >> 2)];
    } else if (g.sign) {
      load8(g.gate_b + pn * g.ld_gate_b + blk * 8, m.wv);
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) m.wv[k] = 0.f;
    }
  }
  return m;
}

// mix_norm of one row (one wavefront, lane l: columns 8 l .. 8 l + 7) from its x values v and, when
// mixing, its x0 values v0.
NOISE_DEV void mix_norm_row(const noise_mixnorm_t& g, const MixPre& m, int row, int lane, float (&v)[8],
                            const float (&v0)[8]) {
  const int c = lane * 8;
  if (g.x0) {
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = m.lr * v[k] + m.l0 * v0[k];
    store8(g.x + (int64_t)row * D + c, v);
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) ss += v[k] * v[k];
  ss = wave_sum_dpp(ss);
  const float rr = rsqrtf(ss * (1.0f / D) + 1.1920928955078125e-07f);
  float h[8];
  uint32_t packed[4];
  if (g.gain) {  // F.rms_norm's weight: (x rr) gain
#pragma unroll
    for (int k = 0; k < 4; ++k)
      packed[k] = pack_bf2(v[2 * k] * rr * m.gn[2 * k], v[2 * k + 1] * rr * m.gn[2 * k + 1]);
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) packed[k] = pack_bf2(v[2 * k] * rr, v[2 * k + 1] * rr);
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    h[2 * k] = bf_lo(packed[k]);
    h[2 * k + 1] = bf_hi(packed[k]);
  }
  *reinterpret_cast<uint4*>(g.h + (int64_t)row * D + c) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    if (j >= g.nb) break;
    float d = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) d += h[k] * m.bv[j][k];
    d = wave_sum_dpp(d);
    if (lane == 0) g.u[(int64_t)row * g.ldu + j] = d;
  }
  if (g.gate_w) {
    // Channels 0..31 live in lanes 0..3 (8 each). Lane l < 32 forms the partial logit of gate
    // l / 4 over channel block l % 4; lanes 32..63 form the same block's partial dot with the
    // gate's noise vector b (replicated eight times). Both are summed over the 4 lanes of a group.
    const int blk = lane & 3;
    float hb[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) hb[k] = __shfl(h[k], blk, 64);
    float part = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) part += hb[k] * m.wv[k];
    part = group_sum(part, 4);
    const float nd = __shfl(part, 32, 64);  // h[:32] . b_gate
    if (lane < 32 && blk == 0) {
      const int q = lane >> 2;
      float z = part;
      if (g.sign) z += m.s * nd * m.ga;
      g.gate[(int64_t)row * 8 + q] = 2.0f / (1.0f + expf(-z));
    }
  }
}


// NEXT: the first layer's mix_norm (noise_mixnorm_t `nx`, mixing with x0 = this row) follows on
// the row still in registers; it writes the stream nx.x instead of the plain copy x.
template <bool NEXT>
__global__ __launch_bounds__(256) void embed_norm_kernel(
    const float* __restrict__ table, int64_t ld_table, int vocab, const int64_t* __restrict__ idx,
    int64_t idx_stride, int T, int M, const float* __restrict__ sign, const float* __restrict__ a, int64_t lda,
    const float* __restrict__ b, int64_t ldb, int shift, float* __restrict__ x0, float* __restrict__ x,
    const noise_mixnorm_t nx) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  MixPre m;
  if constexpr (NEXT) m = mix_pre(nx, row, lane);
  const int p = row / T, t = row - p * T;
  const int64_t tok = idx[p * idx_stride + t];
  const int c = lane * 8;
  float v[8];
  if (tok < 0 || tok >= vocab) {  // out-of-range id: poison the row so the loss is non-finite
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = __builtin_nanf("");
  } else {
    load8(table + tok * ld_table + c, v);
    if (sign) {
      const int64_t pn = p >> shift;
      const float sa = sign[p] * a[pn * lda + tok];
      float bv[8];
      load8(b + pn * ldb + c, bv);
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] += sa * bv[k];
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) ss += v[k] * v[k];
  ss = wave_sum(ss);
  const float r = rsqrtf(ss * (1.0f / D) + 1.1920928955078125e-07f);
#pragma unroll
  for (int k = 0; k < 8; ++k) v[k] *= r;
  store8(x0 + (int64_t)row * D + c, v);
  if constexpr (NEXT) {
    float w[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) w[k] = v[k];
    mix_norm_row(nx, m, row, lane, w, v);
  } else {
    if (x) store8(x + (int64_t)row * D + c, v);
  }
}

__global__ __launch_bounds__(256) void mix_norm_kernel(const noise_mixnorm_t g) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= g.M) return;
  const MixPre m = mix_pre(g, row, lane);
  float v[8], v0[8];
  load8(g.x + (int64_t)row * D + lane * 8, v);
  if (g.x0) load8(g.x0 + (int64_t)row * D + lane * 8, v0);
  mix_norm_row(g, m, row, lane, v, v0);
}

// One wavefront per row of the [M, 1536] fp32 q | k | v block.
__global__ __launch_bounds__(256) void rope_norm_ve_kernel(const noise_rope_t g) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= g.M) return;
  const int p = row / g.T, t = row - p * g.T;
  const float* src = g.qkv + (int64_t)row * 1536;
  uint16_t* dst = g.out + (int64_t)row * 1536;
  // q and k: lane -> head lane / 8, dims e*4 .. e*4+3 paired with +32.
  const int head = lane >> 3, e = (lane & 7) * 4;
  float cs[4], sn[4];
  {
    float4 c4 = *reinterpret_cast<const float4*>(g.cos + (int64_t)t * 32 + e);
    float4 s4 = *reinterpret_cast<const float4*>(g.sin + (int64_t)t * 32 + e);
    cs[0] = c4.x; cs[1] = c4.y; cs[2] = c4.z; cs[3] = c4.w;
    sn[0] = s4.x; sn[1] = s4.y; sn[2] = s4.z; sn[3] = s4.w;
  }
#pragma unroll
  for (int part = 0; part < 2; ++part) {
    const int base = part * 512 + head * 64 + e;
    float4 a4 = *reinterpret_cast<const float4*>(src + base);
    float4 b4 = *reinterpret_cast<const float4*>(src + base + 32);
    float x1[4] = {a4.x, a4.y, a4.z, a4.w}, x2[4] = {b4.x, b4.y, b4.z, b4.w};
    float o1[4], o2[4], ss = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      o1[k] = x1[k] * cs[k] + x2[k] * sn[k];
      o2[k] = x1[k] * -sn[k] + x2[k] * cs[k];
      ss += o1[k] * o1[k] + o2[k] * o2[k];
    }
    ss = group_sum(ss, 8);
    const float r = rsqrtf(ss * (1.0f / 64) + 1.1920928955078125e-07f);
    *reinterpret_cast<uint2*>(dst + base) = make_uint2(pack_bf2(o1[0] * r, o1[1] * r), pack_bf2(o1[2] * r, o1[3] * r));
    *reinterpret_cast<uint2*>(dst + base + 32) =
        make_uint2(pack_bf2(o2[0] * r, o2[1] * r), pack_bf2(o2[2] * r, o2[3] * r));
  }
  // v: lane -> columns lane*8 .. +7 (head lane / 8).
  const int c = lane * 8;
  float v[8];
  load8(src + 1024 + c, v);
  if (g.gate) {
    const float gt = g.gate[(int64_t)row * 8 + (c >> 6)];
    const int64_t tok = g.idx[p * g.idx_stride + t];
    float ve[8];
    if (tok < 0 || tok >= g.vocab) {
#pragma unroll
      for (int k = 0; k < 8; ++k) ve[k] = __builtin_nanf("");
    } else {
      load8(g.ve_table + tok * 512 + c, ve);
      if (g.sign) {
        const int64_t pn = p >> g.member_shift;
        const float sa = g.sign[p] * g.ve_a[pn * g.ld_ve_a + tok];
        float bv[8];
        load8(g.ve_b + pn * g.ld_ve_b + c, bv);
#pragma unroll
        for (int k = 0; k < 8; ++k) ve[k] += sa * bv[k];
      }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] += gt * ve[k];
  }
  *reinterpret_cast<uint4*>(dst + 1024 + c) =
      make_uint4(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]), pack_bf2(v[4], v[5]), pack_bf2(v[6], v[7]));
}

}  // namespace

extern "C" int noise_embed_norm(const float* table, int64_t ld_table, int vocab, int d,
                                const int64_t* idx, int64_t idx_stride, int T, int members,
                                const float* sign,
                                const float* a, int64_t lda, const float* b, int64_t ldb,
                                int member_shift, float* x0, float* x, void* stream) {
  NOISE_REQUIRE(d == D, "embed_norm: d=%d, only 512 is supported", d);
  NOISE_REQUIRE(table && idx && x0 && T > 0 && members >= 0 && vocab > 0 && ld_table >= d &&
                    ld_table % 4 == 0,
                "embed_norm: bad arguments");
  NOISE_REQUIRE(!sign || (a && b && lda >= vocab && ldb >= d && ldb % 4 == 0),
                "embed_norm: perturbation needs a [*, vocab] and b [*, d] (4-float aligned rows)");
  const int64_t M = (int64_t)members * T;
  NOISE_REQUIRE(M < (1ll << 31), "embed_norm: too many rows");
  if (M == 0) return NOISE_OK;
  embed_norm_kernel<false><<<(int)((M + 3) / 4), 256, 0, (hipStream_t)stream>>>(
      table, ld_table, vocab, idx, idx_stride, T, (int)M, sign, a, lda, b, ldb, member_shift, x0, x,
      noise_mixnorm_t{});
  return noise::check_launch("embed_norm");
}

extern "C" int noise_embed_mix_norm(const float* table, int64_t ld_table, int vocab, int d,
                                    const int64_t* idx, int64_t idx_stride, int T, int members,
                                    const float* sign, const float* a, int64_t lda, const float* b, int64_t ldb,
                                    int member_shift, float* x0, const noise_mixnorm_t* next, void* stream) {
  NOISE_REQUIRE(next, "embed_mix_norm: null mix_norm record");
  const noise_mixnorm_t& g = *next;
  NOISE_REQUIRE(g.x && g.h && g.x0 == x0 && g.T == T && (int64_t)g.M == (int64_t)members * T,
                "embed_mix_norm: the mix_norm must mix with this x0 over the same members * T rows");
  // the same checks as the two launches it replaces
  int rc = noise_embed_norm(table, ld_table, vocab, d, idx, idx_stride, T, 0, sign, a, lda, b, ldb, member_shift,
                            x0, nullptr, stream);
  if (rc != NOISE_OK) return rc;
  noise_mixnorm_t empty = g;
  empty.M = 0;
  rc = noise_mix_norm(&empty, stream);
  if (rc != NOISE_OK) return rc;
  const int64_t M = (int64_t)members * T;
  NOISE_REQUIRE(M < (1ll << 31), "embed_mix_norm: too many rows");
  if (M == 0) return NOISE_OK;
  embed_norm_kernel<true><<<(int)((M + 3) / 4), 256, 0, (hipStream_t)stream>>>(
      table, ld_table, vocab, idx, idx_stride, T, (int)M, sign, a, lda, b, ldb, member_shift, x0, nullptr, g);
  return noise::check_launch("embed_mix_norm");
}

extern "C" int noise_mix_norm(const noise_mixnorm_t* args, void* stream) {
  NOISE_REQUIRE(args && args->x && args->h && args->M >= 0 && args->T > 0, "mix_norm: bad arguments");
  const noise_mixnorm_t& g = *args;
  NOISE_REQUIRE(g.nb >= 0 && g.nb <= 3, "mix_norm: nb=%d out of range", g.nb);
  NOISE_REQUIRE(g.nb == 0 || (g.u && g.ldb >= D && g.ldb % 4 == 0 && g.ldu >= g.nb),
                "mix_norm: dots need u, ldb >= 512 (multiple of 4) and ldu >= nb");
  for (int j = 0; j < g.nb; ++j) NOISE_REQUIRE(g.b[j], "mix_norm: null b[%d]", j);
  NOISE_REQUIRE(!g.x0 || (g.resid && g.mix), "mix_norm: mixing needs the lambda scalars");
  NOISE_REQUIRE(!(g.x0 && g.sign) || (g.eps_resid && g.eps_mix), "mix_norm: perturbed mixing needs eps");
  NOISE_REQUIRE(!g.gate_w || (g.gate && (!g.sign || (g.gate_a && g.gate_b && g.ld_gate_b % 4 == 0))),
                "mix_norm: gate needs output and perturbation vectors");
  NOISE_REQUIRE(((uintptr_t)g.gain % 16) == 0, "mix_norm: gain must be 16-byte aligned");
  if (g.M == 0) return NOISE_OK;
  mix_norm_kernel<<<(g.M + 3) / 4, 256, 0, (hipStream_t)stream>>>(g);
  return noise::check_launch("mix_norm");
}

extern "C" int noise_rope_norm_ve(const noise_rope_t* args, void* stream) {
  NOISE_REQUIRE(args && args->qkv && args->out && args->cos && args->sin && args->M >= 0 && args->T > 0,
                "rope_norm_ve: bad arguments");
  const noise_rope_t& g = *args;
  NOISE_REQUIRE(!g.gate || (g.ve_table && g.idx && g.vocab > 0), "rope_norm_ve: gate needs the VE table and idx");
  NOISE_REQUIRE(!(g.gate && g.sign) || (g.ve_a && g.ve_b && g.ld_ve_b % 4 == 0),
                "rope_norm_ve: perturbed VE needs a and b");
  if (g.M == 0) return NOISE_OK;
  rope_norm_ve_kernel<<<(g.M + 3) / 4, 256, 0, (hipStream_t)stream>>>(g);
  return noise::check_launch("rope_norm_ve");
}
