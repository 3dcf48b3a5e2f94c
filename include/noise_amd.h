/* libnoise_amd -- C ABI of the MI355X (gfx950) kernels behind Noise's population-perturbed
 * forward pass and its EGGROLL update.
 *
 * Conventions shared by every entry point:
 *  - all pointers are device pointers owned by the caller; the library never frees them;
 *  - bf16 tensors are passed as uint16_t bit patterns, row-major, with explicit row strides
 *    (in elements);
 *  - rows of a population activation are member-major: row = member * T + token;
 *  - `stream` is a hipStream_t passed as an opaque pointer (NULL = the default stream);
 *    launches are asynchronous and nothing synchronises the device;
 *  - the return value is a status (NOISE_OK on success); noise_last_error() describes the
 *    most recent failure of the calling thread.
 *
 * A member p evaluates the weights W + sign[p] * a_p b_p^T of every matrix (a_p in R^out,
 * b_p in R^in; train/val/eggroll.py:56-58), so x (W + s a b^T)^T = x W^T + s (x . b) a^T.
 * The dot products u = x . b are produced by the kernel that writes x (a norm, the attention
 * or the relu^2 epilogue) and consumed by the epilogue of the GEMM that reads x. Perturbation
 * vectors of member p live at row (p >> member_shift) of their arrays: shift 0 for one row per
 * member, 1 for one row per antithetic pair.
 */
#ifndef NOISE_AMD_H
#define NOISE_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NOISE_OK 0
#define NOISE_EINVAL 1     /* shape / argument error (Python: ValueError) */
#define NOISE_EHIP 2       /* HIP runtime error (Python: RuntimeError) */
#define NOISE_ENONFINITE 3 /* non-finite value (Python: FloatingPointError) */

const char* noise_last_error(void);
int noise_abi_version(void); /* 2: noise_mixnorm_t.gain */

/* ---- rank-1 perturbation of a GEMM's output columns ---------------------------------- */
typedef struct {
  const float* sign;    /* [members] +-sigma; NULL = unperturbed (no rank-1 term) */
  int rows_per_member;  /* T: row r belongs to member r / T */
  int member_shift;     /* noise row of member p = p >> member_shift */
  int seg_cols;         /* output columns per segment (a multiple of 128) */
  int nseg;             /* 1..3 segments side by side (e.g. q | k | v) */
  int u_parts;          /* u of a row = sum of u_parts consecutive floats */
  int64_t lda;          /* row stride of every a[s] (floats) */
  int64_t ldu;          /* row stride of every u[s] (floats) */
  const float* a[3];    /* segment s: a [noise rows, seg_cols] */
  const float* u[3];    /* segment s: u [M, ...], the dots x . b of the GEMM input rows */
} noise_rank1_t;

#define NOISE_EPI_BF16 0       /* C (bf16)  = A W^T + rank-1 */
#define NOISE_EPI_F32 1        /* C (fp32)  = A W^T + rank-1 */
#define NOISE_EPI_ADD_F32 2    /* C (fp32) += A W^T + rank-1          (residual add) */
#define NOISE_EPI_RELU2_BF16 3 /* C (bf16)  = relu(A W^T + rank-1)^2, and
                                  u_next[r, c / 64] = sum over that 64-column group of
                                  bf16(C[r, c]) * b_next[member(r), c] */

/* x W^T + sign (x . b) a^T for A [M, K] bf16 and W [N, K] bf16 (the bf16 weight copy).
 * Replaces `lowrank` (train/val/eggroll.py:56-58) together with the ops fused around it:
 * the residual adds of eggroll.py:92-93 (NOISE_EPI_ADD_F32) and the relu^2 of eggroll.py:93
 * (NOISE_EPI_RELU2_BF16). Requires N % 128 == 0 and K % 64 == 0. */
int noise_lowrank_gemm(const uint16_t* A, int64_t lda, const uint16_t* W, int64_t ldw,
                       int M, int N, int K, const noise_rank1_t* r1, int mode,
                       void* C, int64_t ldc, const float* b_next, int64_t ld_bnext,
                       float* u_next, int64_t ld_unext, void* stream);

/* ---- fused relu^2 MLP -------------------------------------------------------------------- */
#define NOISE_MLP_NORM 1     /* h = bf16(norm(in)) (RMSNorm, no gain); else h = bf16(in) */
#define NOISE_MLP_RESIDUAL 2 /* out = in + mlp(h); else out = mlp(h) */
typedef struct {
  const float* in;           /* fp32 [*, 512]: row t of member p at in + p*member_stride_in + t*ld_in */
  int64_t ld_in, member_stride_in; /* member_stride_in 0: one set of rows shared by every member */
  float* out;                /* fp32 [*, 512], indexed alike with ld_out / member_stride_out; may be in
                                (then with the same strides); members' rows must not overlap */
  int64_t ld_out, member_stride_out;
  int T, members, flags;
  const uint16_t* w_fc;      /* mlp.c_fc.weight as packed by noise_mlp_pack */
  const uint16_t* w_proj;    /* mlp.c_proj.weight as packed by noise_mlp_pack */
  const float* sign;         /* [members] +-sigma; NULL = unperturbed */
  int member_shift;          /* noise row of member p = p >> member_shift */
  const float* a_fc;         /* [noise rows, 2048] (c_fc out) */
  int64_t ld_a_fc;
  const float* b_fc;         /* [noise rows, 512] (c_fc in) */
  int64_t ld_b_fc;
  const float* a_proj;       /* [noise rows, 512] (c_proj out) */
  int64_t ld_a_proj;
  const float* b_proj;       /* [noise rows, 2048] (c_proj in) */
  int64_t ld_b_proj;
  /* Optional (NULL = none): the next layer's residual mixing + norm + dots, run on the finished
   * rows in the epilogue, as noise_mix_norm would run them on `out` afterwards. Needs flags
   * NORM | RESIDUAL, next->x == out, next->M == members * T with out contiguous
   * (ld_out 512, member_stride_out T * 512), and next->h 16-byte aligned. */
  const struct noise_mixnorm_s* next;
  /* Optional (attn_y NULL = none): the attention c_proj first, on the input rows:
   * in + attn_y attn_w^T + sign (sum of attn_u's parts) attn_a^T, then the MLP on that (flags
   * NORM | RESIDUAL). attn_y: bf16 [members * T, >= 512], row p * T + t; attn_w: the bf16 copy of
   * attn.c_proj.weight [512 out, 512 in]; attn_u: [rows, >= attn_parts] per-head y . b dots;
   * attn_a: [noise rows, 512]. */
  const uint16_t* attn_y;
  int64_t ld_attn_y;
  const uint16_t* attn_w;
  const float* attn_u;
  int64_t ld_attn_u;
  int attn_parts;
  const float* attn_a;
  int64_t ld_attn_a;
} noise_mlp_t;

/* out = [in +] c_proj(relu(c_fc(h) + rank-1)^2) + rank-1 in one launch, the [rows, 2048] hidden
 * kept on chip: replaces `x + lowrank(c_proj, relu(lowrank(c_fc, norm(x)))^2)`
 * (train/val/eggroll.py:93 with `lowrank` eggroll.py:56-58; utils/model.py:100-107). Cast points:
 * h and the relu^2 hidden are rounded to bf16 (GEMM operands), the rank-1 dots use those rounded
 * values with fp32 b, everything else is fp32. in, w_fc, w_proj and the noise rows must be
 * 16-byte aligned (leading dimensions multiples of 4 floats). */
int noise_mlp_fused(const noise_mlp_t* args, void* stream);

/* Packs the MLP weights into the bf16 operand layouts noise_mlp_fused reads (each 2 MiB, 16-byte
 * aligned; either pair of pointers may be NULL): mlp.c_fc.weight (fp32 [2048, ld_fc >= 512]) as
 * [2048][512] and mlp.c_proj.weight (fp32 [512, ld_proj >= 2048]) as [64 chunks][512][32], both
 * with every 16-deep k-step in the order the fused kernel's MFMA accumulators deliver it. No
 * counterpart in the reference: the weight-copy step of the bf16 GEMMs (autocast, eggroll.py:144). */
int noise_mlp_pack(const float* w_fc, int64_t ld_fc, const float* w_proj, int64_t ld_proj,
                   uint16_t* fc_packed, uint16_t* proj_packed, void* stream);

/* ---- embedding ------------------------------------------------------------------------ */
/* x0[p*T + t] = norm(W[i] + sign[p] a_p[i] b_p) with i = idx[p*idx_stride + t] (idx_stride 0:
 * one sequence shared by every member), fp32 [members*T, d]; x (if not NULL) receives a copy.
 * An id outside [0, vocab) yields a NaN row. Replaces `lowrank_embed` + `norm` (train/val/eggroll.py:61-63, 74;
 * utils/model.py:46-47). d must be 512. */
int noise_embed_norm(const float* table, int64_t ld_table, int vocab, int d,
                     const int64_t* idx, int64_t idx_stride, int T, int members, const float* sign,
                     const float* a, int64_t lda, const float* b, int64_t ldb, int member_shift,
                     float* x0, float* x, void* stream);

struct noise_mixnorm_s;
/* noise_embed_norm followed by the first layer's noise_mix_norm in one launch, on the rows still in
 * registers: `next` mixes with this x0 (next->x0 == x0) over the same members * T rows and writes
 * the stream next->x, h, the dots and the gate (the plain copy x of noise_embed_norm is not
 * written). Replaces eggroll.py:74 (`x = x0 = norm(lowrank_embed(...))`) together with the first
 * iteration of eggroll.py:77-81, 88. */
int noise_embed_mix_norm(const float* table, int64_t ld_table, int vocab, int d,
                         const int64_t* idx, int64_t idx_stride, int T, int members, const float* sign,
                         const float* a, int64_t lda, const float* b, int64_t ldb, int member_shift,
                         float* x0, const struct noise_mixnorm_s* next, void* stream);

/* ---- residual mixing + RMSNorm + the dots of the consuming GEMMs ------------------------ */
typedef struct noise_mixnorm_s {
  float* x;             /* [M, 512] fp32 stream (updated in place when mixing) */
  const float* x0;      /* [M, 512] fp32 normalised embedding; NULL = no mixing */
  int M, T, member_shift;
  const float* sign;    /* [members]; NULL = unperturbed */
  const float* resid;   /* device scalar lambda_r[i] (resid_lambdas + i) */
  const float* mix;     /* device scalar lambda_0[i] (x0_lambdas + i) */
  const float* eps_resid; /* eps of resid_lambdas at layer i: eps_resid[(p>>shift)*ld_eps] */
  const float* eps_mix;
  int64_t ld_eps;
  uint16_t* h;          /* out: bf16(norm(x)) [M, 512] */
  int nb;               /* 0..3 vectors b to dot with bf16(h) */
  const float* b[3];    /* b[j]: [noise rows, 512] */
  int64_t ldb;
  float* u;             /* out: u[r * ldu + j] = bf16(h_r) . b_j */
  int64_t ldu;
  const float* gate_w;  /* ve_gate W [8, 32] fp32, NULL = no gate */
  const float* gate_a;  /* [noise rows, 8] */
  const float* gate_b;  /* [noise rows, 32] */
  int64_t ld_gate_a, ld_gate_b;
  float* gate;          /* out: 2 sigmoid(h[:32] (Wg + s a b^T)^T) [M, 8] */
  const float* gain;    /* [512] RMSNorm gain: h = bf16(norm(x) * gain) (F.rms_norm's weight);
                           NULL = none, as the reference's `norm` (utils/model.py:46-47) */
} noise_mixnorm_t;

/* Replaces the per-layer mixing (train/val/eggroll.py:77-79), `norm` (eggroll.py:81, 93, 94),
 * the x @ b halves of `lowrank` (eggroll.py:58) and the value-embedding gate
 * (eggroll.py:88; utils/model.py:89). */
int noise_mix_norm(const noise_mixnorm_t* args, void* stream);

/* ---- rotary + q/k RMSNorm + value embedding --------------------------------------------- */
typedef struct {
  const float* qkv;     /* [M, 1536] fp32: q | k | v from noise_lowrank_gemm */
  uint16_t* out;        /* [M, 1536] bf16: norm(rot(q)) | norm(rot(k)) | v + gate * ve */
  int M, T, member_shift;
  const float* cos;     /* [T, 32] fp32 holding the bf16 rotary table values */
  const float* sin;
  const float* gate;    /* [M, 8] or NULL (no value embedding at this layer) */
  const float* ve_table; /* [vocab, 512] fp32 */
  const int64_t* idx;   /* token of row p*T + t: idx[p * idx_stride + t] */
  int64_t idx_stride;
  int vocab;
  const float* sign;
  const float* ve_a;    /* [noise rows, vocab] */
  const float* ve_b;    /* [noise rows, 512] */
  int64_t ld_ve_a, ld_ve_b;
} noise_rope_t;

/* Replaces apply_rotary_emb + norm on q, k (utils/model.py:55-58; eggroll.py:90) and
 * v + gate * lowrank_embed(value_embeds) (eggroll.py:85-89). */
int noise_rope_norm_ve(const noise_rope_t* args, void* stream);

/* The q|k|v projection with noise_rope_norm_ve fused into its epilogue, without the fp32
 * intermediate: rope->out [M, 1536] bf16 = rope_norm_ve(A W^T + rank-1) for W = [Wq; Wk; Wv]
 * [1536, K] bf16 and the three rank-1 segments of r1 (512 columns each). Replaces `lowrank`
 * (train/val/eggroll.py:56-58) for c_q, c_k, c_v together with apply_rotary_emb + norm
 * (utils/model.py:55-58; eggroll.py:90) and the value-embedding add (eggroll.py:85-89).
 * rope->qkv is not read; rope->M must equal M; r1->rows_per_member must equal rope->T; with a
 * value embedding, ve_table and ve_b are 16-byte aligned and ld_ve_b is a multiple of 4. */
int noise_qkv_rope_gemm(const uint16_t* A, int64_t lda, const uint16_t* W, int64_t ldw, int M, int K,
                        const noise_rank1_t* r1, const noise_rope_t* rope, void* stream);

/* ---- windowed causal attention ---------------------------------------------------------- */
typedef struct {
  const uint16_t* qkv;  /* [M, ldqkv] bf16, q at column 0, k at 512, v at 1024 (head h at h*64) */
  int64_t ldqkv;
  uint16_t* y;          /* out [M, 512] bf16 */
  int members, T, heads, window;
  float scale;          /* 1/sqrt(64); must lie in (0, 0.25] */
  const float* b_proj;  /* c_proj b [noise rows, 512] or NULL: u_proj[r*8 + h] = y_h . b_h */
  int64_t ld_b_proj;
  int member_shift;
  float* u_proj;        /* [M, heads] */
  float* moments;       /* NULL or [members, heads, 2, 64]: mean over t of y and y^2 */
  float* scratch;       /* moments partials: [members*heads*ceil(T/256), 2, 64] floats */
} noise_attention_t;

/* Softmax(q k^T * scale) v over keys s - window .. s (utils/model.py:17-31; eggroll.py:91),
 * plus the per-(member, head) first and second moments of the output over tokens. The softmax is
 * shifted by the constant 64 * scale rather than a running maximum: exact (up to bf16 rounding of
 * the probabilities) for scores -80 < q.k * scale < 96, which unit-rms and N(0, 1) rows satisfy. */
int noise_window_attention(const noise_attention_t* args, void* stream);

/* ---- RMSNorm'd hidden -> perturbed fp32 head -> soft-cap -> cross-entropy --------------- */
typedef struct {
  const uint16_t* h;     /* [M, 512] bf16 norm(x) */
  const uint16_t* w_hi;  /* [V, 512] bf16(W) */
  const uint16_t* w_lo;  /* [V, 512] bf16(W - bf16(W)): W ~ w_hi + w_lo to ~2^-17; NULL = the
                            bf16 head alone (the reference trainer's autocast product) */
  int M, V, T, member_shift;
  const float* sign;
  const float* a;        /* [noise rows, V] */
  int64_t lda;
  const float* u;        /* [M] h . b */
  const int64_t* targets; /* target of row p*T + t: targets[p * targets_stride + t] */
  int64_t targets_stride;
  float* ce;             /* out [M] per-token cross-entropy */
  int64_t ignore_index;  /* a row whose target equals this gets ce = 0 (F.cross_entropy's
                            ignore_index: -100 by default, -1 in GPT.forward); any other target
                            outside [0, V) gives ce = NaN */
  float* logits;         /* NULL, or out [M, ld_logits] fp32: the capped logits 15 tanh(z / 15) */
  int64_t ld_logits;     /* >= V */
} noise_head_t;

/* logits = h (W + s a b^T)^T in fp32 accuracy, 15 tanh(logits / 15), cross-entropy against
 * the target (train/val/eggroll.py:94-102; utils/model.py:203-209), and, when `logits` is set,
 * the capped logits themselves (utils/model.py:203-204, 210). V % 64 == 0; V % 256 == 0 as well
 * unless T and M are multiples of 256, V <= 4096, a has 16-byte aligned rows and no logits are
 * asked for (the shape of the population step, taken by a row-resident kernel). */
int noise_head_ce(const noise_head_t* args, void* stream);

/* out[p] = mean over t of ce[p*T + t] (eggroll.py:102). */
int noise_member_mean(const float* ce, int members, int T, float* out, void* stream);

/* ---- EGGROLL update -------------------------------------------------------------------- */
/* The perturbation rows of n pairs, gathered from the shared noise buffer (train/val/eggroll.py:
 * 122-128, `Eggroll.noise`: buffer[offsets[name][directions] + arange(sum(shape))]): for every
 * row d < n and parameter k < nparams, out[d * ld_out + starts[k] + i] = buffer[o + min(i,
 * widths[k] - 1)] for i < widths[k] rounded up to 4, o = offsets[k * ld_offsets + directions[d]]
 * (the int64 [nparams, >= pairs] table of `Eggroll.offsets`, eggroll.py:116-120). widths and
 * starts are host arrays (nparams <= 64; starts 4-aligned, increasing, disjoint); out 16-byte
 * aligned with ld_out % 4 == 0. A direction outside [0, pairs) or a slice outside the buffer gives
 * NaN columns. */
int noise_pair_gather(const float* buffer, int64_t buffer_len, const int64_t* offsets, int64_t ld_offsets,
                      int64_t pairs, const int64_t* directions, int n, int nparams, const int* widths,
                      const int* starts, float* out, int64_t ld_out, void* stream);

/* f_j = L[2j+1] - L[2j], f /= (std(f) + 1e-8) (unbiased std), weight[i] = sum_{j = i mod pairs}
 * f_j (train/val/eggroll.py:151-154). n_losses even; weight [pairs]. Raises NOISE_ENONFINITE
 * through *status_out (device int) if a loss is not finite. */
int noise_fitness(const float* losses, int n_losses, int pairs, float* weight,
                  int* status_out, void* stream);

/* The rank-normalised variant of noise_fitness: f_j = L[2j+1] - L[2j] replaced by its centred rank
 * ranked[j] = rank(f_j) / (n - 1) - 0.5 (n = n_losses / 2; rank = position in a stable ascending sort:
 * ties keep index order, NaN after every number, as torch.argsort(stable=True)), then
 * weight[i] = sum over j = i mod pairs of ranked[j] in ascending j. Extends the z-score of
 * train/val/eggroll.py:151-154 (config 4's "rank-normalised fitness"). ranked: [n] fp32 output. */
int noise_fitness_ranks(const float* losses, int n_losses, int pairs, float* weight, float* ranked,
                        int* status_out, void* stream);

/* G[o, i] (+)= scale * sum_j w[j] a_j[o] b_j[i], with a_j = a_base + a_off[j],
 * b_j = b_base + b_off[j] (train/val/eggroll.py:155-163 with scale = -1/n; a vector
 * parameter is out = L, in = 1 with b_j = 1 when b_base is NULL). */
int noise_es_gradient(const float* w, int n, const float* a_base, const int64_t* a_off,
                      const float* b_base, const int64_t* b_off, int out, int in, float scale,
                      int accumulate, float* G, float* work, int64_t work_elems, void* stream);

/* The gradients of up to 64 parameters in one launch (train/val/eggroll.py:155-163: the loop over
 * every parameter of the model, scale = -1/n). Parameter k, shape [outs[k], ins[k]] (ins[k] == 1
 * for a vector), takes pair j's noise from the slice buffer[o .. o + outs[k] + ins[k]) with
 * o = offsets[k * ld_offsets + j] (the reference's noise(), eggroll.py:122-128): a_j is its first
 * outs[k] values, b_j the next ins[k] (b_j = 1 for a vector), and
 * grads[k][o, i] = scale * sum_j w_j a_j[o] b_j[i] (+= with accumulate). One pass over the pairs
 * per 64 x 64 tile: each parameter's result is bit-identical to noise_es_gradient's with no
 * workspace. A slice outside the buffer makes its pair's terms NaN. outs, ins and grads are host
 * arrays of nparams entries (grads: device pointers, row-major [outs[k], ins[k]]). */
int noise_es_gradient_params(const float* w, int n, const float* buffer, int64_t buffer_len,
                             const int64_t* offsets, int64_t ld_offsets, int nparams, const int* outs,
                             const int* ins, float* const* grads, float scale, int accumulate,
                             void* stream);

/* Floats of `work` with which noise_es_gradient splits the pair sum over more workgroups (a
 * fixed split and a fixed-order reduction: the same result on every call); with less (or NULL)
 * it makes one pass over every pair. No counterpart in the reference: workspace sizing. */
int64_t noise_es_gradient_work(int n, int out, int in);

/* noise_es_gradient for callers that cannot allocate (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc); no counterpart in the reference. The split pair sum keeps its
 * partial tiles in a fixed array the library holds on each device until the process ends
 * (noise_es_gradient_noalloc_capacity() floats, 32 MiB: enough for 1536 pairs of a [4096, 512]
 * gradient); a call that would need more returns NOISE_EINVAL. Same kernels, split and result as
 * noise_es_gradient with a large enough workspace. No allocation and no HIP call besides the
 * launches (the first call on a device looks the array's address up once). Calls on one device
 * share the array: calls that overlap in time on one GPU (different streams) race. The calling
 * thread's current device must be the stream's device. */
int noise_es_gradient_noalloc(const float* w, int n, const float* a_base, const int64_t* a_off,
                              const float* b_base, const int64_t* b_off, int out, int in, float scale,
                              int accumulate, float* G, void* stream);
int64_t noise_es_gradient_noalloc_capacity(void);

/* AdamW over a flat fp32 buffer (torch.optim.AdamW semantics, eggroll.py:164-167, 205):
 * param *= 1 - lr wd; m = lerp(m, g, 1 - b1); v = b2 v + (1 - b2) g^2;
 * param -= lr / (1 - b1^t) * m / (sqrt(v) / sqrt(1 - b2^t) + eps). */
int noise_adamw(float* param, const float* grad, float* exp_avg, float* exp_avg_sq, int64_t n,
                float lr, float beta1, float beta2, float eps, float weight_decay, int step,
                void* stream);

/* noise_adamw that leaves param, exp_avg and exp_avg_sq untouched when *status != NOISE_OK
 * (status: a device int, such as the one noise_fitness writes), read on the device, so the update
 * can be queued before the status is read back. No counterpart in the reference, whose step has
 * no non-finite check. */
int noise_adamw_unless(float* param, const float* grad, float* exp_avg, float* exp_avg_sq, int64_t n,
                       float lr, float beta1, float beta2, float eps, float weight_decay, int step,
                       const int* status, void* stream);

/* bf16 copy of an fp32 buffer (hi), and optionally the residual bf16(x - hi) (lo). */
int noise_cast_bf16(const float* x, int64_t n, uint16_t* hi, uint16_t* lo, void* stream);

/* noise_cast_bf16 over `count` (<= 64) buffers in one launch: hi[k][i] = bf16(x[k][i]) and, where lo
 * and lo[k] are non-NULL, lo[k][i] = bf16(x[k][i] - hi[k][i]), for i < n[k]. x, n, hi, lo are host
 * arrays of device pointers / sizes. Bit-identical to one noise_cast_bf16 per buffer. No
 * counterpart in the reference: the bf16 weight copies its autocast forms inside each product. */
int noise_cast_bf16_many(int count, const float* const* x, const int64_t* n, uint16_t* const* hi,
                         uint16_t* const* lo, void* stream);

/* ---- Soft-capped log-sum-exp probes of the readout head ----------------------------------
 * cap(v) = 15 tanh(v / 15). A target y < 0 masks its token (output 0); a target >= V makes the
 * token's outputs NaN (the reference's gather would fault). */

/* out[i, v] = (CE(cap(raw_i + sigma e_v), y_i) - CE(cap(raw_i - sigma e_v), y_i)) / (2 sigma),
 * in the closed form log1p(w_v expm1(cap(raw_v +- sigma) - cap(raw_v))) with the target
 * correction (train/val/run.py:100-111; train/speedrun/run.py:57-68). raw is fp32 or, with
 * raw_is_bf16, bf16 bit patterns; rows of V elements at stride ld_raw; out fp32 [n, ld_out]. */
int noise_coordinate_differences(const void* raw, int raw_is_bf16, int64_t ld_raw, const int64_t* y,
                                 int n, int V, float sigma, float* out, int64_t ld_out, void* stream);

typedef struct {
  const float* base;      /* [n, V] W x of the clean streams, row stride ld_base */
  int64_t ld_base;
  const float* C;         /* [P, V] row j = W D_j, row stride ld_C */
  int64_t ld_C;
  const int64_t* rows;    /* row_derivatives: [n, K] indices into C's rows (stride ld_rows) */
  int64_t ld_rows;
  const int64_t* y;       /* [n] targets */
  const float* steps;     /* [n] step of each token's moves */
  const float* sq;        /* [n] |x|^2 */
  const float* dots;      /* [n, P] (cycle) or [n, K] (rows): x . D, row stride ld_dots */
  int64_t ld_dots;
  const float* dir_sq;    /* [P] (cycle) or [n, K] with row stride ld_dir_sq (rows): |D|^2 */
  int64_t ld_dir_sq;
  int n, P, K, V;
  int width;              /* the stream width the RMS norm divides |x|^2 by */
  float* clean_sum;       /* workspace [n]: sum_v exp(cap(z0_v) - 15) of each clean token */
  float* out;             /* [n, P] (cycle) or [n, K] (rows), row stride ld_out */
  int64_t ld_out;
} noise_probe_t;

/* Forward differences of each token's readout loss along every direction of a cycle:
 * inv = rsqrt((sq + 2 s dots_j + s^2 dir_sq_j) / width + eps), z = (base + s C_j) inv,
 * out[i, j] = (LSE(cap(z)) - cap(z_y) - clean_i) / s_i (train/val/run.py:154-167;
 * train/speedrun/run.py:90-103). Two launches on `stream`: the clean sums, then the probes. */
int noise_cycle_derivatives(const noise_probe_t* args, void* stream);

/* The same along each token's own rows of C: direction k of token i is C[rows[i, k]]
 * (train/val/run.py:170-183). A row index outside [0, P) makes that output NaN. */
int noise_row_derivatives(const noise_probe_t* args, void* stream);

/* ---- Chain moves with every attention held (chain_chunk, train/val/run.py:307-351, own = None)
 * Rows are (token i, move p) pairs, row = i * P + p, W wide. */

/* dx0 = norm(e_i + move_row) - x0_i, delta = mix * dx0 (run.py:324-326; mix = lam_r[0] + lam_0[0]). */
int noise_chain_start(const float* e, const float* x0, const float* move, int m, int P, int W,
                      float mix, float* dx0, float* delta, void* stream);

typedef struct {
  float* delta;            /* [m * P, W] moves, updated in place */
  const float* dx0;        /* NULL, or [m * P, W] moves of x0 (site < 0) */
  int mix;                 /* first delta = lam_r delta + lam_0 dx0 (every block after the first) */
  float lam_r, lam_0;
  const float* mid;        /* [m, W] the block's clean mid stream */
  const int64_t* idx;      /* [m, ld_idx] routed units of each token, in [0, H) (else NaN) */
  int64_t ld_idx;
  const float* hs;         /* [m, ld_hs] their clean pre-activations */
  int64_t ld_hs;
  const uint16_t* w_fc;    /* [H, W] bf16 c_fc.weight (16-byte aligned) */
  const uint16_t* w_out_t; /* [H, W] bf16 c_proj.weight transposed (16-byte aligned) */
  int m, P, W, k, H;       /* W % 256 == 0, W <= 2048, k % 128 == 0 */
  uint16_t* dz;            /* workspace [m * P, W] bf16 (16-byte aligned, as the next three) */
  uint16_t* wf;            /* workspace [m, k, W] bf16 */
  uint16_t* wo;            /* workspace [m, W, k] bf16 */
  uint16_t* g;             /* workspace [m * P, k] bf16 */
} noise_chain_block_t;

/* One block of the chain (run.py:327-350): the optional mix, dz = norm_difference(mid, delta) in
 * bf16, dh = bf16(dz W_fc[idx]^T), g = bf16((relu(h + dh) - relu(h))(relu(h + dh) + relu(h))),
 * delta += bf16(g W_out_t[idx]). */
int noise_chain_block(const noise_chain_block_t* args, void* stream);

typedef struct {
  float* delta;            /* [m * P, W] moves at the block's input, updated in place */
  const float* dx0;        /* NULL, or [m * P, W] moves of x0 (site < 0) */
  int mix;                 /* first delta = lam_r delta + lam_0 dx0 (then call noise_chain_block with mix 0) */
  float lam_r, lam_0;
  const float* x;          /* [m, W] the block's clean input stream */
  const int64_t* pos;      /* [m] positions, in [0, T) (else NaN) */
  const float* w_q;        /* [W, W] fp32 c_q.weight */
  const uint16_t* top_keys;   /* [m, heads, K, 64] bf16 rotated, normed keys */
  const uint16_t* top_values; /* [m, heads, K, 64] bf16 values */
  const float* top_p;      /* [m, heads, K] their clean probabilities */
  const float* rest;       /* [m, heads, 64] the held keys' share of the clean output */
  const float* w_proj_t;   /* [W, W] fp32 c_proj.weight transposed */
  const float* cos_t;      /* [T, 32] rotary tables */
  const float* sin_t;
  int T, m, P, W, heads, K; /* W = 64 heads, W % 256 == 0, W <= 2048, 1 <= K <= 64 */
  uint16_t* a3;            /* workspace [m * P + m, 3 W] bf16 (16-byte aligned, as the next three) */
  float* dr;               /* workspace [m * P + m, W] fp32 */
  uint16_t* wq3;           /* workspace [W, 3 W] bf16 */
  uint16_t* wp3;           /* workspace [W, 3 W] bf16 */
} noise_chain_query_t;

/* The own-query step of a block (run.py:284-304 and 326-331, own = ('routed', ...)): the optional
 * mix, then delta += (change of the token's attention output when its query moves with its
 * input stream and only its top keys' logits move) c_proj^T. Replaces query_change_routed; the
 * two fp32 products run as three bf16 MFMA products each (hi/lo halves). */
int noise_chain_query(const noise_chain_query_t* args, void* stream);

typedef struct {
  float* delta;            /* [m * P, W] moves at the block's input, updated in place */
  const float* dx0;        /* NULL, or [m * P, W] moves of x0 (site < 0) */
  int mix;                 /* first delta = lam_r delta + lam_0 dx0 (then call noise_chain_block with mix 0) */
  float lam_r, lam_0;
  const float* x;          /* [m, W] the block's clean input stream */
  const int64_t* pos;      /* [m] positions, in [0, T) (else NaN) */
  const int64_t* rel;      /* [m] the same positions within the key window (no allowed key: NaN) */
  const float* w_q;        /* [W, W] fp32 c_q.weight */
  const uint16_t* keys;    /* [heads, S, 64] bf16 rotated, normed keys of the chunk's key window */
  const uint16_t* values;  /* [heads, S, 64] bf16 values */
  const float* w_proj_t;   /* [W, W] fp32 c_proj.weight transposed */
  const float* cos_t;      /* [T, 32] rotary tables */
  const float* sin_t;
  int T, m, P, W, heads, S, window; /* W = 64 heads, W % 256 == 0, W <= 2048, 0 <= window < 4096 */
  uint16_t* a3;            /* workspaces as in noise_chain_query_t */
  float* dr;
  uint16_t* wq3;
  uint16_t* wp3;
} noise_chain_query_window_t;

/* The own-query step with own = ('window', ...) (run.py:256-281 and 332-335): as
 * noise_chain_query, over every key t of the token's window (0 <= rel - t <= window) with the
 * clean softmax p0 computed per token. Replaces query_change. */
int noise_chain_query_window(const noise_chain_query_window_t* args, void* stream);

typedef struct {
  const float* delta;      /* [m * P, W] */
  const float* xL;         /* [m, W] clean top stream */
  const float* base;       /* [m, ld_base] xL W^T */
  int64_t ld_base;
  const uint16_t* weight;  /* [V, W] bf16 head weight (the reference's weight_t transposed) */
  const float* target_w;   /* [m, W] fp32 head rows of the targets */
  const int64_t* y;        /* [m] targets; < 0 masks the token, >= V gives NaN */
  const float* scale;      /* [m, ld_scale] step of each move */
  int64_t ld_scale;
  int m, P, W, V;          /* V % 256 == 0 */
  float* out;              /* [m, ld_out] */
  int64_t ld_out;
  uint16_t* dbf;           /* workspace [m * P, W] bf16 (16-byte aligned) */
  float* inv;              /* workspace [m * P] */
  float* zy;               /* workspace [m * P] */
  float* clean;            /* workspace [2 m] */
} noise_chain_head_t;

/* The head of the chain (run.py:341-351): z = (base + bf16(bf16(delta) W^T)) inv, inv from
 * |xL + delta|, LSE of the capped z over V fused into the head product, the target term in fp32,
 * out = (moved - clean) / scale. */
int noise_chain_head(const noise_chain_head_t* args, void* stream);

#ifdef __cplusplus
}
#endif
#endif
