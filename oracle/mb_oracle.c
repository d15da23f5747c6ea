/*
 * CPU ORACLE for the MOSS-TTS-Nano decoder hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * It checks the HIP library's results; it is never the thing measured or
 * shipped.  Only tests/, __graft_entry__.smoke() and the cpu_baseline leg of
 * bench.py may load it; the product path (the HIP library under mockbird_amd/)
 * never links or calls it.
 *
 * It is a plain-C restatement of the reference's algorithm, written from the
 * reference's CPU restatement and WGSL kernels:
 *   - RoPE + ring write ........ tools/onnx-probe/ref-decode.mjs:111-124,
 *                                src/lib/tts/engine/kernels-decode.ts:216-241,
 *                                kernels-batch.ts:194-234
 *   - wrap / eviction rule ..... kernels-decode.ts:679-714 (slot = pos % C,
 *                                slots[slot] = pos) and :590-667 (live mask)
 *   - decode attention ......... ref-decode.mjs:138-161, kernels-decode.ts:254-327
 *   - causal prefill attention . kernels-batch.ts:246-350, ref-decode.mjs:175-204
 *   - layer / model ............ ref-decode.mjs:85-110 (LN, GEMV, GELU),
 *                                :163-174 (embedRow), :175-234 (prefill,
 *                                decodeStep), :238-286 (localStep, argmax),
 *                                :378-421 (frame loop order)
 *   - greedy rules ............. src/lib/tts/engine/policy.ts:273-302
 *
 * Arithmetic follows ref-decode.mjs: every reduction (dot products, LN
 * moments, softmax) is carried in double (acc_t) and each op's output is stored as
 * fp32, as the JS reference does with Float32Array buffers.  Two places
 * deliberately follow the ONNX graph (the reference's ORT CPU path) instead of
 * the JS restatement, because the reference's own ORT fixture
 * (tests/fixtures/golden/prefill-195rows-layer0-k.f32) fixes them:
 *   - the RoPE angle is the fp32 product float(pos) * inv_freq_f32 with the
 *     fp32 inv_freq table the graph carries, and the rotation is evaluated as
 *     fp32 Mul/Mul/Add (x*cos + rotate_half(x)*sin) with fp32 cos/sin;
 *   - embeddings are summed in fp32 in channel order (ref-decode.mjs:163-174
 *     accumulates into a Float32Array, which rounds every add to fp32).
 *
 * Ring layout in this file is the reference's: per layer and sequence,
 * [slot][head*64 + dim] (prefill.ts:55-56), K and V in separate arrays, plus
 * slot_pos[slot] = absolute position stored in that slot (-1 = empty).
 *
 * Build: oracle/Makefile.  liboracle.so (the checker) is built with
 * -ffp-contract=off: the fp32 RoPE below must not be fused into FMAs.
 *
 * The same source also builds liboracle_fp32.so with -DOR_ACC=float and
 * FMA contraction on: every reduction is then carried in fp32, as ORT's MLAS
 * kernels do.  That build is only the CPU throughput baseline (the stand-in
 * for the reference's ORT-wasm path); it is never used as a checker.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define OR_D 768
#define OR_H 12
#define OR_HD 64
#define OR_QKV 2304
#define OR_FFN 3072
#define OR_NVQ 16
#define OR_ROW 17
#define OR_PAD 1024
#define OR_CODES 1024
#define OR_EPS 1e-5

/* Accumulator type of every dot product, moment and softmax sum. */
#ifndef OR_ACC
#define OR_ACC double
#endif
typedef OR_ACC acc_t;

/* fp32 inverse frequencies 1 / 10000^(2i/64) exactly as the exported graph
 * carries them (the fp32 values torch produces for
 * 1.0 / (10000 ** (arange(0, 64, 2).float() / 64))).  Six entries differ from
 * the correctly rounded value by one ulp; the ORT fixture distinguishes them. */
static const uint32_t OR_INV_FREQ_BITS[32] = {
    0x3f800000u, 0x3f3ff911u, 0x3f0ff59au, 0x3ed7e89bu, 0x3ea1e89bu, 0x3e72d423u,
    0x3e361887u, 0x3e088d77u, 0x3dcccccdu, 0x3d99940du, 0x3d6655c2u, 0x3d2cba15u,
    0x3d0186e3u, 0x3cc2434fu, 0x3c91ad39u, 0x3c5a7bf2u, 0x3c23d70au, 0x3bf5b9b0u,
    0x3bb8449cu, 0x3b8a2e77u, 0x3b4f3e38u, 0x3b1b690du, 0x3ae91528u, 0x3aaec98eu,
    0x3a83126fu, 0x3a44948cu, 0x3a136a16u, 0x39dd1725u, 0x39a5cb60u, 0x3978a815u,
    0x393a7753u, 0x390bd472u};

static float bits_to_f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

void or_inv_freq(float* out) {
  for (int i = 0; i < 32; i++) out[i] = bits_to_f(OR_INV_FREQ_BITS[i]);
}

/* Round an fp32 value to bf16 (round to nearest, ties to even) and return it
 * widened back to fp32. */
float or_bf16_round(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7f800000u) == 0x7f800000u) { /* inf / nan: truncate, keep quiet */
    u &= 0xffff0000u;
    if (x != x) u |= 0x00400000u;
  } else {
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
  }
  float r;
  memcpy(&r, &u, 4);
  return r;
}

void or_bf16_round_array(const float* x, int64_t n, float* out) {
  for (int64_t i = 0; i < n; i++) out[i] = or_bf16_round(x[i]);
}

/* cos/sin of one RoPE pair at an absolute position (fp32 angle, fp32 result). */
static void rope_cs(int64_t pos, int i, float* c, float* s) {
  float a = (float)pos * bits_to_f(OR_INV_FREQ_BITS[i]);
  *c = (float)cos((double)a);
  *s = (float)sin((double)a);
}

/* RoPE over n_heads 64-wide heads (ref-decode.mjs:114-124): pair (2i, 2i+1)
 * shares frequency i; out[2i] = x[2i]*c - x[2i+1]*s, out[2i+1] = x[2i+1]*c + x[2i]*s. */
void or_rope(const float* x, int n_heads, int64_t pos, float* out) {
  for (int i = 0; i < 32; i++) {
    float c, s;
    rope_cs(pos, i, &c, &s);
    for (int h = 0; h < n_heads; h++) {
      const float x0 = x[h * 64 + 2 * i], x1 = x[h * 64 + 2 * i + 1];
      const float a0 = x0 * c, b0 = (-x1) * s;
      const float a1 = x1 * c, b1 = x0 * s;
      out[h * 64 + 2 * i] = a0 + b0;
      out[h * 64 + 2 * i + 1] = a1 + b1;
    }
  }
}

/* ------------------------------------------------------------------ ring */

/* Slot of an absolute position (kernels-decode.ts:709: slot = pos % C).  With
 * wrap == 0 the reference's non-wrapping global ring is modelled instead: the
 * slot IS the position and a position >= C is an error (decode.ts:719-724). */
int or_slot_of(int64_t pos, int C, int wrap) {
  if (pos < 0) return -1;
  if (!wrap) return pos < C ? (int)pos : -1;
  return (int)(pos % C);
}

/* Is a slot holding absolute position `stored` visible to a query at `cur`?
 * kernels-decode.ts:608-611: stored >= 0 && 0 <= cur - stored < C. */
int or_slot_live(int64_t stored, int64_t cur, int C) {
  if (stored < 0) return 0;
  const int64_t d = cur - stored;
  return d >= 0 && d < C;
}

/* Write n[b] consecutive rows of fused qkv (q | k | v, head-major, row stride
 * `qkv_stride` floats) for sequences b in [0, B), starting at absolute
 * position pos0[b], into per-sequence rings ringK/ringV[b][C][768] and
 * slot_pos[b][C].  q is roped into q_out[b][row][768] (row stride 768 * rows_max).
 * kv_bf16 rounds stored K and V to bf16.  Returns 0, or -1 when wrap == 0 and
 * a position does not fit the ring. */
int or_ring_write(int B, int C, int wrap, int kv_bf16, int rows_max, const float* qkv,
                  int64_t qkv_stride, const int32_t* pos0, const int32_t* n, float* q_out,
                  float* ringK, float* ringV, int32_t* slot_pos) {
  for (int b = 0; b < B; b++)
    for (int r = 0; r < n[b]; r++)
      if (or_slot_of((int64_t)pos0[b] + r, C, wrap) < 0) return -1;
  for (int b = 0; b < B; b++) {
    for (int r = 0; r < n[b]; r++) {
      const int64_t pos = (int64_t)pos0[b] + r;
      const int slot = or_slot_of(pos, C, wrap);
      const float* row = qkv + ((int64_t)b * rows_max + r) * qkv_stride;
      float* kd = ringK + ((int64_t)b * C + slot) * OR_D;
      float* vd = ringV + ((int64_t)b * C + slot) * OR_D;
      if (q_out) or_rope(row, OR_H, pos, q_out + ((int64_t)b * rows_max + r) * OR_D);
      or_rope(row + OR_D, OR_H, pos, kd);
      memcpy(vd, row + 2 * OR_D, OR_D * sizeof(float));
      if (kv_bf16)
        for (int i = 0; i < OR_D; i++) {
          kd[i] = or_bf16_round(kd[i]);
          vd[i] = or_bf16_round(vd[i]);
        }
      slot_pos[(int64_t)b * C + slot] = (int32_t)pos;
    }
  }
  return 0;
}

/* One query row against the live slots of a ring, per head (ref-decode.mjs:
 * 138-161 with the live mask of kernels-decode.ts:608-611).  Scale 0.125,
 * reductions in acc_t.  No live slot gives a zero row. */
static void attend_one(const float* q, int64_t cur, int C, const float* K, const float* V,
                       const int32_t* sp, float* out, acc_t* scores) {
  for (int h = 0; h < OR_H; h++) {
    acc_t mx = -INFINITY;
    for (int j = 0; j < C; j++) {
      if (!or_slot_live(sp[j], cur, C)) {
        scores[j] = -INFINITY;
        continue;
      }
      acc_t s = 0;
      const float* kr = K + (int64_t)j * OR_D + h * OR_HD;
      for (int d = 0; d < OR_HD; d++) s += (acc_t)q[h * OR_HD + d] * (acc_t)kr[d];
      scores[j] = s * (acc_t)0.125;
      if (scores[j] > mx) mx = scores[j];
    }
    acc_t sum = 0;
    for (int j = 0; j < C; j++) {
      scores[j] = scores[j] == -INFINITY ? 0 : (acc_t)exp((double)(scores[j] - mx));
      sum += scores[j];
    }
    acc_t acc[OR_HD];
    for (int d = 0; d < OR_HD; d++) acc[d] = 0;
    for (int j = 0; j < C; j++) {
      if (scores[j] == 0) continue;
      const acc_t p = scores[j] / sum;
      const float* vr = V + (int64_t)j * OR_D + h * OR_HD;
      for (int d = 0; d < OR_HD; d++) acc[d] += p * (acc_t)vr[d];
    }
    for (int d = 0; d < OR_HD; d++) out[h * OR_HD + d] = sum > 0 ? (float)acc[d] : 0.0f;
  }
}

/* Decode attention for B sequences: q[b][768] at position pos[b] against ring
 * b.  out[b][768]. */
void or_decode_attention(int B, int C, const float* q, const int32_t* pos, const float* ringK,
                         const float* ringV, const int32_t* slot_pos, float* out) {
#pragma omp parallel
  {
    acc_t* scores = (acc_t*)malloc(sizeof(acc_t) * (size_t)C);
#pragma omp for schedule(dynamic, 1)
    for (int b = 0; b < B; b++)
      attend_one(q + (int64_t)b * OR_D, pos[b], C, ringK + (int64_t)b * C * OR_D,
                 ringV + (int64_t)b * C * OR_D, slot_pos + (int64_t)b * C,
                 out + (int64_t)b * OR_D, scores);
    free(scores);
  }
}

/* Causal prefill attention (kernels-batch.ts:246-350): roped queries
 * q[b][r][768] (row stride 768, rows_max rows per sequence) at positions
 * pos0[b] + r, r < n[b], each attending the ring's live slots at or before its
 * own position.  The ring already holds all n[b] rows (the reference writes
 * the whole prompt's K/V before scoring).  out[b][r][768]. */
void or_prefill_attention(int B, int C, int rows_max, const float* q, const int32_t* pos0,
                          const int32_t* n, const float* ringK, const float* ringV,
                          const int32_t* slot_pos, float* out) {
  const int64_t total = (int64_t)B * rows_max;
#pragma omp parallel
  {
    acc_t* scores = (acc_t*)malloc(sizeof(acc_t) * (size_t)C);
    int32_t* sp = (int32_t*)malloc(sizeof(int32_t) * (size_t)C);
#pragma omp for schedule(dynamic, 4)
    for (int64_t t = 0; t < total; t++) {
      const int b = (int)(t / rows_max), r = (int)(t % rows_max);
      if (r >= n[b]) continue;
      const int64_t cur = (int64_t)pos0[b] + r;
      /* causal: slots holding a later position than the query are masked */
      for (int j = 0; j < C; j++) {
        const int32_t s = slot_pos[(int64_t)b * C + j];
        sp[j] = (s > cur) ? -1 : s;
      }
      attend_one(q + t * OR_D, cur, C, ringK + (int64_t)b * C * OR_D,
                 ringV + (int64_t)b * C * OR_D, sp, out + t * OR_D, scores);
    }
    free(scores);
    free(sp);
  }
}

/* ---------------------------------------------------------- layer pieces */

/* LayerNorm eps 1e-5 over n features (ref-decode.mjs:85-99). */
void or_layernorm(const float* x, const float* w, const float* b, int n, float* out) {
  acc_t m = 0;
  for (int i = 0; i < n; i++) m += x[i];
  m /= n;
  acc_t v = 0;
  for (int i = 0; i < n; i++) {
    const acc_t d = x[i] - m;
    v += d * d;
  }
  v /= n;
  const acc_t inv = (acc_t)(1.0 / sqrt((double)v + OR_EPS));
  for (int i = 0; i < n; i++)
    out[i] = (float)((x[i] - m) * inv * (w ? (acc_t)w[i] : (acc_t)1) + (b ? (acc_t)b[i] : (acc_t)0));
}

/* Rows [m0, m1) x columns [n0, n1) of y = x W + bias; acc holds n1 - n0. */
static void gemm_block(int K, int N, const float* x, const float* W, const float* bias, float* y,
                       int m0, int m1, int n0, int n1, acc_t* acc) {
  for (int m = m0; m < m1; m++) {
    for (int n = n0; n < n1; n++) acc[n - n0] = bias ? bias[n] : 0;
    const float* xr = x + (int64_t)m * K;
    for (int k = 0; k < K; k++) {
      const acc_t xv = xr[k];
      const float* wr = W + (int64_t)k * N;
      for (int n = n0; n < n1; n++) acc[n - n0] += xv * (acc_t)wr[n];
    }
    for (int n = n0; n < n1; n++) y[(int64_t)m * N + n] = (float)acc[n - n0];
  }
}

/* y[m][n] = bias[n] + sum_k x[m][k] * W[k][n], W [K, N] row-major
 * (ref-decode.mjs:100-108; kernels-batch.ts:156-184), summed over k in order.
 * Threads split the rows, or the columns when there are fewer rows than
 * threads; every output is the same sum either way. */
void or_gemm(int M, int K, int N, const float* x, const float* W, const float* bias, float* y) {
#ifdef _OPENMP
  const int nt = omp_in_parallel() ? 1 : omp_get_max_threads();
#else
  const int nt = 1;
#endif
  if (M >= nt || nt == 1) {
#pragma omp parallel if (nt > 1)
    {
      acc_t* acc = (acc_t*)malloc(sizeof(acc_t) * (size_t)N);
#pragma omp for schedule(static)
      for (int m = 0; m < M; m++) gemm_block(K, N, x, W, bias, y, m, m + 1, 0, N, acc);
      free(acc);
    }
    return;
  }
  const int blk = 256;
  const int nb = (N + blk - 1) / blk;
#pragma omp parallel
  {
    acc_t* acc = (acc_t*)malloc(sizeof(acc_t) * blk);
#pragma omp for schedule(dynamic, 1)
    for (int j = 0; j < nb; j++) {
      const int n0 = j * blk, n1 = n0 + blk < N ? n0 + blk : N;
      gemm_block(K, N, x, W, bias, y, 0, M, n0, n1, acc);
    }
    free(acc);
  }
}

/* GELU, tanh approximation (ref-decode.mjs:109-110; kernels-decode.ts:373-385). */
float or_gelu_tanh(float v) {
  const double x = v;
  return (float)(0.5 * x * (1.0 + tanh(0.7978845608028654 * (x + 0.044715 * x * x * x))));
}

/* ----------------------------------------------------------------- model */

typedef struct {
  const float *ln1_w, *ln1_b, *attn_w, *attn_b, *proj_w, *proj_b;
  const float *ln2_w, *ln2_b, *fc_in_w, *fc_in_b, *fc_out_w, *fc_out_b;
} or_layer;

typedef struct {
  int n_layers, vocab;
  const or_layer* layers;
  const float *lnf_w, *lnf_b;
  const float* wte;                   /* [vocab][768] */
  const float* audio_emb[OR_NVQ];     /* [1024][768] each */
  or_layer local;
  const float *local_lnf_w, *local_lnf_b;
  const float* text_head;             /* [768][vocab] */
  const float* audio_heads[OR_NVQ];   /* [768][1024] each */
  int audio_end_id, assistant_id;     /* 7, 9 */
  double penalty;                     /* 1.2, a JS number in the reference */
  int penalty_f32;                    /* 1: the WGSL engine's f32 penalty arithmetic */
} or_model;

/* Embed one 17-wide row: wte[row[0]] + sum_k audio_k[row[1+k]], pads skipped,
 * accumulated in fp32 in channel order (ref-decode.mjs:163-174,
 * promptRows.ts:21-36). */
void or_embed_row(const or_model* M, const int32_t* row, float* x) {
  for (int j = 0; j < OR_D; j++) x[j] = M->wte[(int64_t)row[0] * OR_D + j];
  for (int k = 0; k < OR_NVQ; k++) {
    const int id = row[k + 1];
    if (id == OR_PAD) continue;
    const float* e = M->audio_emb[k] + (int64_t)id * OR_D;
    for (int j = 0; j < OR_D; j++) x[j] = x[j] + e[j];
  }
}

/* One layer over S rows of one sequence whose K/V ring is (K, V, sp) with
 * capacity C: rows sit at positions pos0 .. pos0+S-1.  hs[S][768] is updated
 * in place (ref-decode.mjs:175-204 per layer; :207-234 is the S == 1 case). */
static int layer_rows(const or_layer* L, int C, int wrap, int kv_bf16, int S, int64_t pos0,
                      float* hs, float* K, float* V, int32_t* sp) {
  float* norm = (float*)calloc((size_t)S * OR_FFN, sizeof(float));
  float* qkv = (float*)malloc(sizeof(float) * (size_t)S * OR_QKV);
  float* q = (float*)malloc(sizeof(float) * (size_t)S * OR_D);
  float* ctx = (float*)malloc(sizeof(float) * (size_t)S * OR_D);
  float* proj = (float*)malloc(sizeof(float) * (size_t)S * OR_FFN);
  int rc = 0;
  for (int i = 0; i < S; i++)
    or_layernorm(hs + (int64_t)i * OR_D, L->ln1_w, L->ln1_b, OR_D, norm + (int64_t)i * OR_D);
  or_gemm(S, OR_D, OR_QKV, norm, L->attn_w, L->attn_b, qkv);
  const int32_t p0 = (int32_t)pos0, nn = S;
  rc = or_ring_write(1, C, wrap, kv_bf16, S, qkv, OR_QKV, &p0, &nn, q, K, V, sp);
  if (rc == 0) {
    or_prefill_attention(1, C, S, q, &p0, &nn, K, V, sp, ctx);
    or_gemm(S, OR_D, OR_D, ctx, L->proj_w, L->proj_b, proj);
    for (int64_t i = 0; i < (int64_t)S * OR_D; i++) hs[i] = hs[i] + proj[i];
    for (int i = 0; i < S; i++)
      or_layernorm(hs + (int64_t)i * OR_D, L->ln2_w, L->ln2_b, OR_D, norm + (int64_t)i * OR_D);
    or_gemm(S, OR_D, OR_FFN, norm, L->fc_in_w, L->fc_in_b, proj);
    for (int64_t i = 0; i < (int64_t)S * OR_FFN; i++) proj[i] = or_gelu_tanh(proj[i]);
    or_gemm(S, OR_FFN, OR_D, proj, L->fc_out_w, L->fc_out_b, norm);
    for (int64_t i = 0; i < (int64_t)S * OR_D; i++) hs[i] = hs[i] + norm[i];
  }
  free(norm);
  free(qkv);
  free(q);
  free(ctx);
  free(proj);
  return rc;
}

/* Global prefill of one sequence: S rows ids[S][17] at positions 0..S-1 into
 * rings K/V[layer][C][768], sp[layer][C].  hidden_out[S][768] receives ln_f of
 * every row (ref-decode.mjs:175-204).  Returns 0 or -1 (ring too small). */
int or_model_prefill(const or_model* M, int C, int wrap, int kv_bf16, int S,
                     const int32_t* ids, float* K, float* V, int32_t* sp, float* hidden_out) {
  if (S < 1 || S > C) return -1; /* the prompt must fit the ring (prefill.ts:136) */
  float* hs = (float*)malloc(sizeof(float) * (size_t)S * OR_D);
  int rc = 0;
  for (int i = 0; i < S; i++) or_embed_row(M, ids + (int64_t)i * OR_ROW, hs + (int64_t)i * OR_D);
  for (int l = 0; l < M->n_layers && rc == 0; l++)
    rc = layer_rows(&M->layers[l], C, wrap, kv_bf16, S, 0, hs, K + (int64_t)l * C * OR_D,
                    V + (int64_t)l * C * OR_D, sp + (int64_t)l * C);
  if (rc == 0)
    for (int i = 0; i < S; i++)
      or_layernorm(hs + (int64_t)i * OR_D, M->lnf_w, M->lnf_b, OR_D, hidden_out + (int64_t)i * OR_D);
  free(hs);
  return rc;
}

/* One global decode step of one sequence: embed row17, run every layer at
 * `pos` (appending K/V), ln_f into hidden[768] (ref-decode.mjs:207-234). */
int or_model_decode_step(const or_model* M, int C, int wrap, int kv_bf16, const int32_t* row17,
                         int pos, float* K, float* V, int32_t* sp, float* hidden) {
  float hs[OR_D];
  int rc = 0;
  or_embed_row(M, row17, hs);
  for (int l = 0; l < M->n_layers && rc == 0; l++)
    rc = layer_rows(&M->layers[l], C, wrap, kv_bf16, 1, pos, hs, K + (int64_t)l * C * OR_D,
                    V + (int64_t)l * C * OR_D, sp + (int64_t)l * C);
  if (rc == 0) or_layernorm(hs, M->lnf_w, M->lnf_b, OR_D, hidden);
  return rc;
}

/* Greedy argmax with the HuggingFace repetition penalty over a 1024-bit seen
 * mask (policy.ts:273-290, ref-decode.mjs:273-286): scores of seen ids are
 * multiplied by the penalty when negative, divided when not; strict '>' so a
 * tie keeps the lowest id.  The penalty and the penalised score are doubles,
 * as in the JS reference (GEN.audio_repetition_penalty is the JS number 1.2,
 * mossTtsRuntime.js:506-521).  Returns the winning id; *best_out / *second_out get the
 * winning and runner-up penalised scores (for margin reports). */
int or_argmax_penalty_prec(const float* logits, int n, const uint32_t* seen, double penalty,
                           int f32, double* best_out, double* second_out) {
  int any = 0;
  for (int w = 0; w < (n + 31) / 32; w++) any |= seen[w] != 0;
  const int apply = any && penalty != 1.0;
  const float pf = (float)penalty;
  int best = 0;
  double bv = -INFINITY, sv = -INFINITY;
  for (int i = 0; i < n; i++) {
    double s = logits[i];
    if (apply && ((seen[i >> 5] >> (i & 31)) & 1u)) {
      if (f32) { /* ARGMAX_PENALTY, kernels-decode.ts:454-461: f32 penalty and arithmetic */
        const float x = logits[i];
        s = x < 0.0f ? (double)(x * pf) : (double)(x / pf);
      } else {
        s = s < 0 ? s * penalty : s / penalty;
      }
    }
    if (s > bv) {
      sv = bv;
      bv = s;
      best = i;
    } else if (s > sv) {
      sv = s;
    }
  }
  if (best_out) *best_out = bv;
  if (second_out) *second_out = sv;
  return best;
}

int or_argmax_penalty(const float* logits, int n, const uint32_t* seen, double penalty,
                      double* best_out, double* second_out) {
  return or_argmax_penalty_prec(logits, n, seen, penalty, 0, best_out, second_out);
}

/* Continue/stop decision (policy.ts:297-302, kernels-decode.ts:487-518): two
 * double dot products with text_head columns end and assistant; continue iff
 * assistant >= end. */
int or_text_decide(const or_model* M, const float* h, double* end_out, double* asst_out) {
  double e = 0.0, a = 0.0;
  for (int d = 0; d < OR_D; d++) {
    e += (double)h[d] * (double)M->text_head[(int64_t)d * M->vocab + M->audio_end_id];
    a += (double)h[d] * (double)M->text_head[(int64_t)d * M->vocab + M->assistant_id];
  }
  if (end_out) *end_out = e;
  if (asst_out) *asst_out = a;
  return a >= e;
}

/* One local-head step (ref-decode.mjs:238-272): the input embedding x[768] at
 * frame-local position `step` through the 1-layer local transformer whose
 * 17-slot cache is (K, V, sp); h[768] = local ln_f. */
static void local_step(const or_model* M, const float* x, int step, float* K, float* V,
                       int32_t* sp, float* h) {
  float e[OR_D];
  memcpy(e, x, sizeof e);
  layer_rows(&M->local, OR_ROW, 0, 0, 1, step, e, K, V, sp);
  or_layernorm(e, M->local_lnf_w, M->local_lnf_b, OR_D, h);
}

/* The 17-step local frame head for one voice (ref-decode.mjs:383-412,
 * decode.ts:788-939).  seen[16][32] is the per-channel repetition history and
 * is updated.  Writes codes[16] and returns 1 (continue) or 0 (stop; codes
 * untouched).  margins[17] (optional): step 0 gets asst - end, steps 1..16 the
 * gap between the winning and runner-up penalised logit. */
int or_local_frame(const or_model* M, const float* hidden, uint32_t* seen, int32_t* codes,
                   double* margins) {
  float* K = (float*)calloc((size_t)OR_ROW * OR_D, sizeof(float));
  float* V = (float*)calloc((size_t)OR_ROW * OR_D, sizeof(float));
  int32_t sp[OR_ROW];
  for (int i = 0; i < OR_ROW; i++) sp[i] = -1;
  float h[OR_D], x[OR_D], logits[OR_CODES];
  double e, a;
  local_step(M, hidden, 0, K, V, sp, h);
  const int cont = or_text_decide(M, h, &e, &a);
  if (margins) margins[0] = a - e;
  if (cont) {
    int prev = 0;
    for (int ch = 0; ch < OR_NVQ; ch++) {
      if (ch == 0) {
        for (int j = 0; j < OR_D; j++) x[j] = M->wte[(int64_t)M->assistant_id * OR_D + j];
      } else {
        const float* t = M->audio_emb[ch - 1] + (int64_t)prev * OR_D;
        memcpy(x, t, sizeof x);
      }
      local_step(M, x, ch + 1, K, V, sp, h);
      or_gemm(1, OR_D, OR_CODES, h, M->audio_heads[ch], NULL, logits);
      double bv, sv;
      const int tok = or_argmax_penalty_prec(logits, OR_CODES, seen + ch * 32, M->penalty,
                                             M->penalty_f32, &bv, &sv);
      if (margins) margins[ch + 1] = bv - sv;
      codes[ch] = tok;
      seen[ch * 32 + (tok >> 5)] |= 1u << (tok & 31);
      prev = tok;
    }
  }
  free(K);
  free(V);
  return cont;
}

/* Local-head steps 0 .. max_step with no greedy choice, the conformance probe
 * DecodeRunner.nextFrameSteps (decode.ts:970-1030): step 0 takes `hidden`,
 * step 1 the assistant-slot text embedding, step s >= 2 the embedding of
 * codes[s - 2] on channel s - 2.  out[768] = local ln_f of step max_step. */
void or_local_steps(const or_model* M, const float* hidden, int max_step, const int32_t* codes,
                    float* out) {
  float* K = (float*)calloc((size_t)OR_ROW * OR_D, sizeof(float));
  float* V = (float*)calloc((size_t)OR_ROW * OR_D, sizeof(float));
  int32_t sp[OR_ROW];
  for (int i = 0; i < OR_ROW; i++) sp[i] = -1;
  float x[OR_D];
  for (int step = 0; step <= max_step; step++) {
    if (step == 0)
      memcpy(x, hidden, sizeof x);
    else if (step == 1)
      memcpy(x, M->wte + (int64_t)M->assistant_id * OR_D, sizeof x);
    else
      memcpy(x, M->audio_emb[step - 2] + (int64_t)codes[step - 2] * OR_D, sizeof x);
    local_step(M, x, step, K, V, sp, out);
  }
  free(K);
  free(V);
}

/* The local frame head teacher-forced with given codes: the 17 steps of
 * or_local_frame (ref-decode.mjs:383-412) with codes[ch] fed to step ch + 2
 * in place of the greedy choice.  text2[0] / text2[1] receive step 0's
 * audio_end and assistant dot products (or_text_decide), logits[ch][1024]
 * the audio head of channel ch on step ch + 1 before any penalty
 * (ref-decode.mjs:401-402). */
void or_local_logits(const or_model* M, const float* hidden, const int32_t* codes, double* text2,
                     float* logits) {
  float* K = (float*)calloc((size_t)OR_ROW * OR_D, sizeof(float));
  float* V = (float*)calloc((size_t)OR_ROW * OR_D, sizeof(float));
  int32_t sp[OR_ROW];
  for (int i = 0; i < OR_ROW; i++) sp[i] = -1;
  float h[OR_D], x[OR_D];
  local_step(M, hidden, 0, K, V, sp, h);
  or_text_decide(M, h, &text2[0], &text2[1]);
  for (int ch = 0; ch < OR_NVQ; ch++) {
    if (ch == 0)
      memcpy(x, M->wte + (int64_t)M->assistant_id * OR_D, sizeof x);
    else
      memcpy(x, M->audio_emb[ch - 1] + (int64_t)codes[ch - 1] * OR_D, sizeof x);
    local_step(M, x, ch + 1, K, V, sp, h);
    or_gemm(1, OR_D, OR_CODES, h, M->audio_heads[ch], NULL, logits + (int64_t)ch * OR_CODES);
  }
  free(K);
  free(V);
}

/* Prompt rows of buildVoiceCloneRows with empty templates (policy.ts:49-80):
 * [audio_start] + one audio row per code frame + [audio_end] + text rows +
 * [audio_start].  Returns the row count (n_frames + n_text + 3). */
int or_build_rows(int n_frames, const int32_t* codes, int n_text, const int32_t* text,
                  int32_t* rows) {
  int r = 0;
  const int AUDIO_START = 6, AUDIO_END = 7, USER_SLOT = 8;
#define OR_TEXT_ROW(id)                                          \
  do {                                                           \
    for (int j = 0; j < OR_ROW; j++) rows[r * OR_ROW + j] = OR_PAD; \
    rows[r * OR_ROW] = (id);                                     \
    r++;                                                         \
  } while (0)
  OR_TEXT_ROW(AUDIO_START);
  for (int f = 0; f < n_frames; f++) {
    rows[r * OR_ROW] = USER_SLOT;
    for (int j = 0; j < OR_NVQ; j++) rows[r * OR_ROW + 1 + j] = codes[f * OR_NVQ + j];
    r++;
  }
  OR_TEXT_ROW(AUDIO_END);
  for (int t = 0; t < n_text; t++) OR_TEXT_ROW(text[t]);
  OR_TEXT_ROW(AUDIO_START);
#undef OR_TEXT_ROW
  return r;
}

/* ------------------------------------------------------ batched helpers */
/* The batched forms run independent voices on OpenMP threads; each voice's
 * own arithmetic is exactly the single-voice function above (nested parallel
 * regions inside are inactive, so every GEMM runs single-threaded per voice;
 * a single voice runs outside the voice loop and its GEMMs use the threads).
 * Ring arrays are per voice: K/V[b][layer][C][768], sp[b][layer][C]. */

int or_model_prefill_batch(const or_model* M, int B, int C, int wrap, int kv_bf16, int rows_max,
                           const int32_t* n_rows, const int32_t* ids, float* K, float* V,
                           int32_t* sp, float* last_hidden) {
  int rc = 0;
  const int64_t ring = (int64_t)M->n_layers * C;
#pragma omp parallel for schedule(dynamic, 1) reduction(| : rc) if (B > 1)
  for (int b = 0; b < B; b++) {
    float* hid = (float*)malloc(sizeof(float) * (size_t)(n_rows[b] > 0 ? n_rows[b] : 1) * OR_D);
    int r = or_model_prefill(M, C, wrap, kv_bf16, n_rows[b], ids + (int64_t)b * rows_max * OR_ROW,
                             K + b * ring * OR_D, V + b * ring * OR_D, sp + b * ring, hid);
    if (r == 0)
      memcpy(last_hidden + (int64_t)b * OR_D, hid + (int64_t)(n_rows[b] - 1) * OR_D,
             sizeof(float) * OR_D);
    free(hid);
    rc |= (r != 0);
  }
  return rc ? -1 : 0;
}

int or_model_decode_step_batch(const or_model* M, int B, int C, int wrap, int kv_bf16,
                               const int32_t* rows17, const int32_t* pos, float* K, float* V,
                               int32_t* sp, float* hidden) {
  int rc = 0;
  const int64_t ring = (int64_t)M->n_layers * C;
#pragma omp parallel for schedule(dynamic, 1) reduction(| : rc) if (B > 1)
  for (int b = 0; b < B; b++)
    rc |= or_model_decode_step(M, C, wrap, kv_bf16, rows17 + (int64_t)b * OR_ROW, pos[b],
                               K + b * ring * OR_D, V + b * ring * OR_D, sp + b * ring,
                               hidden + (int64_t)b * OR_D) != 0;
  return rc ? -1 : 0;
}

void or_local_frame_batch(const or_model* M, int B, const float* hidden, uint32_t* seen,
                          int32_t* codes, int32_t* cont, double* margins) {
#pragma omp parallel for schedule(dynamic, 1) if (B > 1)
  for (int b = 0; b < B; b++)
    cont[b] = or_local_frame(M, hidden + (int64_t)b * OR_D, seen + (int64_t)b * OR_NVQ * 32,
                             codes + (int64_t)b * OR_NVQ, margins ? margins + (int64_t)b * 17 : NULL);
}
