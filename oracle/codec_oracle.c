/*
 * CPU ORACLE for the codec decoder -- TEST INFRASTRUCTURE ONLY.
 *
 * Part of liboracle.so (see mb_oracle.c): only tests/, __graft_entry__ and
 * bench.py's CPU baseline may load it; the HIP library never does.
 *
 * A plain-C restatement of the reference's streaming codec decoder, one
 * voice, one position at a time, in the reference's order
 * (src/lib/tts/engine/codec.ts:470-765, encodeFrame):
 *   RVQ front ........ RVQ_ACCUM / RVQ_PROJECT, kernels-decode.ts:537-574
 *   per stage ........ input projection once per position (codec.ts:536-557),
 *                      then per layer and per position: LayerNorm (LAYERNORM_1),
 *                      qkv GEMV (GEMV_NOB), RoPE + ring write at the absolute
 *                      position (ROPE_SPLIT_CODEC, kernels-decode.ts:679-714),
 *                      windowed ring attention (ATTEND_RING_CODEC, :590-667),
 *                      out GEMV, layer-scale add (LAYER_SCALE_ADD, :360-371),
 *                      LayerNorm, FFN with exact GELU (GELU_ERF, :392-415),
 *                      layer-scale add; then the output projection
 *                      (codec.ts:717-735) and the x2 upsample (UPSAMPLE2, :722-745)
 *   head ............. CODEC_HEAD, kernels-decode.ts:747-768
 *
 * Each stage's ring has exactly `context` slots, slot = position % context
 * (kernels-decode.ts:709), and a query at position cur sees slot j iff
 * slot_pos[j] >= 0 and 0 <= cur - slot_pos[j] < context (:608-611).  Dot
 * products, LayerNorm moments and the softmax are carried in double with
 * fp32 results (as mb_oracle.c); the layer-scale add is the reference's fp32
 * multiply then add; erf is Abramowitz & Stegun 7.1.26, the reference's.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define CO_D 256
#define CO_H 4
#define CO_HD 64
#define CO_FFN 1024
#define CO_RVQ 512
#define CO_RVQ_OUT 768
#define CO_ENTRY 8
#define CO_NVQ 16
#define CO_CODES 1024
#define CO_STAGES 4
#define CO_SAMPLES 3840
#define CO_LATENT 240

void or_rope(const float* x, int n_heads, int64_t pos, float* out);
void or_layernorm(const float* x, const float* w, const float* b, int n, float* out);
float or_bf16_round(float x);

typedef struct {
  const float *qkv, *o, *f1, *f2; /* [256][768], [256][256], [256][1024], [1024][256] */
  const float *ln1_w, *ln1_b, *ln2_w, *ln2_b, *s1, *s2; /* [256] */
} or_codec_layer;

typedef struct {
  const float* rvq_w[CO_NVQ];    /* [512][8] per quantiser */
  const float* rvq_b[CO_NVQ];    /* [512] */
  const float* rvq_book[CO_NVQ]; /* [1024][8] */
  const float* rvq_out;          /* [768][512] (output-major, as the graph stores it) */
  const float* rvq_out_b;        /* [768] */
  int layers[CO_STAGES];
  int context[CO_STAGES];
  const float* in_proj[CO_STAGES];  /* [192 | 384][256] */
  const float* out_proj[CO_STAGES]; /* [256][768 | 240] */
  const or_codec_layer* layer;      /* every layer, stage by stage */
  int kv_bf16;                      /* store ring K/V rounded to bf16 */
} or_codec;

/* erf by Abramowitz & Stegun 7.1.26, |error| <= 1.5e-7 (GELU_ERF's form). */
double or_erf_as(double x) {
  const double sgn = x >= 0.0 ? 1.0 : -1.0;
  const double ax = fabs(x);
  const double t = 1.0 / (1.0 + 0.3275911 * ax);
  const double poly =
      ((((1.061405429 * t - 1.453152027) * t + 1.421413741) * t - 0.284496736) * t + 0.254829592) * t;
  return sgn * (1.0 - poly * exp(-ax * ax));
}

float or_gelu_erf(float v) {
  const double x = v;
  return (float)(0.5 * x * (1.0 + or_erf_as(x * 0.7071067811865476)));
}

/* y[n] = sum_k x[k] W[k][n] for W [K][N] row-major, double accumulation. */
static void gemv(const float* x, const float* W, int K, int N, float* y) {
  double acc[CO_FFN > CO_RVQ_OUT ? CO_FFN : CO_RVQ_OUT];
  for (int n = 0; n < N; n++) acc[n] = 0.0;
  for (int k = 0; k < K; k++) {
    const double xv = x[k];
    const float* wr = W + (int64_t)k * N;
    for (int n = 0; n < N; n++) acc[n] += xv * (double)wr[n];
  }
  for (int n = 0; n < N; n++) y[n] = (float)acc[n];
}

/* Slots per layer summed over the stages: the size of one voice's rings is
 * or_codec_slots() * 256 floats for K (and for V) and or_codec_slots() ints. */
int64_t or_codec_slots(const or_codec* W) {
  int64_t n = 0;
  for (int s = 0; s < CO_STAGES; s++) n += (int64_t)W->layers[s] * W->context[s];
  return n;
}

/* RVQ front for one frame: codes[16] -> stage0 [4][192]. */
void or_codec_rvq(const or_codec* W, const int32_t* codes, float* stage0) {
  float acc[CO_RVQ];
  for (int n = 0; n < CO_RVQ; n++) {
    double a = 0.0;
    for (int k = 0; k < CO_NVQ; k++) {
      const int32_t code = codes[k];
      double dot = 0.0;
      if (code >= 0 && code < CO_CODES)
        for (int j = 0; j < CO_ENTRY; j++)
          dot += (double)W->rvq_w[k][n * CO_ENTRY + j] * (double)W->rvq_book[k][code * CO_ENTRY + j];
      a += dot + (double)W->rvq_b[k][n];
    }
    acc[n] = (float)a;
  }
  for (int n = 0; n < CO_RVQ_OUT; n++) {
    double g = W->rvq_out_b[n];
    for (int i = 0; i < CO_RVQ; i++) g += (double)acc[i] * (double)W->rvq_out[(int64_t)n * CO_RVQ + i];
    stage0[(n & 3) * 192 + (n >> 2)] = (float)g;
  }
}

/* One query at `cur` against one layer's ring of `C` slots, 4 heads.
 * `live` is scratch for C slot indices. */
static void attend(const float* q, int64_t cur, int C, const float* K, const float* V,
                   const int32_t* sp, float* out, double* scores, int* live) {
  int nl = 0;
  for (int j = 0; j < C; j++) {
    const int64_t d = cur - (int64_t)sp[j];
    if (sp[j] >= 0 && d >= 0 && d < C) live[nl++] = j;
  }
  for (int h = 0; h < CO_H; h++) {
    double qd[CO_HD];
    for (int i = 0; i < CO_HD; i++) qd[i] = q[h * CO_HD + i];
    /* each score is its own sum over i in ascending order; four slots' sums
     * run side by side so their dependency chains overlap */
    int t = 0;
    for (; t + 4 <= nl; t += 4) {
      const float* k0 = K + (int64_t)live[t] * CO_D + h * CO_HD;
      const float* k1 = K + (int64_t)live[t + 1] * CO_D + h * CO_HD;
      const float* k2 = K + (int64_t)live[t + 2] * CO_D + h * CO_HD;
      const float* k3 = K + (int64_t)live[t + 3] * CO_D + h * CO_HD;
      double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
      for (int i = 0; i < CO_HD; i++) {
        s0 += qd[i] * (double)k0[i];
        s1 += qd[i] * (double)k1[i];
        s2 += qd[i] * (double)k2[i];
        s3 += qd[i] * (double)k3[i];
      }
      scores[t] = s0 * 0.125;
      scores[t + 1] = s1 * 0.125;
      scores[t + 2] = s2 * 0.125;
      scores[t + 3] = s3 * 0.125;
    }
    for (; t < nl; t++) {
      const float* kr = K + (int64_t)live[t] * CO_D + h * CO_HD;
      double s = 0.0;
      for (int i = 0; i < CO_HD; i++) s += qd[i] * (double)kr[i];
      scores[t] = s * 0.125;
    }
    double mx = -INFINITY;
    for (t = 0; t < nl; t++)
      if (scores[t] > mx) mx = scores[t];
    /* the softmax and P V over the live slots in ascending slot order */
    double sum = 0.0;
    for (t = 0; t < nl; t++) {
      scores[t] = exp(scores[t] - mx);
      sum += scores[t];
    }
    double acc[CO_HD];
    for (int i = 0; i < CO_HD; i++) acc[i] = 0.0;
    for (t = 0; t < nl; t++) {
      if (scores[t] == 0.0) continue;
      const float* vr = V + (int64_t)live[t] * CO_D + h * CO_HD;
      for (int i = 0; i < CO_HD; i++) acc[i] += scores[t] * (double)vr[i];
    }
    for (int i = 0; i < CO_HD; i++) out[h * CO_HD + i] = sum > 0.0 ? (float)(acc[i] / sum) : 0.0f;
  }
}

/* Decode n_frames frames of one voice: codes [n][16] -> pcm [2][n * 3840]
 * (pcm row stride `pcm_stride` floats, so a caller may write frames into a
 * longer buffer).  ringK / ringV [or_codec_slots][256], slot_pos
 * [or_codec_slots] (-1 = empty) and pos[4] (the next position of each stage)
 * carry the voice's state across calls.  Returns 0, or -1 on allocation
 * failure. */
int or_codec_decode(const or_codec* W, float* ringK, float* ringV, int32_t* slot_pos,
                    int32_t* pos, int n_frames, const int32_t* codes, float* pcm,
                    int64_t pcm_stride) {
  int maxC = 0;
  for (int s = 0; s < CO_STAGES; s++)
    if (W->context[s] > maxC) maxC = W->context[s];
  float* in = (float*)malloc(sizeof(float) * 64 * 384);
  float* x = (float*)malloc(sizeof(float) * 32 * CO_D);
  float* out = (float*)malloc(sizeof(float) * 32 * CO_RVQ_OUT);
  double* scores = (double*)malloc(sizeof(double) * (size_t)maxC);
  int* live = (int*)malloc(sizeof(int) * (size_t)maxC);
  if (!in || !x || !out || !scores || !live) {
    free(in); free(x); free(out); free(scores); free(live);
    return -1;
  }
  float h[CO_D], qkv[3 * CO_D], q[CO_D], ctx[CO_D], proj[CO_D], ffn[CO_FFN];
  for (int f = 0; f < n_frames; f++) {
    or_codec_rvq(W, codes + (int64_t)f * CO_NVQ, in);
    int in_w = 192;
    int64_t slot0 = 0;
    const or_codec_layer* L = W->layer;
    for (int s = 0; s < CO_STAGES; s++) {
      const int n = 4 << s, C = W->context[s];
      const int out_w = s == CO_STAGES - 1 ? CO_LATENT : CO_RVQ_OUT;
      for (int i = 0; i < n; i++) gemv(in + (int64_t)i * in_w, W->in_proj[s], in_w, CO_D, x + (int64_t)i * CO_D);
      for (int l = 0; l < W->layers[s]; l++, L++, slot0 += C) {
        float* K = ringK + slot0 * CO_D;
        float* V = ringV + slot0 * CO_D;
        int32_t* sp = slot_pos + slot0;
        for (int i = 0; i < n; i++) {
          float* xi = x + (int64_t)i * CO_D;
          const int64_t p = (int64_t)pos[s] + i;
          or_layernorm(xi, L->ln1_w, L->ln1_b, CO_D, h);
          gemv(h, L->qkv, CO_D, 3 * CO_D, qkv);
          const int slot = (int)(p % C);
          or_rope(qkv, CO_H, p, q);
          or_rope(qkv + CO_D, CO_H, p, K + (int64_t)slot * CO_D);
          memcpy(V + (int64_t)slot * CO_D, qkv + 2 * CO_D, CO_D * sizeof(float));
          if (W->kv_bf16)
            for (int d = 0; d < CO_D; d++) {
              K[(int64_t)slot * CO_D + d] = or_bf16_round(K[(int64_t)slot * CO_D + d]);
              V[(int64_t)slot * CO_D + d] = or_bf16_round(V[(int64_t)slot * CO_D + d]);
            }
          sp[slot] = (int32_t)p;
          attend(q, p, C, K, V, sp, ctx, scores, live);
          gemv(ctx, L->o, CO_D, CO_D, proj);
          for (int d = 0; d < CO_D; d++) xi[d] = xi[d] + L->s1[d] * proj[d];
          or_layernorm(xi, L->ln2_w, L->ln2_b, CO_D, h);
          gemv(h, L->f1, CO_D, CO_FFN, ffn);
          for (int d = 0; d < CO_FFN; d++) ffn[d] = or_gelu_erf(ffn[d]);
          gemv(ffn, L->f2, CO_FFN, CO_D, proj);
          for (int d = 0; d < CO_D; d++) xi[d] = xi[d] + L->s2[d] * proj[d];
        }
      }
      for (int i = 0; i < n; i++) gemv(x + (int64_t)i * CO_D, W->out_proj[s], CO_D, out_w, out + (int64_t)i * out_w);
      pos[s] += n;
      if (s < CO_STAGES - 1) {
        /* new[2t + r][m] = old[t][2m + r] */
        for (int t = 0; t < n; t++)
          for (int r = 0; r < 2; r++)
            for (int m = 0; m < 384; m++)
              in[(int64_t)(2 * t + r) * 384 + m] = out[(int64_t)t * CO_RVQ_OUT + 2 * m + r];
        in_w = 384;
      }
    }
    /* audio[c][t * 120 + j] = latent[t][2j + c] */
    for (int c = 0; c < 2; c++)
      for (int t = 0; t < 32; t++)
        for (int j = 0; j < 120; j++)
          pcm[(int64_t)c * pcm_stride + (int64_t)f * CO_SAMPLES + t * 120 + j] =
              out[(int64_t)t * CO_LATENT + 2 * j + c];
  }
  free(in);
  free(x);
  free(out);
  free(scores);
  free(live);
  return 0;
}

/* Several voices on OpenMP threads: voice b's rings at ringK + b *
 * or_codec_slots * 256 (likewise V, slot_pos + b * or_codec_slots), pos +
 * 4b, codes [n][B][16], pcm [B][2][n * 3840]. */
int or_codec_decode_batch(const or_codec* W, int B, float* ringK, float* ringV,
                          int32_t* slot_pos, int32_t* pos, int n_frames, const int32_t* codes,
                          float* pcm) {
  const int64_t S = or_codec_slots(W);
  const int64_t T = (int64_t)n_frames * CO_SAMPLES;
  int bad = 0;
#pragma omp parallel for schedule(dynamic, 1) reduction(| : bad)
  for (int b = 0; b < B; b++) {
    int32_t* c = (int32_t*)malloc(sizeof(int32_t) * (size_t)n_frames * CO_NVQ);
    if (!c) {
      bad |= 1;
      continue;
    }
    for (int f = 0; f < n_frames; f++)
      memcpy(c + (int64_t)f * CO_NVQ, codes + ((int64_t)f * B + b) * CO_NVQ, CO_NVQ * sizeof(int32_t));
    bad |= or_codec_decode(W, ringK + (int64_t)b * S * CO_D, ringV + (int64_t)b * S * CO_D,
                           slot_pos + (int64_t)b * S, pos + 4 * b, n_frames, c,
                           pcm + (int64_t)b * 2 * T, T) != 0;
    free(c);
  }
  return bad ? -1 : 0;
}
