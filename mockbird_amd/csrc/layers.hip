// Per-layer glue of the decoder on gfx950: LayerNorm, row embedding, the
// local head's embeddings, the continue/stop text-head decision, greedy
// argmax with the repetition penalty, and frame-row feedback.
#include "mb_internal.h"
#include "pick.h"

namespace mb {

// ---------------------------------------------------------------- LayerNorm

// One wave per row of WIDTH = 256 * NV (the model's 768, the codec's 256;
// 4 NV values per lane): mean, then the centred second moment, eps 1e-5,
// y = (x - mean) * rsqrt * w + b (LAYERNORM_ROWS, kernels-batch.ts:99-147;
// LAYERNORM_1, kernels-decode.ts:168-202; ref-decode.mjs:85-99).
// src_row (optional) maps output row i to input row src_row[i].
template <int NV>
__global__ __launch_bounds__(256) void k_layernorm(const float* __restrict__ x, int64_t ldx,
                                                   const int32_t* __restrict__ src_row, int M,
                                                   const float* __restrict__ w,
                                                   const float* __restrict__ bb,
                                                   float* __restrict__ y, int64_t ldy) {
  constexpr float kInvW = 1.f / (256.f * NV);
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const float* xr = x + (int64_t)(src_row ? src_row[row] : row) * ldx;
  float v[4 * NV];
#pragma unroll
  for (int i = 0; i < NV; i++) {
    const float4 t = *(const float4*)(xr + i * 256 + lane * 4);
    v[i * 4] = t.x; v[i * 4 + 1] = t.y; v[i * 4 + 2] = t.z; v[i * 4 + 3] = t.w;
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4 * NV; i++) s += v[i];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
  const float mean = s * kInvW;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < 4 * NV; i++) {
    const float d = v[i] - mean;
    q = fmaf(d, d, q);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) q += __shfl_xor(q, off);
  const float inv = 1.f / sqrtf(q * kInvW + 1e-5f);
  float* yr = y + (int64_t)row * ldy;
#pragma unroll
  for (int i = 0; i < NV; i++) {
    const int c = i * 256 + lane * 4;
    const float4 ww = *(const float4*)(w + c), bv = *(const float4*)(bb + c);
    *(float4*)(yr + c) = make_float4((v[i * 4] - mean) * inv * ww.x + bv.x,
                                     (v[i * 4 + 1] - mean) * inv * ww.y + bv.y,
                                     (v[i * 4 + 2] - mean) * inv * ww.z + bv.z,
                                     (v[i * 4 + 3] - mean) * inv * ww.w + bv.w);
  }
}

int launch_layernorm(mb_ctx* ctx, const float* x, int64_t ldx, const int32_t* src_row, int M,
                     const float* w, const float* b, float* y, int64_t ldy, int width) {
  if (M <= 0) return MB_OK;
  const dim3 grid((unsigned)((M + 3) / 4));
  if (width == D)
    hipLaunchKernelGGL(k_layernorm<3>, grid, dim3(256), 0, ctx->stream, x, ldx, src_row, M, w, b,
                       y, ldy);
  else if (width == 256)
    hipLaunchKernelGGL(k_layernorm<1>, grid, dim3(256), 0, ctx->stream, x, ldx, src_row, M, w, b,
                       y, ldy);
  else
    return fail(ctx, MB_ERR_ARG, "LayerNorm over rows of %d is not built", width);
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

// ------------------------------------------------------------------ embedding

// x[row] = wte[ids[row][0]] + sum_k audio_k[ids[row][1+k]], pad (1024) skipped,
// summed in fp32 in channel order (EMBED_ROWS, kernels-batch.ts:45-92;
// embedRowFor, promptRows.ts:21-36).  An id outside its table contributes
// nothing (the host rejects such ids before launching).
// With `codes` (ids null) row b is the frame row [assistant_id, codes[b][0..15]]
// (buildFrameRow, policy.ts:83-88) read from the chosen codes directly.
__global__ __launch_bounds__(256) void k_embed_rows(const int32_t* __restrict__ ids, int M,
                                                    const float* __restrict__ wte, int vocab,
                                                    AudioTables audio, float* __restrict__ x,
                                                    const int32_t* __restrict__ codes,
                                                    int assistant_id) {
  const int row = blockIdx.x;
  if (row >= M) return;
  // the row's 16 audio ids: ids[row][1..16], or the row's chosen codes
  const int32_t* aid = ids ? ids + (int64_t)row * ROW + 1 : codes + (int64_t)row * NVQ;
  // Every table read is issued before the first add (ids clamped into their
  // tables, the skipped ones then left out of the sum), so a row costs one
  // memory round trip, not one per channel; the sum keeps channel order.
  static_assert(D % 256 == 0, "whole rows per block");
  constexpr int DI = D / 256;
  const int t = ids ? ids[(int64_t)row * ROW] : assistant_id;
  const bool tv = t >= 0 && t < vocab;
  const int tc = tv ? t : 0;
  float tw[DI], av[NVQ][DI];
#pragma unroll
  for (int i = 0; i < DI; i++) tw[i] = wte[(int64_t)tc * D + threadIdx.x + 256 * i];
  bool ok[NVQ];
#pragma unroll
  for (int k = 0; k < NVQ; k++) {
    const int a = aid[k];
    ok[k] = a != PAD && a >= 0 && a < CODES;
    const int ac = ok[k] ? a : 0;
#pragma unroll
    for (int i = 0; i < DI; i++) av[k][i] = audio.t[k][(int64_t)ac * D + threadIdx.x + 256 * i];
  }
#pragma unroll
  for (int i = 0; i < DI; i++) {
    float acc = tv ? tw[i] : 0.f;
#pragma unroll
    for (int k = 0; k < NVQ; k++) acc = ok[k] ? acc + av[k][i] : acc;
    x[(int64_t)row * D + threadIdx.x + 256 * i] = acc;
  }
}

int launch_embed_rows(mb_ctx* ctx, const int32_t* ids, int M, const float* wte, int vocab,
                      const AudioTables& audio, float* x, const int32_t* codes, int assistant_id) {
  if (M <= 0) return MB_OK;
  if (!ids == !codes) return fail(ctx, MB_ERR_ARG, "frame rows come from ids or from codes");
  hipLaunchKernelGGL(k_embed_rows, dim3((unsigned)M), dim3(256), 0, ctx->stream, ids, M, wte, vocab,
                     audio, x, codes, assistant_id);
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

// The local head's step embeddings (EMBED_ROW_LOCAL modes 1 and 2,
// kernels-decode.ts:96-124; ref-decode.mjs:238-251):
//   step 1:  wte[assistant_id]
//   step s>1: audio_{s-2}[tokens[b][s-2]]  (the previous channel's code)
__global__ __launch_bounds__(256) void k_embed_local(int step, int B, const float* __restrict__ wte,
                                                     int assistant_id, AudioTables audio,
                                                     const int32_t* __restrict__ tokens,
                                                     float* __restrict__ x) {
  const int b = blockIdx.x;
  if (b >= B) return;
  const float* src;
  if (step == 1) {
    src = wte + (int64_t)assistant_id * D;
  } else {
    int t = tokens[b * NVQ + step - 2];
    t = t < 0 ? 0 : (t >= CODES ? CODES - 1 : t);
    src = audio.t[step - 2] + (int64_t)t * D;
  }
  for (int d = threadIdx.x; d < D; d += 256) x[(int64_t)b * D + d] = src[d];
}

int launch_embed_local(mb_ctx* ctx, int step, int B, const float* wte, int assistant_id,
                       const AudioTables& audio, const int32_t* tokens, float* x) {
  hipLaunchKernelGGL(k_embed_local, dim3((unsigned)B), dim3(256), 0, ctx->stream, step, B, wte,
                     assistant_id, audio, tokens, x);
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

// ------------------------------------------------------------ greedy choice

// Row b of x = row `tok` of a [*][768] table, one wave: three 16-byte
// copies per lane.
__device__ __forceinline__ void copy_row(const float* __restrict__ table, int tok,
                                         float* __restrict__ x, int b, int lane) {
  const float4* src = (const float4*)(table + (int64_t)tok * D);
  float4* dst = (float4*)(x + (int64_t)b * D);
#pragma unroll
  for (int i = 0; i < D / 4 / 64; i++) dst[lane + 64 * i] = src[lane + 64 * i];
}

// Continue/stop: two double-precision dot products of the step-0 hidden
// state with text-head columns end_id and assistant_id; continue iff
// assistant >= end (TEXT_HEAD_DECIDE kernels-decode.ts:487-518,
// decideAssistantStop policy.ts:297-302).  One wave per sequence.  With
// `alive`, a sequence already stopped (alive[b] == 0) stays stopped.  With
// `x`, the wave also writes step 1's input row, wte[assistant_id]
// (EMBED_ROW_LOCAL mode 1, kernels-decode.ts:96-124).  With `te`, the two
// dot products go to te[b] = (end, assistant).
__global__ __launch_bounds__(256) void k_text_decide(const float* __restrict__ h, int B,
                                                     const float* __restrict__ head, int vocab,
                                                     int end_id, int assistant_id,
                                                     const int32_t* __restrict__ alive,
                                                     int32_t* __restrict__ cont,
                                                     const float* __restrict__ wte,
                                                     float* __restrict__ x,
                                                     double* __restrict__ te) {
  const int lane = threadIdx.x & 63;
  const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (b >= B) return;
  // every read issued before the first product (one round trip): the
  // alive flag, the row of h and the two head columns (strided, one line each)
  const bool was_alive = !alive || alive[b];
  constexpr int DI = D / 64;
  float hv[DI], he[DI], ha[DI];
#pragma unroll
  for (int i = 0; i < DI; i++) {
    const int d = lane + 64 * i;
    hv[i] = h[(int64_t)b * D + d];
    he[i] = head[(int64_t)d * vocab + end_id];
    ha[i] = head[(int64_t)d * vocab + assistant_id];
  }
  if (x) copy_row(wte, assistant_id, x, b, lane);
  double e = 0.0, a = 0.0;
#pragma unroll
  for (int i = 0; i < DI; i++) {
    const double xv = hv[i];
    e += xv * (double)he[i];
    a += xv * (double)ha[i];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    e += __shfl_xor(e, off);
    a += __shfl_xor(a, off);
  }
  if (lane == 0) {
    cont[b] = a >= e && was_alive ? 1 : 0;
    if (te) {
      te[2 * b] = e;
      te[2 * b + 1] = a;
    }
  }
}

int launch_text_decide(mb_ctx* ctx, const float* h, int B, const float* head, int vocab, int end_id,
                       int assistant_id, const int32_t* alive, int32_t* cont, const float* wte,
                       float* x, double* te) {
  hipLaunchKernelGGL(k_text_decide, dim3((unsigned)((B + 3) / 4)), dim3(256), 0, ctx->stream, h, B,
                     head, vocab, end_id, assistant_id, alive, cont, wte, x, te);
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

// The greedy code choice of channel `ch` for every sequence: the penalised
// argmax of its 1024 logits (choice_load / choice_take, pick.h) goes to tokens[b][ch],
// and the seen bit is set only for sequences that continue (the reference
// stops before drawing codes).  One wave per sequence; the seen word the
// update changes is already in a register, so the update is a store with no
// load in front of it.  With `x`, the wave also writes the next step's input
// row, next_emb[winner] (EMBED_ROW_LOCAL mode 2: the next step embeds this
// channel's code).  Channels rec0 .. ch-1 were picked by the one-row
// projections of the steps after them (PickIn, pick.h), which only read the
// seen sets: their winners, already in tokens, are recorded here.
__global__ __launch_bounds__(256) void k_argmax_penalty(const float* __restrict__ logits, int B,
                                                        int ch, int rec0, double penalty, int f32,
                                                        uint32_t* __restrict__ seen,
                                                        const int32_t* __restrict__ cont,
                                                        int32_t* __restrict__ tokens,
                                                        const float* __restrict__ next_emb,
                                                        float* __restrict__ x) {
  const int lane = threadIdx.x & 63;
  const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (b >= B) return;
  uint32_t* sm = seen + ((int64_t)b * NVQ + ch) * 32;
  const bool go_on = !cont || cont[b];  // loaded with the logits, not after the choice
  const int rt = lane >= rec0 && lane < ch ? tokens[b * NVQ + lane] : 0;
  const ChoiceIn c = choice_load(logits + (int64_t)b * CODES, sm, lane);
  const int tok = choice_take(c, penalty, f32, lane);
  const uint32_t wtok = __shfl(c.word, (tok >> 5) * 2);
  if (lane == 0) {
    tokens[b * NVQ + ch] = tok;
    if (go_on) sm[tok >> 5] = wtok | (1u << (tok & 31));
  }
  if (go_on && lane >= rec0 && lane < ch)
    seen[((int64_t)b * NVQ + lane) * 32 + (rt >> 5)] |= 1u << (rt & 31);
  if (x) copy_row(next_emb, tok, x, b, lane);
}

int launch_argmax_penalty(mb_ctx* ctx, const float* logits, int B, int ch, int rec0,
                          double penalty, bool penalty_f32, uint32_t* seen, const int32_t* cont,
                          int32_t* tokens, const float* next_emb, float* x) {
  if (rec0 < 0 || rec0 > ch) return fail(ctx, MB_ERR_ARG, "channels %d .. %d to record", rec0, ch);
  hipLaunchKernelGGL(k_argmax_penalty, dim3((unsigned)((B + 3) / 4)), dim3(256), 0, ctx->stream,
                     logits, B, ch, rec0, penalty, (int)penalty_f32, seen, cont, tokens, next_emb,
                     x);
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

// Frame row fed back to the global transformer: [assistant_id, codes...]
// (buildFrameRow, policy.ts:83-88).
__global__ void k_frame_rows(const int32_t* __restrict__ tokens, int B, int assistant_id,
                             int32_t* __restrict__ rows17) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B * ROW) return;
  const int b = i / ROW, c = i % ROW;
  rows17[i] = c == 0 ? assistant_id : tokens[b * NVQ + c - 1];
}

int launch_frame_rows(mb_ctx* ctx, const int32_t* tokens, int B, int assistant_id, int32_t* rows17) {
  hipLaunchKernelGGL(k_frame_rows, dim3((unsigned)((B * ROW + 255) / 256)), dim3(256), 0,
                     ctx->stream, tokens, B, assistant_id, rows17);
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

// End of a device-resident frame: frame f's codes and continue flags go to
// codes[f][B][16] and cont_out[f][B] (f read from *frame_idx, then advanced),
// every sequence that continued moves to its next position, and one that
// stopped is latched in alive[].  One workgroup, so the counter update
// follows every read of it.
__global__ __launch_bounds__(256) void k_frame_emit(const int32_t* __restrict__ tokens,
                                                    const int32_t* __restrict__ cont, int B,
                                                    int32_t* __restrict__ frame_idx,
                                                    int32_t* __restrict__ codes,
                                                    int32_t* __restrict__ cont_out,
                                                    int32_t* __restrict__ pos,
                                                    int32_t* __restrict__ alive) {
  __shared__ int f;
  if (threadIdx.x == 0) f = *frame_idx;
  __syncthreads();
  for (int i = threadIdx.x; i < B * NVQ; i += blockDim.x) codes[(int64_t)f * B * NVQ + i] = tokens[i];
  for (int b = threadIdx.x; b < B; b += blockDim.x) {
    const int c = cont[b];
    cont_out[(int64_t)f * B + b] = c;
    alive[b] = c;
    if (c) pos[b] += 1;
  }
  __syncthreads();
  if (threadIdx.x == 0) *frame_idx = f + 1;
}

int launch_frame_emit(mb_ctx* ctx, const int32_t* tokens, const int32_t* cont, int B,
                      int32_t* frame_idx, int32_t* codes, int32_t* cont_out, int32_t* pos,
                      int32_t* alive) {
  hipLaunchKernelGGL(k_frame_emit, dim3(1), dim3(256), 0, ctx->stream, tokens, cont, B, frame_idx,
                     codes, cont_out, pos, alive);
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

}  // namespace mb
