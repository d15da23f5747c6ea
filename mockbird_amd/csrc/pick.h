// The greedy code choice of one audio channel, as a device function shared
// by the argmax kernel (layers.hip) and by the one-row GEMVs that take the
// choice over from it (gemm.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mb_internal.h"

namespace mb {

// Greedy argmax over one row of 1024 logits with the HuggingFace repetition
// penalty on the channel's seen set (`sm`, 32 words): a seen id's score is
// multiplied by the penalty when negative and divided when not
// (argmaxWithRepetitionPenalty, policy.ts:273-290; ARGMAX_PENALTY,
// kernels-decode.ts:428-478).  Penalty and score are doubles, as the JS
// numbers of the reference's CPU path are (audio_repetition_penalty is the
// double 1.2, mossTtsRuntime.js:506-521); with `f32` (wave-uniform) they are
// f32, as in the WGSL engine: the penalty rounded to f32 and a correctly
// rounded f32 multiply or divide (taken in double and rounded once to f32,
// which for a product or quotient of two floats is the correctly rounded f32
// result, since 53 >= 2 * 24 + 2), whose result the double compare then
// orders exactly as an f32 compare would.  The penalty applies once the
// channel has emitted anything (policy.ts:282).  Strict '>' keeps the lowest
// id on ties and a NaN never wins.
//
// One wave, every lane returning the winner.  Lane l takes ids 16l ..
// 16l+15: choice_load issues its four 16-byte logit loads and the one seen
// word that holds their 16 bits (lanes 2w and 2w + 1 hold word w), so a
// caller can put other loads behind them before choice_take waits; ties are
// broken within the lane (ascending ids) and across lanes (the lower id on
// equal values).

// What one lane reads for the choice: its 16 logits and its seen word.
struct ChoiceIn {
  float4 v[4];
  uint32_t word;
};

__device__ __forceinline__ ChoiceIn choice_load(const float* __restrict__ lrow,
                                                const uint32_t* __restrict__ sm, int lane) {
  static_assert(CODES == 64 * 16, "one wave covers the codebook, 16 ids per lane");
  ChoiceIn c;
  const float4* lp = (const float4*)(lrow + 16 * lane);
#pragma unroll
  for (int q = 0; q < 4; q++) c.v[q] = lp[q];
  c.word = sm[lane >> 1];
  return c;
}

// A penalty above 1 only lowers a score (a seen id's positive score is
// divided by it, a negative one multiplied), so a seen id can win only if
// its raw logit reaches the best unseen one.  The choice therefore takes the best unseen
// id first, in float (the raw scores are floats, compared exactly), reduces
// its value across the wave, and penalises only the seen ids at or above it
// -- rarely more than one in a wave -- instead of every seen id: each
// penalised score is a double division.  Any other penalty penalises every
// seen id.  The winner is the scan's: the
// highest score, the lowest id among equal ones, never an id whose score is
// -inf or NaN (a strict '>' from -inf never takes them).
__device__ __forceinline__ int choice_take(const ChoiceIn& c, double penalty, int f32, int lane) {
  float v[16];
#pragma unroll
  for (int q = 0; q < 4; q++) {
    v[4 * q] = c.v[q].x; v[4 * q + 1] = c.v[q].y; v[4 * q + 2] = c.v[q].z; v[4 * q + 3] = c.v[q].w;
  }
  const uint32_t bits = (c.word >> (16 * (lane & 1))) & 0xffffu;
  const bool any = __ballot(c.word != 0u) != 0ull;
  const uint32_t pen = any && penalty != 1.0 ? bits : 0u;  // the ids this lane penalises
  float bu = -INFINITY;
  int idx = 0x7fffffff;
#pragma unroll
  for (int j = 0; j < 16; j++) {
    if (!((pen >> j) & 1u) && v[j] > bu) {
      bu = v[j];
      idx = 16 * lane + j;
    }
  }
  float top = bu;  // the best unseen score of the wave (never NaN)
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) top = fmaxf(top, __shfl_xor(top, off));
  const float thr = penalty > 1.0 ? top : -INFINITY;
  double best = bu;
  const float pf = (float)penalty;
#pragma unroll
  for (int j = 0; j < 16; j++) {
    if (((pen >> j) & 1u) && v[j] >= thr) {
      double s;
      if (f32)  // f32 result: the double product / quotient of two floats rounded once
        s = (double)(float)(v[j] < 0.f ? (double)v[j] * (double)pf : (double)v[j] / (double)pf);
      else
        s = v[j] < 0.f ? (double)v[j] * penalty : (double)v[j] / penalty;
      const int id = 16 * lane + j;
      if (s > best || (s == best && s > -INFINITY && id < idx)) {
        best = s;
        idx = id;
      }
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const double ob = __shfl_xor(best, off);
    const int oi = __shfl_xor(idx, off);
    if (ob > best || (ob == best && oi < idx)) {
      best = ob;
      idx = oi;
    }
  }
  return idx == 0x7fffffff ? 0 : idx;
}

// One voice's choice for channel `ch`, made by the one-row projection of the
// next local step instead of a launch of its own: every wave of that launch
// takes the same choice from the same logits and reads its input row,
// emb[winner], straight from the channel's code embedding table; block 0's
// first wave also writes the winner to tokens[ch] and the row to x (the
// step's residual).  The seen set is only read here: the launch that picks
// the frame's last channel records these channels' winners (each channel's
// set is read by that channel's choice alone, once per frame).  A frame that
// a cancellation cuts short therefore records none of its choices.
struct PickIn {
  const float* logits;   // [1024]: channel ch's audio-head logits
  const uint32_t* seen;  // [NVQ][32]: the voice's seen sets
  int32_t* tokens;       // [NVQ]
  const float* emb;      // channel ch's code embedding table [1024][768]
  float* x;              // [768]
  double penalty;
  int ch, f32;
};

__device__ __forceinline__ ChoiceIn pick_load(const PickIn& p, int lane) {
  return choice_load(p.logits, p.seen + (int64_t)p.ch * 32, lane);
}

__device__ __forceinline__ const float* pick_row(const PickIn& p, const ChoiceIn& c, int lane,
                                                 bool writer) {
  const int tok = choice_take(c, p.penalty, p.f32, lane);
  const float* row = p.emb + (int64_t)tok * D;
  if (writer) {
    if (lane == 0) p.tokens[p.ch] = tok;
#pragma unroll
    for (int i = 0; i < D / 4 / 64; i++)
      ((float4*)p.x)[lane + 64 * i] = ((const float4*)row)[lane + 64 * i];
  }
  return row;
}

}  // namespace mb
