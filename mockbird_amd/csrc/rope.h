// RoPE as the graph evaluates it, shared by the ring writes (ring.hip) and
// the codec's window attention, which appends its own rows (prefill.hip).
#pragma once
#include "mb_internal.h"

namespace mb {

// inv_freq of the 32 pairs of a 64-dim head, as the graph's fp32 constants
// (each translation unit keeps its own copy)
static __constant__ uint32_t c_inv_freq_bits[32] = {
    kInvFreqBits[0], kInvFreqBits[1], kInvFreqBits[2], kInvFreqBits[3], kInvFreqBits[4],
    kInvFreqBits[5], kInvFreqBits[6], kInvFreqBits[7], kInvFreqBits[8], kInvFreqBits[9],
    kInvFreqBits[10], kInvFreqBits[11], kInvFreqBits[12], kInvFreqBits[13], kInvFreqBits[14],
    kInvFreqBits[15], kInvFreqBits[16], kInvFreqBits[17], kInvFreqBits[18], kInvFreqBits[19],
    kInvFreqBits[20], kInvFreqBits[21], kInvFreqBits[22], kInvFreqBits[23], kInvFreqBits[24],
    kInvFreqBits[25], kInvFreqBits[26], kInvFreqBits[27], kInvFreqBits[28], kInvFreqBits[29],
    kInvFreqBits[30], kInvFreqBits[31]};

// cos/sin of pair `i` at absolute position `pos`: the angle is the fp32
// product float(pos) * inv_freq[i] (as the graph's fp32 Einsum forms it), and
// cos/sin of that fp32 angle are evaluated in double and rounded to fp32.
// Positions below kRopeTab read the context's table (built on the host with
// the same recipe); later ones are evaluated here.
__device__ __forceinline__ void rope_cs(const float2* __restrict__ tab, int32_t pos, int i,
                                        float& c, float& s) {
  if (pos < kRopeTab) {
    const float2 t = tab[(int64_t)pos * 32 + i];
    c = t.x;
    s = t.y;
    return;
  }
  const float a = __fmul_rn((float)pos, __uint_as_float(c_inv_freq_bits[i]));
  double sd, cd;
  sincos((double)a, &sd, &cd);
  c = (float)cd;
  s = (float)sd;
}

// One rotated pair, evaluated as the graph does it: fp32 Mul, Mul, Add with
// rotate_half(x) = (-x1, x0) -- never fused into an FMA (the library is built
// with -ffp-contract=off, so only explicit fmaf calls fuse).
__device__ __forceinline__ void rope_pair(float x0, float x1, float c, float s, float& o0,
                                          float& o1) {
  o0 = __fadd_rn(__fmul_rn(x0, c), __fmul_rn(-x1, s));
  o1 = __fadd_rn(__fmul_rn(x1, c), __fmul_rn(x0, s));
}

}  // namespace mb
