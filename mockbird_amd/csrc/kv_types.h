// Element conversions and 16-byte vector load/store helpers for fp32 and bf16
// rows (bf16 is stored as the upper 16 bits of an fp32 pattern; the store
// rounds to nearest, ties to even), and cross-lane folds.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mb {

__host__ __device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7f800000u) == 0x7f800000u) {  // inf / nan: keep, quiet the nan
    const uint32_t nan = (u & 0x007fffffu) ? 0x0040u : 0u;
    return (uint16_t)((u >> 16) | nan);
  }
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
}

// Unpack one 16-byte vector: 4 fp32 or 8 bf16 values.
template <bool BF16>
__device__ __forceinline__ void unpack(const uint4& v, float* out) {
  if (BF16) {
    out[0] = bf16_lo(v.x); out[1] = bf16_hi(v.x);
    out[2] = bf16_lo(v.y); out[3] = bf16_hi(v.y);
    out[4] = bf16_lo(v.z); out[5] = bf16_hi(v.z);
    out[6] = bf16_lo(v.w); out[7] = bf16_hi(v.w);
  } else {
    out[0] = __uint_as_float(v.x); out[1] = __uint_as_float(v.y);
    out[2] = __uint_as_float(v.z); out[3] = __uint_as_float(v.w);
  }
}

// Load 8 consecutive elements starting at element `off` (16-byte aligned).
template <bool BF16>
__device__ __forceinline__ void load8(const void* base, int64_t off, float* out) {
  if (BF16) {
    const uint4 v = *(const uint4*)((const uint16_t*)base + off);
    unpack<true>(v, out);
  } else {
    const uint4 a = *(const uint4*)((const float*)base + off);
    const uint4 b = *(const uint4*)((const float*)base + off + 4);
    unpack<false>(a, out);
    unpack<false>(b, out + 4);
  }
}

// Store 8 consecutive elements starting at element `off` (16-byte aligned).
template <bool BF16>
__device__ __forceinline__ void store8(void* base, int64_t off, const float* in) {
  if (BF16) {
    uint4 v;
    v.x = pack_bf16(in[0], in[1]);
    v.y = pack_bf16(in[2], in[3]);
    v.z = pack_bf16(in[4], in[5]);
    v.w = pack_bf16(in[6], in[7]);
    *(uint4*)((uint16_t*)base + off) = v;
  } else {
    float* p = (float*)base + off;
    *(float4*)p = make_float4(in[0], in[1], in[2], in[3]);
    *(float4*)(p + 4) = make_float4(in[4], in[5], in[6], in[7]);
  }
}

// Reduce over the four lane groups that share a column (lanes i, i^16,
// i^32, i^48) with the gfx950 cross-row swaps: v_permlane32_swap pairs lane
// i with i^32 and v_permlane16_swap pairs i with i^16, both without an LDS
// round trip.  Each step combines the two values of a pair in the same order
// on both lanes, so all four lanes end with bit-identical results.
template <class Op>
__device__ __forceinline__ float col_reduce(float x, Op op) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = op(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return op(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float col_max(float x) {
  return col_reduce(x, [](float u, float v) { return fmaxf(u, v); });
}
__device__ __forceinline__ float col_sum(float x) {
  return col_reduce(x, [](float u, float v) { return u + v; });
}

}  // namespace mb
