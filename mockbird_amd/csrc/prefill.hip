// Causal prefill attention on MFMA (gfx950), flash-style: no S x S score
// matrix is ever materialised (the reference writes [12, S, S] scores and
// probabilities, kernels-batch.ts:246-350, and caps S at 256, prefill.ts:136).
//
// One workgroup = 64 query rows of one (sequence, head); each of its 4 waves
// owns 16 query columns.  The kernel computes S^T = K Q^T so that the
// accumulator tile (lane l holds rows (l/16)*4 + j, column l%16) is already
// the B operand of the next MFMA: for bf16 that is v_mfma_f32_16x16x16_bf16
// (B lane l = rows (l/16)*4 + j, column l%16), so P^T goes from the softmax
// straight into O^T += V^T P^T without an LDS round trip.  Per 64-slot K/V
// tile a wave issues 8 (bf16: 16x16x32) or 64 (fp32: 16x16x4) MFMAs for the
// scores and 16 / 64 for P V.
//
// Queries: row r of sequence b sits at position cur = pos0[b] + r and sees
// the ring slots whose stored position p satisfies 0 <= cur - p < C (the
// window rule of kernels-decode.ts:608-611, which implies p <= cur: causal).
// Slots are visited in physical order, 64 at a time, up to
// min(last position in the tile + 1, C).
#include "kv_types.h"
#include "mb_internal.h"

namespace mb {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int KT = 64;    // slots per K/V tile
constexpr int QT = 64;    // query rows per workgroup
constexpr int KPAD = 72;  // bf16 LDS row stride (144 B) to spread banks
constexpr int FPAD = 68;  // fp32 LDS row stride (272 B)

__device__ __forceinline__ bool live_slot(int32_t p, int64_t cur, int C) {
  const int64_t d = cur - p;
  return p >= 0 && d >= 0 && d < C;
}

// Reduce over the four lane groups that share a query column (l%16).
__device__ __forceinline__ float col_max(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}
__device__ __forceinline__ float col_sum(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}

// ---------------------------------------------------------------- bf16 MMA

// Q bf16 [B][rows_max][768] (roped), K/V bf16 ring, fp32 output.
__global__ __launch_bounds__(256) void k_flash_bf16(
    const uint16_t* __restrict__ q, Rows q_rows, const int32_t* __restrict__ pos0,
    const int32_t* __restrict__ n_rows, const uint16_t* __restrict__ ring_k,
    const uint16_t* __restrict__ ring_v, const int32_t* __restrict__ slot_pos,
    int64_t ring_seq_stride, int C, float* __restrict__ out, Rows out_rows) {
  __shared__ uint16_t Ks[KT * KPAD];   // [slot][dim]
  __shared__ uint16_t Vt[HD * KPAD];   // [dim][slot]
  __shared__ int32_t Ps[KT];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qcol = lane & 15, grp = lane >> 4;
  const int b = blockIdx.z, h = blockIdx.y;
  const int qtile = gridDim.x - 1 - blockIdx.x;  // longest (latest) tiles first
  const int n = n_rows[b];
  if (qtile * QT >= n) return;  // uniform per workgroup, before any barrier
  const int r = qtile * QT + wave * 16 + qcol;
  const bool qvalid = r < n;
  const int64_t cur = qvalid ? (int64_t)pos0[b] + r : -1;
  const int rlast = min(qtile * QT + QT, n) - 1;
  const int64_t kv_end64 = (int64_t)pos0[b] + rlast + 1;
  const int kv_end = kv_end64 < C ? (int)kv_end64 : C;

  // B operand of the score MFMA: Q[r][32*kc + 8*grp + 0..7], scaled by 0.125 (exact)
  bf16x8_t qb[2];
#pragma unroll
  for (int kc = 0; kc < 2; kc++) {
    uint4 raw = make_uint4(0, 0, 0, 0);
    if (qvalid)
      raw = *(const uint4*)(q + row_at(q_rows, b, r) + h * HD + kc * 32 + grp * 8);
    float f[8];
    unpack<true>(raw, f);
#pragma unroll
    for (int i = 0; i < 8; i++) qb[kc][i] = (__bf16)(f[i] * 0.125f);
  }
  const uint16_t* kb = ring_k + (int64_t)b * ring_seq_stride + (int64_t)h * C * HD;
  const uint16_t* vb = ring_v + (int64_t)b * ring_seq_stride + (int64_t)h * C * HD;
  const int32_t* sp = slot_pos + (int64_t)b * C;

  f32x4_t acc[4];
#pragma unroll
  for (int d = 0; d < 4; d++) acc[d] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;

  for (int t0 = 0; t0 < kv_end; t0 += KT) {
    __syncthreads();
    // stage K [slot][dim] and V^T [dim][slot]; thread -> (slot, 8-dim chunk), 2 passes
#pragma unroll
    for (int pass = 0; pass < 2; pass++) {
      const int sl = pass * 32 + (tid >> 3), dc = (tid & 7) * 8;
      const int slot = t0 + sl;
      uint4 kv = make_uint4(0, 0, 0, 0), vv = make_uint4(0, 0, 0, 0);
      if (slot < kv_end) {
        kv = *(const uint4*)(kb + (int64_t)slot * HD + dc);
        vv = *(const uint4*)(vb + (int64_t)slot * HD + dc);
      }
      *(uint4*)(Ks + sl * KPAD + dc) = kv;
      const uint16_t* ve = (const uint16_t*)&vv;
#pragma unroll
      for (int i = 0; i < 8; i++) Vt[(dc + i) * KPAD + sl] = ve[i];
    }
    if (tid < KT) Ps[tid] = (t0 + tid < kv_end) ? sp[t0 + tid] : -1;
    __syncthreads();

    // S^T blocks: rows = slots sb*16 + grp*4 + j, column = this lane's query
    float s[4][4];
    float mt = -INFINITY;
#pragma unroll
    for (int sb = 0; sb < 4; sb++) {
      f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < 2; kc++) {
        const bf16x8_t a = *(const bf16x8_t*)(Ks + (sb * 16 + qcol) * KPAD + kc * 32 + grp * 8);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qb[kc], c, 0, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const bool ok = live_slot(Ps[sb * 16 + grp * 4 + j], cur, C);
        s[sb][j] = ok ? c[j] : -INFINITY;
        mt = fmaxf(mt, s[sb][j]);
      }
    }
    mt = col_max(mt);
    const float mn = fmaxf(m, mt);
    const float mu = mn == -INFINITY ? 0.f : mn;
    const float scale = __expf(m - mu);
    float ls = 0.f;
    i16x4_t pb[4];
#pragma unroll
    for (int sb = 0; sb < 4; sb++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float p = __expf(s[sb][j] - mu);
        const __bf16 pbf = (__bf16)p;
        ls += (float)pbf;  // the sum uses the same rounded weights the MMA sees
        pb[sb][j] = __builtin_bit_cast(short, pbf);
      }
    l = l * scale + col_sum(ls);
    m = mn;
#pragma unroll
    for (int d = 0; d < 4; d++) acc[d] *= scale;
    // O^T[d-block] += V^T[d-block rows][slots] * P^T[slots][queries]
#pragma unroll
    for (int sb = 0; sb < 4; sb++)
#pragma unroll
      for (int d = 0; d < 4; d++) {
        const i16x4_t a = *(const i16x4_t*)(Vt + (d * 16 + qcol) * KPAD + sb * 16 + grp * 4);
        acc[d] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, pb[sb], acc[d], 0, 0, 0);
      }
  }
  if (!qvalid) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  float* op = out + row_at(out_rows, b, r) + h * HD;
#pragma unroll
  for (int d = 0; d < 4; d++)
    *(float4*)(op + d * 16 + grp * 4) =
        make_float4(acc[d][0] * inv, acc[d][1] * inv, acc[d][2] * inv, acc[d][3] * inv);
}

// ---------------------------------------------------------------- fp32 MMA

// Q fp32 [B][rows_max][768] (roped), K/V fp32 or bf16 ring (widened exactly
// into LDS), fp32 output, v_mfma_f32_16x16x4f32.  The score MMA's k index
// (0..3 per instruction, 16 instructions) is mapped to dim grp*16 + kc so a
// lane reads 16 consecutive dims of its K row and of its Q row.  In P V the
// instruction (sb, j) sums over k = grp, i.e. over slots sb*16 + grp*4 + j,
// which is exactly the score element the lane already holds.
template <bool KV_BF16>
__global__ __launch_bounds__(256) void k_flash_f32(
    const float* __restrict__ q, Rows q_rows, const int32_t* __restrict__ pos0,
    const int32_t* __restrict__ n_rows, const void* __restrict__ ring_k,
    const void* __restrict__ ring_v, const int32_t* __restrict__ slot_pos,
    int64_t ring_seq_stride, int C, float* __restrict__ out, Rows out_rows) {
  __shared__ float Ks[KT * FPAD];  // [slot][dim]
  __shared__ float Vs[KT * FPAD];  // [slot][dim]
  __shared__ int32_t Ps[KT];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qcol = lane & 15, grp = lane >> 4;
  const int b = blockIdx.z, h = blockIdx.y;
  const int qtile = gridDim.x - 1 - blockIdx.x;
  const int n = n_rows[b];
  if (qtile * QT >= n) return;
  const int r = qtile * QT + wave * 16 + qcol;
  const bool qvalid = r < n;
  const int64_t cur = qvalid ? (int64_t)pos0[b] + r : -1;
  const int rlast = min(qtile * QT + QT, n) - 1;
  const int64_t kv_end64 = (int64_t)pos0[b] + rlast + 1;
  const int kv_end = kv_end64 < C ? (int)kv_end64 : C;

  float qv[16];
  {
    const float* qp = q + (qvalid ? row_at(q_rows, b, r) : 0) + h * HD + grp * 16;
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      float4 t = qvalid ? *(const float4*)(qp + i) : make_float4(0.f, 0.f, 0.f, 0.f);
      qv[i] = t.x * 0.125f; qv[i + 1] = t.y * 0.125f; qv[i + 2] = t.z * 0.125f; qv[i + 3] = t.w * 0.125f;
    }
  }
  constexpr int E = KV_BF16 ? 2 : 4;
  const char* kb = (const char*)ring_k + ((int64_t)b * ring_seq_stride + (int64_t)h * C * HD) * E;
  const char* vb = (const char*)ring_v + ((int64_t)b * ring_seq_stride + (int64_t)h * C * HD) * E;
  const int32_t* sp = slot_pos + (int64_t)b * C;

  f32x4_t acc[4];
#pragma unroll
  for (int d = 0; d < 4; d++) acc[d] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;

  for (int t0 = 0; t0 < kv_end; t0 += KT) {
    __syncthreads();
    // stage K and V [slot][dim] as fp32; thread -> (slot, 8-dim chunk), 2 passes
#pragma unroll
    for (int pass = 0; pass < 2; pass++) {
      const int sl = pass * 32 + (tid >> 3), dc = (tid & 7) * 8;
      const int slot = t0 + sl;
      float kf[8], vf[8];
      if (slot < kv_end) {
        load8<KV_BF16>(kb, (int64_t)slot * HD + dc, kf);
        load8<KV_BF16>(vb, (int64_t)slot * HD + dc, vf);
      } else {
#pragma unroll
        for (int i = 0; i < 8; i++) kf[i] = vf[i] = 0.f;
      }
      *(float4*)(Ks + sl * FPAD + dc) = make_float4(kf[0], kf[1], kf[2], kf[3]);
      *(float4*)(Ks + sl * FPAD + dc + 4) = make_float4(kf[4], kf[5], kf[6], kf[7]);
      *(float4*)(Vs + sl * FPAD + dc) = make_float4(vf[0], vf[1], vf[2], vf[3]);
      *(float4*)(Vs + sl * FPAD + dc + 4) = make_float4(vf[4], vf[5], vf[6], vf[7]);
    }
    if (tid < KT) Ps[tid] = (t0 + tid < kv_end) ? sp[t0 + tid] : -1;
    __syncthreads();

    float s[4][4];
    float mt = -INFINITY;
#pragma unroll
    for (int sb = 0; sb < 4; sb++) {
      f32x4_t c = {0.f, 0.f, 0.f, 0.f};
      const float* krow = Ks + (sb * 16 + qcol) * FPAD + grp * 16;
#pragma unroll
      for (int kc = 0; kc < 16; kc += 4) {
        const float4 a4 = *(const float4*)(krow + kc);
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.x, qv[kc], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.y, qv[kc + 1], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.z, qv[kc + 2], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.w, qv[kc + 3], c, 0, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const bool ok = live_slot(Ps[sb * 16 + grp * 4 + j], cur, C);
        s[sb][j] = ok ? c[j] : -INFINITY;
        mt = fmaxf(mt, s[sb][j]);
      }
    }
    mt = col_max(mt);
    const float mn = fmaxf(m, mt);
    const float mu = mn == -INFINITY ? 0.f : mn;
    const float scale = __expf(m - mu);
    float ls = 0.f;
#pragma unroll
    for (int sb = 0; sb < 4; sb++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        s[sb][j] = __expf(s[sb][j] - mu);
        ls += s[sb][j];
      }
    l = l * scale + col_sum(ls);
    m = mn;
#pragma unroll
    for (int d = 0; d < 4; d++) acc[d] *= scale;
#pragma unroll
    for (int sb = 0; sb < 4; sb++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float* vrow = Vs + (sb * 16 + grp * 4 + j) * FPAD + qcol;
#pragma unroll
        for (int d = 0; d < 4; d++)
          acc[d] = __builtin_amdgcn_mfma_f32_16x16x4f32(vrow[d * 16], s[sb][j], acc[d], 0, 0, 0);
      }
  }
  if (!qvalid) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  float* op = out + row_at(out_rows, b, r) + h * HD;
#pragma unroll
  for (int d = 0; d < 4; d++)
    *(float4*)(op + d * 16 + grp * 4) =
        make_float4(acc[d][0] * inv, acc[d][1] * inv, acc[d][2] * inv, acc[d][3] * inv);
}

int launch_prefill_attention(mb_ctx* ctx, const RingView& ring, int B, int rows_max,
                             const void* q, int q_dtype, const Rows& q_rows, const int32_t* pos0,
                             const int32_t* n_rows, float* out, const Rows& out_rows) {
  if (q_dtype == MB_DT_BF16 && !ring.bf16)
    return fail(ctx, MB_ERR_ARG, "bf16 queries need a bf16 ring (the bf16 MFMA path)");
  if (B > 65535) return fail(ctx, MB_ERR_ARG, "at most 65535 sequences per prefill call");
  if (B == 0 || rows_max == 0) return MB_OK;
  dim3 grid((unsigned)((rows_max + QT - 1) / QT), H, (unsigned)B);
  if (q_dtype == MB_DT_BF16)
    hipLaunchKernelGGL(k_flash_bf16, grid, dim3(256), 0, ctx->stream, (const uint16_t*)q, q_rows,
                       pos0, n_rows, (const uint16_t*)ring.k, (const uint16_t*)ring.v, ring.sp,
                       ring.seq_stride, ring.C, out, out_rows);
  else if (ring.bf16)
    hipLaunchKernelGGL(k_flash_f32<true>, grid, dim3(256), 0, ctx->stream, (const float*)q, q_rows,
                       pos0, n_rows, ring.k, ring.v, ring.sp, ring.seq_stride, ring.C, out, out_rows);
  else
    hipLaunchKernelGGL(k_flash_f32<false>, grid, dim3(256), 0, ctx->stream, (const float*)q,
                       q_rows, pos0, n_rows, ring.k, ring.v, ring.sp, ring.seq_stride, ring.C, out,
                       out_rows);
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

}  // namespace mb
