// fp32 GEMM on MFMA for the projections of the decoder (gfx950):
//   C[M][N] (=, +=) epi(A[M][K] * W[K][N] + bias[N])
// with W row-major [K, N] exactly as the exported graph stores its MatMul
// initialisers (no transposition, docs section 9.1; GEMM_NT in
// kernels-batch.ts:156-184 and GEMV in kernels-decode.ts:127-142 compute the
// same product one output per lane).
//
// v_mfma_f32_16x16x4f32 keeps fp32 products, so the projections stay inside
// the 1e-4 logits bar; four waves in a 2x2 arrangement, each owning TM x TN
// blocks of 16x16.  A 16-deep K slice is staged in LDS per iteration: A as
// [m][k] and W transposed to [n][k], so a lane fetches the four k values it
// feeds to four consecutive MFMAs with one 16-byte LDS read (lane group g
// covers k = 4g .. 4g+3 of the slice; the sum over the slice is the same
// product in a different order).  The next slice's global loads are issued
// before the current slice's MFMAs.
#include <type_traits>
#include <utility>

#include "kv_types.h"
#include "lds_dma.h"
#include "mb_internal.h"
#include "pick.h"

namespace mb {

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

typedef float f32x8_t __attribute__((ext_vector_type(8)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// v = hi + lo in bf16 halves: hi = bf16(v), lo = bf16(v - hi), both rounded
// to nearest even.  The high halves are converted in pairs and their fp32
// values taken from the packed words (a shift, a mask), so a value costs
// three VALU operations.
__device__ __forceinline__ void split_bf16x8(const float (&v)[8], bf16x8_t& hi, bf16x8_t& lo) {
  uint32_t hw[4];
  f32x8_t rest;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const bf16x2_t h = __builtin_convertvector((f32x2_t){v[2 * i], v[2 * i + 1]}, bf16x2_t);
    hw[i] = __builtin_bit_cast(uint32_t, h);
    rest[2 * i] = v[2 * i] - __uint_as_float(hw[i] << 16);
    rest[2 * i + 1] = v[2 * i + 1] - __uint_as_float(hw[i] & 0xffff0000u);
  }
  hi = __builtin_bit_cast(bf16x8_t, make_uint4(hw[0], hw[1], hw[2], hw[3]));
  lo = __builtin_convertvector(rest, bf16x8_t);
}

constexpr int GBK = 16;   // K slice
constexpr int GPAD = 20;  // LDS row stride in floats (16 + 4)

// GELU with the tanh approximation, 0.5 v (1 + tanh(u)) with
// u = 0.7978845608 (v + 0.044715 v^3) (kernels-decode.ts:373-385), evaluated
// as v / (1 + exp(-2u)): 0.5 (1 + tanh(u)) is the logistic function of 2u, so
// the two forms are equal, and this one needs one exponential and no
// cancellation (exp(-2u) overflowing to inf gives -0, the limit).
__device__ __forceinline__ float gelu_tanh(float v) {
  const float u = 0.7978845608028654f * (v + 0.044715f * v * v * v);
  return v / (1.f + __expf(-2.f * u));
}

// Exact GELU 0.5 v (1 + erf(v / sqrt 2)), the codec decoder's activation,
// with erf from Abramowitz & Stegun 7.1.26 (|error| <= 1.5e-7), the form
// GELU_ERF evaluates (kernels-decode.ts:392-415).
__device__ __forceinline__ float erf_as(float x) {
  const float sgn = x >= 0.f ? 1.f : -1.f;
  const float ax = fabsf(x);
  const float t = 1.f / (1.f + 0.3275911f * ax);
  const float poly =
      ((((1.061405429f * t + -1.453152027f) * t + 1.421413741f) * t + -0.284496736f) * t +
       0.254829592f) * t;
  return sgn * (1.f - poly * expf(-ax * ax));
}
__device__ __forceinline__ float gelu_erf(float v) {
  return 0.5f * v * (1.f + erf_as(v * 0.7071067811865476f));
}

// Compile-time epilogue dispatch: f(std::integral_constant<int, EPI>{}).
template <class F>
static void with_epi(int epi, F f) {
  switch (epi) {
    case EPI_GELU: f(std::integral_constant<int, EPI_GELU>{}); break;
    case EPI_ADD: f(std::integral_constant<int, EPI_ADD>{}); break;
    case EPI_SCALE_ADD: f(std::integral_constant<int, EPI_SCALE_ADD>{}); break;
    case EPI_GELU_ERF: f(std::integral_constant<int, EPI_GELU_ERF>{}); break;
    default: f(std::integral_constant<int, EPI_STORE>{}); break;
  }
}

// f(std::integral_constant<int, i>{}) for i = 0 .. N - 1, so a body can index
// register arrays with a compile-time i however large it is (an unrolled loop
// may be left rolled, and the arrays then live in scratch memory).
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

template <int TM, int TN, int EPI>
__global__ __launch_bounds__(256) void k_gemm(const float* __restrict__ A, int64_t lda,
                                              const float* __restrict__ W, int N, int K,
                                              const float* __restrict__ bias, float* __restrict__ Cm,
                                              int64_t ldc, int M) {
  constexpr int BM = 2 * TM * 16, BN = 2 * TN * 16;
  constexpr int A_LOADS = BM * GBK / 4 / 256 > 0 ? BM * GBK / 4 / 256 : 1;  // float4 per thread
  constexpr int B_LOADS = BN * GBK / 4 / 256 > 0 ? BN * GBK / 4 / 256 : 1;
  __shared__ float As[BM * GPAD];
  __shared__ float Bt[BN * GPAD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col16 = lane & 15, g = lane >> 4;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

  f32x4_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  float4 ra[A_LOADS], rb[B_LOADS];
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_LOADS; i++) {
      const int idx = tid + i * 256;  // float4 index in the BM x 16 slice
      const int row = idx >> 2, kq = (idx & 3) * 4;
      ra[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (idx < BM * 4 && m0 + row < M) ra[i] = *(const float4*)(A + (int64_t)(m0 + row) * lda + k0 + kq);
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; i++) {
      const int idx = tid + i * 256;  // float4 index in the 16 x BN slice
      const int k = idx / (BN / 4), nq = (idx % (BN / 4)) * 4;
      rb[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (idx < BN * 4) rb[i] = *(const float4*)(W + (int64_t)(k0 + k) * N + n0 + nq);
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int i = 0; i < A_LOADS; i++) {
      const int idx = tid + i * 256;
      if (idx < BM * 4) *(float4*)(As + (idx >> 2) * GPAD + (idx & 3) * 4) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; i++) {
      const int idx = tid + i * 256;
      if (idx < BN * 4) {
        const int k = idx / (BN / 4), nq = (idx % (BN / 4)) * 4;
        Bt[(nq + 0) * GPAD + k] = rb[i].x;
        Bt[(nq + 1) * GPAD + k] = rb[i].y;
        Bt[(nq + 2) * GPAD + k] = rb[i].z;
        Bt[(nq + 3) * GPAD + k] = rb[i].w;
      }
    }
  };

  load(0);
  for (int k0 = 0; k0 < K; k0 += GBK) {
    __syncthreads();
    stash();
    __syncthreads();
    if (k0 + GBK < K) load(k0 + GBK);
    float4 a4[TM], b4[TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
      a4[i] = *(const float4*)(As + ((wm * TM + i) * 16 + col16) * GPAD + g * 4);
#pragma unroll
    for (int j = 0; j < TN; j++)
      b4[j] = *(const float4*)(Bt + ((wn * TN + j) * 16 + col16) * GPAD + g * 4);
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a4[i].x, b4[j].x, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a4[i].y, b4[j].y, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a4[i].z, b4[j].z, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a4[i].w, b4[j].w, acc[i][j], 0, 0, 0);
      }
  }

  // lane holds C[row0 + g*4 + r][col0 + col16] of each 16x16 block
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const int col = n0 + (wn * TN + j) * 16 + col16;
      const float bv = bias ? bias[col] : 0.f;  // the scale for EPI_SCALE_ADD
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int row = m0 + (wm * TM + i) * 16 + g * 4 + r;
        if (row >= M) continue;
        float* cp = Cm + (int64_t)row * ldc + col;
        float v;
        if (EPI == EPI_SCALE_ADD) {
          v = *cp + bv * acc[i][j][r];
        } else {
          v = acc[i][j][r] + bv;
          if (EPI == EPI_GELU) v = gelu_tanh(v);
          if (EPI == EPI_GELU_ERF) v = gelu_erf(v);
          if (EPI == EPI_ADD) v = *cp + v;
        }
        *cp = v;
      }
    }
}

template <int TM, int TN>
static void gemm_launch(mb_ctx* ctx, int epi, const float* A, int64_t lda, const float* W, int N,
                        int K, const float* bias, float* Cm, int64_t ldc, int M) {
  constexpr int BM = 2 * TM * 16, BN = 2 * TN * 16;
  dim3 grid((unsigned)(N / BN), (unsigned)((M + BM - 1) / BM));
  with_epi(epi, [&](auto e) {
    hipLaunchKernelGGL((k_gemm<TM, TN, decltype(e)::value>), grid, dim3(256), 0, ctx->stream, A,
                       lda, W, N, K, bias, Cm, ldc, M);
  });
}

// ---------------------------------------------------------------------------
// Streaming GEMM for decode-sized M (and mid-sized M with few tiles, see
// launch_gemm): W is read straight
// from HBM in the MFMA B-operand layout, one 16-byte load per lane, with no
// LDS staging.  In 16x16x4 step t of a 16-deep k group, lane (l16 = lane & 15,
// r = lane >> 4) feeds A[m0 + l16][k + 4r + t] and W[k + 4r + t][n + 4*l16 + j]
// to column block j (j = 0..3), so block j's MFMA column c is the real column
// n + 4c + j.  The products over t and r cover k .. k+15 exactly once, and a
// lane's four column blocks end up holding four adjacent real columns, which
// the epilogue writes as one float4.
//
// A workgroup owns MT rows x 64 columns and a k range; its four waves take
// four consecutive quarters of that range and add their sums through LDS in
// wave order.  Each wave streams its quarter in 16-deep chunks through ST
// register stages (chunk c in stage c % ST, ST - 1 chunks in flight ahead of
// the MFMAs).  Across workgroups the k range may be split S ways (gridDim.z):
// each split writes its sum to part[split][M][N] and k_gemm_reduce adds the
// splits in split order, so every output is the same fixed-order sum on every
// run.
constexpr int kStreamMaxM = 1024;
constexpr int kStreamChunk = 16;  // k rows per wave per pipeline stage
constexpr int kStreamMaxSplit = 8;

// epilogue4 on operands already in registers: b = bias (or the scale of
// EPI_SCALE_ADD), has_bias = whether there is one, c = the output's old value
template <int EPI>
__device__ __forceinline__ float4 epilogue_regs(float4 v, float4 b, bool has_bias, float4 c) {
  if (EPI == EPI_SCALE_ADD)
    return make_float4(c.x + b.x * v.x, c.y + b.y * v.y, c.z + b.z * v.z, c.w + b.w * v.w);
  if (has_bias) {
    v.x += b.x; v.y += b.y; v.z += b.z; v.w += b.w;
  }
  if (EPI == EPI_GELU) {
    v.x = gelu_tanh(v.x); v.y = gelu_tanh(v.y); v.z = gelu_tanh(v.z); v.w = gelu_tanh(v.w);
  }
  if (EPI == EPI_GELU_ERF) {
    v.x = gelu_erf(v.x); v.y = gelu_erf(v.y); v.z = gelu_erf(v.z); v.w = gelu_erf(v.w);
  }
  if (EPI == EPI_ADD) {
    v.x = c.x + v.x; v.y = c.y + v.y; v.z = c.z + v.z; v.w = c.w + v.w;
  }
  return v;
}

template <int EPI>
__device__ __forceinline__ float4 epilogue4(float4 v, const float* __restrict__ bias, int n,
                                            const float* cp) {
  if (EPI == EPI_SCALE_ADD) {  // bias holds the per-column scale
    const float4 c = *(const float4*)cp, sc = *(const float4*)(bias + n);
    return make_float4(c.x + sc.x * v.x, c.y + sc.y * v.y, c.z + sc.z * v.z, c.w + sc.w * v.w);
  }
  if (bias) {
    const float4 b = *(const float4*)(bias + n);
    v.x += b.x; v.y += b.y; v.z += b.z; v.w += b.w;
  }
  if (EPI == EPI_GELU) {
    v.x = gelu_tanh(v.x); v.y = gelu_tanh(v.y); v.z = gelu_tanh(v.z); v.w = gelu_tanh(v.w);
  }
  if (EPI == EPI_GELU_ERF) {
    v.x = gelu_erf(v.x); v.y = gelu_erf(v.y); v.z = gelu_erf(v.z); v.w = gelu_erf(v.w);
  }
  if (EPI == EPI_ADD) {
    const float4 c = *(const float4*)cp;
    v.x = c.x + v.x; v.y = c.y + v.y; v.z = c.z + v.z; v.w = c.w + v.w;
  }
  return v;
}

// Two floats stored, and four loaded, as device-coherent accesses
// (agent-scope relaxed atomics: sc1 stores and loads on gfx950).
__device__ __forceinline__ void store_coherent(float* p, float a, float b) {
  const uint64_t v = (uint64_t)__float_as_uint(a) | ((uint64_t)__float_as_uint(b) << 32);
  __hip_atomic_store((uint64_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float4 load_coherent(const float* p) {
  const uint64_t lo = __hip_atomic_load((const uint64_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t hi = __hip_atomic_load((const uint64_t*)p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float4(__uint_as_float((uint32_t)lo), __uint_as_float((uint32_t)(lo >> 32)),
                     __uint_as_float((uint32_t)hi), __uint_as_float((uint32_t)(hi >> 32)));
}

// The end of a streaming tile, shared by k_gemm_stream and k_gemm_x3: the
// four waves' partial sums of an MT x 64 tile (acc[i][j][e] = row 16i + 4r +
// e, column n + j of the wave's k range) are added in wave order and the
// tile is stored (S == 1: epilogue; S > 1: this split's partial).  With LNF,
// sx / sxx / x0 are the lane's sums of x - x0 and (x - x0)^2 over the A
// values it streamed (rows 16i + l16, k group r of every k step) and K is
// the row width.
//
// With tile counters (cnt, S > 1) the splits finish the tile themselves: each
// writes its partial and counts itself in on its tile's counter; the one that
// counts last adds the S partials in split order (whichever split that is,
// the sum is the same), applies the epilogue and sets the counter back to
// zero for the next launch.  Without counters k_gemm_reduce does that in a
// second launch.  The splits of a tile run on different XCDs, whose L2 caches
// are not coherent with each other; a device-scope fence would write back and
// invalidate the whole L2 of every workgroup's XCD, so instead the partials
// move with device-coherent accesses: agent-scope relaxed atomic stores and
// loads (global_store / global_load with sc1), the stores waited for
// (vmcnt(0)) before the counter's atomic add.
// The epilogue operands of a lane's stores, loaded before the k loop so the
// tile's end waits on no memory round trip of its own: the bias (or scale),
// the folded LayerNorm's c and d at columns n .. n+3, and for the residual
// epilogues the old output values of the rows 16i + 4r + wave it stores.
template <int MI>
struct EpiRegs {
  float4 b, cv, dv, c[MI];
};

template <int MI, int EPI, bool LNF>
__device__ __forceinline__ void epi_prefetch(EpiRegs<MI>& pre, const float* __restrict__ bias,
                                             const float* __restrict__ Cm, int64_t ldc, int M,
                                             const float* __restrict__ lnc,
                                             const float* __restrict__ lnd) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = blockIdx.x * 64 + 4 * (lane & 15), r = lane >> 4;
  const int m0 = blockIdx.y * (16 * MI);
  // no bias: any in-bounds address, the value is never used
  pre.b = *(const float4*)(bias ? bias + n : Cm);
  pre.cv = pre.dv = make_float4(0.f, 0.f, 0.f, 0.f);
  if (LNF) {
    pre.cv = *(const float4*)(lnc + n);
    pre.dv = *(const float4*)(lnd + n);
  }
  if (EPI == EPI_ADD || EPI == EPI_SCALE_ADD) {
#pragma unroll
    for (int i = 0; i < MI; i++)
      pre.c[i] = *(const float4*)(Cm + (int64_t)min(m0 + 16 * i + 4 * r + wave, M - 1) * ldc + n);
  }
}

template <int MI, int EPI, bool LNF, bool PRE = false>
__device__ __forceinline__ void stream_finish(f32x4_t (&acc)[MI][4], float (&sx)[MI],
                                              float (&sxx)[MI], const float (&x0)[MI], int K,
                                              const float* __restrict__ bias,
                                              float* __restrict__ Cm, int64_t ldc, int M,
                                              int N, float* __restrict__ part,
                                              const float* __restrict__ lnc,
                                              const float* __restrict__ lnd,
                                              int32_t* __restrict__ cnt = nullptr,
                                              const EpiRegs<MI>* pre = nullptr) {
  __shared__ float red[4][2][4][4][64];  // [wave][block][column block][element][lane]
  __shared__ float4 stat[LNF ? 4 : 1][MI][16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, r = lane >> 4;
  const int n = blockIdx.x * 64 + 4 * l16;
  const int m0 = blockIdx.y * (16 * MI);
  const int S = gridDim.z, split = blockIdx.z;
  if (LNF) {
    // a row's four k groups sit in lanes l16 + 16r: fold them, then lanes
    // r = 0 publish the wave's quarter of the row sums
#pragma unroll
    for (int i = 0; i < MI; i++) {
      sx[i] += __shfl_xor(sx[i], 16);
      sx[i] += __shfl_xor(sx[i], 32);
      sxx[i] += __shfl_xor(sxx[i], 16);
      sxx[i] += __shfl_xor(sxx[i], 32);
      if (lane < 16) stat[wave][i][lane] = make_float4(sx[i], sxx[i], x0[i], 0.f);
    }
  }

  // Add the four waves' sums and finish the tile on all four waves: the
  // partial tiles go through LDS two 16-row blocks at a time, and wave w
  // takes element w of every accumulator -- row 16i + 4r + w, columns
  // n .. n+3 -- summing the waves in wave order (the same order on every run).
  const float inv_k = 1.f / (float)K;
  float4 cv = make_float4(0.f, 0.f, 0.f, 0.f), dv = cv;
  if (PRE) {
    cv = pre->cv;
    dv = pre->dv;
  } else if (LNF) {
    cv = *(const float4*)(lnc + n);
    dv = *(const float4*)(lnd + n);
  }
#pragma unroll
  for (int i0 = 0; i0 < MI; i0 += 2) {
    if (i0 > 0) __syncthreads();  // the previous group's reads are done
#pragma unroll
    for (int ii = 0; ii < 2; ii++) {
      if (i0 + ii >= MI) break;
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int e = 0; e < 4; e++) red[wave][ii][j][e][lane] = acc[i0 + ii][j][e];
    }
    __syncthreads();
#pragma unroll
    for (int ii = 0; ii < 2; ii++) {
      const int i = i0 + ii;
      if (i >= MI) break;
      float o[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        float t = red[0][ii][j][wave][lane];
        t += red[1][ii][j][wave][lane];
        t += red[2][ii][j][wave][lane];
        t += red[3][ii][j][wave][lane];
        o[j] = t;
      }
      const int rl = 4 * r + wave;
      const int row = m0 + 16 * i + rl;
      if (LNF) {
        const float4 q0 = stat[0][i][rl], q1 = stat[1][i][rl], q2 = stat[2][i][rl], q3 = stat[3][i][rl];
        const float s1 = ((q0.x + q1.x) + q2.x) + q3.x;
        const float s2 = ((q0.y + q1.y) + q2.y) + q3.y;
        const float ms = s1 * inv_k;  // mean of x - x0
        const float var = fmaxf(s2 * inv_k - ms * ms, 0.f);
        const float mean = q0.z + ms;
        const float rstd = 1.f / sqrtf(var + 1e-5f);
        o[0] = rstd * (o[0] - mean * cv.x) + dv.x;
        o[1] = rstd * (o[1] - mean * cv.y) + dv.y;
        o[2] = rstd * (o[2] - mean * cv.z) + dv.z;
        o[3] = rstd * (o[3] - mean * cv.w) + dv.w;
      }
      if (row >= M) continue;
      if (S > 1) {
        float* pp = part + ((int64_t)split * M + row) * N + n;
        if (cnt) {
          store_coherent(pp, o[0], o[1]);
          store_coherent(pp + 2, o[2], o[3]);
        } else {
          *(float4*)pp = make_float4(o[0], o[1], o[2], o[3]);
        }
        continue;
      }
      float* cp = Cm + (int64_t)row * ldc + n;
      const float4 ov = make_float4(o[0], o[1], o[2], o[3]);
      if (PRE)
        *(float4*)cp = epilogue_regs<EPI>(ov, pre->b, bias != nullptr, pre->c[i]);
      else
        *(float4*)cp = epilogue4<EPI>(ov, bias, n, cp);
    }
  }
  if (S == 1 || !cnt) return;
  __shared__ int last;
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0): this split's partial stores are done
  __syncthreads();
  const int tile = blockIdx.y * gridDim.x + blockIdx.x;
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(&cnt[tile], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == S - 1;
  __syncthreads();
  if (!last) return;
  const int64_t stride = (int64_t)M * N;
#pragma unroll
  for (int u = 0; u < MI; u++) {
    const int q = threadIdx.x + 256 * u;  // float4 of the 16 MI x 64 tile
    const int row = m0 + (q >> 4), col = blockIdx.x * 64 + (q & 15) * 4;
    if (row >= M) continue;
    const float* pp = part + (int64_t)row * N + col;
    float4 sum = load_coherent(pp);
    for (int sp = 1; sp < S; sp++) {
      const float4 v = load_coherent(pp + sp * stride);
      sum.x += v.x; sum.y += v.y; sum.z += v.z; sum.w += v.w;
    }
    float* cp = Cm + (int64_t)row * ldc + col;
    *(float4*)cp = epilogue4<EPI>(sum, bias, col, cp);
  }
  if (threadIdx.x == 0) __hip_atomic_store(&cnt[tile], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// With LNF the A rows are the raw residual stream x and the LayerNorm in
// front of the projection is folded in: W holds diag(gamma) * W, and
//   LN(x) W = rstd (x W' - mean c) + d,   c = 1 W',  d = beta W
// (c, d from k_fold_ln), so the kernel only needs each row's mean and rstd.
// It accumulates them from the A values it streams anyway -- sums of
// x - x0 and (x - x0)^2 with x0 = x[row][0], so the variance does not cancel
// -- which requires the workgroup to see the whole row (S == 1, K == 768).
template <int MT, int ST, int EPI, bool LNF, bool TILED>
__global__ __launch_bounds__(256) void k_gemm_stream(
    const float* __restrict__ A, int64_t lda, const float* __restrict__ W, int N, int kw,
    const float* __restrict__ bias, float* __restrict__ Cm, int64_t ldc, int M,
    float* __restrict__ part, const float* __restrict__ lnc, const float* __restrict__ lnd) {
  constexpr int MI = MT / 16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, r = lane >> 4;
  const int n = blockIdx.x * 64 + 4 * l16;
  const int m0 = blockIdx.y * MT;
  const int S = gridDim.z, split = blockIdx.z;

  f32x4_t acc[MI][4];
#pragma unroll
  for (int i = 0; i < MI; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float x0[MI], sx[MI], sxx[MI];

  {
    // Rows past M read row M - 1 (in bounds, no branch); their sums are
    // never stored.
    const float* Ap[MI];
#pragma unroll
    for (int i = 0; i < MI; i++) Ap[i] = A + (int64_t)min(m0 + 16 * i + l16, M - 1) * lda + 4 * r;
    if (LNF) {
#pragma unroll
      for (int i = 0; i < MI; i++) {
        x0[i] = Ap[i][-4 * r];
        sx[i] = 0.f;
        sxx[i] = 0.f;
      }
    }
    // TILED: W column-block-major, [N / 64][K][64] (launch_tile_w), so a
    // workgroup streams one contiguous strip instead of 256 bytes of every row
    const int64_t wstride = TILED ? 64 : N;
    const float* Wp = TILED ? W + (int64_t)blockIdx.x * 64 * (4 * S * kw) + 4 * r * 64 + 4 * l16
                            : W + (int64_t)4 * r * N + n;
    float4 a[ST][MI], w[ST][4];
    auto load = [&](int st, int k) {
#pragma unroll
      for (int t = 0; t < 4; t++) w[st][t] = *(const float4*)(Wp + (int64_t)(k + t) * wstride);
#pragma unroll
      for (int i = 0; i < MI; i++) a[st][i] = *(const float4*)(Ap[i] + k);
    };
    auto mma = [&](int st) {
      if (LNF) {
#pragma unroll
        for (int i = 0; i < MI; i++) {
          const float e0 = a[st][i].x - x0[i], e1 = a[st][i].y - x0[i];
          const float e2 = a[st][i].z - x0[i], e3 = a[st][i].w - x0[i];
          sx[i] += (e0 + e1) + (e2 + e3);
          sxx[i] = fmaf(e0, e0, fmaf(e1, e1, fmaf(e2, e2, fmaf(e3, e3, sxx[i]))));
        }
      }
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const float4 wt = w[st][t];
#pragma unroll
        for (int i = 0; i < MI; i++) {
          const float av = t == 0 ? a[st][i].x : t == 1 ? a[st][i].y : t == 2 ? a[st][i].z : a[st][i].w;
          acc[i][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, wt.x, acc[i][0], 0, 0, 0);
          acc[i][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, wt.y, acc[i][1], 0, 0, 0);
          acc[i][2] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, wt.z, acc[i][2], 0, 0, 0);
          acc[i][3] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, wt.w, acc[i][3], 0, 0, 0);
        }
      }
    };
    // Prefetch ST - 1 chunks, then per chunk: issue the load ST - 1 ahead and
    // run the MFMAs of the oldest stage.  Past the end the last chunk is
    // re-read (in bounds, unused), so the loop body has no load branch and
    // each stage's MFMAs wait only for that stage's loads.  The main loop
    // runs whole groups of ST chunks with no branch inside: a stage skipped
    // on some path would leave its load pending at the loop header, and the
    // compiler then drains every load in flight there (vmcnt(0)) on every
    // iteration.  The nc mod ST chunks left over (already in flight) follow.
    const int k0 = (split * 4 + wave) * kw, k1 = k0 + kw, nc = kw / kStreamChunk;
#pragma unroll
    for (int s = 0; s < ST - 1; s++) load(s, min(k0 + s * kStreamChunk, k1 - kStreamChunk));
    int c = 0;
    for (; c + ST <= nc; c += ST) {
#pragma unroll
      for (int s = 0; s < ST; s++) {
        load((s + ST - 1) % ST, min(k0 + (c + s + ST - 1) * kStreamChunk, k1 - kStreamChunk));
        __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the MFMAs
        mma(s);
      }
    }
#pragma unroll
    for (int s = 0; s < ST - 1; s++)
      if (c + s < nc) mma(s);
  }

  stream_finish<MI, EPI, LNF>(acc, sx, sxx, x0, 4 * S * kw, bias, Cm, ldc, M, N, part, lnc, lnd);
}

// ---------------------------------------------------------------------------
// Split-bf16 streaming GEMM, the decode-sized projections of bf16-KV
// contexts.  The streaming kernel's tiling (MT rows x 64 columns per
// workgroup, the four waves on consecutive quarters of each split's k range,
// stream_finish), with each fp32 product taken as three bf16 products on
// v_mfma_f32_16x16x32_bf16: a = ah + al and w = wh + wl with ah = bf16(a),
// al = bf16(a - ah) (likewise w), and a w ~ al wh + ah wl + ah wh summed in
// fp32.  What is left out -- al wl and the rounding of al and wl -- is
// within about 2^-16 |a w| per product (an fp32 product keeps 2^-24).  A
// 32-deep k block costs three 16-cycle MFMAs where fp32 takes eight of 32
// cycles, for the same bytes streamed: W is split once into its two bf16
// halves (launch_split_w), A on the fly.
//
// Wx (launch_split_w): per 64-column strip s and 32-deep k block kb, 8 KB as
// [column block j][half h (hi, lo)][lane][8 bf16], lane l of block j holding
// W[32 kb + 8 (l >> 4) + t][64 s + 4 (l & 15) + j] for t = 0..7: the B
// operand of one MFMA, one 16-byte load per lane.  MFMA column c of block j
// is real column 4c + j, as in the streaming kernel, so stream_finish writes
// four adjacent columns per lane.
//
// A: lane (l16, r) feeds A[row 16i + l16][32 kb + 8r .. + 7] to the MFMAs,
// but loading that directly puts 16 rows (16 cache lines) in each quarter
// wave of a load -- four times the W loads' lines per byte, and measured the
// slower stream.  So A is loaded row-contiguous (8 lanes per 128-byte row
// line, load p covering rows 8p .. 8p + 7 of the tile's 32-deep block) and
// each wave passes its block through its own slice of LDS: written 16-byte
// chunk c of row R at chunk c ^ (R & 7), read back as the MFMA fragments
// (both conflict-free).  A wave only reads what it wrote, so this needs no
// barrier; the compiler sees every load and orders the LDS traffic.
constexpr int kX3Block = 32;  // k per MFMA step
constexpr int kX3BlockU4 = 512;  // uint4 per 64-column x 32-deep block (8 KB)

//
// W1 (bf16 weight storage): W is bf16-exact, so it has no remainder half:
// the copy holds only the high halves ([column block j][lane][8], 4 KB per
// 64-column x 32-deep block, launch_split_w1) and each product is the two
// bf16 products al w + ah w.  GAM: the LayerNorm's gamma multiplies A on the
// fly (A's LayerNorm sums stay those of the raw rows), gamma[32 kb + 8 r ..
// + 7] loaded with each block.
template <int MT, int ST, int EPI, bool LNF, bool W1 = false, bool GAM = false>
__global__ __launch_bounds__(256) void k_gemm_x3(
    const float* __restrict__ A, int64_t lda, const uint4* __restrict__ Wx, int N, int kw,
    const float* __restrict__ bias, float* __restrict__ Cm, int64_t ldc, int M,
    float* __restrict__ part, const float* __restrict__ lnc, const float* __restrict__ lnd,
    int32_t* __restrict__ cnt, const float* __restrict__ gamma) {
  constexpr int BU4 = W1 ? kX3BlockU4 / 2 : kX3BlockU4;  // uint4 per 64 x 32 weight block
  constexpr int NH = W1 ? 1 : 2;                          // weight halves
  constexpr int MI = MT / 16, AL = MT / 8;  // row blocks; A loads per block (8 rows each)
  __shared__ f32x4_t Ablk[4][MT * 8];       // per wave: MT rows x 8 chunks of 4 floats
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, r = lane >> 4;
  const int m0 = blockIdx.y * MT;
  const int S = gridDim.z, split = blockIdx.z;
  const int K = 4 * S * kw;

  EpiRegs<MI> pre;
  epi_prefetch<MI, EPI, LNF>(pre, bias, Cm, ldc, M, lnc, lnd);
  f32x4_t acc[MI][4];
#pragma unroll
  for (int i = 0; i < MI; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float x0[MI], sx[MI], sxx[MI];

  {
    // Rows past M read row M - 1 (in bounds, no branch); their sums are
    // never stored.
    if (LNF) {
#pragma unroll
      for (int i = 0; i < MI; i++) {
        x0[i] = A[(int64_t)min(m0 + 16 * i + l16, M - 1) * lda];
        sx[i] = 0.f;
        sxx[i] = 0.f;
      }
    }
    // row-contiguous load order: load p, lane (crow, cchunk) = row 8p + crow,
    // chunk cchunk; element offsets fit 32 bits (launch_gemm_x3 checks M lda)
    const int crow = lane >> 3, cchunk = lane & 7;
    uint32_t aoff[AL];
#pragma unroll
    for (int p = 0; p < AL; p++) aoff[p] = (uint32_t)(min(m0 + 8 * p + crow, M - 1) * lda + 4 * cchunk);
    // (8p + crow) & 7 == crow and (16i + l16) & 7 == l16 & 7: one swizzled
    // base per lane, rows apart by immediate offsets
    f32x4_t* const Aw = Ablk[wave] + crow * 8 + (cchunk ^ crow);
    const f32x4_t* const Ar0 = Ablk[wave] + l16 * 8 + ((2 * r) ^ (l16 & 7));
    const f32x4_t* const Ar1 = Ablk[wave] + l16 * 8 + ((2 * r + 1) ^ (l16 & 7));
    const uint4* Wb = Wx + (int64_t)blockIdx.x * (K / kX3Block) * BU4 + lane;
    f32x4_t a[ST][AL];
    uint4 w[ST][4][NH];
    f32x4_t g[ST][2];
    auto load = [&](auto st_, int kb) {
      constexpr int st = decltype(st_)::value;
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int h = 0; h < NH; h++) w[st][j][h] = Wb[(int64_t)kb * BU4 + (NH * j + h) * 64];
#pragma unroll
      for (int p = 0; p < AL; p++) a[st][p] = *(const f32x4_t*)(A + kb * kX3Block + aoff[p]);
      if (GAM) {
        g[st][0] = *(const f32x4_t*)(gamma + kb * kX3Block + 8 * r);
        g[st][1] = *(const f32x4_t*)(gamma + kb * kX3Block + 8 * r + 4);
      }
    };
    auto mma = [&](auto st_) {
      constexpr int st = decltype(st_)::value;
#pragma unroll
      for (int p = 0; p < AL; p++) Aw[p * 64] = a[st][p];
      bf16x8_t ah[MI], al[MI];
#pragma unroll
      for (int i = 0; i < MI; i++) {
        const f32x4_t v0 = Ar0[i * 128], v1 = Ar1[i * 128];
        float v[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
        if (LNF) {
          float s1 = 0.f, s2 = sxx[i];
#pragma unroll
          for (int e = 0; e < 8; e++) {
            const float d = v[e] - x0[i];
            s1 += d;
            s2 = fmaf(d, d, s2);
          }
          sx[i] += s1;
          sxx[i] = s2;
        }
        if (GAM) {
#pragma unroll
          for (int e = 0; e < 4; e++) {
            v[e] = __fmul_rn(v[e], g[st][0][e]);
            v[e + 4] = __fmul_rn(v[e + 4], g[st][1][e]);
          }
        }
        split_bf16x8(v, ah[i], al[i]);
      }
      // the three products of every (i, j) in turn, so consecutive MFMAs are
      // independent; each accumulator takes them in the same order
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const bf16x8_t wh = __builtin_bit_cast(bf16x8_t, w[st][j][0]);
#pragma unroll
        for (int i = 0; i < MI; i++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[i], wh, acc[i][j], 0, 0, 0);
      }
      if constexpr (!W1) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const bf16x8_t wl = __builtin_bit_cast(bf16x8_t, w[st][j][NH - 1]);
#pragma unroll
          for (int i = 0; i < MI; i++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[i], wl, acc[i][j], 0, 0, 0);
        }
      }
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const bf16x8_t wh = __builtin_bit_cast(bf16x8_t, w[st][j][0]);
#pragma unroll
        for (int i = 0; i < MI; i++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[i], wh, acc[i][j], 0, 0, 0);
      }
    };
    // The streaming kernel's pipeline over 32-deep k blocks: ST - 1 blocks in
    // flight, whole groups of ST with no branch inside, the rest after.
    const int nc = kw / kX3Block, kb0 = (split * 4 + wave) * nc, kb1 = kb0 + nc - 1;
    static_for<ST - 1>([&](auto s_) {
      constexpr int s = decltype(s_)::value;
      load(std::integral_constant<int, s>{}, min(kb0 + s, kb1));
    });
    int c = 0;
    for (; c + ST <= nc; c += ST) {
      static_for<ST>([&](auto s_) {
        constexpr int s = decltype(s_)::value;
        load(std::integral_constant<int, (s + ST - 1) % ST>{}, min(kb0 + c + s + ST - 1, kb1));
        __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the MFMAs
        mma(s_);
      });
    }
    static_for<ST - 1>([&](auto s_) {
      if (c + decltype(s_)::value < nc) mma(s_);
    });
  }

  stream_finish<MI, EPI, LNF, true>(acc, sx, sxx, x0, K, bias, Cm, ldc, M, N, part, lnc, lnd, cnt,
                                    &pre);
}

// C = epi(sum over splits of part, in split order, + bias); one float4 per thread.
template <int EPI>
__global__ __launch_bounds__(256) void k_gemm_reduce(const float* __restrict__ part, int S, int M,
                                                     int N, const float* __restrict__ bias,
                                                     float* __restrict__ Cm, int64_t ldc) {
  const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int q = N / 4;
  if (u >= (int64_t)M * q) return;
  const int row = (int)(u / q), col = (int)(u % q) * 4;
  const float* p = part + (int64_t)row * N + col;
  const int64_t stride = (int64_t)M * N;
  float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
  int s = 0;
  for (; s + 4 <= S; s += 4) {
    float4 v[4];
#pragma unroll
    for (int t = 0; t < 4; t++) v[t] = *(const float4*)(p + (s + t) * stride);
#pragma unroll
    for (int t = 0; t < 4; t++) {
      sum.x += v[t].x; sum.y += v[t].y; sum.z += v[t].z; sum.w += v[t].w;
    }
  }
  for (; s < S; s++) {
    const float4 v = *(const float4*)(p + s * stride);
    sum.x += v.x; sum.y += v.y; sum.z += v.z; sum.w += v.w;
  }
  float* cp = Cm + (int64_t)row * ldc + col;
  *(float4*)cp = epilogue4<EPI>(sum, bias, col, cp);
}

// part_ext (optional, part_cap floats) holds the split-K partials instead of
// the context's growable scratch.
template <int MT, int ST, bool LNF>
static int stream_launch(mb_ctx* ctx, int epi, const float* A, int64_t lda, const float* W, int N,
                         int K, const float* bias, float* Cm, int64_t ldc, int M, int S,
                         const float* lnc, const float* lnd, bool tiled, float* part_ext = nullptr,
                         size_t part_cap = 0) {
  const int tx = N / 64, ty = (M + MT - 1) / MT;
  float* part = nullptr;
  if (S > 1) {
    const size_t need = (size_t)S * M * N;
    if (part_ext) {
      if (need > part_cap)
        return fail(ctx, MB_ERR_ARG, "gemm split-K partials need %zu floats, the buffer holds %zu",
                    need, part_cap);
      part = part_ext;
    } else {
      part = (float*)scratch(ctx, "gemm_part", need * 4);
    }
    if (!part) return fail(ctx, MB_ERR_NOMEM, "gemm split-K partials (%d x %d x %d)", S, M, N);
  }
  dim3 grid((unsigned)tx, (unsigned)ty, (unsigned)S);
  const int kw = K / (4 * S);
  if (LNF && epi != EPI_STORE && epi != EPI_GELU && epi != EPI_GELU_ERF)
    return fail(ctx, MB_ERR_ARG, "folded LayerNorm gemm has no epilogue %d", epi);
  with_epi(epi, [&](auto e) {
    constexpr int E = decltype(e)::value;
    // folded weights (LNF) always come tiled from launch_fold_ln
    if constexpr (LNF) {
      if constexpr (E == EPI_STORE || E == EPI_GELU || E == EPI_GELU_ERF)
        hipLaunchKernelGGL((k_gemm_stream<MT, ST, E, true, true>), grid, dim3(256), 0, ctx->stream,
                           A, lda, W, N, kw, bias, Cm, ldc, M, part, lnc, lnd);
    } else if (tiled) {
      hipLaunchKernelGGL((k_gemm_stream<MT, ST, E, false, true>), grid, dim3(256), 0, ctx->stream,
                         A, lda, W, N, kw, bias, Cm, ldc, M, part, lnc, lnd);
    } else {
      hipLaunchKernelGGL((k_gemm_stream<MT, ST, E, false, false>), grid, dim3(256), 0, ctx->stream,
                         A, lda, W, N, kw, bias, Cm, ldc, M, part, lnc, lnd);
    }
  });
  if (S > 1) {
    const unsigned rb = (unsigned)(((int64_t)M * (N / 4) + 255) / 256);
    with_epi(epi, [&](auto e) {
      hipLaunchKernelGGL(k_gemm_reduce<decltype(e)::value>, dim3(rb), dim3(256), 0, ctx->stream,
                         part, S, M, N, bias, Cm, ldc);
    });
  }
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

// Row tile and k split of the streaming kernel for an M x N x K projection
// (see launch_gemm); `whole_rows` forbids a split (LayerNorm folding needs
// every k of a row in one workgroup).
static void stream_shape(int M, int N, int K, bool whole_rows, int& mt, int& S) {
  const int tx = N / 64;
  auto tiles = [&](int m) { return (int64_t)tx * ((M + m - 1) / m); };
  mt = 64;
  for (int cand : {16, 32, 48}) {
    if (tiles(cand) <= 256) {
      mt = cand;
      break;
    }
  }
  S = 1;
  if (K >= 2048 && !whole_rows) {
    // From 96 rows up, 32-row tiles split over k read each W column block
    // half as often as 16-row tiles at the same workgroup count.  Measured on
    // 768 x 3072 (fc_out, W from HBM) at M = 96 / 128 / 192 / 256: 12.5 /
    // 13.8 / 15.7 / 19.5 us, where 16-row tiles at their best split took
    // 16.2 / 16.0 / 22.4 / 23.1 us; at M <= 64 the 16-row tiles stay ahead.
    if (mt == 16 && M >= 96 && tiles(32) * 2 <= 256) mt = 32;
    for (int s = kStreamMaxSplit; s > 1; s--) {
      if (K % (4 * kStreamChunk * s) == 0 && tiles(mt) * s <= 256) {
        S = s;
        break;
      }
    }
  }
}

// Per-tile arrival counters of the split-K tiles that finish themselves
// (stream_finish), zero between launches: zeroed once when allocated (a fill
// kernel), and each tile's last split sets its counter back to zero.
constexpr int kTileCounters = 8192;
static int tile_counters(mb_ctx* ctx, int32_t*& cnt) {
  const bool fresh = !ctx->scratch["gemm_tile_cnt"].ptr;
  cnt = (int32_t*)scratch(ctx, "gemm_tile_cnt", kTileCounters * sizeof(int32_t));
  if (!cnt) return fail(ctx, MB_ERR_NOMEM, "split gemm tile counters");
  return fresh ? launch_fill_i32(ctx, cnt, kTileCounters, 0) : MB_OK;
}

template <int MT, int ST, bool LNF, bool W1 = false, bool GAM = false>
static int x3_launch(mb_ctx* ctx, int epi, const float* A, int64_t lda, const uint4* Wx, int N,
                     int K, const float* bias, float* Cm, int64_t ldc, int M, int S,
                     const float* lnc, const float* lnd, const float* gamma = nullptr) {
  const dim3 grid((unsigned)(N / 64), (unsigned)((M + MT - 1) / MT), (unsigned)S);
  float* part = nullptr;
  int32_t* cnt = nullptr;
  if (S > 1) {
    // its own buffer: only device-coherent accesses ever touch it
    part = (float*)scratch(ctx, "gemm_part_coherent", (size_t)S * M * N * 4);
    if (!part) return fail(ctx, MB_ERR_NOMEM, "gemm split-K partials (%d x %d x %d)", S, M, N);
    if ((int64_t)grid.x * grid.y > kTileCounters)
      return fail(ctx, MB_ERR_ARG, "split gemm has %u tiles, the counters cover %d", grid.x * grid.y,
                  kTileCounters);
    int rc = tile_counters(ctx, cnt);
    if (rc) return rc;
  }
  const int kw = K / (4 * S);
  with_epi(epi, [&](auto e) {
    constexpr int E = decltype(e)::value;
    if constexpr (LNF) {
      if constexpr (E == EPI_STORE || E == EPI_GELU || E == EPI_GELU_ERF)
        hipLaunchKernelGGL((k_gemm_x3<MT, ST, E, true, W1, GAM>), grid, dim3(256), 0, ctx->stream,
                           A, lda, Wx, N, kw, bias, Cm, ldc, M, part, lnc, lnd, cnt, gamma);
    } else if constexpr (!GAM) {
      hipLaunchKernelGGL((k_gemm_x3<MT, ST, E, false, W1, false>), grid, dim3(256), 0, ctx->stream,
                         A, lda, Wx, N, kw, bias, Cm, ldc, M, part, lnc, lnd, cnt, gamma);
    }
  });
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

// ---------------------------------------------------------------------------
// Split-bf16 products at prefill-sized M (bf16-KV contexts, the codec on bf16
// rings): the product of k_gemm_x3 -- each fp32 product as bf16 products of
// high and low halves (three, or two with bf16 weights), within about 2^-16 of
// the fp32 product, fp32 sums -- on the same split weight copies, tiled for
// many rows.  A workgroup owns BM = 32 MI rows x 128 columns (two 64-column
// weight strips) over all of k, so it adds nothing across workgroups or
// waves: wave (wm, wn) owns rows wm 16 MI .. + 16 MI and strip wn, MI x 4
// MFMA blocks, and sums its k blocks in order.  Per 32-deep k block the
// workgroup's A rows (fp32) and both strips' weight blocks reach LDS by the
// load unit (global_load_lds_dwordx4, 1 KB per wave instruction, the pieces
// dealt evenly over the four waves), D stages deep; one barrier per block
// publishes a stage and frees the one the next loads overwrite.  A lands in
// the swizzled [row][16-byte chunk] layout of k_gemm_x3's fragment reads,
// the weights as they lie in memory (16 bytes per lane = its B operand).
// With LNF the LayerNorm in front is folded in exactly as there: the waves
// add up x - x0 and (x - x0)^2 of their rows from the A values they read
// (x0 = x[row][0]) and apply rstd and mean per row in the epilogue, which
// takes a row's sums from the lane that formed them (a lane swap).  GAM: the
// LayerNorm scale applied to A on the fly (bf16 weights), from a per-wave
// copy of the block's 32 scales in the stage.
template <int MI, bool W1, bool GAM>
constexpr int xt_stage_bytes() {
  return (4 * MI + 8 * (W1 ? 1 : 2)) * 1024 + (GAM ? 4 * 256 : 0);
}

template <int MI, int D, int EPI, bool LNF, bool W1 = false, bool GAM = false, int OCC = 2>
__global__ __launch_bounds__(256, OCC) void k_gemm_xt(
    const float* __restrict__ A, int64_t lda, const uint4* __restrict__ Wx, int N, int K,
    const float* __restrict__ bias, float* __restrict__ Cm, int64_t ldc, int M,
    const float* __restrict__ lnc, const float* __restrict__ lnd,
    const float* __restrict__ gamma) {
  constexpr int NH = W1 ? 1 : 2;                          // weight halves
  constexpr int BU4 = W1 ? kX3BlockU4 / 2 : kX3BlockU4;  // uint4 per 64 x 32 weight block
  constexpr int BM = 32 * MI;
  constexpr int AP = BM / 8;       // A pieces per block (8 rows of 128 bytes each)
  constexpr int WP = 2 * 4 * NH;   // weight pieces per block (two strips)
  static_assert((AP + WP) % 4 == 0, "the pieces divide over the four waves");
  constexpr int PW = (AP + WP) / 4;              // pieces per wave per block
  constexpr int LOADS = PW + (GAM ? 1 : 0);      // its loads per block
  constexpr int STAGE = xt_stage_bytes<MI, W1, GAM>();
  static_assert(D >= 2 && (D - 2) * LOADS <= 63, "vmcnt holds at most 63 loads");
  __shared__ __align__(16) char lds[D * STAGE];
  // the wave index in a scalar register: every choice made from it below is
  // a scalar branch, not a masked one
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int l16 = lane & 15, r = lane >> 4;
  const int m0 = blockIdx.y * BM, strip0 = 2 * blockIdx.x;
  const int nkb = K / kX3Block;

  f32x4_t acc[MI][4];
#pragma unroll
  for (int i = 0; i < MI; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float x0[MI], sx[MI], sxx[MI];
  if (LNF) {
    // rows past M read row M - 1 (in bounds); their sums are never stored
#pragma unroll
    for (int i = 0; i < MI; i++) {
      x0[i] = A[(int64_t)min(m0 + wm * 16 * MI + 16 * i + l16, M - 1) * lda];
      sx[i] = 0.f;
      sxx[i] = 0.f;
    }
  }
  // This wave's pieces of a block: piece wave * PW + t.  An A piece p holds
  // rows 8p .. 8p + 7: slot 64 p + l of the stage gets row 8p + (l >> 3),
  // chunk (l & 7) ^ (l >> 3) (byte offsets fit 32 bits: the launcher checks
  // M lda); a weight piece q holds piece q mod 4 NH of strip q / (4 NH).
  uint32_t poff[PW];
  int64_t pbase[PW];  // A pieces: 0; weight pieces: uint4 offset of block 0
#pragma unroll
  for (int t = 0; t < PW; t++) {
    const int pi = wave * PW + t;
    if (pi < AP) {
      const int row = min(m0 + 8 * pi + (lane >> 3), M - 1);
      poff[t] = (uint32_t)((row * lda + 4 * ((lane & 7) ^ (lane >> 3))) * 4);
      pbase[t] = -1;
    } else {
      const int q = pi - AP, s = q / (4 * NH), qq = q % (4 * NH);
      poff[t] = (uint32_t)(lane * 16);
      pbase[t] = (int64_t)(strip0 + s) * nkb * BU4 + qq * 64;
    }
  }
  auto issue = [&](int st, int kb) {
    char* const sp = lds + st * STAGE;
#pragma unroll
    for (int t = 0; t < PW; t++) {
      const uint32_t dst = lds_addr(sp + (wave * PW + t) * 1024);
      if (pbase[t] < 0)
        dma16(A + kb * kX3Block, poff[t], dst);
      else
        dma16(Wx + pbase[t] + (int64_t)kb * BU4, poff[t], dst);
    }
    if (GAM)
      dma4(gamma + kb * kX3Block, min(lane, 31) * 4, lds_addr(sp + (AP + WP) * 1024 + wave * 256));
  };
  auto mma = [&](int st) {
    const char* const sp = lds + st * STAGE;
    uint4 w[4][NH];
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int h = 0; h < NH; h++)
        w[j][h] = *(const uint4*)(sp + (AP + wn * 4 * NH + NH * j + h) * 1024 + 16 * lane);
    f32x4_t g0 = {}, g1 = {};
    if (GAM) {
      const float* gp = (const float*)(sp + (AP + WP) * 1024 + wave * 256);
      g0 = *(const f32x4_t*)(gp + 8 * r);
      g1 = *(const f32x4_t*)(gp + 8 * r + 4);
    }
    const f32x4_t* const Ab = (const f32x4_t*)sp + (wm * 16 * MI + l16) * 8;
    bf16x8_t ah[MI], al[MI];
#pragma unroll
    for (int i = 0; i < MI; i++) {
      const f32x4_t v0 = Ab[i * 128 + ((2 * r) ^ (l16 & 7))];
      const f32x4_t v1 = Ab[i * 128 + ((2 * r + 1) ^ (l16 & 7))];
      float v[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
      if (LNF) {
        float s1 = 0.f, s2 = sxx[i];
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const float d = v[e] - x0[i];
          s1 += d;
          s2 = fmaf(d, d, s2);
        }
        sx[i] += s1;
        sxx[i] = s2;
      }
      if (GAM) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
          v[e] = __fmul_rn(v[e], g0[e]);
          v[e + 4] = __fmul_rn(v[e + 4], g1[e]);
        }
      }
      split_bf16x8(v, ah[i], al[i]);
    }
    // the products in k_gemm_x3's order: lo x hi, hi x lo, hi x hi
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const bf16x8_t wh = __builtin_bit_cast(bf16x8_t, w[j][0]);
#pragma unroll
      for (int i = 0; i < MI; i++)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[i], wh, acc[i][j], 0, 0, 0);
    }
    if constexpr (!W1) {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const bf16x8_t wl = __builtin_bit_cast(bf16x8_t, w[j][NH - 1]);
#pragma unroll
        for (int i = 0; i < MI; i++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[i], wl, acc[i][j], 0, 0, 0);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const bf16x8_t wh = __builtin_bit_cast(bf16x8_t, w[j][0]);
#pragma unroll
      for (int i = 0; i < MI; i++)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[i], wh, acc[i][j], 0, 0, 0);
    }
  };
#pragma unroll
  for (int s = 0; s < D - 1; s++) issue(s, min(s, nkb - 1));
  for (int c = 0; c < nkb; c++) {
    MB_WAIT_VMCNT64((D - 2) * LOADS);  // this wave's pieces of block c have landed
    __syncthreads();  // every wave's have, and no wave still reads stage (c - 1) mod D
    issue((c + D - 1) % D, min(c + D - 1, nkb - 1));  // past the end: reloads, never read
    mma(c % D);
  }
  MB_WAIT_VMCNT(0);  // the reloads past the end have landed before the workgroup ends

  // lane (l16, r) holds rows 16 i + 4 r + e, columns 4 l16 + j of its strip;
  // its rows' LayerNorm sums sit in lane 4 r + e (each row's sums are the
  // four k groups' of lanes l16 + 16 r, folded first)
  const float inv_k = 1.f / (float)K;
  const int n = (strip0 + wn) * 64 + 4 * l16;
  float4 cv = make_float4(0.f, 0.f, 0.f, 0.f), dv = cv;
  if (LNF) {
#pragma unroll
    for (int i = 0; i < MI; i++) {
      sx[i] += __shfl_xor(sx[i], 16);
      sx[i] += __shfl_xor(sx[i], 32);
      sxx[i] += __shfl_xor(sxx[i], 16);
      sxx[i] += __shfl_xor(sxx[i], 32);
    }
    cv = *(const float4*)(lnc + n);
    dv = *(const float4*)(lnd + n);
  }
#pragma unroll
  for (int i = 0; i < MI; i++) {
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int row = m0 + wm * 16 * MI + 16 * i + 4 * r + e;
      float o[4] = {acc[i][0][e], acc[i][1][e], acc[i][2][e], acc[i][3][e]};
      if (LNF) {
        const float s1 = __shfl(sx[i], 4 * r + e), s2 = __shfl(sxx[i], 4 * r + e);
        const float ms = s1 * inv_k;  // mean of x - x0
        const float var = fmaxf(s2 * inv_k - ms * ms, 0.f);
        const float mean = __shfl(x0[i], 4 * r + e) + ms;
        const float rstd = 1.f / sqrtf(var + 1e-5f);
        o[0] = rstd * (o[0] - mean * cv.x) + dv.x;
        o[1] = rstd * (o[1] - mean * cv.y) + dv.y;
        o[2] = rstd * (o[2] - mean * cv.z) + dv.z;
        o[3] = rstd * (o[3] - mean * cv.w) + dv.w;
      }
      if (row >= M) continue;
      float* cp = Cm + (int64_t)row * ldc + n;
      *(float4*)cp = epilogue4<EPI>(make_float4(o[0], o[1], o[2], o[3]), bias, n, cp);
    }
  }
}

template <int MI, int D, int OCC, bool LNF, bool W1, bool GAM>
static void xt_go(mb_ctx* ctx, int epi, const float* A, int64_t lda, const uint4* Wx, int N,
                  int K, const float* bias, float* Cm, int64_t ldc, int M, const float* lnc,
                  const float* lnd, const float* gamma) {
  const dim3 grid((unsigned)(N / 128), (unsigned)((M + 32 * MI - 1) / (32 * MI)));
  with_epi(epi, [&](auto e) {
    constexpr int E = decltype(e)::value;
    if constexpr (LNF) {
      if constexpr (E == EPI_STORE || E == EPI_GELU || E == EPI_GELU_ERF)
        hipLaunchKernelGGL((k_gemm_xt<MI, D, E, true, W1, GAM, OCC>), grid, dim3(256), 0, ctx->stream,
                           A, lda, Wx, N, K, bias, Cm, ldc, M, lnc, lnd, gamma);
    } else if constexpr (!GAM) {
      hipLaunchKernelGGL((k_gemm_xt<MI, D, E, false, W1, false, OCC>), grid, dim3(256), 0, ctx->stream,
                         A, lda, Wx, N, K, bias, Cm, ldc, M, lnc, lnd, gamma);
    }
  });
}

template <int MI, bool LNF, bool W1, bool GAM>
static int xt_launch(mb_ctx* ctx, int epi, const float* A, int64_t lda, const uint4* Wx, int N,
                     int K, const float* bias, float* Cm, int64_t ldc, int M, const float* lnc,
                     const float* lnd, const float* gamma, bool three) {
  // Two workgroups per CU, with three stages where they still fit the 160 KB
  // of LDS (else two).  Measured at 8192 rows (QKV / O / fc_in / fc_out):
  // one workgroup per CU with four stages took 162 / 66 / 193 / 221 us
  // against 118 / 42 / 130 / 136 us.  `three`: three workgroups per CU with
  // two stages each (64-row tiles; see the caller).
  constexpr int SB = xt_stage_bytes<MI, W1, GAM>();
  if constexpr (6 * SB <= 160 * 1024) {
    if (three) {
      xt_go<MI, 2, 3, LNF, W1, GAM>(ctx, epi, A, lda, Wx, N, K, bias, Cm, ldc, M, lnc, lnd, gamma);
      MB_HIP(ctx, hipGetLastError());
      return MB_OK;
    }
  }
  xt_go<MI, 3 * SB <= 80 * 1024 ? 3 : 2, 2, LNF, W1, GAM>(ctx, epi, A, lda, Wx, N, K, bias, Cm,
                                                          ldc, M, lnc, lnd, gamma);
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

template <bool W1>
static int gemm_x3_any(mb_ctx* ctx, int epi, const float* A, int64_t lda, const void* Wx, int N,
                       int K, const float* bias, float* Cm, int64_t ldc, int M, const float* lnc,
                       const float* lnd, const float* gamma) {
  if (M <= 0) return MB_OK;
  if (M <= kGemvMaxM)
    return fail(ctx, MB_ERR_STATE, "split-bf16 gemm takes more than %d rows (M %d)", kGemvMaxM, M);
  const bool lnf = lnc != nullptr;
  if (lnf && (!lnd || (epi != EPI_STORE && epi != EPI_GELU && epi != EPI_GELU_ERF)))
    return fail(ctx, MB_ERR_ARG, "folded LayerNorm gemm has no epilogue %d", epi);
  if (gamma && !lnf) return fail(ctx, MB_ERR_ARG, "gamma on A goes with a folded LayerNorm");
  const uint4* W = (const uint4*)Wx;
  if (!gemm_streams(M, N)) {
    // prefill-sized M: the tiled kernel, MI row blocks per wave -- the most
    // that still gives every CU a workgroup
    if (N % 128 || K % kX3Block || lda % 4 || ldc % 4 || (int64_t)M * lda >= (int64_t)1 << 30 ||
        ((uintptr_t)A & 15) || ((uintptr_t)Wx & 15) || ((uintptr_t)Cm & 15) ||
        ((uintptr_t)bias & 15) || ((uintptr_t)lnc & 15) || ((uintptr_t)lnd & 15) ||
        ((uintptr_t)gamma & 15))
      return fail(ctx, MB_ERR_ARG, "split-bf16 gemm shape/alignment unsupported (M %d N %d K %d)",
                  M, N, K);
    // (128-row tiles over 64-row ones at 8192 rows: QKV 118 against 130 us,
    // both at two workgroups per CU.)  Where the 128-row tiles leave the last
    // of their rounds (512 per round, two per CU) part full and 64-row tiles
    // fill at least one round of 768, the 64-row tiles run three per CU with
    // two stages each: at 8192 rows QKV (1152 tiles of 128 rows, 2.25 rounds)
    // 106.8 -> 102.6 us, O and fc_out (384 tiles) 36.8 -> 34.9 and 126.5 ->
    // 117.8 us, the 256-voice codec frame 2.146 -> 2.130 ms (same GPU,
    // alternating); fc_in (1536 tiles, three whole rounds) went 118.3 ->
    // 123.8 us that way and keeps the 128-row tiles.
    auto tiles = [&](int mi) { return (int64_t)(N / 128) * ((M + 32 * mi - 1) / (32 * mi)); };
    const bool three = tiles(2) >= 768 && tiles(4) % 512 != 0;
    const int mi = three ? 2 : tiles(4) >= 256 ? 4 : tiles(2) >= 256 ? 2 : 1;
    auto go = [&](auto mi_) {
      constexpr int T = decltype(mi_)::value;
      if (lnf && gamma)
        return xt_launch<T, true, W1, true>(ctx, epi, A, lda, W, N, K, bias, Cm, ldc, M, lnc, lnd,
                                            gamma, three);
      if (lnf)
        return xt_launch<T, true, W1, false>(ctx, epi, A, lda, W, N, K, bias, Cm, ldc, M, lnc,
                                             lnd, nullptr, three);
      return xt_launch<T, false, W1, false>(ctx, epi, A, lda, W, N, K, bias, Cm, ldc, M, nullptr,
                                            nullptr, nullptr, three);
    };
    if (mi == 4) return go(std::integral_constant<int, 4>{});
    if (mi == 2) return go(std::integral_constant<int, 2>{});
    return go(std::integral_constant<int, 1>{});
  }
  if (N % 64 || K % (4 * kX3Block) || lda % 4 || ldc % 4 || (int64_t)M * lda >= INT32_MAX ||
      ((uintptr_t)A & 15) ||
      ((uintptr_t)Wx & 15) || ((uintptr_t)Cm & 15) || ((uintptr_t)bias & 15) ||
      ((uintptr_t)lnc & 15) || ((uintptr_t)lnd & 15) || ((uintptr_t)gamma & 15))
    return fail(ctx, MB_ERR_ARG, "split-bf16 gemm shape/alignment unsupported (M %d N %d K %d)", M,
                N, K);
  int mt, S;
  stream_shape(M, N, K, lnf, mt, S);
  while (S > 1 && K % (4 * kX3Block * S)) S--;
  // 64-row tiles give way to 32-row tiles over at most 1.5 rounds of the
  // chip: 3072 x 768 at 256 rows, W streamed from HBM, took 11.2-12.0 us on
  // 32-row tiles (384 workgroups) against 11.8-12.3 us on 64-row tiles.
  if (mt == 64 && (int64_t)(N / 64) * ((M + 31) / 32) <= 384) mt = 32;
  // Two register stages (one 32-deep block in flight) at every tile height:
  // at 64 and 256 rows every projection shape ran fastest that way (at 256
  // rows O 4.9 us against 5.4 with 4 stages, fc_in on 32-row tiles 11.2
  // against 11.7 with 3; deeper prologues spend longer issuing loads before
  // the first MFMA, and the per-CU load rate, not latency, bounds the rest).
  auto go = [&](auto mt_) {
    constexpr int T = decltype(mt_)::value;
    if (lnf && gamma)
      return x3_launch<T, 2, true, W1, true>(ctx, epi, A, lda, W, N, K, bias, Cm, ldc, M, S, lnc, lnd, gamma);
    if (lnf) return x3_launch<T, 2, true, W1>(ctx, epi, A, lda, W, N, K, bias, Cm, ldc, M, S, lnc, lnd);
    return x3_launch<T, 2, false, W1>(ctx, epi, A, lda, W, N, K, bias, Cm, ldc, M, S, nullptr, nullptr);
  };
  switch (mt) {
    case 16: return go(std::integral_constant<int, 16>{});
    case 32: return go(std::integral_constant<int, 32>{});
    case 48: return go(std::integral_constant<int, 48>{});
    default: return go(std::integral_constant<int, 64>{});
  }
}

int launch_gemm_x3(mb_ctx* ctx, int epi, const float* A, int64_t lda, const void* Wx, int N,
                   int K, const float* bias, float* Cm, int64_t ldc, int M, const float* lnc,
                   const float* lnd) {
  return gemm_x3_any<false>(ctx, epi, A, lda, Wx, N, K, bias, Cm, ldc, M, lnc, lnd, nullptr);
}

int launch_gemm_x2(mb_ctx* ctx, int epi, const float* A, int64_t lda, const void* Wx1, int N,
                   int K, const float* bias, float* Cm, int64_t ldc, int M, const float* lnc,
                   const float* lnd, const float* gamma) {
  return gemm_x3_any<true>(ctx, epi, A, lda, Wx1, N, K, bias, Cm, ldc, M, lnc, lnd, gamma);
}

// ---------------------------------------------------------------------------
// GEMV-sized M (at most kGemvMaxM rows) on row-major or column-block-major
// weights (mb_linear_dev, the codec's few-voice projections; the model's
// decode layers read k-major copies instead, k_gemv_k below).  The product
// reads each weight once and does a few multiply-adds per weight, so its
// time is the weight bytes over the bandwidth the launch reaches, which
// takes many CUs loading at once with every load in flight:
// the streaming kernel puts N / 64 workgroups on the chip at M = 1 (12 for
// the O projection) and walks k in dependent pipeline steps.  Here a
// workgroup owns a strip of SW = 16 columns and all of k, so the grid is
// N / 16 workgroups of NW waves (4, or 8 for k >= 2048).
// Lane (c = lane mod CL, q = lane / CL; CL = SW / 4) of wave w owns columns
// 4c .. 4c + 3 of the strip and, in each block of k, the four rows
// WR w + 4q .. + 3 (WR = 256 / CL rows per wave per block): four float4
// loads of W and one float4 of A per row of A.  A lane issues the loads of
// RB blocks before its first multiply-add (the finishing threads' bias,
// residual and LayerNorm-fold operands before those); its sums run in k
// order, then fold over q (lane swaps) and over the waves (LDS, wave order),
// so every output is the same fixed-order sum on every run.  The strips of
// a 64-column block are numbered 8 apart, so the dispatcher's round-robin
// puts them on one XCD and they share the L2 lines (128 bytes = 32 columns)
// of the weight rows.
//
// With LNF the rows are the raw residual stream and the LayerNorm is folded
// in (Wg, c, d as for the streaming kernel): the workgroup sees every k of
// its rows, and the lanes of column group 0 add up x - x0 and (x - x0)^2 from
// the A values they load anyway (x0 = x[m][0], so the variance does not
// cancel).
template <int EPI, bool LNF, bool TILED, int MR, int NW>
__global__ __launch_bounds__(64 * NW) void k_gemv(
    const float* __restrict__ A, int64_t lda, const float* __restrict__ W, int N, int K,
    const float* __restrict__ bias, float* __restrict__ Cm, int64_t ldc, int M,
    const float* __restrict__ lnc, const float* __restrict__ lnd) {
  constexpr int RB = MR <= 2 ? 6 : MR <= 4 ? 4 : NW == 8 ? 2 : 3;  // k blocks per round of loads
  constexpr int SW = 16;                             // strip width (columns)
  constexpr int CL = SW / 4;                         // lanes (float4 column groups) per row
  constexpr int WR = 256 / CL;                       // rows of k per wave per block
  constexpr int KB = WR * NW;                        // rows of k per block
  constexpr int P = 64 / SW;                         // strips per 64-column block
  __shared__ float4 red[NW][MR][CL];
  __shared__ float2 rowst[LNF ? NW : 1][MR];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane % CL, q = lane / CL;
  // strip: the four strips of 64-column block G are workgroups 32 (G / 8) +
  // 8 s + G mod 8 (s = 0..3); a last group of fewer than 32 strips in order
  const int L = blockIdx.x, strips = N / SW, full = strips - strips % (8 * P);
  const int strip = L < full ? ((L / (8 * P)) * 8 + (L & 7)) * P + ((L >> 3) % P) : L;
  const int n = strip * SW + 4 * c;  // this lane's first column
  const float* Wp = TILED ? W + (int64_t)(n >> 6) * K * 64 + (n & 63) : W + n;
  const int64_t wrow = TILED ? 64 : N;
  // the finishing threads' epilogue operands, loaded under the main loop
  const bool fin = tid < CL * M;
  const int om = tid / CL, oc = tid % CL;
  const int on = strip * SW + 4 * oc;
  float4 ep_bias = make_float4(0.f, 0.f, 0.f, 0.f), ep_c = ep_bias, ep_cv = ep_bias, ep_dv = ep_bias;
  float ep_x0 = 0.f;
  if (fin) {
    if (bias) ep_bias = *(const float4*)(bias + on);
    if (EPI == EPI_ADD || EPI == EPI_SCALE_ADD) ep_c = *(const float4*)(Cm + (int64_t)om * ldc + on);
    if (LNF) {
      ep_cv = *(const float4*)(lnc + on);
      ep_dv = *(const float4*)(lnd + on);
      ep_x0 = A[(int64_t)om * lda];
    }
  }

  float acc[MR][4];
  float s1[MR], s2[MR], x0[MR];
#pragma unroll
  for (int m = 0; m < MR; m++) {
#pragma unroll
    for (int j = 0; j < 4; j++) acc[m][j] = 0.f;
    s1[m] = s2[m] = 0.f;
    x0[m] = LNF && m < M ? A[(int64_t)m * lda] : 0.f;
  }
  const int nblk = (K + KB - 1) / KB;
  for (int b0 = 0; b0 < nblk; b0 += RB) {
    float4 w[RB][4], a[RB][MR];
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
      const int k = (b0 + rb) * KB + wave * WR + 4 * q;
      if (b0 + rb < nblk && k < K) {
#pragma unroll
        for (int r = 0; r < 4; r++) w[rb][r] = *(const float4*)(Wp + (int64_t)(k + r) * wrow);
      }
    }
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
      const int k = (b0 + rb) * KB + wave * WR + 4 * q;
#pragma unroll
      for (int m = 0; m < MR; m++)
        a[rb][m] = b0 + rb < nblk && k < K && m < M ? *(const float4*)(A + (int64_t)m * lda + k)
                                                    : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
      const int k = (b0 + rb) * KB + wave * WR + 4 * q;
      if (b0 + rb >= nblk || k >= K) continue;
#pragma unroll
      for (int m = 0; m < MR; m++) {
        const float av[4] = {a[rb][m].x, a[rb][m].y, a[rb][m].z, a[rb][m].w};
#pragma unroll
        for (int r = 0; r < 4; r++) {
          acc[m][0] = fmaf(av[r], w[rb][r].x, acc[m][0]);
          acc[m][1] = fmaf(av[r], w[rb][r].y, acc[m][1]);
          acc[m][2] = fmaf(av[r], w[rb][r].z, acc[m][2]);
          acc[m][3] = fmaf(av[r], w[rb][r].w, acc[m][3]);
          if (LNF) {
            const float e = av[r] - x0[m];
            s1[m] += e;
            s2[m] = fmaf(e, e, s2[m]);
          }
        }
      }
    }
  }
  // fold q (lanes with the same column group c)
  auto fold = [](float v) {
#pragma unroll
    for (int sh = CL; sh < 16; sh <<= 1) v += __shfl_xor(v, sh);
    return col_sum(v);
  };
#pragma unroll
  for (int m = 0; m < MR; m++) {
    if (m >= M) break;
#pragma unroll
    for (int j = 0; j < 4; j++) acc[m][j] = fold(acc[m][j]);
    if (LNF) {
      s1[m] = fold(s1[m]);
      s2[m] = fold(s2[m]);
    }
  }
  if (q == 0) {
#pragma unroll
    for (int m = 0; m < MR; m++) {
      if (m >= M) break;
      red[wave][m][c] = make_float4(acc[m][0], acc[m][1], acc[m][2], acc[m][3]);
      if (LNF && c == 0) rowst[wave][m] = make_float2(s1[m], s2[m]);
    }
  }
  __syncthreads();
  // thread t < CL M finishes row t / CL, columns 4 (t mod CL) .. + 3 of the strip
  if (!fin) return;
  float4 o = red[0][om][oc];
#pragma unroll
  for (int w2 = 1; w2 < NW; w2++) {
    const float4 v = red[w2][om][oc];
    o.x += v.x; o.y += v.y; o.z += v.z; o.w += v.w;
  }
  if (LNF) {
    const float inv_k = 1.f / (float)K;
    float t1 = rowst[0][om].x, t2 = rowst[0][om].y;
#pragma unroll
    for (int w2 = 1; w2 < NW; w2++) {
      t1 += rowst[w2][om].x;
      t2 += rowst[w2][om].y;
    }
    const float ms = t1 * inv_k;  // mean of x - x0
    const float var = fmaxf(t2 * inv_k - ms * ms, 0.f);
    const float mean = ep_x0 + ms;
    const float rstd = 1.f / sqrtf(var + 1e-5f);
    o.x = rstd * (o.x - mean * ep_cv.x) + ep_dv.x;
    o.y = rstd * (o.y - mean * ep_cv.y) + ep_dv.y;
    o.z = rstd * (o.z - mean * ep_cv.z) + ep_dv.z;
    o.w = rstd * (o.w - mean * ep_cv.w) + ep_dv.w;
  }
  *(float4*)(Cm + (int64_t)om * ldc + on) = epilogue_regs<EPI>(o, ep_bias, bias != nullptr, ep_c);
}

template <bool LNF>
static int gemv_launch(mb_ctx* ctx, int epi, const float* A, int64_t lda, const float* W, int N,
                       int K, const float* bias, float* Cm, int64_t ldc, int M, bool tiled,
                       const float* lnc, const float* lnd) {
  if (LNF && epi != EPI_STORE && epi != EPI_GELU && epi != EPI_GELU_ERF)
    return fail(ctx, MB_ERR_ARG, "folded LayerNorm gemm has no epilogue %d", epi);
  // Deep k (fc_out's 3072) runs on 8 waves, so one round of loads covers
  // more of it.  (8- and 4-column strips, for more workgroups at small N,
  // were slower on every decode shape but 768 x 3072: their 32- and 16-byte
  // row pieces read HBM less efficiently.)
  const dim3 grid((unsigned)(N / 16));
  const bool deep = K >= 2048;
  with_epi(epi, [&](auto e) {
    constexpr int E = decltype(e)::value;
    auto go = [&](auto mr) {
      constexpr int MRv = decltype(mr)::value;
      auto launch = [&](auto nw) {
        constexpr int NWv = decltype(nw)::value;
        if constexpr (LNF) {
          if constexpr (E == EPI_STORE || E == EPI_GELU || E == EPI_GELU_ERF)
            hipLaunchKernelGGL((k_gemv<E, true, true, MRv, NWv>), grid, dim3(64 * NWv), 0,
                               ctx->stream, A, lda, W, N, K, bias, Cm, ldc, M, lnc, lnd);
        } else if (tiled) {
          hipLaunchKernelGGL((k_gemv<E, false, true, MRv, NWv>), grid, dim3(64 * NWv), 0,
                             ctx->stream, A, lda, W, N, K, bias, Cm, ldc, M, lnc, lnd);
        } else {
          hipLaunchKernelGGL((k_gemv<E, false, false, MRv, NWv>), grid, dim3(64 * NWv), 0,
                             ctx->stream, A, lda, W, N, K, bias, Cm, ldc, M, lnc, lnd);
        }
      };
      if (deep) launch(std::integral_constant<int, 8>{});
      else launch(std::integral_constant<int, 4>{});
    };
    if (M <= 1) go(std::integral_constant<int, 1>{});
    else if (M <= 2) go(std::integral_constant<int, 2>{});
    else if (M <= 4) go(std::integral_constant<int, 4>{});
    else go(std::integral_constant<int, 8>{});
  });
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

// ---------------------------------------------------------------------------
// GEMV on k-major weights: Wk[n][k] = W[k][n] (launch_kmajor_w), for the
// model's decode-sized projections, which keep such a copy.  A column's
// weights are then one contiguous run of K floats, so wave w of workgroup g
// computes column n = 4g + w alone: lane l reads the float4s at k = 4l +
// 256i (a wave reads 1 KB contiguous per load) and the matching float4 of
// every A row, all issued before the first multiply-add, and the wave folds
// its 64 lanes (lane swaps) -- no LDS, no barrier.  With LNF the wave also
// sums x - x0 and (x - x0)^2 over the rows it loads (x0 = x[m][0]) and
// applies the folded LayerNorm itself.  The grid is N / 4 workgroups (192
// for 768 outputs, 768 for 3072), and every output is a fixed-order sum.
// KC > 0: K == KC known at compile time, so every round of loads is a fixed
// set of unconditional loads (no branch around a load: the compiler then
// leaves them in flight across the epilogue operands' waits); KC = 0: any K,
// in a run-time loop.
// (At most 4 waves per SIMD are asked for: a grid is N / 4 workgroups, one
// column per wave, so at 768 and 3072 columns there are 0.75 and 3 waves per
// SIMD, and the registers go to keeping every load of a round in flight.)
template <int EPI, bool LNF, int MR, int KC = 0, bool PICK = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 4))) void k_gemv_k(
    const float* __restrict__ A, int64_t lda, const float* __restrict__ Wk, int N, int K,
    const float* __restrict__ bias, float* __restrict__ Cm, int64_t ldc, int M,
    const float* __restrict__ lnc, const float* __restrict__ lnd, PickIn pk) {
  static_assert(!PICK || (MR == 1 && KC == D && LNF && EPI == EPI_STORE), "PICK: one row of 768");
  constexpr int RI = MR <= 2 ? 12 : MR <= 4 ? 6 : 3;  // k steps (256 rows each) per round of loads
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = blockIdx.x * 4 + wave;
  const float* wp = Wk + (int64_t)n * K;
  // Every load is unconditional (addresses clamped into the operands, the
  // values of rows >= M and of k >= K never used), so the compiler counts the
  // same loads on every path: the weight loads issue right behind the
  // epilogue operands instead of after a wait for them.
  const int le = min(lane, M - 1);  // lane m < M finishes row m
  const float* bp = bias ? bias : A;
  float ep_b = bp[bias ? n : 0], ep_c = 0.f, ep_cv = 0.f, ep_dv = 0.f;
  if (EPI == EPI_ADD || EPI == EPI_SCALE_ADD) ep_c = Cm[(int64_t)le * ldc + n];
  if (LNF) {
    ep_cv = lnc[n];
    ep_dv = lnd[n];
  }
  float acc[MR], s1[MR], s2[MR], x0[MR];
#pragma unroll
  for (int m = 0; m < MR; m++) {
    acc[m] = s1[m] = s2[m] = 0.f;
    x0[m] = LNF && !PICK ? A[(int64_t)min(m, M - 1) * lda] : 0.f;
  }
  const float* Ar = A;  // PICK: the chosen code's embedding row
  const int Kx = KC > 0 ? KC : K;  // a constant where the launch fixed it
  // one k step (256 k): lane l's float4 at k = 256 step + 4 l.  Lanes past K
  // (only in a last, partial step) add zeros: no branch, so no load is sunk
  // into one.
  auto step_mac = [&](int st, float4 w, const float4* a) {
    const bool in = st * 256 + 4 * lane < Kx;
    if (!in) w = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int m = 0; m < MR; m++) {
      acc[m] = fmaf(a[m].x, w.x, acc[m]);
      acc[m] = fmaf(a[m].y, w.y, acc[m]);
      acc[m] = fmaf(a[m].z, w.z, acc[m]);
      acc[m] = fmaf(a[m].w, w.w, acc[m]);
      if (LNF) {
        const float x0m = in ? x0[m] : 0.f;
        const float e[4] = {in ? a[m].x - x0m : 0.f, in ? a[m].y - x0m : 0.f,
                            in ? a[m].z - x0m : 0.f, in ? a[m].w - x0m : 0.f};
#pragma unroll
        for (int j = 0; j < 4; j++) {
          s1[m] += e[j];
          s2[m] = fmaf(e[j], e[j], s2[m]);
        }
      }
    }
  };
  auto load_w = [&](int st, float4& w) { w = *(const float4*)(wp + min(st * 256 + 4 * lane, Kx - 4)); };
  auto load_a = [&](int st, float4* a) {
    const int k = min(st * 256 + 4 * lane, Kx - 4);
#pragma unroll
    for (int m = 0; m < MR; m++) a[m] = *(const float4*)(Ar + (int64_t)min(m, M - 1) * lda + k);
  };
  auto step_load = [&](int st, float4& w, float4* a) {
    load_w(st, w);
    load_a(st, a);
  };
  if constexpr (KC > 0) {
    constexpr int SPR = (KC + 255) / 256;
    constexpr int RK = SPR < RI ? SPR : RI;
    static_assert(!PICK || RK == SPR, "PICK: one round of loads");
    static_for<(SPR + RK - 1) / RK>([&](auto r_) {
      constexpr int r = decltype(r_)::value;
      constexpr int NI = (r + 1) * RK <= SPR ? RK : SPR - r * RK;
      float4 w[NI], a[NI][MR];
      if constexpr (PICK) {
        // the choice's logits first, the weights behind them, then the
        // choice (waiting for the logits only) and the chosen row
        const ChoiceIn c = pick_load(pk, lane);
#pragma unroll
        for (int i = 0; i < NI; i++) load_w(i, w[i]);
        Ar = pick_row(pk, c, lane, blockIdx.x == 0 && wave == 0);
        x0[0] = Ar[0];
#pragma unroll
        for (int i = 0; i < NI; i++) load_a(i, a[i]);
      } else {
#pragma unroll
        for (int i = 0; i < NI; i++) step_load(r * RK + i, w[i], a[i]);
      }
      asm volatile("" ::: "memory");  // the round's loads stay in front, none sunk into a branch
#pragma unroll
      for (int i = 0; i < NI; i++) step_mac(r * RK + i, w[i], a[i]);
    });
  } else {
    const int steps = (K + 255) >> 8;
    for (int i0 = 0; i0 < steps; i0 += RI) {
      float4 w[RI], a[RI][MR];
#pragma unroll
      for (int i = 0; i < RI; i++) step_load(i0 + i, w[i], a[i]);
#pragma unroll
      for (int i = 0; i < RI; i++) step_mac(i0 + i, w[i], a[i]);
    }
  }
  auto fold = [](float v) {
#pragma unroll
    for (int sh = 1; sh < 16; sh <<= 1) v += __shfl_xor(v, sh);
    return col_sum(v);
  };
  float mine = 0.f, m1 = 0.f, m2 = 0.f, mx0 = 0.f;
#pragma unroll
  for (int m = 0; m < MR; m++) {
    if (m >= M) break;
    const float t = fold(acc[m]);
    if (lane == m) mine = t;
    if (LNF) {
      const float u1 = fold(s1[m]), u2 = fold(s2[m]);
      if (lane == m) {
        m1 = u1;
        m2 = u2;
        mx0 = x0[m];
      }
    }
  }
  if (lane >= M) return;
  if (!bias) ep_b = 0.f;
  float o = mine;
  if (LNF) {
    const float inv_k = 1.f / (float)K;
    const float ms = m1 * inv_k;  // mean of x - x0
    const float var = fmaxf(m2 * inv_k - ms * ms, 0.f);
    const float rstd = 1.f / sqrtf(var + 1e-5f);
    o = rstd * (o - (mx0 + ms) * ep_cv) + ep_dv;
  }
  if (EPI == EPI_SCALE_ADD) {
    o = ep_c + ep_b * o;
  } else {
    if (bias) o += ep_b;
    if (EPI == EPI_GELU) o = gelu_tanh(o);
    if (EPI == EPI_GELU_ERF) o = gelu_erf(o);
    if (EPI == EPI_ADD) o = ep_c + o;
  }
  Cm[(int64_t)lane * ldc + n] = o;
}

int launch_gemv_k(mb_ctx* ctx, int epi, const float* A, int64_t lda, const float* Wk, int N, int K,
                  const float* bias, float* Cm, int64_t ldc, int M, const float* lnc,
                  const float* lnd, const PickIn* pick) {
  if (M <= 0) return MB_OK;
  const bool lnf = lnc != nullptr;
  if (pick) {
    if (M != 1 || K != D || !lnf || !lnd || epi != EPI_STORE || N % 4 || ((uintptr_t)Wk & 15))
      return fail(ctx, MB_ERR_ARG, "gemv with the code choice: one row of %d, folded LayerNorm "
                  "(M %d N %d K %d)", D, M, N, K);
    hipLaunchKernelGGL((k_gemv_k<EPI_STORE, true, 1, D, true>), dim3((unsigned)(N / 4)), dim3(256),
                       0, ctx->stream, A, lda, Wk, N, K, bias, Cm, ldc, M, lnc, lnd, *pick);
    MB_HIP(ctx, hipGetLastError());
    return MB_OK;
  }
  if (M > kGemvMaxM || N % 4 || K % 4 || lda % 4 || ((uintptr_t)A & 15) || ((uintptr_t)Wk & 15) ||
      (lnf && !lnd))
    return fail(ctx, MB_ERR_ARG, "k-major gemv shape/alignment unsupported (M %d N %d K %d)", M, N, K);
  if (lnf && epi != EPI_STORE && epi != EPI_GELU && epi != EPI_GELU_ERF)
    return fail(ctx, MB_ERR_ARG, "folded LayerNorm gemm has no epilogue %d", epi);
  const dim3 grid((unsigned)(N / 4));
  // one row at the model's two widths: k loops fixed at compile time
  const int kc = M == 1 && (K == D || K == FFN) ? K : 0;
  with_epi(epi, [&](auto e) {
    constexpr int E = decltype(e)::value;
    auto go = [&](auto mr) {
      constexpr int MRv = decltype(mr)::value;
      auto launch = [&](auto kc_) {
        constexpr int KCv = decltype(kc_)::value;
        if (lnf) {
          if constexpr (E == EPI_STORE || E == EPI_GELU || E == EPI_GELU_ERF)
            hipLaunchKernelGGL((k_gemv_k<E, true, MRv, KCv>), grid, dim3(256), 0, ctx->stream, A,
                               lda, Wk, N, K, bias, Cm, ldc, M, lnc, lnd, PickIn{});
        } else {
          hipLaunchKernelGGL((k_gemv_k<E, false, MRv, KCv>), grid, dim3(256), 0, ctx->stream, A,
                             lda, Wk, N, K, bias, Cm, ldc, M, lnc, lnd, PickIn{});
        }
      };
      if constexpr (MRv == 1) {
        if (kc == D) return launch(std::integral_constant<int, D>{});
        if (kc == FFN) return launch(std::integral_constant<int, FFN>{});
      }
      launch(std::integral_constant<int, 0>{});
    };
    if (M <= 1) go(std::integral_constant<int, 1>{});
    else if (M <= 2) go(std::integral_constant<int, 2>{});
    else if (M <= 4) go(std::integral_constant<int, 4>{});
    else go(std::integral_constant<int, 8>{});
  });
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

// The attention's output projection at up to kPartsMaxSeqs rows, reading
// the attention as per-wave partials (k_attn_unit's PARTS form): part holds,
// for row m, head h and wave w < nwp, acc[64], max and sum at
// ((m * 12 + h) * nwp + w) * PART.  Each workgroup first merges them into its
// input rows in LDS -- per (row, head) the waves' states weighted by
// exp(max_w - max) and divided by the weighted sum, the fold k_attn_unit does
// through LDS within one block -- with its weight loads already in flight,
// then takes k_gemv_k16's products (one wave per column, 8 bf16 weights per
// lane and 512-k step) and epilogue.  Only the bf16-weight store runs it: with
// fp32 weights the merged path measured no faster per frame than the unit
// attention followed by k_gemv_k.
template <int EPI, int MR>
__global__ __launch_bounds__(256) void k_gemv_parts(const float* part, int nwp,
                                                    const uint16_t* __restrict__ Wk, int N,
                                                    const float* __restrict__ bias,
                                                    float* __restrict__ Cm, int64_t ldc, int M) {
  constexpr int K = D, ST = (K + 511) / 512;
  __shared__ __align__(16) float xs[MR][K];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = blockIdx.x * 4 + wave;
  uint4 w16[ST];
#pragma unroll
  for (int st = 0; st < ST; st++)
    w16[st] = *(const uint4*)(Wk + (int64_t)n * K + min(st * 512 + 8 * lane, K - 8));
  const int le = min(lane, M - 1);
  const float ep_b = bias ? bias[n] : 0.f;
  const float ep_c = (EPI == EPI_ADD || EPI == EPI_SCALE_ADD) ? Cm[(int64_t)le * ldc + n] : 0.f;
  // (row, 4-dim quad) pairs over the 256 threads; each issues all of its
  // partials' loads at once (unused ones re-read the last partial), so a
  // pair costs one round trip
  constexpr int NP = 16;
  for (int i = threadIdx.x; i < M * (K / 4); i += 256) {
    const int m = i / (K / 4), q = i % (K / 4), h = q / 16, d4 = (q % 16) * 4;
    const float* pb = part + (int64_t)(m * H + h) * nwp * PART;
    float2 ml[NP];
    float4 av[NP];
#pragma unroll
    for (int v = 0; v < NP; v++) {
      const float* pv = pb + min(v, nwp - 1) * PART;
      ml[v] = *(const float2*)(pv + 64);
      av[v] = *(const float4*)(pv + d4);
    }
    __builtin_amdgcn_sched_barrier(0);  // every load above issues before the first use
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < NP; v++)
      if (v < nwp) mx = fmaxf(mx, ml[v].x);
    // an empty wave (max -inf) weighs 0, so no branch holds a load back
    float L = 0.f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int v = 0; v < NP; v++) {
      const float sv = v < nwp && ml[v].x != -INFINITY ? __expf(ml[v].x - mx) : 0.f;
      L += ml[v].y * sv;
      o.x = fmaf(sv, av[v].x, o.x);
      o.y = fmaf(sv, av[v].y, o.y);
      o.z = fmaf(sv, av[v].z, o.z);
      o.w = fmaf(sv, av[v].w, o.w);
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    *(float4*)&xs[m][h * HD + d4] = make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
  }
  __syncthreads();
  float acc[MR];
#pragma unroll
  for (int m = 0; m < MR; m++) acc[m] = 0.f;
#pragma unroll
  for (int st = 0; st < ST; st++) {
    // lanes past K (the second step's upper half) add zeros
    const bool in = st * 512 + 8 * lane < K;
    const int k = min(st * 512 + 8 * lane, K - 8);
    const uint32_t wb[4] = {in ? w16[st].x : 0u, in ? w16[st].y : 0u, in ? w16[st].z : 0u,
                            in ? w16[st].w : 0u};
    float wf[8];
#pragma unroll
    for (int t = 0; t < 4; t++) {
      wf[2 * t] = __uint_as_float(wb[t] << 16);
      wf[2 * t + 1] = __uint_as_float(wb[t] & 0xFFFF0000u);
    }
#pragma unroll
    for (int m = 0; m < MR; m++) {
      const float4 a0 = *(const float4*)&xs[min(m, M - 1)][k];
      const float4 a1 = *(const float4*)&xs[min(m, M - 1)][k + 4];
      const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
      for (int t = 0; t < 8; t++) acc[m] = fmaf(av[t], wf[t], acc[m]);
    }
  }
  float mine = 0.f;
#pragma unroll
  for (int m = 0; m < MR; m++) {
    if (m >= M) break;
    float v = acc[m];
#pragma unroll
    for (int sh = 1; sh < 16; sh <<= 1) v += __shfl_xor(v, sh);
    v = col_sum(v);
    if (lane == m) mine = v;
  }
  if (lane >= M) return;
  float o = mine;
  if (EPI == EPI_SCALE_ADD) {
    o = ep_c + ep_b * o;
  } else {
    if (bias) o += ep_b;
    if (EPI == EPI_GELU) o = gelu_tanh(o);
    if (EPI == EPI_GELU_ERF) o = gelu_erf(o);
    if (EPI == EPI_ADD) o = ep_c + o;
  }
  Cm[(int64_t)lane * ldc + n] = o;
}

int launch_gemv_k_parts(mb_ctx* ctx, int epi, const float* part, int nwp, const uint16_t* Wk,
                        int N, const float* bias, float* Cm, int64_t ldc, int M) {
  if (M <= 0) return MB_OK;
  if (M > kPartsMaxSeqs || N % 4 || nwp < 1 || nwp > 16 || ((uintptr_t)part & 15) ||
      ((uintptr_t)Wk & 15))
    return fail(ctx, MB_ERR_ARG, "partials gemv shape unsupported (M %d N %d, %d partials)", M, N,
                nwp);
  const dim3 grid((unsigned)(N / 4));
  with_epi(epi, [&](auto e) {
    constexpr int E = decltype(e)::value;
    auto go = [&](auto mr) {
      constexpr int MRv = decltype(mr)::value;
      hipLaunchKernelGGL((k_gemv_parts<E, MRv>), grid, dim3(256), 0, ctx->stream, part, nwp, Wk, N,
                         bias, Cm, ldc, M);
    };
    if (M <= 1) go(std::integral_constant<int, 1>{});
    else if (M <= 2) go(std::integral_constant<int, 2>{});
    else if (M <= 4) go(std::integral_constant<int, 4>{});
    else go(std::integral_constant<int, 8>{});
  });
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

// ---------------------------------------------------------------------------
// bf16 weight storage (mb_set_weight_storage): the projection weights are
// rounded to bf16 once (k_round_bf16) and the decode-sized kernels read them
// as bf16 -- half the bytes -- with fp32 products and accumulation.  The
// LayerNorm's gamma stays on the activation side (gamma[k] x[k] w[k][n] in
// the kernel; c and d come from the rounded W, launch_fold_ln), so every
// product is one of the rounded weights exactly as the model holds it.
//
// k_gemv_k16: k_gemv_k on a bf16 k-major copy Wk16[n][k] = W[k][n].  Lane l
// reads 8 consecutive k per load (k = 8 l + 512 i: a wave reads 1 KB
// contiguous per load), with the matching two float4 of every A row (and of
// gamma with GAM), all issued before the first multiply-add.  The LayerNorm
// sums of LNF are taken over the raw rows, as in k_gemv_k.
template <int EPI, bool LNF, bool GAM, int MR, int KC = 0, bool PICK = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 4))) void k_gemv_k16(
    const float* __restrict__ A, int64_t lda, const uint16_t* __restrict__ Wk, int N, int K,
    const float* __restrict__ bias, float* __restrict__ Cm, int64_t ldc, int M,
    const float* __restrict__ lnc, const float* __restrict__ lnd,
    const float* __restrict__ gamma, PickIn pk) {
  static_assert(!PICK || (MR == 1 && KC == D && LNF && EPI == EPI_STORE), "PICK: one row of 768");
  constexpr int RI = MR <= 2 ? 6 : MR <= 4 ? 3 : 2;  // k steps (512 each) per round of loads
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = blockIdx.x * 4 + wave;
  const uint16_t* wp = Wk + (int64_t)n * K;
  // unconditional, clamped loads, as in k_gemv_k
  const int le = min(lane, M - 1);
  const float* bp = bias ? bias : A;
  float ep_b = bp[bias ? n : 0], ep_c = 0.f, ep_cv = 0.f, ep_dv = 0.f;
  if (EPI == EPI_ADD || EPI == EPI_SCALE_ADD) ep_c = Cm[(int64_t)le * ldc + n];
  if (LNF) {
    ep_cv = lnc[n];
    ep_dv = lnd[n];
  }
  float acc[MR], s1[MR], s2[MR], x0[MR];
#pragma unroll
  for (int m = 0; m < MR; m++) {
    acc[m] = s1[m] = s2[m] = 0.f;
    x0[m] = LNF && !PICK ? A[(int64_t)min(m, M - 1) * lda] : 0.f;
  }
  const float* Ar = A;  // PICK: the chosen code's embedding row
  const int Kx = KC > 0 ? KC : K;  // a constant where the launch fixed it
  auto load_w = [&](int st, uint4& w, float4* g) {
    const int k = min(st * 512 + 8 * lane, Kx - 8);
    w = *(const uint4*)(wp + k);
    if (GAM) {
      g[0] = *(const float4*)(gamma + k);
      g[1] = *(const float4*)(gamma + k + 4);
    }
  };
  auto load_a = [&](int st, float4 (*a)[2]) {
    const int k = min(st * 512 + 8 * lane, Kx - 8);
#pragma unroll
    for (int m = 0; m < MR; m++) {
      const float* ar = Ar + (int64_t)min(m, M - 1) * lda + k;
      a[m][0] = *(const float4*)ar;
      a[m][1] = *(const float4*)(ar + 4);
    }
  };
  auto step_load = [&](int st, uint4& w, float4* g, float4 (*a)[2]) {
    load_w(st, w, g);
    load_a(st, a);
  };
  // lanes past K (only in a last, partial step) add zeros, with no branch
  auto step_mac = [&](int st, const uint4& w, const float4* g, const float4 (*a)[2]) {
    const bool in = st * 512 + 8 * lane < Kx;
    const uint32_t wb[4] = {in ? w.x : 0u, in ? w.y : 0u, in ? w.z : 0u, in ? w.w : 0u};
    float wf[8], gf[8];
#pragma unroll
    for (int t = 0; t < 4; t++) {
      wf[2 * t] = __uint_as_float(wb[t] << 16);
      wf[2 * t + 1] = __uint_as_float(wb[t] & 0xFFFF0000u);
    }
    if (GAM) {
      gf[0] = g[0].x; gf[1] = g[0].y; gf[2] = g[0].z; gf[3] = g[0].w;
      gf[4] = g[1].x; gf[5] = g[1].y; gf[6] = g[1].z; gf[7] = g[1].w;
    }
#pragma unroll
    for (int m = 0; m < MR; m++) {
      const float av[8] = {a[m][0].x, a[m][0].y, a[m][0].z, a[m][0].w,
                           a[m][1].x, a[m][1].y, a[m][1].z, a[m][1].w};
#pragma unroll
      for (int t = 0; t < 8; t++) {
        acc[m] = fmaf(GAM ? __fmul_rn(av[t], gf[t]) : av[t], wf[t], acc[m]);
        if (LNF) {
          const float e = in ? av[t] - x0[m] : 0.f;
          s1[m] += e;
          s2[m] = fmaf(e, e, s2[m]);
        }
      }
    }
  };
  if constexpr (KC > 0) {
    constexpr int SPR = (KC + 511) / 512;
    constexpr int RK = SPR < RI ? SPR : RI;
    static_assert(!PICK || RK == SPR, "PICK: one round of loads");
    static_for<(SPR + RK - 1) / RK>([&](auto r_) {
      constexpr int r = decltype(r_)::value;
      constexpr int NI = (r + 1) * RK <= SPR ? RK : SPR - r * RK;
      uint4 w[NI];
      float4 g[NI][2], a[NI][MR][2];
      if constexpr (PICK) {
        // as in k_gemv_k: the choice's logits, the weights, the choice, the row
        const ChoiceIn c = pick_load(pk, lane);
#pragma unroll
        for (int i = 0; i < NI; i++) load_w(i, w[i], g[i]);
        Ar = pick_row(pk, c, lane, blockIdx.x == 0 && wave == 0);
        x0[0] = Ar[0];
#pragma unroll
        for (int i = 0; i < NI; i++) load_a(i, a[i]);
      } else {
#pragma unroll
        for (int i = 0; i < NI; i++) step_load(r * RK + i, w[i], g[i], a[i]);
      }
      asm volatile("" ::: "memory");  // the round's loads stay in front, none sunk into a branch
#pragma unroll
      for (int i = 0; i < NI; i++) step_mac(r * RK + i, w[i], g[i], a[i]);
    });
  } else {
    const int steps = (K + 511) >> 9;
    for (int i0 = 0; i0 < steps; i0 += RI) {
      uint4 w[RI];
      float4 g[RI][2], a[RI][MR][2];
#pragma unroll
      for (int i = 0; i < RI; i++) step_load(i0 + i, w[i], g[i], a[i]);
#pragma unroll
      for (int i = 0; i < RI; i++) step_mac(i0 + i, w[i], g[i], a[i]);
    }
  }
  auto fold = [](float v) {
#pragma unroll
    for (int sh = 1; sh < 16; sh <<= 1) v += __shfl_xor(v, sh);
    return col_sum(v);
  };
  float mine = 0.f, m1 = 0.f, m2 = 0.f, mx0 = 0.f;
#pragma unroll
  for (int m = 0; m < MR; m++) {
    if (m >= M) break;
    const float t = fold(acc[m]);
    if (lane == m) mine = t;
    if (LNF) {
      const float u1 = fold(s1[m]), u2 = fold(s2[m]);
      if (lane == m) {
        m1 = u1;
        m2 = u2;
        mx0 = x0[m];
      }
    }
  }
  if (lane >= M) return;
  if (!bias) ep_b = 0.f;
  float o = mine;
  if (LNF) {
    const float inv_k = 1.f / (float)K;
    const float ms = m1 * inv_k;  // mean of x - x0
    const float var = fmaxf(m2 * inv_k - ms * ms, 0.f);
    const float rstd = 1.f / sqrtf(var + 1e-5f);
    o = rstd * (o - (mx0 + ms) * ep_cv) + ep_dv;
  }
  if (EPI == EPI_SCALE_ADD) {
    o = ep_c + ep_b * o;
  } else {
    if (bias) o += ep_b;
    if (EPI == EPI_GELU) o = gelu_tanh(o);
    if (EPI == EPI_GELU_ERF) o = gelu_erf(o);
    if (EPI == EPI_ADD) o = ep_c + o;
  }
  Cm[(int64_t)lane * ldc + n] = o;
}

int launch_gemv_k16(mb_ctx* ctx, int epi, const float* A, int64_t lda, const uint16_t* Wk,
                    int N, int K, const float* bias, float* Cm, int64_t ldc, int M,
                    const float* lnc, const float* lnd, const float* gamma,
                    const PickIn* pick) {
  if (M <= 0) return MB_OK;
  const bool lnf = lnc != nullptr;
  if (pick) {
    if (M != 1 || K != D || !lnf || !lnd || epi != EPI_STORE || N % 4 || ((uintptr_t)Wk & 15) ||
        ((uintptr_t)gamma & 15))
      return fail(ctx, MB_ERR_ARG, "gemv with the code choice: one row of %d, folded LayerNorm "
                  "(M %d N %d K %d)", D, M, N, K);
    if (gamma)
      hipLaunchKernelGGL((k_gemv_k16<EPI_STORE, true, true, 1, D, true>), dim3((unsigned)(N / 4)),
                         dim3(256), 0, ctx->stream, A, lda, Wk, N, K, bias, Cm, ldc, M, lnc, lnd,
                         gamma, *pick);
    else
      hipLaunchKernelGGL((k_gemv_k16<EPI_STORE, true, false, 1, D, true>), dim3((unsigned)(N / 4)),
                         dim3(256), 0, ctx->stream, A, lda, Wk, N, K, bias, Cm, ldc, M, lnc, lnd,
                         gamma, *pick);
    MB_HIP(ctx, hipGetLastError());
    return MB_OK;
  }
  if (M > kGemvMaxM || N % 4 || K % 8 || lda % 4 || ((uintptr_t)A & 15) || ((uintptr_t)Wk & 15) ||
      ((uintptr_t)gamma & 15) || (lnf && !lnd))
    return fail(ctx, MB_ERR_ARG, "bf16 k-major gemv shape/alignment unsupported (M %d N %d K %d)", M, N, K);
  if (lnf && epi != EPI_STORE && epi != EPI_GELU && epi != EPI_GELU_ERF)
    return fail(ctx, MB_ERR_ARG, "folded LayerNorm gemm has no epilogue %d", epi);
  const dim3 grid((unsigned)(N / 4));
  const int kc = M == 1 && (K == D || K == FFN) ? K : 0;  // as launch_gemv_k
  with_epi(epi, [&](auto e) {
    constexpr int E = decltype(e)::value;
    auto go = [&](auto mr) {
      constexpr int MRv = decltype(mr)::value;
      auto launch = [&](auto kc_) {
        constexpr int KCv = decltype(kc_)::value;
        if (lnf) {
          if constexpr (E == EPI_STORE || E == EPI_GELU || E == EPI_GELU_ERF) {
            if (gamma)
              hipLaunchKernelGGL((k_gemv_k16<E, true, true, MRv, KCv>), grid, dim3(256), 0,
                                 ctx->stream, A, lda, Wk, N, K, bias, Cm, ldc, M, lnc, lnd, gamma,
                                 PickIn{});
            else
              hipLaunchKernelGGL((k_gemv_k16<E, true, false, MRv, KCv>), grid, dim3(256), 0,
                                 ctx->stream, A, lda, Wk, N, K, bias, Cm, ldc, M, lnc, lnd, gamma,
                                 PickIn{});
          }
        } else {
          hipLaunchKernelGGL((k_gemv_k16<E, false, false, MRv, KCv>), grid, dim3(256), 0,
                             ctx->stream, A, lda, Wk, N, K, bias, Cm, ldc, M, lnc, lnd, gamma,
                             PickIn{});
        }
      };
      if constexpr (MRv == 1) {
        if (kc == D) return launch(std::integral_constant<int, D>{});
        if (kc == FFN) return launch(std::integral_constant<int, FFN>{});
      }
      launch(std::integral_constant<int, 0>{});
    };
    if (M <= 1) go(std::integral_constant<int, 1>{});
    else if (M <= 2) go(std::integral_constant<int, 2>{});
    else if (M <= 4) go(std::integral_constant<int, 4>{});
    else go(std::integral_constant<int, 8>{});
  });
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

// Wr = bf16(W) (round to nearest even), kept as fp32: the rounded weights
// every later copy and the fp32 paths derive from.
__global__ __launch_bounds__(256) void k_round_bf16(const float* __restrict__ W, int64_t n,
                                                    float* __restrict__ Wr) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) Wr[i] = (float)(__bf16)W[i];
}

int launch_round_bf16(mb_ctx* ctx, const float* W, int64_t n, float* Wr) {
  hipLaunchKernelGGL(k_round_bf16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, ctx->stream, W,
                     n, Wr);
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

// Wk16[n][k] = bf16(W[k][n]) (W [K][N] row-major, already bf16-exact where
// it comes from k_round_bf16).
__global__ __launch_bounds__(256) void k_kmajor_w16(const float* __restrict__ W, int K, int N,
                                                    uint16_t* __restrict__ Wk) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)K * N) return;
  const int k = (int)(i % K);
  const int64_t n = i / K;
  Wk[i] = __builtin_bit_cast(uint16_t, (__bf16)W[(int64_t)k * N + n]);
}

int launch_kmajor_w16(mb_ctx* ctx, const float* W, int K, int N, uint16_t* Wk) {
  const int64_t n = (int64_t)K * N;
  hipLaunchKernelGGL(k_kmajor_w16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, ctx->stream, W,
                     K, N, Wk);
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

// Wk[n][k] = gamma[k] * W[k][n] (W [K][N] row-major; gamma null: 1), one
// thread per output element, rounded as k_fold_ln rounds its product, so a
// folded k-major copy holds the same values as the folded tiled one.
__global__ __launch_bounds__(256) void k_kmajor_w(const float* __restrict__ W, int K, int N,
                                                  const float* __restrict__ gamma,
                                                  float* __restrict__ Wk) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)K * N) return;
  const int k = (int)(i % K);
  const int64_t n = i / K;
  const float w = W[(int64_t)k * N + n];
  Wk[i] = gamma ? __fmul_rn(gamma[k], w) : w;
}

int launch_kmajor_w(mb_ctx* ctx, const float* W, int K, int N, const float* gamma, float* Wk) {
  const int64_t n = (int64_t)K * N;
  hipLaunchKernelGGL(k_kmajor_w, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, ctx->stream, W,
                     K, N, gamma, Wk);
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

// W' = diag(gamma) W, c = column sums of W', d = beta W: the folded form of
// "LayerNorm, then x W" used by the LNF streaming kernel.  One thread per
// column; c and d are summed in double in k order and rounded once.  W' is
// written column-block-major ([N / 64][K][64]), the layout the streaming
// kernel reads contiguously.
__global__ __launch_bounds__(256) void k_tile_w(const float* __restrict__ W, int K, int N,
                                                float* __restrict__ Wt) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // one output element
  if (i >= (int64_t)K * N) return;
  const int c = (int)(i & 63);
  const int64_t rest = i >> 6;
  const int k = (int)(rest % K), cb = (int)(rest / K);
  Wt[i] = W[(int64_t)k * N + cb * 64 + c];
}

// Wt = W ([K][N] row-major) in column-block-major order [N / 64][K][64].
int launch_tile_w(mb_ctx* ctx, const float* W, int K, int N, float* Wt) {
  if (N % 64) return fail(ctx, MB_ERR_ARG, "tiled projection width %d is not a multiple of 64", N);
  const int64_t n = (int64_t)K * N;
  hipLaunchKernelGGL(k_tile_w, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, ctx->stream, W, K,
                     N, Wt);
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

// The split-bf16 operand layout of k_gemm_x3 from an fp32 W, column-block-
// major [N / 64][K][64] (tiled) or row-major [K][N]: one thread per 16-byte
// piece (strip, k block, column block j, half h, lane), 8 bf16 of one column.
__global__ __launch_bounds__(256) void k_split_w(const float* __restrict__ Wt, int K, int N,
                                                 bool tiled, uint4* __restrict__ Wx) {
  const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (u >= (int64_t)(N / 64) * (K / kX3Block) * kX3BlockU4) return;
  const int lane = (int)(u & 63), h = (int)((u >> 6) & 1), j = (int)((u >> 7) & 3);
  const int64_t blk = u >> 9;  // strip * (K / 32) + k block
  const int nkb = K / kX3Block;
  const int64_t strip = blk / nkb;
  const int kb = (int)(blk % nkb);
  const int64_t k = kb * kX3Block + 8 * (lane >> 4), ld = tiled ? 64 : N;
  const float* src = (tiled ? Wt + strip * K * 64 : Wt + strip * 64) + k * ld + 4 * (lane & 15) + j;
  bf16x8_t out;
#pragma unroll
  for (int t = 0; t < 8; t++) {
    const float v = src[t * ld];
    const __bf16 hi = (__bf16)v;
    out[t] = h ? (__bf16)(v - (float)hi) : hi;
  }
  Wx[u] = __builtin_bit_cast(uint4, out);
}

// The W1 layout of k_gemm_x3 (bf16 weight storage): the high halves only,
// per (strip, k block, column block j, lane) one 16-byte piece.
__global__ __launch_bounds__(256) void k_split_w1(const float* __restrict__ Wt, int K, int N,
                                                  bool tiled, uint4* __restrict__ Wx) {
  const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (u >= (int64_t)(N / 64) * (K / kX3Block) * (kX3BlockU4 / 2)) return;
  const int lane = (int)(u & 63), j = (int)((u >> 6) & 3);
  const int64_t blk = u >> 8;  // strip * (K / 32) + k block
  const int nkb = K / kX3Block;
  const int64_t strip = blk / nkb;
  const int kb = (int)(blk % nkb);
  const int64_t k = kb * kX3Block + 8 * (lane >> 4), ld = tiled ? 64 : N;
  const float* src = (tiled ? Wt + strip * K * 64 : Wt + strip * 64) + k * ld + 4 * (lane & 15) + j;
  bf16x8_t out;
#pragma unroll
  for (int t = 0; t < 8; t++) out[t] = (__bf16)src[t * ld];
  Wx[u] = __builtin_bit_cast(uint4, out);
}

int launch_split_w1(mb_ctx* ctx, const float* Wt, int K, int N, void* Wx, bool tiled) {
  if (N % 64 || K % kX3Block)
    return fail(ctx, MB_ERR_ARG, "bf16 weights need N %% 64 == 0 and K %% 32 == 0 (K %d N %d)", K, N);
  const int64_t n = (int64_t)(N / 64) * (K / kX3Block) * (kX3BlockU4 / 2);
  hipLaunchKernelGGL(k_split_w1, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, ctx->stream, Wt,
                     K, N, tiled, (uint4*)Wx);
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

int launch_split_w(mb_ctx* ctx, const float* Wt, int K, int N, void* Wx, bool tiled) {
  if (N % 64 || K % kX3Block)
    return fail(ctx, MB_ERR_ARG, "split-bf16 weights need N %% 64 == 0 and K %% 32 == 0 (K %d N %d)",
                K, N);
  const int64_t n = (int64_t)(N / 64) * (K / kX3Block) * kX3BlockU4;
  hipLaunchKernelGGL(k_split_w, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, ctx->stream, Wt, K,
                     N, tiled, (uint4*)Wx);
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

__global__ __launch_bounds__(256) void k_fold_ln(const float* __restrict__ W, int K, int N,
                                                 const float* __restrict__ gamma,
                                                 const float* __restrict__ beta,
                                                 float* __restrict__ Wg, float* __restrict__ c,
                                                 float* __restrict__ d) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  float* wg = Wg + (int64_t)(n >> 6) * K * 64 + (n & 63);  // column-block-major, as launch_tile_w
  double sc = 0.0, sd = 0.0;
  for (int k = 0; k < K; k++) {
    const float w = W[(int64_t)k * N + n];
    const float g = __fmul_rn(gamma[k], w);
    wg[(int64_t)k * 64] = g;
    sc += (double)g;
    sd += (double)beta[k] * (double)w;
  }
  c[n] = (float)sc;
  d[n] = (float)sd;
}

int launch_fold_ln(mb_ctx* ctx, const float* W, int K, int N, const float* gamma,
                   const float* beta, float* Wg, float* c, float* d) {
  if (N % 64) return fail(ctx, MB_ERR_ARG, "folded projection width %d is not a multiple of 64", N);
  hipLaunchKernelGGL(k_fold_ln, dim3((unsigned)((N + 255) / 256)), dim3(256), 0, ctx->stream, W, K,
                     N, gamma, beta, Wg, c, d);
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

// The streaming kernel takes M < kStreamMaxM, and larger M while its 64-row
// tiling needs at most two rounds of the chip (<= 512 workgroups): measured on
// the codec's shapes it beat the LDS-tiled kernel everywhere there (8192 x 256
// x 1024: 43.6 against 61.0 us; 4096 x 256 x 1024: 22.3 against 40.1 us;
// 1024 x 768 x 768: 16.2 against 31.2 us; 2048 x 768 x 256: 15.8 against
// 16.9 us), and lost beyond (8192 x 768 x 256: 47.9 against 40.5 us).
bool gemm_streams(int M, int N) {
  return M < kStreamMaxM || (int64_t)((M + 63) / 64) * (N / 64) <= 512;
}

// out = epi(LN(x) W + bias) with the LayerNorm folded in (Wg, c, d from
// launch_fold_ln); K is the row width (the workgroup sees whole rows).  Where
// the streaming kernel does not take the shape (gemm_streams) it returns
// MB_ERR_STATE, so the caller runs the LayerNorm and the GEMM apart.
int launch_gemm_ln(mb_ctx* ctx, int epi, const float* x, int64_t ldx, const float* Wg, int N,
                   int K, const float* c, const float* d, const float* bias, float* Cm,
                   int64_t ldc, int M) {
  if (M <= 0) return MB_OK;
  if (!gemm_streams(M, N)) return MB_ERR_STATE;
  if (K % 64 || N % 64 || ldx % 4 || ldc % 4 || ((uintptr_t)x & 15) || ((uintptr_t)Wg & 15) ||
      ((uintptr_t)Cm & 15) || ((uintptr_t)bias & 15) || ((uintptr_t)c & 15) || ((uintptr_t)d & 15))
    return fail(ctx, MB_ERR_ARG, "folded gemm shape/alignment unsupported (M %d N %d K %d)", M, N, K);
  if (M <= kGemvMaxM) return gemv_launch<true>(ctx, epi, x, ldx, Wg, N, K, bias, Cm, ldc, M, true, c, d);
  int mt, S;
  stream_shape(M, N, K, true, mt, S);
  switch (mt) {
    case 16: return stream_launch<16, 2, true>(ctx, epi, x, ldx, Wg, N, K, bias, Cm, ldc, M, 1, c, d, true);
    case 32: return stream_launch<32, 2, true>(ctx, epi, x, ldx, Wg, N, K, bias, Cm, ldc, M, 1, c, d, true);
    case 48: return stream_launch<48, 2, true>(ctx, epi, x, ldx, Wg, N, K, bias, Cm, ldc, M, 1, c, d, true);
    default: return stream_launch<64, 2, true>(ctx, epi, x, ldx, Wg, N, K, bias, Cm, ldc, M, 1, c, d, true);
  }
}

// At most kGemvMaxM rows: the GEMV kernel.  M < kStreamMaxM, or few enough
// 64-row tiles: the streaming kernel.  Its
// row tile is the smallest of
// 16 / 32 / 48 / 64 rows that keeps the grid at most one workgroup per CU
// (256 CUs), so the projection runs as one round; K = 3072 projections with
// few tiles split K over up to 8 workgroups (fixed-order reduce), on 32-row
// tiles from 96 rows up (stream_shape).  Measured
// on the decode projections (M = 1, 64, 256; N x K = 2304 x 768, 768 x 768,
// 3072 x 768, 768 x 3072, 1024 x 768) these choices were the fastest of a
// sweep over tile, pipeline depth and split; 16-deep chunks in two register
// stages (one chunk in flight): re-measured once the loop no longer drained
// its loads at every iteration, two stages matched or beat three and four
// (QKV at 256 rows 12.6 against 13.1 us; the codec's 64-voice frame 1.22
// against 1.25 ms).
// Larger M: the LDS-tiled kernel with the largest tile that still gives the
// chip (256 CUs) a block per CU (128 x 128 only from K = 512 up), else the
// smallest tile.
size_t gemm_partial_floats(int M, int N, int K) {
  if (M <= kGemvMaxM) return 0;
  if (M <= 0 || !gemm_streams(M, N)) return 0;
  int mt, S;
  stream_shape(M, N, K, false, mt, S);
  return S > 1 ? (size_t)S * M * N : 0;
}

int launch_gemm(mb_ctx* ctx, int epi, const float* A, int64_t lda, const float* W, int N, int K,
                const float* bias, float* Cm, int64_t ldc, int M, bool w_tiled, float* part,
                size_t part_cap) {
  if (M <= 0) return MB_OK;
  if (w_tiled && !gemm_streams(M, N))
    return fail(ctx, MB_ERR_STATE, "tiled weights need the streaming kernel (M %d N %d)", M, N);
  if (N % 64 || K % 64 || lda % 4 || ldc % 4 || ((uintptr_t)A & 15) ||
      ((uintptr_t)W & 15) || ((uintptr_t)Cm & 15) || ((uintptr_t)bias & 15))
    return fail(ctx, MB_ERR_ARG, "gemm shape/alignment unsupported (M %d N %d K %d)", M, N, K);
  if (M <= kGemvMaxM)
    return gemv_launch<false>(ctx, epi, A, lda, W, N, K, bias, Cm, ldc, M, w_tiled, nullptr, nullptr);
  if (gemm_streams(M, N)) {
    int mt, S;
    stream_shape(M, N, K, false, mt, S);
    switch (mt) {
      case 16: return stream_launch<16, 2, false>(ctx, epi, A, lda, W, N, K, bias, Cm, ldc, M, S, nullptr, nullptr, w_tiled, part, part_cap);
      case 32: return stream_launch<32, 2, false>(ctx, epi, A, lda, W, N, K, bias, Cm, ldc, M, S, nullptr, nullptr, w_tiled, part, part_cap);
      case 48: return stream_launch<48, 2, false>(ctx, epi, A, lda, W, N, K, bias, Cm, ldc, M, S, nullptr, nullptr, w_tiled, part, part_cap);
      default: return stream_launch<64, 2, false>(ctx, epi, A, lda, W, N, K, bias, Cm, ldc, M, S, nullptr, nullptr, w_tiled, part, part_cap);
    }
  }
  auto blocks = [&](int bm, int bn) { return (int64_t)((M + bm - 1) / bm) * (N / bn); };
  // 128 x 128 tiles need a long k loop to pay off: at K = 256 (the codec's
  // d = 256 projections) 64 x 64 tiles were faster on every measured shape
  // (8192 x 768: 41.1 against 53.0 us; 4096 x 1024: 28.9 against 34.4 us),
  // at K = 768 / 3072 (prefill) the 128 x 128 tiles were.
  if (N % 128 == 0 && K >= 512 && blocks(128, 128) >= 256)
    gemm_launch<4, 4>(ctx, epi, A, lda, W, N, K, bias, Cm, ldc, M);
  else if (N % 64 == 0 && blocks(64, 64) >= 256)
    gemm_launch<2, 2>(ctx, epi, A, lda, W, N, K, bias, Cm, ldc, M);
  else if (N % 64 == 0 && blocks(32, 64) >= 256)
    gemm_launch<1, 2>(ctx, epi, A, lda, W, N, K, bias, Cm, ldc, M);
  else
    gemm_launch<1, 1>(ctx, epi, A, lda, W, N, K, bias, Cm, ldc, M);
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

}  // namespace mb
