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
#include "mb_internal.h"

namespace mb {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int GBK = 16;   // K slice
constexpr int GPAD = 20;  // LDS row stride in floats (16 + 4)

__device__ __forceinline__ float gelu_tanh(float v) {
  // 0.5 v (1 + tanh(0.7978845608 (v + 0.044715 v^3))), kernels-decode.ts:373-385
  const float inner = 0.7978845608028654f * (v + 0.044715f * v * v * v);
  return 0.5f * v * (1.f + tanhf(inner));
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
      const float bv = bias ? bias[col] : 0.f;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int row = m0 + (wm * TM + i) * 16 + g * 4 + r;
        if (row >= M) continue;
        float v = acc[i][j][r] + bv;
        float* cp = Cm + (int64_t)row * ldc + col;
        if (EPI == EPI_GELU) v = gelu_tanh(v);
        if (EPI == EPI_ADD) v = *cp + v;
        *cp = v;
      }
    }
}

template <int TM, int TN>
static void gemm_launch(mb_ctx* ctx, int epi, const float* A, int64_t lda, const float* W, int N,
                        int K, const float* bias, float* Cm, int64_t ldc, int M) {
  constexpr int BM = 2 * TM * 16, BN = 2 * TN * 16;
  dim3 grid((unsigned)(N / BN), (unsigned)((M + BM - 1) / BM));
  if (epi == EPI_GELU)
    hipLaunchKernelGGL((k_gemm<TM, TN, EPI_GELU>), grid, dim3(256), 0, ctx->stream, A, lda, W, N, K,
                       bias, Cm, ldc, M);
  else if (epi == EPI_ADD)
    hipLaunchKernelGGL((k_gemm<TM, TN, EPI_ADD>), grid, dim3(256), 0, ctx->stream, A, lda, W, N, K,
                       bias, Cm, ldc, M);
  else
    hipLaunchKernelGGL((k_gemm<TM, TN, EPI_STORE>), grid, dim3(256), 0, ctx->stream, A, lda, W, N,
                       K, bias, Cm, ldc, M);
}

// Pick the largest tile that still gives the chip (256 CUs) a block per CU,
// else the smallest tile.
int launch_gemm(mb_ctx* ctx, int epi, const float* A, int64_t lda, const float* W, int N, int K,
                const float* bias, float* Cm, int64_t ldc, int M) {
  if (M <= 0) return MB_OK;
  if (N % 32 || K % GBK || lda % 4 || ldc % 4 || ((uintptr_t)A & 15) || ((uintptr_t)W & 15))
    return fail(ctx, MB_ERR_ARG, "gemm shape/alignment unsupported (M %d N %d K %d)", M, N, K);
  auto blocks = [&](int bm, int bn) { return (int64_t)((M + bm - 1) / bm) * (N / bn); };
  if (N % 128 == 0 && blocks(128, 128) >= 256)
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
