// mb_linear_noalloc_dev: the projection of mb_linear_dev for callers that
// cannot allocate device memory (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc).  Its only scratch -- the streaming
// kernel's split-K partials, which mb_linear_dev keeps in the context's
// growable scratch -- lives here in a static device array instead.
//
// The array is 4 MiB on every GPU the library runs on, held until the process
// ends.  That covers every split the streaming kernel chooses: a split of S
// ways over T row x column tiles is taken only when S * T <= 256, and one tile
// is at most 64 rows x 64 columns, so S * M * N <= 64 * 64 * 256 floats.
//
// Every call on one GPU shares that GPU's array: two calls that overlap on
// one GPU (two streams, two threads, two contexts) race on it.  Each split
// writes its whole slice of partials before the reduce reads it, so nothing
// in the array needs to start at zero.
#include <mutex>

#include "mb_internal.h"

namespace {
constexpr size_t kScratchFloats = (size_t)1 << 20;
constexpr int kMaxDevices = 64;
}  // namespace

static __device__ __align__(256) float scratch[kScratchFloats];

namespace mb {
namespace {
std::mutex g_mu;
// The array's address on each device; the array's host-side name is no
// device address, so kernels only ever receive these.
float* g_scratch[kMaxDevices] = {};
}  // namespace

int noalloc_init(mb_ctx* ctx) {
  if (ctx->device < 0 || ctx->device >= kMaxDevices)
    return fail(ctx, MB_ERR_ARG, "device %d out of [0, %d)", ctx->device, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_scratch[ctx->device]) return MB_OK;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(::scratch));
  if (e != hipSuccess) return hip_fail(ctx, e, "hipGetSymbolAddress(scratch)");
  g_scratch[ctx->device] = (float*)p;
  return MB_OK;
}

}  // namespace mb

using namespace mb;

extern "C" int mb_linear_noalloc_dev(mb_ctx* ctx, int M, int N, int K, const float* A, int64_t lda,
                                     const float* W, const float* bias, float* C, int64_t ldc,
                                     int epi) {
  MB_DEVICE_GUARD(ctx);
  if (!ctx) return MB_ERR_ARG;
  if (M < 0 || N < 1 || K < 1) return fail(ctx, MB_ERR_ARG, "linear shape M %d N %d K %d", M, N, K);
  if (epi < EPI_STORE || epi > EPI_GELU_ERF) return fail(ctx, MB_ERR_ARG, "unknown epilogue %d", epi);
  if (epi == EPI_SCALE_ADD && !bias)
    return fail(ctx, MB_ERR_ARG, "MB_EPI_SCALE_ADD needs the scale vector in `bias`");
  if (M == 0) return MB_OK;
  if (!A || !W || !C) return fail(ctx, MB_ERR_ARG, "null pointer");
  if (lda < K || ldc < N) return fail(ctx, MB_ERR_ARG, "leading dimension below the row width");
  const size_t need = gemm_partial_floats(M, N, K);
  if (need > kScratchFloats)
    return fail(ctx, MB_ERR_ARG,
                "M %d N %d K %d needs %zu floats of split-K partials; the static scratch holds %zu",
                M, N, K, need, kScratchFloats);
  float* part = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_mu);
    part = g_scratch[ctx->device];
  }
  if (!part) return fail(ctx, MB_ERR_STATE, "the static scratch of device %d is not set up", ctx->device);
  return launch_gemm(ctx, epi, A, lda, W, N, K, bias, C, ldc, M, false, part, kScratchFloats);
}
