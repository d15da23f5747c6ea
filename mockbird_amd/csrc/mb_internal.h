// Internal declarations shared by the HIP translation units of libmockbird_hip.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <map>
#include <string>
#include <vector>

#include "../../include/mockbird_hip.h"

namespace mb {

constexpr int D = 768;      // hidden width
constexpr int H = 12;       // heads
constexpr int HD = 64;      // head dim
constexpr int QKV = 2304;   // fused q | k | v
constexpr int FFN = 3072;   // MLP width
constexpr int NVQ = 16;     // audio channels
constexpr int ROW = 17;     // prompt row width
constexpr int PAD = 1024;   // audio pad id
constexpr int CODES = 1024; // codebook size

// One attention partial per (sequence, head, split): 64 accumulators, the
// running max and the running sum, padded to 68 floats (16-byte aligned).
constexpr int PART = 68;

// Positions whose RoPE cos/sin come from the context's table.
constexpr int kRopeTab = 65536;

// fp32 inverse frequencies of the exported graph (torch's fp32 values of
// 1 / 10000^(2i/64)); six entries sit one ulp away from the correctly rounded
// value, and the reference's ORT K fixture fixes which.
constexpr uint32_t kInvFreqBits[32] = {
    0x3f800000u, 0x3f3ff911u, 0x3f0ff59au, 0x3ed7e89bu, 0x3ea1e89bu, 0x3e72d423u,
    0x3e361887u, 0x3e088d77u, 0x3dcccccdu, 0x3d99940du, 0x3d6655c2u, 0x3d2cba15u,
    0x3d0186e3u, 0x3cc2434fu, 0x3c91ad39u, 0x3c5a7bf2u, 0x3c23d70au, 0x3bf5b9b0u,
    0x3bb8449cu, 0x3b8a2e77u, 0x3b4f3e38u, 0x3b1b690du, 0x3ae91528u, 0x3aaec98eu,
    0x3a83126fu, 0x3a44948cu, 0x3a136a16u, 0x39dd1725u, 0x39a5cb60u, 0x3978a815u,
    0x393a7753u, 0x390bd472u};

struct DeviceTensor {
  float* ptr = nullptr;
  std::vector<int64_t> dims;
  int64_t numel = 0;
};

// Growable device scratch used by the host-pointer entry points.
struct Scratch {
  void* ptr = nullptr;
  size_t bytes = 0;
};

}  // namespace mb

struct mb_ctx {
  mb_config cfg{};
  int device = 0;
  hipStream_t own_stream = nullptr;
  hipStream_t stream = nullptr;
  std::string err;

  // Rings, per layer and sequence, head-major across slots:
  //   K/V element (layer, seq, head, slot, dim) at
  //   (((layer * max_seqs + seq) * H + head) * C + slot) * 64 + dim
  // in kv_dtype; slot_pos (layer, seq, slot) at (layer * max_seqs + seq) * C + slot.
  void* ring_k = nullptr;
  void* ring_v = nullptr;
  int32_t* slot_pos = nullptr;
  size_t ring_bytes = 0;  // bytes of ring_k (== ring_v)

  // RoPE cos/sin for positions [0, kRopeTab): (cos, sin) of pair i at
  // position p in rope_tab[p * 32 + i]; later positions are computed in-kernel.
  float2* rope_tab = nullptr;


  std::map<std::string, mb::DeviceTensor> weights;
  std::map<std::string, mb::Scratch> scratch;
  int64_t device_bytes = 0;
  std::atomic<int> cancel{0};
};

namespace mb {

// Record an error message on the context and return `code`.
int fail(mb_ctx* ctx, int code, const char* fmt, ...) __attribute__((format(printf, 3, 4)));

// hipError_t -> MB_ERR_HIP with the call site in the message.
int hip_fail(mb_ctx* ctx, hipError_t e, const char* what);

#define MB_HIP(ctx, call)                                   \
  do {                                                      \
    hipError_t e_ = (call);                                 \
    if (e_ != hipSuccess) return mb::hip_fail((ctx), e_, #call); \
  } while (0)

// Device scratch named `name` of at least `bytes`, kept between calls.
void* scratch(mb_ctx* ctx, const char* name, size_t bytes);

inline size_t kv_elem_bytes(const mb_ctx* ctx) { return ctx->cfg.kv_dtype == MB_KV_BF16 ? 2 : 4; }

// Element offset of (layer, seq, head=0, slot=0, dim=0) in ring_k / ring_v.
inline int64_t ring_base(const mb_ctx* ctx, int layer, int seq) {
  return ((int64_t)layer * ctx->cfg.max_seqs + seq) * H * (int64_t)ctx->cfg.capacity * HD;
}
inline int64_t slot_base(const mb_ctx* ctx, int layer, int seq) {
  return ((int64_t)layer * ctx->cfg.max_seqs + seq) * (int64_t)ctx->cfg.capacity;
}

// Kernel launchers (ring.hip).
int launch_ring_write(mb_ctx* ctx, int layer, int B, int rows_max, const void* qkv, int qkv_dtype,
                      int64_t qkv_row_stride, int64_t qkv_seq_stride, const int32_t* pos0,
                      const int32_t* n_rows, void* q_out, int q_dtype, int64_t q_row_stride,
                      int64_t q_seq_stride);
int launch_decode_attention(mb_ctx* ctx, int layer, int B, const float* q, int64_t q_stride,
                            const int32_t* pos, int32_t max_pos, float* out, int64_t out_stride);
int launch_fill_i32(mb_ctx* ctx, int32_t* p, int64_t n, int32_t value);
int launch_fill_kv(mb_ctx* ctx, void* p, int64_t n, float value);
int launch_prefill_attention(mb_ctx* ctx, int layer, int B, int rows_max, const void* q,
                             int q_dtype, int64_t q_row_stride, int64_t q_seq_stride,
                             const int32_t* pos0, const int32_t* n_rows, float* out,
                             int64_t out_row_stride, int64_t out_seq_stride);

}  // namespace mb
