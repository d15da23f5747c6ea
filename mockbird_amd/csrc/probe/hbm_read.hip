// Measurement only (not part of the decoder library): the HBM read ceiling
// that bench.py reports beside the decode-attention roofline.  One kernel
// streams a buffer front to back with 16-byte non-temporal loads, 16 loads
// of 1 KB per wave in flight, each wave reading its own contiguous 256 KB,
// and folds the data into a value it stores only if it matches an
// impossible pattern (so the loads are not optimised away).  Built into
// libmb_probe.so by mockbird_amd/build.py.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace {

constexpr size_t kWaveBytes = 256 << 10;

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void k_stream_read(const char* __restrict__ buf,
                                                     unsigned* __restrict__ sink) {
  const int lane = threadIdx.x & 63;
  const size_t wave = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const char* p = buf + wave * kWaveBytes + lane * 16;
  unsigned acc = 0;
  for (size_t off = 0; off < kWaveBytes; off += 16 * 1024) {
    u32x4_t r[16];
#pragma unroll
    for (int u = 0; u < 16; u++) r[u] = __builtin_nontemporal_load((const u32x4_t*)(p + off + u * 1024));
#pragma unroll
    for (int u = 0; u < 16; u++) acc ^= r[u].x ^ r[u].y ^ r[u].z ^ r[u].w;
  }
  if (acc == 0x9e3779b9u) sink[wave] = acc;
}

}  // namespace

extern "C" {

// Bytes one launch reads for a buffer of `bytes` (whole 1 MiB blocks of four
// 256 KB waves); 0 when the buffer is too small.
size_t mbp_stream_read_bytes(size_t bytes) { return bytes / (4 * kWaveBytes) * 4 * kWaveBytes; }

// Enqueue one streaming read of the first mbp_stream_read_bytes(bytes) bytes
// of `buf` on `stream` (a hipStream_t).  `sink` must hold one unsigned per
// 256 KB read.  Returns 0 or the hipError_t of the launch.
int mbp_stream_read(const void* buf, size_t bytes, void* stream, unsigned* sink) {
  const size_t blocks = bytes / (4 * kWaveBytes);
  if (!buf || !sink || blocks == 0 || blocks > 0x7fffffff) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(k_stream_read, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     (const char*)buf, sink);
  return (int)hipGetLastError();
}

}  // extern "C"
