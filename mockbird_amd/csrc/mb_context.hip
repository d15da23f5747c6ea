// Context lifetime, errors, weights, ring bookkeeping and the host-pointer
// entry points of the C ABI (include/mockbird_hip.h).  Kernels live in
// ring.hip; this file only allocates, validates, stages and launches.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "kv_types.h"
#include "mb_internal.h"

namespace mb {

const DeviceTensor* find(mb_ctx* ctx, const std::string& name, std::initializer_list<int64_t> dims,
                         std::string& missing) {
  auto it = ctx->weights.find(name);
  if (it == ctx->weights.end()) {
    if (missing.empty()) missing = "weight not uploaded: " + name;
    return nullptr;
  }
  const DeviceTensor& t = it->second;
  if (t.dims.size() != dims.size() || !std::equal(dims.begin(), dims.end(), t.dims.begin())) {
    if (missing.empty()) missing = "weight has the wrong shape: " + name;
    return nullptr;
  }
  return &t;
}

// A device tensor owned by the context under an internal name (freed with
// the uploaded weights); reallocated only when its size changes.
float* internal_tensor(mb_ctx* ctx, const std::string& name, int64_t numel) {
  DeviceTensor& t = ctx->weights[name];
  if (t.ptr && t.numel != numel) {
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipFree(t.ptr);
    ctx->device_bytes -= t.numel * 4;
    t.ptr = nullptr;
  }
  if (!t.ptr) {
    if (hipMalloc(&t.ptr, (size_t)numel * 4) != hipSuccess) {
      ctx->weights.erase(name);
      return nullptr;
    }
    ctx->device_bytes += numel * 4;
    ctx->graph_gen++;
  }
  t.numel = numel;
  t.dims = {numel};
  return t.ptr;
}

void drop_internal(mb_ctx* ctx, const std::string& name) {
  auto it = ctx->weights.find(name);
  if (it == ctx->weights.end()) return;
  if (it->second.ptr) {
    (void)hipStreamSynchronize(ctx->stream);  // no launch in flight still reads it
    (void)hipFree(it->second.ptr);
    ctx->device_bytes -= it->second.numel * 4;
    ctx->graph_gen++;
  }
  ctx->weights.erase(it);
}


int fail(mb_ctx* ctx, int code, const char* fmt, ...) {
  if (ctx) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    ctx->err = buf;
  }
  return code;
}

int hip_fail(mb_ctx* ctx, hipError_t e, const char* what) {
  if (e == hipErrorOutOfMemory)
    return fail(ctx, MB_ERR_NOMEM, "%s: %s", what, hipGetErrorString(e));
  return fail(ctx, MB_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

void* scratch(mb_ctx* ctx, const char* name, size_t bytes) {
  Scratch& s = ctx->scratch[name];
  if (s.bytes >= bytes && s.ptr) return s.ptr;
  if (s.ptr) {
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipFree(s.ptr);
    ctx->device_bytes -= (int64_t)s.bytes;
    s.ptr = nullptr;
    s.bytes = 0;
  }
  size_t want = bytes < 4096 ? 4096 : bytes;
  ctx->graph_gen++;
  if (hipMalloc(&s.ptr, want) != hipSuccess) {
    s.ptr = nullptr;
    return nullptr;
  }
  s.bytes = want;
  ctx->device_bytes += (int64_t)want;
  return s.ptr;
}

}  // namespace mb

using namespace mb;

namespace {

int check_cfg(const mb_config& c, std::string& why) {
  char buf[256];
  if (c.n_layers < 1 || c.n_layers > 64) {
    snprintf(buf, sizeof buf, "n_layers %d out of [1, 64]", c.n_layers);
  } else if (c.capacity < 1 || c.capacity > (1 << 20)) {
    snprintf(buf, sizeof buf, "capacity %d out of [1, 2^20]", c.capacity);
  } else if (c.max_seqs < 1 || c.max_seqs > 65535) {
    snprintf(buf, sizeof buf, "max_seqs %d out of [1, 65535]", c.max_seqs);
  } else if (c.max_rows < 1 || c.max_rows > (1 << 20)) {
    snprintf(buf, sizeof buf, "max_rows %d out of [1, 2^20]", c.max_rows);
  } else if (c.kv_dtype != MB_KV_F32 && c.kv_dtype != MB_KV_BF16) {
    snprintf(buf, sizeof buf, "kv_dtype %d is neither MB_KV_F32 nor MB_KV_BF16", c.kv_dtype);
  } else if (c.wrap != 0 && c.wrap != 1) {
    snprintf(buf, sizeof buf, "wrap must be 0 or 1, got %d", c.wrap);
  } else if (c.vocab < 0) {
    snprintf(buf, sizeof buf, "vocab %d is negative", c.vocab);
  } else if (c.device < 0) {
    snprintf(buf, sizeof buf, "device %d is negative", c.device);
  } else {
    return 0;
  }
  why = buf;
  return 1;
}

// Validate positions of a host-pointer call against the ring's rule.
int check_positions(mb_ctx* ctx, int B, const int32_t* pos0, const int32_t* n_rows, int rows_max) {
  for (int b = 0; b < B; b++) {
    const int64_t n = n_rows ? n_rows[b] : 1;
    if (pos0[b] < 0) return fail(ctx, MB_ERR_ARG, "sequence %d: negative position %d", b, pos0[b]);
    if (n < 0 || n > rows_max || n > ctx->cfg.capacity)
      return fail(ctx, MB_ERR_ARG, "sequence %d: n_rows %lld out of [0, min(%d, capacity %d)]", b,
                  (long long)n, rows_max, ctx->cfg.capacity);
    const int64_t last = (int64_t)pos0[b] + n - 1;
    if (last > INT32_MAX - 1) return fail(ctx, MB_ERR_ARG, "sequence %d: position overflow", b);
    if (!ctx->cfg.wrap && n > 0 && last >= ctx->cfg.capacity)
      return fail(ctx, MB_ERR_RANGE,
                  "decode position %lld exceeds the KV ring (%d slots); it must be sized "
                  "prefill_rows + max_new_frames",
                  (long long)last, ctx->cfg.capacity);
  }
  return MB_OK;
}

int check_common(mb_ctx* ctx, int layer, int B) {
  if (!ctx) return MB_ERR_ARG;
  if (layer < 0 || layer >= ctx->cfg.n_layers)
    return fail(ctx, MB_ERR_ARG, "layer %d out of [0, %d)", layer, ctx->cfg.n_layers);
  if (B < 0 || B > ctx->cfg.max_seqs)
    return fail(ctx, MB_ERR_ARG, "B %d out of [0, %d]", B, ctx->cfg.max_seqs);
  return MB_OK;
}

}  // namespace

extern "C" {

int mb_abi_version(void) { return MB_ABI_VERSION; }

int mb_create(const mb_config* cfg, mb_ctx** out) {
  if (!cfg || !out) return MB_ERR_ARG;
  *out = nullptr;
  std::string why;
  if (check_cfg(*cfg, why)) {
    fprintf(stderr, "mb_create: %s\n", why.c_str());
    return MB_ERR_ARG;
  }
  // the caller's current device is given back on return
  mb::DeviceGuard guard(cfg->device);
  mb_ctx* ctx = new mb_ctx();
  ctx->cfg = *cfg;
  ctx->device = cfg->device;
  int rc = MB_OK;
  do {
    hipError_t e = hipSetDevice(cfg->device);
    if (e != hipSuccess) { rc = hip_fail(ctx, e, "hipSetDevice"); break; }
    {
      int cus = 0, xccs = 0;
      if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, cfg->device) ==
              hipSuccess &&
          hipDeviceGetAttribute(&xccs, hipDeviceAttributeNumberOfXccs, cfg->device) == hipSuccess &&
          xccs > 0 && cus >= xccs) {
        ctx->xcds = xccs;
        ctx->cus_per_xcd = cus / xccs;
      }
    }
    if ((rc = noalloc_init(ctx))) break;
    e = hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking);
    if (e != hipSuccess) { rc = hip_fail(ctx, e, "hipStreamCreate"); break; }
    ctx->stream = ctx->own_stream;
    const int64_t slots = (int64_t)cfg->n_layers * cfg->max_seqs * cfg->capacity;
    ctx->ring_bytes = (size_t)slots * H * HD * kv_elem_bytes(ctx);
    e = hipMalloc(&ctx->ring_k, ctx->ring_bytes);
    if (e != hipSuccess) { rc = hip_fail(ctx, e, "hipMalloc(ring K)"); break; }
    e = hipMalloc(&ctx->ring_v, ctx->ring_bytes);
    if (e != hipSuccess) { rc = hip_fail(ctx, e, "hipMalloc(ring V)"); break; }
    e = hipMalloc(&ctx->slot_pos, (size_t)slots * sizeof(int32_t));
    if (e != hipSuccess) { rc = hip_fail(ctx, e, "hipMalloc(slot_pos)"); break; }
    {
      // (cos, sin) of float(pos) * inv_freq[i], in double, rounded to fp32
      std::vector<float2> tab((size_t)kRopeTab * 32);
      for (int i = 0; i < 32; i++) {
        float inv;
        memcpy(&inv, &kInvFreqBits[i], 4);
        for (int p = 0; p < kRopeTab; p++) {
          const float a = (float)p * inv;
          tab[(size_t)p * 32 + i] = make_float2((float)cos((double)a), (float)sin((double)a));
        }
      }
      e = hipMalloc(&ctx->rope_tab, tab.size() * sizeof(float2));
      if (e != hipSuccess) { rc = hip_fail(ctx, e, "hipMalloc(rope table)"); break; }
      e = hipMemcpy(ctx->rope_tab, tab.data(), tab.size() * sizeof(float2), hipMemcpyHostToDevice);
      if (e != hipSuccess) { rc = hip_fail(ctx, e, "hipMemcpy(rope table)"); break; }
    }
    ctx->device_bytes = 2 * (int64_t)ctx->ring_bytes + slots * 4 + (int64_t)kRopeTab * 32 * 8;
    // every slot empty; K/V zero so a read of an unwritten slot is well defined
    rc = launch_fill_kv(ctx, ctx->ring_k, (int64_t)(ctx->ring_bytes / kv_elem_bytes(ctx)), 0.f);
    if (rc) break;
    rc = launch_fill_kv(ctx, ctx->ring_v, (int64_t)(ctx->ring_bytes / kv_elem_bytes(ctx)), 0.f);
    if (rc) break;
    rc = launch_fill_i32(ctx, ctx->slot_pos, slots, -1);
    if (rc) break;
    e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) { rc = hip_fail(ctx, e, "hipStreamSynchronize"); break; }
  } while (0);
  if (rc != MB_OK) {
    fprintf(stderr, "mb_create: %s\n", ctx->err.c_str());
    mb_destroy(ctx);
    return rc;
  }
  *out = ctx;
  return MB_OK;
}

void mb_destroy(mb_ctx* ctx) {
  MB_DEVICE_GUARD(ctx);
  if (!ctx) return;
  if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
  mb::codec_free(ctx);
  for (auto& kv : ctx->weights) (void)hipFree(kv.second.ptr);
  for (auto& kv : ctx->scratch) (void)hipFree(kv.second.ptr);
  (void)hipFree(ctx->ring_k);
  (void)hipFree(ctx->ring_v);
  (void)hipFree(ctx->slot_pos);
  (void)hipFree(ctx->rope_tab);
  for (void* p : {(void*)ctx->local_k, (void*)ctx->local_v, (void*)ctx->local_sp,
                  (void*)ctx->local_pos, (void*)ctx->seen, (void*)ctx->tokens, (void*)ctx->cont})
    (void)hipFree(p);
  if (ctx->frame_exec) (void)hipGraphExecDestroy(ctx->frame_exec);
  if (ctx->capture_stream) (void)hipStreamDestroy(ctx->capture_stream);
  if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
  delete ctx;
}

const char* mb_last_error(const mb_ctx* ctx) { return ctx ? ctx->err.c_str() : "null context"; }

int mb_set_stream(mb_ctx* ctx, void* hip_stream) {
  if (!ctx) return MB_ERR_ARG;
  ctx->stream = (hipStream_t)hip_stream;
  return MB_OK;
}

void* mb_get_stream(mb_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int mb_synchronize(mb_ctx* ctx) {
  MB_DEVICE_GUARD(ctx);
  if (!ctx) return MB_ERR_ARG;
  MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return MB_OK;
}

int64_t mb_device_bytes(const mb_ctx* ctx) { return ctx ? ctx->device_bytes : 0; }

int mb_cancel(mb_ctx* ctx, int on) {
  if (!ctx) return MB_ERR_ARG;
  ctx->cancel.store(on ? 1 : 0);
  return MB_OK;
}

int mb_upload_tensor(mb_ctx* ctx, const char* name, const float* data, const int64_t* dims,
                     int ndims) {
  MB_DEVICE_GUARD(ctx);
  if (!ctx) return MB_ERR_ARG;
  if (!name || !data || !dims || ndims < 1 || ndims > 4)
    return fail(ctx, MB_ERR_ARG, "mb_upload_tensor: bad arguments");
  if (name[0] == '#')  // the context's own derived tensors live under '#' names
    return fail(ctx, MB_ERR_ARG, "mb_upload_tensor: names starting with '#' are reserved");
  int64_t numel = 1;
  for (int i = 0; i < ndims; i++) {
    if (dims[i] < 1) return fail(ctx, MB_ERR_ARG, "mb_upload_tensor(%s): dim %d is %lld", name, i,
                                 (long long)dims[i]);
    if (dims[i] > ((int64_t)1 << 40) / numel)
      return fail(ctx, MB_ERR_ARG, "mb_upload_tensor(%s): more than 2^40 elements", name);
    numel *= dims[i];
  }
  DeviceTensor& t = ctx->weights[name];
  if (t.ptr && t.numel != numel) {
    MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
    (void)hipFree(t.ptr);
    ctx->device_bytes -= t.numel * 4;
    t.ptr = nullptr;
  }
  if (!t.ptr) {
    hipError_t e = hipMalloc(&t.ptr, (size_t)numel * 4);
    if (e != hipSuccess) {
      ctx->weights.erase(name);
      return hip_fail(ctx, e, "hipMalloc(weight)");
    }
    ctx->device_bytes += numel * 4;
  }
  t.numel = numel;
  t.dims.assign(dims, dims + ndims);
  ctx->model_ok = false;
  ctx->codec_ok = false;
  ctx->graph_gen++;
  MB_HIP(ctx, hipMemcpyAsync(t.ptr, data, (size_t)numel * 4, hipMemcpyHostToDevice, ctx->stream));
  MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return MB_OK;
}

int mb_ring_reset(mb_ctx* ctx, int n, const int32_t* seq_ids) {
  MB_DEVICE_GUARD(ctx);
  if (!ctx) return MB_ERR_ARG;
  const int64_t C = ctx->cfg.capacity;
  if (n < 0) {
    const int64_t slots = (int64_t)ctx->cfg.n_layers * ctx->cfg.max_seqs * C;
    int rc = launch_fill_i32(ctx, ctx->slot_pos, slots, -1);
    if (rc) return rc;
  } else {
    if (n > 0 && !seq_ids) return fail(ctx, MB_ERR_ARG, "mb_ring_reset: seq_ids is null");
    for (int i = 0; i < n; i++)
      if (seq_ids[i] < 0 || seq_ids[i] >= ctx->cfg.max_seqs)
        return fail(ctx, MB_ERR_ARG, "mb_ring_reset: sequence %d out of range", seq_ids[i]);
    for (int l = 0; l < ctx->cfg.n_layers; l++)
      for (int i = 0; i < n; i++) {
        int rc = launch_fill_i32(ctx, ctx->slot_pos + slot_base(ctx, l, seq_ids[i]), C, -1);
        if (rc) return rc;
      }
  }
  MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return MB_OK;
}

int mb_ring_poison(mb_ctx* ctx, int layer, int seq, int n_slots, float sentinel) {
  MB_DEVICE_GUARD(ctx);
  int rc = check_common(ctx, layer, 0);
  if (rc) return rc;
  if (seq < 0 || seq >= ctx->cfg.max_seqs || n_slots < 0 || n_slots > ctx->cfg.capacity)
    return fail(ctx, MB_ERR_ARG, "mb_ring_poison: seq %d / n_slots %d out of range", seq, n_slots);
  const int64_t C = ctx->cfg.capacity;
  const size_t e = kv_elem_bytes(ctx);
  for (int h = 0; h < H; h++) {
    const int64_t off = ring_base(ctx, layer, seq) + (int64_t)h * C * HD;
    rc = launch_fill_kv(ctx, (char*)ctx->ring_k + off * e, (int64_t)n_slots * HD, sentinel);
    if (rc) return rc;
    rc = launch_fill_kv(ctx, (char*)ctx->ring_v + off * e, (int64_t)n_slots * HD, sentinel);
    if (rc) return rc;
  }
  MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return MB_OK;
}

int mb_read_ring(mb_ctx* ctx, int layer, int seq, int slot0, int n, float* k, float* v,
                 int32_t* slot_pos) {
  MB_DEVICE_GUARD(ctx);
  int rc = check_common(ctx, layer, 0);
  if (rc) return rc;
  const int C = ctx->cfg.capacity;
  if (seq < 0 || seq >= ctx->cfg.max_seqs || slot0 < 0 || n < 0 || slot0 + n > C)
    return fail(ctx, MB_ERR_ARG, "mb_read_ring: seq %d slots [%d, %d) out of range", seq, slot0,
                slot0 + n);
  if (n == 0) return MB_OK;
  const size_t e = kv_elem_bytes(ctx);
  std::vector<uint8_t> host((size_t)H * n * HD * e);
  for (int which = 0; which < 2; which++) {
    float* dst = which == 0 ? k : v;
    if (!dst) continue;
    const char* src = (const char*)(which == 0 ? ctx->ring_k : ctx->ring_v);
    for (int h = 0; h < H; h++) {
      const int64_t off = ring_base(ctx, layer, seq) + ((int64_t)h * C + slot0) * HD;
      MB_HIP(ctx, hipMemcpyAsync(host.data() + (size_t)h * n * HD * e, src + off * e,
                                 (size_t)n * HD * e, hipMemcpyDeviceToHost, ctx->stream));
    }
    MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
    // device [head][slot][dim] -> reference [slot][head*64 + dim]
    for (int h = 0; h < H; h++)
      for (int s = 0; s < n; s++)
        for (int d = 0; d < HD; d++) {
          const size_t i = ((size_t)h * n + s) * HD + d;
          float f;
          if (e == 2) {
            uint32_t u = (uint32_t)((const uint16_t*)host.data())[i] << 16;
            memcpy(&f, &u, 4);
          } else {
            f = ((const float*)host.data())[i];
          }
          dst[(size_t)s * D + h * HD + d] = f;
        }
  }
  if (slot_pos) {
    MB_HIP(ctx, hipMemcpyAsync(slot_pos, ctx->slot_pos + slot_base(ctx, layer, seq) + slot0,
                               (size_t)n * 4, hipMemcpyDeviceToHost, ctx->stream));
    MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
  }
  return MB_OK;
}

int mb_write_ring(mb_ctx* ctx, int layer, int seq, int slot0, int n, const float* k,
                  const float* v, const int32_t* slot_pos) {
  MB_DEVICE_GUARD(ctx);
  int rc = check_common(ctx, layer, 0);
  if (rc) return rc;
  const int C = ctx->cfg.capacity;
  if (seq < 0 || seq >= ctx->cfg.max_seqs || slot0 < 0 || n < 0 || slot0 + n > C)
    return fail(ctx, MB_ERR_ARG, "mb_write_ring: seq %d slots [%d, %d) out of range", seq, slot0,
                slot0 + n);
  if (n == 0) return MB_OK;
  // Every stored position must be one the ring's own writes could have left
  // in that slot: empty (-1), or pos mod C (pos itself on a non-wrapping ring).
  if (slot_pos)
    for (int i = 0; i < n; i++) {
      const int32_t p = slot_pos[i], s = slot0 + i;
      const bool ok = p == -1 || (p >= 0 && (ctx->cfg.wrap ? p % C == s : p == s));
      if (!ok)
        return fail(ctx, MB_ERR_ARG, "mb_write_ring: position %d cannot sit in slot %d of a "
                    "%s ring of %d slots", p, s, ctx->cfg.wrap ? "wrapping" : "non-wrapping", C);
    }
  const size_t e = kv_elem_bytes(ctx);
  std::vector<uint8_t> host((size_t)H * n * HD * e);
  for (int which = 0; which < 2; which++) {
    const float* src = which == 0 ? k : v;
    if (!src) continue;
    // reference [slot][head*64 + dim] -> device [head][slot][dim]
    for (int h = 0; h < H; h++)
      for (int s = 0; s < n; s++)
        for (int d = 0; d < HD; d++) {
          const size_t i = ((size_t)h * n + s) * HD + d;
          const float f = src[(size_t)s * D + h * HD + d];
          if (e == 2) ((uint16_t*)host.data())[i] = f32_to_bf16(f);  // the kernels' rounding
          else ((float*)host.data())[i] = f;
        }
    char* dst = (char*)(which == 0 ? ctx->ring_k : ctx->ring_v);
    for (int h = 0; h < H; h++) {
      const int64_t off = ring_base(ctx, layer, seq) + ((int64_t)h * C + slot0) * HD;
      MB_HIP(ctx, hipMemcpyAsync(dst + off * e, host.data() + (size_t)h * n * HD * e,
                                 (size_t)n * HD * e, hipMemcpyHostToDevice, ctx->stream));
    }
    MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
  }
  if (slot_pos) {
    MB_HIP(ctx, hipMemcpyAsync(ctx->slot_pos + slot_base(ctx, layer, seq) + slot0, slot_pos,
                               (size_t)n * 4, hipMemcpyHostToDevice, ctx->stream));
    MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
  }
  return MB_OK;
}

int mb_ring_write_rows_dev(mb_ctx* ctx, int layer, int B, int rows_max, const void* qkv,
                           int qkv_dtype, const int32_t* pos0, const int32_t* n_rows, void* q_out,
                           int q_dtype) {
  MB_DEVICE_GUARD(ctx);
  int rc = check_common(ctx, layer, B);
  if (rc) return rc;
  if (rows_max < 1 || rows_max > ctx->cfg.max_rows)
    return fail(ctx, MB_ERR_ARG, "rows_max %d out of [1, %d]", rows_max, ctx->cfg.max_rows);
  if ((qkv_dtype != MB_DT_F32 && qkv_dtype != MB_DT_BF16) ||
      (q_dtype != MB_DT_F32 && q_dtype != MB_DT_BF16))
    return fail(ctx, MB_ERR_ARG, "unknown dtype");
  if (B == 0) return MB_OK;
  if (!qkv || !pos0 || !n_rows) return fail(ctx, MB_ERR_ARG, "null pointer");
  return launch_ring_write(ctx, global_ring(ctx, layer), B, rows_max, qkv, qkv_dtype,
                           dense_rows(QKV, rows_max), pos0, n_rows, q_out, q_dtype,
                           dense_rows(D, rows_max));
}

int mb_ring_append_dev(mb_ctx* ctx, int layer, int B, const void* qkv, int qkv_dtype,
                       int64_t qkv_stride, const int32_t* pos, float* q_out, int64_t q_stride) {
  MB_DEVICE_GUARD(ctx);
  int rc = check_common(ctx, layer, B);
  if (rc) return rc;
  if (qkv_dtype != MB_DT_F32 && qkv_dtype != MB_DT_BF16)
    return fail(ctx, MB_ERR_ARG, "unknown dtype");
  if (qkv_stride < QKV || (q_out && q_stride < D))
    return fail(ctx, MB_ERR_ARG, "row stride too small");
  if (B == 0) return MB_OK;
  if (!qkv || !pos) return fail(ctx, MB_ERR_ARG, "null pointer");
  return launch_ring_write(ctx, global_ring(ctx, layer), B, 1, qkv, qkv_dtype,
                           dense_rows(qkv_stride, 1), pos, nullptr, q_out, MB_DT_F32,
                           dense_rows(q_stride, 1));
}

int mb_decode_attention_dev(mb_ctx* ctx, int layer, int B, const float* q, int64_t q_stride,
                            const int32_t* pos, int32_t max_pos, float* out, int64_t out_stride) {
  MB_DEVICE_GUARD(ctx);
  int rc = check_common(ctx, layer, B);
  if (rc) return rc;
  if (q_stride < D || out_stride < D) return fail(ctx, MB_ERR_ARG, "row stride too small");
  if (max_pos < 0) return fail(ctx, MB_ERR_ARG, "max_pos %d is negative", max_pos);
  if (B == 0) return MB_OK;
  if (!q || !pos || !out) return fail(ctx, MB_ERR_ARG, "null pointer");
  return launch_attn(ctx, global_ring(ctx, layer), B, 1, q, dense_rows(q_stride, 1), pos, nullptr,
                     (int64_t)max_pos + 1, out, dense_rows(out_stride, 1));
}

int mb_append_attend_dev(mb_ctx* ctx, int layer, int B, const void* qkv, int qkv_dtype,
                         int64_t qkv_stride, const int32_t* pos, int32_t max_pos, float* q_out,
                         int64_t q_stride, float* out, int64_t out_stride) {
  MB_DEVICE_GUARD(ctx);
  int rc = check_common(ctx, layer, B);
  if (rc) return rc;
  if (qkv_dtype != MB_DT_F32 && qkv_dtype != MB_DT_BF16)
    return fail(ctx, MB_ERR_ARG, "unknown dtype");
  if (qkv_stride < QKV || out_stride < D || (q_out && q_stride < D))
    return fail(ctx, MB_ERR_ARG, "row stride too small");
  if (max_pos < 0) return fail(ctx, MB_ERR_ARG, "max_pos %d is negative", max_pos);
  if (!ctx->cfg.wrap && max_pos >= ctx->cfg.capacity)
    return fail(ctx, MB_ERR_RANGE,
                "decode position %d exceeds the KV ring (%d slots); it must be sized "
                "prefill_rows + max_new_frames",
                max_pos, ctx->cfg.capacity);
  if (B == 0) return MB_OK;
  if (!qkv || !pos || !out) return fail(ctx, MB_ERR_ARG, "null pointer");
  return launch_append_attn(ctx, global_ring(ctx, layer), B, qkv, qkv_dtype,
                            dense_rows(qkv_stride, 1), pos, (int64_t)max_pos + 1, q_out,
                            dense_rows(q_stride, 1), out, dense_rows(out_stride, 1));
}

int mb_prefill_attention_dev(mb_ctx* ctx, int layer, int B, int rows_max, const void* q,
                             int q_dtype, const int32_t* pos0, const int32_t* n_rows, float* out) {
  MB_DEVICE_GUARD(ctx);
  int rc = check_common(ctx, layer, B);
  if (rc) return rc;
  if (rows_max < 1 || rows_max > ctx->cfg.max_rows)
    return fail(ctx, MB_ERR_ARG, "rows_max %d out of [1, %d]", rows_max, ctx->cfg.max_rows);
  if (q_dtype != MB_DT_F32 && q_dtype != MB_DT_BF16) return fail(ctx, MB_ERR_ARG, "unknown dtype");
  if (B == 0) return MB_OK;
  if (!q || !pos0 || !n_rows || !out) return fail(ctx, MB_ERR_ARG, "null pointer");
  return launch_prefill_attention(ctx, global_ring(ctx, layer), B, rows_max, q, q_dtype,
                                  dense_rows(D, rows_max), pos0, n_rows, out,
                                  dense_rows(D, rows_max));
}

int mb_linear_dev(mb_ctx* ctx, int M, int N, int K, const float* A, int64_t lda, const float* W,
                  const float* bias, float* C, int64_t ldc, int epi) {
  MB_DEVICE_GUARD(ctx);
  if (!ctx) return MB_ERR_ARG;
  if (M < 0 || N < 1 || K < 1) return fail(ctx, MB_ERR_ARG, "linear shape M %d N %d K %d", M, N, K);
  if (epi < EPI_STORE || epi > EPI_GELU_ERF) return fail(ctx, MB_ERR_ARG, "unknown epilogue %d", epi);
  if (epi == EPI_SCALE_ADD && !bias)
    return fail(ctx, MB_ERR_ARG, "MB_EPI_SCALE_ADD needs the scale vector in `bias`");
  if (M == 0) return MB_OK;
  if (!A || !W || !C) return fail(ctx, MB_ERR_ARG, "null pointer");
  if (lda < K || ldc < N) return fail(ctx, MB_ERR_ARG, "leading dimension below the row width");
  return launch_gemm(ctx, epi, A, lda, W, N, K, bias, C, ldc, M);
}

int mb_split_weights_dev(mb_ctx* ctx, const float* W, int K, int N, void* Wx) {
  MB_DEVICE_GUARD(ctx);
  if (!ctx) return MB_ERR_ARG;
  if (K < 1 || N < 1) return fail(ctx, MB_ERR_ARG, "split weights shape K %d N %d", K, N);
  if (!W || !Wx) return fail(ctx, MB_ERR_ARG, "null pointer");
  if (((uintptr_t)Wx & 15)) return fail(ctx, MB_ERR_ARG, "Wx must be 16-byte aligned");
  return launch_split_w(ctx, W, K, N, Wx, false);
}

int mb_linear_split_dev(mb_ctx* ctx, int M, int N, int K, const float* A, int64_t lda,
                        const void* Wx, const float* bias, float* C, int64_t ldc, int epi) {
  MB_DEVICE_GUARD(ctx);
  if (!ctx) return MB_ERR_ARG;
  if (M < 0 || N < 1 || K < 1) return fail(ctx, MB_ERR_ARG, "linear shape M %d N %d K %d", M, N, K);
  if (epi < EPI_STORE || epi > EPI_GELU_ERF) return fail(ctx, MB_ERR_ARG, "unknown epilogue %d", epi);
  if (epi == EPI_SCALE_ADD && !bias)
    return fail(ctx, MB_ERR_ARG, "MB_EPI_SCALE_ADD needs the scale vector in `bias`");
  if (M == 0) return MB_OK;
  if (!A || !Wx || !C) return fail(ctx, MB_ERR_ARG, "null pointer");
  if (lda < K || ldc < N) return fail(ctx, MB_ERR_ARG, "leading dimension below the row width");
  return launch_gemm_x3(ctx, epi, A, lda, Wx, N, K, bias, C, ldc, M, nullptr, nullptr);
}

// ---------------------------------------------------------- host pointers

int mb_ring_write_rows(mb_ctx* ctx, int layer, int B, int rows_max, const float* qkv,
                       const int32_t* pos0, const int32_t* n_rows, float* q_out) {
  MB_DEVICE_GUARD(ctx);
  int rc = check_common(ctx, layer, B);
  if (rc) return rc;
  if (rows_max < 1 || rows_max > ctx->cfg.max_rows)
    return fail(ctx, MB_ERR_ARG, "rows_max %d out of [1, %d]", rows_max, ctx->cfg.max_rows);
  if (B == 0) return MB_OK;
  if (!qkv || !pos0 || !n_rows) return fail(ctx, MB_ERR_ARG, "null pointer");
  rc = check_positions(ctx, B, pos0, n_rows, rows_max);
  if (rc) return rc;
  const size_t rows = (size_t)B * rows_max;
  float* d_qkv = (float*)scratch(ctx, "qkv", rows * QKV * 4);
  float* d_q = (float*)scratch(ctx, "q", rows * D * 4);
  int32_t* d_pos = (int32_t*)scratch(ctx, "pos", (size_t)B * 8);
  if (!d_qkv || !d_q || !d_pos) return fail(ctx, MB_ERR_NOMEM, "staging allocation failed");
  MB_HIP(ctx, hipMemcpyAsync(d_qkv, qkv, rows * QKV * 4, hipMemcpyHostToDevice, ctx->stream));
  MB_HIP(ctx, hipMemcpyAsync(d_pos, pos0, (size_t)B * 4, hipMemcpyHostToDevice, ctx->stream));
  MB_HIP(ctx, hipMemcpyAsync(d_pos + B, n_rows, (size_t)B * 4, hipMemcpyHostToDevice, ctx->stream));
  rc = launch_ring_write(ctx, global_ring(ctx, layer), B, rows_max, d_qkv, MB_DT_F32,
                         dense_rows(QKV, rows_max), d_pos, d_pos + B, q_out ? d_q : nullptr,
                         MB_DT_F32, dense_rows(D, rows_max));
  if (rc) return rc;
  if (q_out) MB_HIP(ctx, hipMemcpyAsync(q_out, d_q, rows * D * 4, hipMemcpyDeviceToHost, ctx->stream));
  MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return MB_OK;
}

int mb_ring_append(mb_ctx* ctx, int layer, int B, const float* qkv, const int32_t* pos,
                   float* q_out) {
  MB_DEVICE_GUARD(ctx);
  int rc = check_common(ctx, layer, B);
  if (rc) return rc;
  if (B == 0) return MB_OK;
  if (!qkv || !pos) return fail(ctx, MB_ERR_ARG, "null pointer");
  rc = check_positions(ctx, B, pos, nullptr, 1);
  if (rc) return rc;
  float* d_qkv = (float*)scratch(ctx, "qkv", (size_t)B * QKV * 4);
  float* d_q = (float*)scratch(ctx, "q", (size_t)B * D * 4);
  int32_t* d_pos = (int32_t*)scratch(ctx, "pos", (size_t)B * 8);
  if (!d_qkv || !d_q || !d_pos) return fail(ctx, MB_ERR_NOMEM, "staging allocation failed");
  MB_HIP(ctx, hipMemcpyAsync(d_qkv, qkv, (size_t)B * QKV * 4, hipMemcpyHostToDevice, ctx->stream));
  MB_HIP(ctx, hipMemcpyAsync(d_pos, pos, (size_t)B * 4, hipMemcpyHostToDevice, ctx->stream));
  rc = launch_ring_write(ctx, global_ring(ctx, layer), B, 1, d_qkv, MB_DT_F32, dense_rows(QKV, 1),
                         d_pos, nullptr, q_out ? d_q : nullptr, MB_DT_F32, dense_rows(D, 1));
  if (rc) return rc;
  if (q_out) MB_HIP(ctx, hipMemcpyAsync(q_out, d_q, (size_t)B * D * 4, hipMemcpyDeviceToHost, ctx->stream));
  MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return MB_OK;
}

int mb_decode_attention(mb_ctx* ctx, int layer, int B, const float* q, const int32_t* pos,
                        float* out) {
  MB_DEVICE_GUARD(ctx);
  int rc = check_common(ctx, layer, B);
  if (rc) return rc;
  if (B == 0) return MB_OK;
  if (!q || !pos || !out) return fail(ctx, MB_ERR_ARG, "null pointer");
  int32_t max_pos = 0;
  for (int b = 0; b < B; b++) {
    if (pos[b] < 0) return fail(ctx, MB_ERR_ARG, "sequence %d: negative position %d", b, pos[b]);
    if (pos[b] > max_pos) max_pos = pos[b];
  }
  float* d_q = (float*)scratch(ctx, "q", (size_t)B * D * 4);
  float* d_out = (float*)scratch(ctx, "out", (size_t)B * D * 4);
  int32_t* d_pos = (int32_t*)scratch(ctx, "pos", (size_t)B * 8);
  if (!d_q || !d_out || !d_pos) return fail(ctx, MB_ERR_NOMEM, "staging allocation failed");
  MB_HIP(ctx, hipMemcpyAsync(d_q, q, (size_t)B * D * 4, hipMemcpyHostToDevice, ctx->stream));
  MB_HIP(ctx, hipMemcpyAsync(d_pos, pos, (size_t)B * 4, hipMemcpyHostToDevice, ctx->stream));
  rc = launch_attn(ctx, global_ring(ctx, layer), B, 1, d_q, dense_rows(D, 1), d_pos, nullptr,
                   (int64_t)max_pos + 1, d_out, dense_rows(D, 1));
  if (rc) return rc;
  MB_HIP(ctx, hipMemcpyAsync(out, d_out, (size_t)B * D * 4, hipMemcpyDeviceToHost, ctx->stream));
  MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return MB_OK;
}

int mb_append_attend(mb_ctx* ctx, int layer, int B, const float* qkv, const int32_t* pos,
                     float* q_out, float* out) {
  MB_DEVICE_GUARD(ctx);
  int rc = check_common(ctx, layer, B);
  if (rc) return rc;
  if (B == 0) return MB_OK;
  if (!qkv || !pos || !out) return fail(ctx, MB_ERR_ARG, "null pointer");
  rc = check_positions(ctx, B, pos, nullptr, 1);
  if (rc) return rc;
  int32_t max_pos = 0;
  for (int b = 0; b < B; b++) max_pos = pos[b] > max_pos ? pos[b] : max_pos;
  float* d_qkv = (float*)scratch(ctx, "qkv", (size_t)B * QKV * 4);
  float* d_q = (float*)scratch(ctx, "q", (size_t)B * D * 4);
  float* d_out = (float*)scratch(ctx, "out", (size_t)B * D * 4);
  int32_t* d_pos = (int32_t*)scratch(ctx, "pos", (size_t)B * 8);
  if (!d_qkv || !d_q || !d_out || !d_pos) return fail(ctx, MB_ERR_NOMEM, "staging allocation failed");
  MB_HIP(ctx, hipMemcpyAsync(d_qkv, qkv, (size_t)B * QKV * 4, hipMemcpyHostToDevice, ctx->stream));
  MB_HIP(ctx, hipMemcpyAsync(d_pos, pos, (size_t)B * 4, hipMemcpyHostToDevice, ctx->stream));
  rc = launch_append_attn(ctx, global_ring(ctx, layer), B, d_qkv, MB_DT_F32, dense_rows(QKV, 1),
                          d_pos, (int64_t)max_pos + 1, q_out ? d_q : nullptr, dense_rows(D, 1),
                          d_out, dense_rows(D, 1));
  if (rc) return rc;
  if (q_out) MB_HIP(ctx, hipMemcpyAsync(q_out, d_q, (size_t)B * D * 4, hipMemcpyDeviceToHost, ctx->stream));
  MB_HIP(ctx, hipMemcpyAsync(out, d_out, (size_t)B * D * 4, hipMemcpyDeviceToHost, ctx->stream));
  MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return MB_OK;
}

int mb_prefill_attention(mb_ctx* ctx, int layer, int B, int rows_max, const float* q,
                         const int32_t* pos0, const int32_t* n_rows, float* out) {
  MB_DEVICE_GUARD(ctx);
  int rc = check_common(ctx, layer, B);
  if (rc) return rc;
  if (rows_max < 1 || rows_max > ctx->cfg.max_rows)
    return fail(ctx, MB_ERR_ARG, "rows_max %d out of [1, %d]", rows_max, ctx->cfg.max_rows);
  if (B == 0) return MB_OK;
  if (!q || !pos0 || !n_rows || !out) return fail(ctx, MB_ERR_ARG, "null pointer");
  rc = check_positions(ctx, B, pos0, n_rows, rows_max);
  if (rc) return rc;
  const size_t rows = (size_t)B * rows_max;
  float* d_q = (float*)scratch(ctx, "q", rows * D * 4);
  float* d_out = (float*)scratch(ctx, "out", rows * D * 4);
  int32_t* d_pos = (int32_t*)scratch(ctx, "pos", (size_t)B * 8);
  if (!d_q || !d_out || !d_pos) return fail(ctx, MB_ERR_NOMEM, "staging allocation failed");
  MB_HIP(ctx, hipMemcpyAsync(d_q, q, rows * D * 4, hipMemcpyHostToDevice, ctx->stream));
  MB_HIP(ctx, hipMemcpyAsync(d_pos, pos0, (size_t)B * 4, hipMemcpyHostToDevice, ctx->stream));
  MB_HIP(ctx, hipMemcpyAsync(d_pos + B, n_rows, (size_t)B * 4, hipMemcpyHostToDevice, ctx->stream));
  rc = launch_prefill_attention(ctx, global_ring(ctx, layer), B, rows_max, d_q, MB_DT_F32,
                                dense_rows(D, rows_max), d_pos, d_pos + B, d_out,
                                dense_rows(D, rows_max));
  if (rc) return rc;
  MB_HIP(ctx, hipMemcpyAsync(out, d_out, rows * D * 4, hipMemcpyDeviceToHost, ctx->stream));
  MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return MB_OK;
}

}  // extern "C"
