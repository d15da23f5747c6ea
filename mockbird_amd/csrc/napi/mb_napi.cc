// mockbird_hip.node -- the thin N-API binding of libmockbird_hip.so for the
// JavaScript host engine (mockbird_amd/engine/engine.mjs).
//
// The reference host reaches the GPU through WebGPU (src/lib/tts/engine/gpu.ts,
// prefill.ts, decode.ts); this addon is the one place JavaScript meets the C ABI
// of include/mockbird_hip.h.  It holds no state of its own beyond the context
// handle, checks every typed-array length against the sizes the C call will
// read or write (the C ABI trusts its pointers), copies nothing it does not
// have to (typed arrays are passed by their backing store), and turns a
// non-zero status into a thrown Error carrying mb_last_error() and the status
// name as `code` (MB_ERR_RANGE, ...).
//
// The model calls (prefill, decodeStep, localFrame, decodeFrames,
// codecDecode) also come as *Async forms that run the C call on a libuv
// worker thread and return a Promise, so the reference's awaited engine calls
// (gpu.ts:173-272) leave the Node event loop free.  A context runs one call
// at a time, as the reference's runtime never overlaps two engine calls
// (runtime.ts:523-561): while an asynchronous call is in flight every other
// call on that context throws MB_ERR_BUSY.
#include <node_api.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "mockbird_hip.h"

namespace {

constexpr int64_t kD = 768, kQkv = 2304, kRow = 17, kNvq = 16;

const char* status_name(int rc) {
  switch (rc) {
    case MB_ERR_ARG: return "MB_ERR_ARG";
    case MB_ERR_RANGE: return "MB_ERR_RANGE";
    case MB_ERR_HIP: return "MB_ERR_HIP";
    case MB_ERR_STATE: return "MB_ERR_STATE";
    case MB_ERR_CANCELLED: return "MB_ERR_CANCELLED";
    case MB_ERR_NOMEM: return "MB_ERR_NOMEM";
    default: return "MB_ERR_UNKNOWN";
  }
}

// Thrown-error helpers: each returns nullptr so callers can `return throw_*`.
napi_value throw_type(napi_env env, const std::string& msg) {
  napi_throw_type_error(env, "ERR_INVALID_ARG_TYPE", msg.c_str());
  return nullptr;
}
napi_value throw_range(napi_env env, const std::string& msg) {
  napi_throw_range_error(env, "ERR_OUT_OF_RANGE", msg.c_str());
  return nullptr;
}

// An Error with .code = status name and .status = the numeric code.
napi_value status_error(napi_env env, mb_ctx* ctx, int rc) {
  const char* msg = ctx ? mb_last_error(ctx) : "mb_create failed";
  napi_value code, text, err, st;
  napi_create_string_utf8(env, status_name(rc), NAPI_AUTO_LENGTH, &code);
  napi_create_string_utf8(env, msg && *msg ? msg : status_name(rc), NAPI_AUTO_LENGTH, &text);
  napi_create_error(env, code, text, &err);
  napi_create_int32(env, rc, &st);
  napi_set_named_property(env, err, "status", st);
  return err;
}

napi_value throw_status(napi_env env, mb_ctx* ctx, int rc) {
  napi_throw(env, status_error(env, ctx, rc));
  return nullptr;
}

struct Args {
  napi_env env;
  size_t argc = 12;
  napi_value argv[12];
  bool ok = true;
  Args(napi_env e, napi_callback_info info) : env(e) {
    napi_get_cb_info(e, info, &argc, argv, nullptr, nullptr);
  }
  napi_value at(size_t i) {
    if (i < argc) return argv[i];
    napi_value u;
    napi_get_undefined(env, &u);
    return u;
  }
};

bool get_i64(napi_env env, napi_value v, int64_t* out, const char* what) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t != napi_number) {
    throw_type(env, std::string(what) + " must be a number");
    return false;
  }
  double d;
  napi_get_value_double(env, v, &d);
  // range first: converting a NaN or out-of-range double to an integer is undefined
  if (!(d >= -2147483648.0 && d <= 2147483647.0) || d != (double)(int64_t)d) {
    throw_range(env, std::string(what) + " must be a 32-bit integer");
    return false;
  }
  *out = (int64_t)d;
  return true;
}

bool get_int(napi_env env, napi_value v, int* out, const char* what) {
  int64_t x;
  if (!get_i64(env, v, &x, what)) return false;
  *out = (int)x;
  return true;
}

bool get_f64(napi_env env, napi_value v, double* out, const char* what) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t != napi_number) {
    throw_type(env, std::string(what) + " must be a number");
    return false;
  }
  napi_get_value_double(env, v, out);
  return true;
}

bool get_f32(napi_env env, napi_value v, float* out, const char* what) {
  double d;
  if (!get_f64(env, v, &d, what)) return false;
  *out = (float)d;
  return true;
}

// What a JS context handle (an external) points at: the context and whether
// an asynchronous call on it is in flight.  Only the JS thread touches it.
struct Handle {
  mb_ctx* ctx = nullptr;
  bool busy = false;
};

Handle* get_handle(napi_env env, napi_value v) {
  void* p = nullptr;
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t != napi_external || napi_get_value_external(env, v, &p) != napi_ok || !p) {
    throw_type(env, "the first argument must be a live context handle");
    return nullptr;
  }
  Handle* h = (Handle*)p;
  if (!h->ctx) {
    throw_type(env, "the context was destroyed");
    return nullptr;
  }
  if (h->busy) {
    napi_throw_error(env, "MB_ERR_BUSY",
                     "the context is running an asynchronous call: await it before the next call");
    return nullptr;
  }
  return h;
}

mb_ctx* get_ctx(napi_env env, napi_value v) {
  Handle* h = get_handle(env, v);
  return h ? h->ctx : nullptr;
}

// A typed array of the expected element type with at least `need` elements
// (need < 0: any length); `allow_null` accepts null/undefined (-> nullptr).
template <typename T>
bool get_array(napi_env env, napi_value v, napi_typedarray_type want, int64_t need, T** out,
               int64_t* len, const char* what, bool allow_null = false) {
  napi_valuetype vt;
  napi_typeof(env, v, &vt);
  if (allow_null && (vt == napi_null || vt == napi_undefined)) {
    *out = nullptr;
    if (len) *len = 0;
    return true;
  }
  bool is_ta = false;
  napi_is_typedarray(env, v, &is_ta);
  napi_typedarray_type type;
  size_t n = 0, off = 0;
  void* data = nullptr;
  napi_value ab;
  if (!is_ta || napi_get_typedarray_info(env, v, &type, &n, &data, &ab, &off) != napi_ok ||
      type != want) {
    const char* tn = want == napi_float32_array ? "a Float32Array" : "an Int32Array";
    throw_type(env, std::string(what) + " must be " + tn);
    return false;
  }
  if (need >= 0 && (int64_t)n < need) {
    throw_range(env, std::string(what) + " holds " + std::to_string(n) + " elements, needs " +
                         std::to_string(need));
    return false;
  }
  *out = (T*)data;
  if (len) *len = (int64_t)n;
  return true;
}

// A zeroed typed array of n 4-byte elements, or nullptr with a RangeError
// thrown when it cannot be allocated.
napi_value new_typed(napi_env env, int64_t n, napi_typedarray_type type, void** data) {
  napi_value ab, ta;
  void* p = nullptr;
  *data = nullptr;
  if (n < 0 || n > ((int64_t)1 << 32) ||
      napi_create_arraybuffer(env, (size_t)n * 4, &p, &ab) != napi_ok || (n && !p)) {
    throw_range(env, "cannot allocate an output array of " + std::to_string(n) + " elements");
    return nullptr;
  }
  if (n) std::memset(p, 0, (size_t)n * 4);
  if (napi_create_typedarray(env, type, (size_t)n, ab, 0, &ta) != napi_ok) {
    throw_range(env, "cannot create an output array of " + std::to_string(n) + " elements");
    return nullptr;
  }
  *data = p;
  return ta;
}

napi_value new_f32(napi_env env, int64_t n, float** data) {
  void* p;
  napi_value ta = new_typed(env, n, napi_float32_array, &p);
  *data = (float*)p;
  return ta;
}

napi_value new_i32(napi_env env, int64_t n, int32_t** data) {
  void* p;
  napi_value ta = new_typed(env, n, napi_int32_array, &p);
  *data = (int32_t*)p;
  return ta;
}

napi_value num(napi_env env, double x) {
  napi_value v;
  napi_create_double(env, x, &v);
  return v;
}

napi_value undef(napi_env env) {
  napi_value v;
  napi_get_undefined(env, &v);
  return v;
}

bool read_config_field(napi_env env, napi_value obj, const char* key, int32_t* out) {
  bool has = false;
  napi_has_named_property(env, obj, key, &has);
  if (!has) return true;  // keep the default
  napi_value v;
  napi_get_named_property(env, obj, key, &v);
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t == napi_undefined) return true;
  if (t == napi_boolean) {
    bool b;
    napi_get_value_bool(env, v, &b);
    *out = b ? 1 : 0;
    return true;
  }
  int x;
  if (!get_int(env, v, &x, key)) return false;
  *out = x;
  return true;
}

void finalize_ctx(napi_env, void* data, void*) {
  Handle* h = (Handle*)data;
  if (h->ctx) mb_destroy(h->ctx);
  delete h;
}

// ------------------------------------------------------ asynchronous calls

// One C call run on a libuv worker.  The job holds references to the handle,
// the result and every typed array the call reads or writes, so none of them
// can be collected (or their backing stores freed) before it completes.
struct Job {
  napi_async_work work = nullptr;
  napi_deferred deferred = nullptr;
  Handle* h = nullptr;
  std::vector<napi_ref> refs;
  napi_ref result = nullptr;
  std::function<int(mb_ctx*)> call;
  int rc = 0;
};

void job_execute(napi_env, void* data) {
  Job* j = (Job*)data;
  j->rc = j->call(j->h->ctx);
}

void job_complete(napi_env env, napi_status status, void* data) {
  Job* j = (Job*)data;
  j->h->busy = false;
  if (status != napi_ok) {
    napi_value code, text, err;
    napi_create_string_utf8(env, "MB_ERR_UNKNOWN", NAPI_AUTO_LENGTH, &code);
    napi_create_string_utf8(env, "the asynchronous call did not run", NAPI_AUTO_LENGTH, &text);
    napi_create_error(env, code, text, &err);
    napi_reject_deferred(env, j->deferred, err);
  } else if (j->rc) {
    napi_reject_deferred(env, j->deferred, status_error(env, j->h->ctx, j->rc));
  } else {
    napi_value v;
    napi_get_reference_value(env, j->result, &v);
    napi_resolve_deferred(env, j->deferred, v);
  }
  for (napi_ref r : j->refs) napi_delete_reference(env, r);
  napi_delete_reference(env, j->result);
  napi_delete_async_work(env, j->work);
  delete j;
}

// Run `call` now and return `result` (sync), or queue it on a worker and
// return a Promise of `result` (async).  `keep` lists the typed arrays the
// call touches.
napi_value finish(napi_env env, napi_value handle_value, bool async, napi_value result,
                  std::initializer_list<napi_value> keep, std::function<int(mb_ctx*)> call) {
  Handle* h = get_handle(env, handle_value);
  if (!h) return nullptr;
  if (!async) {
    const int rc = call(h->ctx);
    if (rc) return throw_status(env, h->ctx, rc);
    return result;
  }
  Job* j = new Job;
  j->h = h;
  j->call = std::move(call);
  napi_value promise, name;
  napi_create_promise(env, &j->deferred, &promise);
  napi_create_reference(env, result, 1, &j->result);
  napi_ref r;
  napi_create_reference(env, handle_value, 1, &r);
  j->refs.push_back(r);
  for (napi_value v : keep) {
    napi_valuetype t;
    napi_typeof(env, v, &t);
    if (t != napi_object) continue;  // a null optional array
    napi_create_reference(env, v, 1, &r);
    j->refs.push_back(r);
  }
  napi_create_string_utf8(env, "mockbird_hip", NAPI_AUTO_LENGTH, &name);
  if (napi_create_async_work(env, nullptr, name, job_execute, job_complete, j, &j->work) != napi_ok ||
      napi_queue_async_work(env, j->work) != napi_ok) {
    for (napi_ref x : j->refs) napi_delete_reference(env, x);
    napi_delete_reference(env, j->result);
    if (j->work) napi_delete_async_work(env, j->work);
    delete j;
    napi_throw_error(env, "MB_ERR_UNKNOWN", "cannot queue the asynchronous call");
    return nullptr;
  }
  h->busy = true;
  return promise;
}

// ---------------------------------------------------------------- bindings

napi_value AbiVersion(napi_env env, napi_callback_info) { return num(env, mb_abi_version()); }

// create({nLayers, vocab, capacity, maxSeqs, maxRows, kvDtype, wrap, device}) -> handle
napi_value Create(napi_env env, napi_callback_info info) {
  Args a(env, info);
  mb_config cfg{12, 16384, 1024, 1, 512, MB_KV_F32, 1, 0};
  napi_valuetype t;
  napi_typeof(env, a.at(0), &t);
  if (t != napi_object) return throw_type(env, "create() takes a config object");
  napi_value o = a.at(0);
  if (!read_config_field(env, o, "nLayers", &cfg.n_layers) ||
      !read_config_field(env, o, "vocab", &cfg.vocab) ||
      !read_config_field(env, o, "capacity", &cfg.capacity) ||
      !read_config_field(env, o, "maxSeqs", &cfg.max_seqs) ||
      !read_config_field(env, o, "maxRows", &cfg.max_rows) ||
      !read_config_field(env, o, "kvDtype", &cfg.kv_dtype) ||
      !read_config_field(env, o, "wrap", &cfg.wrap) ||
      !read_config_field(env, o, "device", &cfg.device))
    return nullptr;
  mb_ctx* ctx = nullptr;
  int rc = mb_create(&cfg, &ctx);
  if (rc != MB_OK) {
    napi_throw_error(env, status_name(rc), "mb_create failed (bad configuration or no device)");
    return nullptr;
  }
  Handle* handle = new Handle;
  handle->ctx = ctx;
  napi_value h;
  napi_create_external(env, handle, finalize_ctx, nullptr, &h);
  return h;
}

napi_value Destroy(napi_env env, napi_callback_info info) {
  Args a(env, info);
  void* p = nullptr;
  napi_valuetype t;
  napi_typeof(env, a.at(0), &t);
  if (t != napi_external || napi_get_value_external(env, a.at(0), &p) != napi_ok || !p)
    return throw_type(env, "destroy() takes a context handle");
  Handle* h = (Handle*)p;
  if (h->busy) {
    napi_throw_error(env, "MB_ERR_BUSY", "destroy() while an asynchronous call is in flight");
    return nullptr;
  }
  if (h->ctx) mb_destroy(h->ctx);
  h->ctx = nullptr;
  return undef(env);
}

napi_value DeviceBytes(napi_env env, napi_callback_info info) {
  Args a(env, info);
  mb_ctx* ctx = get_ctx(env, a.at(0));
  if (!ctx) return nullptr;
  return num(env, (double)mb_device_bytes(ctx));
}

// uploadTensor(h, name, Float32Array data, dims: number[])
napi_value UploadTensor(napi_env env, napi_callback_info info) {
  Args a(env, info);
  mb_ctx* ctx = get_ctx(env, a.at(0));
  if (!ctx) return nullptr;
  size_t len = 0;
  if (napi_get_value_string_utf8(env, a.at(1), nullptr, 0, &len) != napi_ok)
    return throw_type(env, "name must be a string");
  std::string name(len, '\0');
  napi_get_value_string_utf8(env, a.at(1), &name[0], len + 1, &len);
  bool is_arr = false;
  napi_is_array(env, a.at(3), &is_arr);
  if (!is_arr) return throw_type(env, "dims must be an array of numbers");
  uint32_t nd = 0;
  napi_get_array_length(env, a.at(3), &nd);
  if (nd < 1 || nd > 4) return throw_range(env, "dims must have 1 to 4 entries");
  std::vector<int64_t> dims(nd);
  int64_t numel = 1;
  for (uint32_t i = 0; i < nd; i++) {
    napi_value e;
    napi_get_element(env, a.at(3), i, &e);
    if (!get_i64(env, e, &dims[i], "dims[i]")) return nullptr;
    if (dims[i] <= 0) return throw_range(env, "dims must be positive");
    // the library's own limit, checked before the product can overflow
    if (dims[i] > ((int64_t)1 << 40) / numel)
      return throw_range(env, "dims describe more than 2^40 elements");
    numel *= dims[i];
  }
  float* data;
  int64_t n;
  if (!get_array(env, a.at(2), napi_float32_array, numel, &data, &n, "data")) return nullptr;
  if (n != numel) return throw_range(env, "data length does not match dims for " + name);
  int rc = mb_upload_tensor(ctx, name.c_str(), data, dims.data(), (int)nd);
  if (rc) return throw_status(env, ctx, rc);
  return undef(env);
}

napi_value Cancel(napi_env env, napi_callback_info info) {
  Args a(env, info);
  mb_ctx* ctx = get_ctx(env, a.at(0));
  if (!ctx) return nullptr;
  bool on = true;
  napi_valuetype t;
  napi_typeof(env, a.at(1), &t);
  if (t == napi_boolean) napi_get_value_bool(env, a.at(1), &on);
  int rc = mb_cancel(ctx, on ? 1 : 0);
  if (rc) return throw_status(env, ctx, rc);
  return undef(env);
}

napi_value SetLocalHead(napi_env env, napi_callback_info info) {
  Args a(env, info);
  mb_ctx* ctx = get_ctx(env, a.at(0));
  if (!ctx) return nullptr;
  int end_id, assistant;
  double penalty;
  if (!get_int(env, a.at(1), &end_id, "audioEndTokenId") ||
      !get_int(env, a.at(2), &assistant, "audioAssistantSlotTokenId") ||
      !get_f64(env, a.at(3), &penalty, "repetitionPenalty"))
    return nullptr;
  int rc = mb_set_local_head(ctx, end_id, assistant, penalty);
  if (rc) return throw_status(env, ctx, rc);
  return undef(env);
}

// A two-way string option: sets *second to whether `v` names the second
// choice; throws (and returns false) unless it names one of the two.
bool get_choice(napi_env env, napi_value v, const char* first, const char* second, bool* is_second,
                const char* what) {
  char buf[8] = {0};
  size_t len = 0;
  const std::string msg = std::string(what) + " must be \"" + first + "\" or \"" + second + "\"";
  if (napi_get_value_string_utf8(env, v, buf, sizeof buf, &len) != napi_ok) {
    napi_throw_type_error(env, nullptr, msg.c_str());
    return false;
  }
  const std::string s(buf, len);
  if (s != first && s != second) {
    napi_throw_range_error(env, nullptr, msg.c_str());
    return false;
  }
  *is_second = s == second;
  return true;
}

// setWeightStorage(h, "f32" | "bf16")
napi_value SetWeightStorage(napi_env env, napi_callback_info info) {
  Args a(env, info);
  mb_ctx* ctx = get_ctx(env, a.at(0));
  if (!ctx) return nullptr;
  bool bf16;
  if (!get_choice(env, a.at(1), "f32", "bf16", &bf16, "weight storage")) return nullptr;
  int rc = mb_set_weight_storage(ctx, bf16 ? MB_W_BF16 : MB_W_F32);
  if (rc) return throw_status(env, ctx, rc);
  return undef(env);
}

// setPenaltyPrecision(h, "f64" | "f32"): the CPU path's doubles or the WGSL
// engine's f32 repetition-penalty arithmetic
napi_value SetPenaltyPrecision(napi_env env, napi_callback_info info) {
  Args a(env, info);
  mb_ctx* ctx = get_ctx(env, a.at(0));
  if (!ctx) return nullptr;
  bool f32;
  if (!get_choice(env, a.at(1), "f64", "f32", &f32, "penalty precision")) return nullptr;
  int rc = mb_set_penalty_precision(ctx, f32 ? MB_PENALTY_F32 : MB_PENALTY_F64);
  if (rc) return throw_status(env, ctx, rc);
  return undef(env);
}

// ringReset(h, Int32Array seqIds | null) / clearSeen(h, Int32Array seqIds | null)
template <int (*F)(mb_ctx*, int, const int32_t*)>
napi_value SeqListCall(napi_env env, napi_callback_info info) {
  Args a(env, info);
  mb_ctx* ctx = get_ctx(env, a.at(0));
  if (!ctx) return nullptr;
  int32_t* ids;
  int64_t n;
  if (!get_array(env, a.at(1), napi_int32_array, -1, &ids, &n, "seqIds", true)) return nullptr;
  int rc = F(ctx, ids ? (int)n : -1, ids);
  if (rc) return throw_status(env, ctx, rc);
  return undef(env);
}

napi_value RingPoison(napi_env env, napi_callback_info info) {
  Args a(env, info);
  mb_ctx* ctx = get_ctx(env, a.at(0));
  if (!ctx) return nullptr;
  int layer, seq, n;
  float sentinel;
  if (!get_int(env, a.at(1), &layer, "layer") || !get_int(env, a.at(2), &seq, "seq") ||
      !get_int(env, a.at(3), &n, "nSlots") || !get_f32(env, a.at(4), &sentinel, "sentinel"))
    return nullptr;
  int rc = mb_ring_poison(ctx, layer, seq, n, sentinel);
  if (rc) return throw_status(env, ctx, rc);
  return undef(env);
}

// readRing(h, layer, seq, slot0, n) -> {key, value, slotPos}
napi_value ReadRing(napi_env env, napi_callback_info info) {
  Args a(env, info);
  mb_ctx* ctx = get_ctx(env, a.at(0));
  if (!ctx) return nullptr;
  int layer, seq, slot0, n;
  if (!get_int(env, a.at(1), &layer, "layer") || !get_int(env, a.at(2), &seq, "seq") ||
      !get_int(env, a.at(3), &slot0, "slot0") || !get_int(env, a.at(4), &n, "n"))
    return nullptr;
  if (n < 0) return throw_range(env, "n must be >= 0");
  float *k, *v;
  int32_t* sp;
  napi_value K = new_f32(env, (int64_t)n * kD, &k), V = new_f32(env, (int64_t)n * kD, &v);
  if (!K || !V) return nullptr;
  napi_value S = new_i32(env, n, &sp);
  if (!S) return nullptr;
  int rc = mb_read_ring(ctx, layer, seq, slot0, n, k, v, sp);
  if (rc) return throw_status(env, ctx, rc);
  napi_value o;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "key", K);
  napi_set_named_property(env, o, "value", V);
  napi_set_named_property(env, o, "slotPos", S);
  return o;
}

// writeRing(h, layer, seq, slot0, n, key[n*768] | null, value[n*768] | null,
// slotPos[n] | null): the inverse of readRing; a null part is left as it is
napi_value WriteRing(napi_env env, napi_callback_info info) {
  Args a(env, info);
  mb_ctx* ctx = get_ctx(env, a.at(0));
  if (!ctx) return nullptr;
  int layer, seq, slot0, n;
  if (!get_int(env, a.at(1), &layer, "layer") || !get_int(env, a.at(2), &seq, "seq") ||
      !get_int(env, a.at(3), &slot0, "slot0") || !get_int(env, a.at(4), &n, "n"))
    return nullptr;
  if (n < 0) return throw_range(env, "n must be >= 0");
  float *k, *v;
  int32_t* sp;
  if (!get_array(env, a.at(5), napi_float32_array, (int64_t)n * kD, &k, nullptr, "key", true) ||
      !get_array(env, a.at(6), napi_float32_array, (int64_t)n * kD, &v, nullptr, "value", true) ||
      !get_array(env, a.at(7), napi_int32_array, n, &sp, nullptr, "slotPos", true))
    return nullptr;
  int rc = mb_write_ring(ctx, layer, seq, slot0, n, k, v, sp);
  if (rc) return throw_status(env, ctx, rc);
  return undef(env);
}

// ringAppend(h, layer, B, qkv Float32Array[B*2304], pos Int32Array[B]) -> q Float32Array[B*768]
napi_value RingAppend(napi_env env, napi_callback_info info) {
  Args a(env, info);
  mb_ctx* ctx = get_ctx(env, a.at(0));
  if (!ctx) return nullptr;
  int layer, B;
  if (!get_int(env, a.at(1), &layer, "layer") || !get_int(env, a.at(2), &B, "B")) return nullptr;
  if (B < 0) return throw_range(env, "B must be >= 0");
  float* qkv;
  int32_t* pos;
  if (!get_array(env, a.at(3), napi_float32_array, (int64_t)B * kQkv, &qkv, nullptr, "qkv") ||
      !get_array(env, a.at(4), napi_int32_array, B, &pos, nullptr, "pos"))
    return nullptr;
  float* q;
  napi_value Q = new_f32(env, (int64_t)B * kD, &q);
  if (!Q) return nullptr;
  int rc = mb_ring_append(ctx, layer, B, qkv, pos, q);
  if (rc) return throw_status(env, ctx, rc);
  return Q;
}

// ringWriteRows(h, layer, B, rowsMax, qkv[B*rowsMax*2304], pos0[B], nRows[B]) -> q[B*rowsMax*768]
napi_value RingWriteRows(napi_env env, napi_callback_info info) {
  Args a(env, info);
  mb_ctx* ctx = get_ctx(env, a.at(0));
  if (!ctx) return nullptr;
  int layer, B, R;
  if (!get_int(env, a.at(1), &layer, "layer") || !get_int(env, a.at(2), &B, "B") ||
      !get_int(env, a.at(3), &R, "rowsMax"))
    return nullptr;
  if (B < 0 || R < 0) return throw_range(env, "B and rowsMax must be >= 0");
  float* qkv;
  int32_t *p0, *nr;
  if (!get_array(env, a.at(4), napi_float32_array, (int64_t)B * R * kQkv, &qkv, nullptr, "qkv") ||
      !get_array(env, a.at(5), napi_int32_array, B, &p0, nullptr, "pos0") ||
      !get_array(env, a.at(6), napi_int32_array, B, &nr, nullptr, "nRows"))
    return nullptr;
  float* q;
  napi_value Q = new_f32(env, (int64_t)B * R * kD, &q);
  if (!Q) return nullptr;
  int rc = mb_ring_write_rows(ctx, layer, B, R, qkv, p0, nr, q);
  if (rc) return throw_status(env, ctx, rc);
  return Q;
}

// decodeAttention(h, layer, B, q[B*768], pos[B]) -> out[B*768]
napi_value DecodeAttention(napi_env env, napi_callback_info info) {
  Args a(env, info);
  mb_ctx* ctx = get_ctx(env, a.at(0));
  if (!ctx) return nullptr;
  int layer, B;
  if (!get_int(env, a.at(1), &layer, "layer") || !get_int(env, a.at(2), &B, "B")) return nullptr;
  if (B < 0) return throw_range(env, "B must be >= 0");
  float* q;
  int32_t* pos;
  if (!get_array(env, a.at(3), napi_float32_array, (int64_t)B * kD, &q, nullptr, "q") ||
      !get_array(env, a.at(4), napi_int32_array, B, &pos, nullptr, "pos"))
    return nullptr;
  float* out;
  napi_value O = new_f32(env, (int64_t)B * kD, &out);
  if (!O) return nullptr;
  int rc = mb_decode_attention(ctx, layer, B, q, pos, out);
  if (rc) return throw_status(env, ctx, rc);
  return O;
}

// prefillAttention(h, layer, B, rowsMax, q[B*rowsMax*768], pos0[B], nRows[B]) -> out
napi_value PrefillAttention(napi_env env, napi_callback_info info) {
  Args a(env, info);
  mb_ctx* ctx = get_ctx(env, a.at(0));
  if (!ctx) return nullptr;
  int layer, B, R;
  if (!get_int(env, a.at(1), &layer, "layer") || !get_int(env, a.at(2), &B, "B") ||
      !get_int(env, a.at(3), &R, "rowsMax"))
    return nullptr;
  if (B < 0 || R < 0) return throw_range(env, "B and rowsMax must be >= 0");
  float* q;
  int32_t *p0, *nr;
  if (!get_array(env, a.at(4), napi_float32_array, (int64_t)B * R * kD, &q, nullptr, "q") ||
      !get_array(env, a.at(5), napi_int32_array, B, &p0, nullptr, "pos0") ||
      !get_array(env, a.at(6), napi_int32_array, B, &nr, nullptr, "nRows"))
    return nullptr;
  float* out;
  napi_value O = new_f32(env, (int64_t)B * R * kD, &out);
  if (!O) return nullptr;
  int rc = mb_prefill_attention(ctx, layer, B, R, q, p0, nr, out);
  if (rc) return throw_status(env, ctx, rc);
  return O;
}

// prefill(h, B, rowsMax, ids Int32Array[B*rowsMax*17], nRows Int32Array[B], layerCount?, allRows?)
//   -> Float32Array: [B*768] last-row hidden, or [B*rowsMax*768] with allRows
//   (prefillAsync: a Promise of the same)
template <bool ASYNC>
napi_value Prefill(napi_env env, napi_callback_info info) {
  Args a(env, info);
  if (!get_ctx(env, a.at(0))) return nullptr;
  int B, R, layer_count = 0;
  if (!get_int(env, a.at(1), &B, "B") || !get_int(env, a.at(2), &R, "rowsMax")) return nullptr;
  if (B < 0 || R < 0) return throw_range(env, "B and rowsMax must be >= 0");
  int32_t *ids, *nr;
  if (!get_array(env, a.at(3), napi_int32_array, (int64_t)B * R * kRow, &ids, nullptr, "ids") ||
      !get_array(env, a.at(4), napi_int32_array, B, &nr, nullptr, "nRows"))
    return nullptr;
  napi_valuetype t;
  napi_typeof(env, a.at(5), &t);
  if (t != napi_undefined && t != napi_null && !get_int(env, a.at(5), &layer_count, "layerCount"))
    return nullptr;
  bool all_rows = false;
  napi_typeof(env, a.at(6), &t);
  if (t == napi_boolean) napi_get_value_bool(env, a.at(6), &all_rows);
  all_rows = all_rows || layer_count > 0;
  float* out;
  napi_value O = new_f32(env, (int64_t)B * (all_rows ? R : 1) * kD, &out);
  if (!O) return nullptr;
  return finish(env, a.at(0), ASYNC, O, {a.at(3), a.at(4)}, [=](mb_ctx* ctx) {
    return all_rows ? mb_prefill_rows(ctx, B, R, ids, nr, layer_count, out)
                    : mb_prefill(ctx, B, R, ids, nr, out);
  });
}

// decodeStep(h, B, rows17 Int32Array[B*17], pos Int32Array[B]) -> hidden Float32Array[B*768]
template <bool ASYNC>
napi_value DecodeStep(napi_env env, napi_callback_info info) {
  Args a(env, info);
  if (!get_ctx(env, a.at(0))) return nullptr;
  int B;
  if (!get_int(env, a.at(1), &B, "B")) return nullptr;
  if (B < 0) return throw_range(env, "B must be >= 0");
  int32_t *rows, *pos;
  if (!get_array(env, a.at(2), napi_int32_array, (int64_t)B * kRow, &rows, nullptr, "rows17") ||
      !get_array(env, a.at(3), napi_int32_array, B, &pos, nullptr, "pos"))
    return nullptr;
  float* out;
  napi_value O = new_f32(env, (int64_t)B * kD, &out);
  if (!O) return nullptr;
  return finish(env, a.at(0), ASYNC, O, {a.at(2), a.at(3)},
                [=](mb_ctx* ctx) { return mb_decode_step(ctx, B, rows, pos, out); });
}

// localFrame(h, B, hidden Float32Array[B*768]) -> {codes Int32Array[B*16], cont Int32Array[B]}
template <bool ASYNC>
napi_value LocalFrame(napi_env env, napi_callback_info info) {
  Args a(env, info);
  if (!get_ctx(env, a.at(0))) return nullptr;
  int B;
  if (!get_int(env, a.at(1), &B, "B")) return nullptr;
  if (B < 0) return throw_range(env, "B must be >= 0");
  float* hidden;
  if (!get_array(env, a.at(2), napi_float32_array, (int64_t)B * kD, &hidden, nullptr, "hidden"))
    return nullptr;
  int32_t *codes, *cont;
  napi_value Cd = new_i32(env, (int64_t)B * kNvq, &codes), Ct = new_i32(env, B, &cont);
  if (!Cd || !Ct) return nullptr;
  napi_value o;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "codes", Cd);
  napi_set_named_property(env, o, "cont", Ct);
  return finish(env, a.at(0), ASYNC, o, {a.at(2)},
                [=](mb_ctx* ctx) { return mb_local_frame(ctx, B, hidden, codes, cont); });
}

// localSteps(h, B, hidden[B*768], maxStep) -> Float32Array[B*768]
napi_value LocalSteps(napi_env env, napi_callback_info info) {
  Args a(env, info);
  mb_ctx* ctx = get_ctx(env, a.at(0));
  if (!ctx) return nullptr;
  int B, max_step;
  if (!get_int(env, a.at(1), &B, "B")) return nullptr;
  if (B < 0) return throw_range(env, "B must be >= 0");
  float* hidden;
  if (!get_array(env, a.at(2), napi_float32_array, (int64_t)B * kD, &hidden, nullptr, "hidden") ||
      !get_int(env, a.at(3), &max_step, "maxStep"))
    return nullptr;
  float* out;
  napi_value O = new_f32(env, (int64_t)B * kD, &out);
  if (!O) return nullptr;
  int rc = mb_local_steps(ctx, B, hidden, max_step, out);
  if (rc) return throw_status(env, ctx, rc);
  return O;
}

// decodeFrames(h, B, nFrames, hidden Float32Array[B*768] (in/out), pos Int32Array[B] (in/out))
//   -> {codes Int32Array[nFrames*B*16], cont Int32Array[nFrames*B]}
template <bool ASYNC>
napi_value DecodeFrames(napi_env env, napi_callback_info info) {
  Args a(env, info);
  if (!get_ctx(env, a.at(0))) return nullptr;
  int B, nf;
  if (!get_int(env, a.at(1), &B, "B") || !get_int(env, a.at(2), &nf, "nFrames")) return nullptr;
  if (B < 0 || nf < 0) return throw_range(env, "B and nFrames must be >= 0");
  float* hidden;
  int32_t* pos;
  if (!get_array(env, a.at(3), napi_float32_array, (int64_t)B * kD, &hidden, nullptr, "hidden") ||
      !get_array(env, a.at(4), napi_int32_array, B, &pos, nullptr, "pos"))
    return nullptr;
  int32_t *codes, *cont;
  napi_value Cd = new_i32(env, (int64_t)nf * B * kNvq, &codes);
  if (!Cd) return nullptr;
  napi_value Ct = new_i32(env, (int64_t)nf * B, &cont);
  if (!Ct) return nullptr;
  napi_value o;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "codes", Cd);
  napi_set_named_property(env, o, "cont", Ct);
  return finish(env, a.at(0), ASYNC, o, {a.at(3), a.at(4)},
                [=](mb_ctx* ctx) { return mb_decode_frames(ctx, B, nf, hidden, pos, codes, cont); });
}

// A 4-element array field of a config object (each entry an integer).
bool read_config_quad(napi_env env, napi_value obj, const char* key, int32_t* out) {
  bool has = false;
  napi_has_named_property(env, obj, key, &has);
  if (!has) return true;  // keep the default
  napi_value v;
  napi_get_named_property(env, obj, key, &v);
  bool is_array = false;
  napi_is_array(env, v, &is_array);
  uint32_t len = 0;
  if (is_array) napi_get_array_length(env, v, &len);
  if (!is_array || len != 4) {
    throw_type(env, std::string(key) + " must be an array of 4 integers");
    return false;
  }
  for (uint32_t i = 0; i < 4; i++) {
    napi_value e;
    napi_get_element(env, v, i, &e);
    int x;
    if (!get_int(env, e, &x, key)) return false;
    out[i] = x;
  }
  return true;
}

// codecInit(h, {maxVoices, kvDtype, layers: [4], context: [4]})
//   (the codec's shape defaults: layers 4/2/2/4, windows 500/1696/2480/3248)
napi_value CodecInit(napi_env env, napi_callback_info info) {
  Args a(env, info);
  mb_ctx* ctx = get_ctx(env, a.at(0));
  if (!ctx) return nullptr;
  mb_codec_config cfg{1, MB_KV_F32, {4, 2, 2, 4}, {500, 1696, 2480, 3248}};
  napi_valuetype t;
  napi_typeof(env, a.at(1), &t);
  if (t != napi_undefined) {
    if (t != napi_object) return throw_type(env, "codecInit() takes a config object");
    napi_value o = a.at(1);
    if (!read_config_field(env, o, "maxVoices", &cfg.max_voices) ||
        !read_config_field(env, o, "kvDtype", &cfg.kv_dtype) ||
        !read_config_quad(env, o, "layers", cfg.layers) ||
        !read_config_quad(env, o, "context", cfg.context))
      return nullptr;
  }
  int rc = mb_codec_init(ctx, &cfg);
  if (rc) return throw_status(env, ctx, rc);
  return undef(env);
}

// codecDecode(h, B, nFrames, codes Int32Array[nFrames*B*16])
//   -> pcm Float32Array[B*2*nFrames*3840] (per voice: left, then right)
template <bool ASYNC>
napi_value CodecDecode(napi_env env, napi_callback_info info) {
  Args a(env, info);
  if (!get_ctx(env, a.at(0))) return nullptr;
  int B, nf;
  if (!get_int(env, a.at(1), &B, "B") || !get_int(env, a.at(2), &nf, "nFrames")) return nullptr;
  if (B < 0 || nf < 0) return throw_range(env, "B and nFrames must be >= 0");
  int32_t* codes;
  if (!get_array(env, a.at(3), napi_int32_array, (int64_t)nf * B * kNvq, &codes, nullptr, "codes"))
    return nullptr;
  float* pcm;
  napi_value P = new_f32(env, (int64_t)B * 2 * nf * 3840, &pcm);
  if (!P) return nullptr;
  return finish(env, a.at(0), ASYNC, P, {a.at(3)},
                [=](mb_ctx* ctx) { return mb_codec_decode(ctx, B, nf, codes, pcm); });
}

napi_value LastError(napi_env env, napi_callback_info info) {
  Args a(env, info);
  mb_ctx* ctx = get_ctx(env, a.at(0));
  if (!ctx) return nullptr;
  napi_value s;
  napi_create_string_utf8(env, mb_last_error(ctx), NAPI_AUTO_LENGTH, &s);
  return s;
}

napi_value Init(napi_env env, napi_value exports) {
  struct Fn {
    const char* name;
    napi_callback cb;
  } fns[] = {
      {"abiVersion", AbiVersion},
      {"create", Create},
      {"destroy", Destroy},
      {"deviceBytes", DeviceBytes},
      {"uploadTensor", UploadTensor},
      {"cancel", Cancel},
      {"setLocalHead", SetLocalHead},
      {"setWeightStorage", SetWeightStorage},
      {"setPenaltyPrecision", SetPenaltyPrecision},
      {"ringReset", SeqListCall<mb_ring_reset>},
      {"clearSeen", SeqListCall<mb_clear_seen>},
      {"ringPoison", RingPoison},
      {"readRing", ReadRing},
      {"writeRing", WriteRing},
      {"ringAppend", RingAppend},
      {"ringWriteRows", RingWriteRows},
      {"decodeAttention", DecodeAttention},
      {"prefillAttention", PrefillAttention},
      {"prefill", Prefill<false>},
      {"prefillAsync", Prefill<true>},
      {"decodeStep", DecodeStep<false>},
      {"decodeStepAsync", DecodeStep<true>},
      {"localFrame", LocalFrame<false>},
      {"localFrameAsync", LocalFrame<true>},
      {"localSteps", LocalSteps},
      {"decodeFrames", DecodeFrames<false>},
      {"decodeFramesAsync", DecodeFrames<true>},
      {"codecInit", CodecInit},
      {"codecReset", SeqListCall<mb_codec_reset>},
      {"codecDecode", CodecDecode<false>},
      {"codecDecodeAsync", CodecDecode<true>},
      {"lastError", LastError},
  };
  for (const Fn& f : fns) {
    napi_value v;
    napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.cb, nullptr, &v);
    napi_set_named_property(env, exports, f.name, v);
  }
  napi_value kv;
  napi_create_object(env, &kv);
  napi_set_named_property(env, kv, "F32", num(env, MB_KV_F32));
  napi_set_named_property(env, kv, "BF16", num(env, MB_KV_BF16));
  napi_set_named_property(env, exports, "KV", kv);
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)
