// KV ring kernels for gfx950: RoPE + ring write (append / prefill rows) and
// the split-softmax single-query attention over a wrapping ring.
//
// Ring layout in HBM (per layer, sequence and head, slots contiguous):
//   K[(((layer * max_seqs + seq) * 12 + head) * C + slot) * 64 + dim]
// so one (sequence, head) window is one contiguous run of C * 64 elements and
// a wave streams it with 16-byte loads; the reference's [slot][head*64+dim]
// order (prefill.ts:55-56) is produced only on read-back.
#include "mb_internal.h"
#include "kv_types.h"

namespace mb {

__constant__ uint32_t c_inv_freq_bits[32] = {
    kInvFreqBits[0], kInvFreqBits[1], kInvFreqBits[2], kInvFreqBits[3], kInvFreqBits[4],
    kInvFreqBits[5], kInvFreqBits[6], kInvFreqBits[7], kInvFreqBits[8], kInvFreqBits[9],
    kInvFreqBits[10], kInvFreqBits[11], kInvFreqBits[12], kInvFreqBits[13], kInvFreqBits[14],
    kInvFreqBits[15], kInvFreqBits[16], kInvFreqBits[17], kInvFreqBits[18], kInvFreqBits[19],
    kInvFreqBits[20], kInvFreqBits[21], kInvFreqBits[22], kInvFreqBits[23], kInvFreqBits[24],
    kInvFreqBits[25], kInvFreqBits[26], kInvFreqBits[27], kInvFreqBits[28], kInvFreqBits[29],
    kInvFreqBits[30], kInvFreqBits[31]};

// ------------------------------------------------------------------ fills

__global__ void k_fill_i32(int32_t* __restrict__ p, int64_t n, int32_t value) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = value;
}

template <bool BF16>
__global__ void k_fill_kv(void* __restrict__ p, int64_t n, float value) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    if (BF16)
      ((uint16_t*)p)[i] = f32_to_bf16(value);
    else
      ((float*)p)[i] = value;
  }
}

static int grid_for(int64_t n, int block) {
  int64_t g = (n + block - 1) / block;
  if (g > 65536) g = 65536;
  return (int)(g < 1 ? 1 : g);
}

int launch_fill_i32(mb_ctx* ctx, int32_t* p, int64_t n, int32_t value) {
  if (n <= 0) return MB_OK;
  hipLaunchKernelGGL(k_fill_i32, dim3(grid_for(n, 256)), dim3(256), 0, ctx->stream, p, n, value);
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

int launch_fill_kv(mb_ctx* ctx, void* p, int64_t n, float value) {
  if (n <= 0) return MB_OK;
  if (ctx->cfg.kv_dtype == MB_KV_BF16)
    hipLaunchKernelGGL(k_fill_kv<true>, dim3(grid_for(n, 256)), dim3(256), 0, ctx->stream, p, n,
                       value);
  else
    hipLaunchKernelGGL(k_fill_kv<false>, dim3(grid_for(n, 256)), dim3(256), 0, ctx->stream, p, n,
                       value);
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

// ------------------------------------------------------------ RoPE + write

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

// Each thread owns 8 consecutive dims (4 RoPE pairs) of one head of one row:
// 96 threads per row.  It reads q, k, v (2 x 16 B each for fp32 input),
// writes the roped q, the roped K and the raw V into the ring with 16-byte
// stores (bf16: one 16-byte store each), and the head-0 / dims-0 thread
// records the slot's position.  Rows with r >= n_rows[b], negative positions
// or (non-wrapping ring) pos >= C are skipped; the host rejects them first.
// With more than C rows in one call only the last C reach the ring.
template <bool IN_BF16, bool KV_BF16, bool Q_BF16>
__global__ __launch_bounds__(256) void k_ring_write(
    const void* __restrict__ qkv, Rows qkv_rows, const int32_t* __restrict__ pos0,
    const int32_t* __restrict__ n_rows, int rows_max, int B, void* __restrict__ q_out,
    Rows q_rows, void* __restrict__ ring_k, void* __restrict__ ring_v,
    int32_t* __restrict__ slot_pos, int64_t ring_seq_stride, int C, int wrap,
    const float2* __restrict__ rope_tab) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row_id = t / 96;
  if (row_id >= (int64_t)B * rows_max) return;
  const int part = (int)(t % 96), head = part >> 3, d0 = (part & 7) * 8;
  const int b = (int)(row_id / rows_max), r = (int)(row_id % rows_max);
  const int n = n_rows ? n_rows[b] : 1;
  if (r >= n) return;
  const int64_t p64 = (int64_t)pos0[b] + r;
  if (p64 < 0 || p64 > INT32_MAX || (!wrap && p64 >= C)) return;
  const int32_t pos = (int32_t)p64;
  const int slot = wrap ? (int)(p64 % C) : (int)p64;

  float q[8], k[8], v[8];
  const int64_t roff = row_at(qkv_rows, b, r) + head * HD + d0;
  load8<IN_BF16>(qkv, roff, q);
  load8<IN_BF16>(qkv, roff + D, k);
  load8<IN_BF16>(qkv, roff + 2 * D, v);

  float qo[8], ko[8];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    float c, s;
    rope_cs(rope_tab, pos, (d0 >> 1) + j, c, s);
    rope_pair(q[2 * j], q[2 * j + 1], c, s, qo[2 * j], qo[2 * j + 1]);
    rope_pair(k[2 * j], k[2 * j + 1], c, s, ko[2 * j], ko[2 * j + 1]);
  }
  if (q_out) store8<Q_BF16>(q_out, row_at(q_rows, b, r) + head * HD + d0, qo);
  // a row that a later row of the same call overwrites is never stored, so
  // every slot is written at most once per call (deterministic contents)
  if (n > C && r < n - C) return;
  const int64_t koff = (int64_t)b * ring_seq_stride + ((int64_t)head * C + slot) * HD + d0;
  store8<KV_BF16>(ring_k, koff, ko);
  store8<KV_BF16>(ring_v, koff, v);
  if (part == 0) slot_pos[(int64_t)b * C + slot] = pos;
}

RingView global_ring(const mb_ctx* ctx, int layer) {
  RingView v;
  const size_t e = kv_elem_bytes(ctx);
  v.k = (char*)ctx->ring_k + ring_base(ctx, layer, 0) * e;
  v.v = (char*)ctx->ring_v + ring_base(ctx, layer, 0) * e;
  v.sp = ctx->slot_pos + slot_base(ctx, layer, 0);
  v.seq_stride = (int64_t)H * ctx->cfg.capacity * HD;
  v.C = ctx->cfg.capacity;
  v.wrap = ctx->cfg.wrap;
  v.bf16 = ctx->cfg.kv_dtype == MB_KV_BF16;
  return v;
}

int launch_ring_write(mb_ctx* ctx, const RingView& ring, int B, int rows_max, const void* qkv,
                      int qkv_dtype, const Rows& qkv_rows, const int32_t* pos0,
                      const int32_t* n_rows, void* q_out, int q_dtype, const Rows& q_rows) {
  const int64_t threads = (int64_t)B * rows_max * 96;
  const int64_t blocks = (threads + 255) / 256;
  if (blocks > INT32_MAX) return fail(ctx, MB_ERR_ARG, "too many rows in one call");
  if (blocks == 0) return MB_OK;
  const bool in_bf16 = qkv_dtype == MB_DT_BF16, kv_bf16 = ring.bf16, q_bf16 = q_dtype == MB_DT_BF16;
#define MB_RW(A, Bq, Cq)                                                                        \
  hipLaunchKernelGGL((k_ring_write<A, Bq, Cq>), dim3((unsigned)blocks), dim3(256), 0, ctx->stream, \
                     qkv, qkv_rows, pos0, n_rows, rows_max, B, q_out, q_rows, ring.k, ring.v,     \
                     ring.sp, ring.seq_stride, ring.C, ring.wrap, ctx->rope_tab)
  if (in_bf16) {
    if (kv_bf16) { if (q_bf16) MB_RW(true, true, true); else MB_RW(true, true, false); }
    else { if (q_bf16) MB_RW(true, false, true); else MB_RW(true, false, false); }
  } else {
    if (kv_bf16) { if (q_bf16) MB_RW(false, true, true); else MB_RW(false, true, false); }
    else { if (q_bf16) MB_RW(false, false, true); else MB_RW(false, false, false); }
  }
#undef MB_RW
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

// ------------------------------------------------------- decode attention

// Sum over aligned groups of LR lanes (8 or 16) with DPP row permutes:
// quad swaps (xor 1, xor 2), then the half-row mirror (lane i <-> 7-i) and,
// for 16, the row mirror (lane i <-> 15-i).  Every lane of the group ends
// with the same sum (each step adds two values that are equal across pairs).
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                                              0xF, 0xF, false));
}
template <int LR>
__device__ __forceinline__ float group_sum(float x) {
  x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp<0x141>(x);  // row_half_mirror
  if (LR == 16) x += dpp<0x140>(x);  // row_mirror
  return x;
}

// Merge two online-softmax states (m, l, acc[]) in place.
template <int VD>
__device__ __forceinline__ void merge_state(float& m, float& l, float* acc, float mo, float lo,
                                            const float* acco) {
  const float mn = fmaxf(m, mo);
  if (mn == -INFINITY) return;  // both empty
  const float sa = __expf(m - mn), sb = __expf(mo - mn);
  l = l * sa + lo * sb;
#pragma unroll
  for (int i = 0; i < VD; i++) acc[i] = acc[i] * sa + acco[i] * sb;
  m = mn;
}

// One wave per (query, head, split).  A query is row r of sequence b at
// position cur = pos0[b] + r; it attends the slots of its ring whose stored
// position p satisfies 0 <= cur - p < C (kernels-decode.ts:608-611), which
// are all inside physical slots [0, min(cur + 1, C)).  Split `s` covers
// slots [s * split_len, (s + 1) * split_len) of that range.
//
// Lane layout: LR = 64 / VD lanes hold one 64-dim row (VD dims each, one
// 16-byte load), so a wave covers G = VD consecutive slots -- 1 KB of one
// (sequence, head) run -- per load instruction; U loads of K and V are issued
// before any is used.  Scores are reduced across the LR lanes with DPP; each
// lane group keeps its own online-softmax state (max, sum, VD accumulators)
// and the G groups are merged with cross-row shuffles at the end.
//
// Liveness: for each tile of 256 slots every lane loads the stored positions
// of 4 slots and the wave turns them into four 64-bit ballot masks, so the
// per-slot test in the hot loop is a bit lookup, not a memory access.
//
// With one split the normalised row is written directly; with several each
// wave writes a partial (acc[64], max, sum) for k_attn_combine.
template <bool KV_BF16, int U>
__global__ __launch_bounds__(256) void k_attn_split(
    const float* __restrict__ q, Rows q_rows, const int32_t* __restrict__ pos0,
    const int32_t* __restrict__ n_rows, int rows, const void* __restrict__ ring_k,
    const void* __restrict__ ring_v, const int32_t* __restrict__ slot_pos,
    int64_t ring_seq_stride, int C, int split_len, int nsplit, float* __restrict__ part,
    float* __restrict__ out, Rows out_rows) {
  constexpr int VD = KV_BF16 ? 8 : 4;
  constexpr int LR = 64 / VD;
  constexpr int G = VD;
  constexpr int TILE = 256;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int head = blockIdx.y * 4 + wave;
  const int qidx = blockIdx.x / nsplit, split = blockIdx.x % nsplit;
  const int b = qidx / rows, r = qidx % rows;
  if (n_rows && r >= n_rows[b]) return;  // uniform per wave; no barriers in this kernel
  const int g = lane / LR, sub = lane % LR;
  const int64_t cur = (int64_t)pos0[b] + r;
  const int nvalid = cur < 0 ? 0 : (int)(cur + 1 < C ? cur + 1 : C);
  const int s0 = split * split_len;
  const int s1 = min(s0 + split_len, nvalid);

  float qv[VD];
  {
    const float* qp = q + row_at(q_rows, b, r) + head * HD + sub * VD;
#pragma unroll
    for (int i = 0; i < VD; i += 4) {
      const float4 t = *(const float4*)(qp + i);
      // 0.125 = 2^-3: pre-scaling q is exact
      qv[i] = t.x * 0.125f; qv[i + 1] = t.y * 0.125f; qv[i + 2] = t.z * 0.125f; qv[i + 3] = t.w * 0.125f;
    }
  }
  const char* kbase = (const char*)ring_k +
      ((int64_t)b * ring_seq_stride + (int64_t)head * C * HD + sub * VD) * (KV_BF16 ? 2 : 4);
  const char* vbase = (const char*)ring_v +
      ((int64_t)b * ring_seq_stride + (int64_t)head * C * HD + sub * VD) * (KV_BF16 ? 2 : 4);
  constexpr int ROWB = HD * (KV_BF16 ? 2 : 4);  // bytes of one slot's 64-dim row
  const int32_t* sp = slot_pos + (int64_t)b * C;

  float m = -INFINITY, l = 0.f, acc[VD];
#pragma unroll
  for (int i = 0; i < VD; i++) acc[i] = 0.f;

  for (int t0 = s0; t0 < s1; t0 += TILE) {
    const int t1 = min(t0 + TILE, s1);
    uint64_t live[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const int idx = t0 + 4 * lane + c;
      const int64_t p = idx < t1 ? (int64_t)sp[idx] : -1;
      const int64_t dlt = cur - p;
      live[c] = __ballot(p >= 0 && dlt >= 0 && dlt < C);
    }
    for (int base = t0; base < t1; base += G * U) {
      uint4 kr[U], vr[U];
      bool ok[U];
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int slot = base + u * G + g;
        const int i = slot - t0;
        ok[u] = slot < t1 && ((live[i & 3] >> (i >> 2)) & 1ull);
        const int sl = slot < t1 ? slot : t0;
        kr[u] = *(const uint4*)(kbase + (int64_t)sl * ROWB);
        vr[u] = *(const uint4*)(vbase + (int64_t)sl * ROWB);
      }
      float sc[U];
      float mx = m;
#pragma unroll
      for (int u = 0; u < U; u++) {
        float kf[VD];
        unpack<KV_BF16>(kr[u], kf);
        float dot = 0.f;
#pragma unroll
        for (int i = 0; i < VD; i++) dot = fmaf(qv[i], kf[i], dot);
        dot = group_sum<LR>(dot);
        sc[u] = ok[u] ? dot : -INFINITY;
        mx = fmaxf(mx, sc[u]);
      }
      if (mx == -INFINITY) continue;  // nothing live yet in this lane group
      const float scale = __expf(m - mx);
      l *= scale;
#pragma unroll
      for (int i = 0; i < VD; i++) acc[i] *= scale;
#pragma unroll
      for (int u = 0; u < U; u++) {
        const float p = __expf(sc[u] - mx);
        l += p;
        float vf[VD];
        unpack<KV_BF16>(vr[u], vf);
#pragma unroll
        for (int i = 0; i < VD; i++) acc[i] = fmaf(p, vf[i], acc[i]);
      }
      m = mx;
    }
  }

  // fold the G lane groups: lanes sub, sub+LR, sub+2LR, ... hold the same dims
#pragma unroll
  for (int off = LR; off < 64; off <<= 1) {
    const float mo = __shfl_xor(m, off);
    const float lo = __shfl_xor(l, off);
    float ao[VD];
#pragma unroll
    for (int i = 0; i < VD; i++) ao[i] = __shfl_xor(acc[i], off);
    merge_state<VD>(m, l, acc, mo, lo, ao);
  }
  if (g != 0) return;
  if (nsplit == 1) {
    const float inv = l > 0.f ? 1.f / l : 0.f;
    float* op = out + row_at(out_rows, b, r) + head * HD + sub * VD;
#pragma unroll
    for (int i = 0; i < VD; i += 4)
      *(float4*)(op + i) = make_float4(acc[i] * inv, acc[i + 1] * inv, acc[i + 2] * inv, acc[i + 3] * inv);
  } else {
    float* pp = part + (((int64_t)qidx * H + head) * nsplit + split) * PART;
#pragma unroll
    for (int i = 0; i < VD; i += 4)
      *(float4*)(pp + sub * VD + i) = make_float4(acc[i], acc[i + 1], acc[i + 2], acc[i + 3]);
    if (sub == 0) {
      pp[64] = m;
      pp[65] = l;
    }
  }
}

// Fold the split partials of one (query, head) -- one wave, lane = dim.
// Lane s first holds split s's (max, sum) (nsplit <= 64), the wave forms the
// global max and each split's weight, then every lane sums its dim over the
// splits with independent loads.
__global__ __launch_bounds__(256) void k_attn_combine(
    const float* __restrict__ part, int nsplit, const int32_t* __restrict__ n_rows, int rows,
    int64_t units, float* __restrict__ out, Rows out_rows) {
  const int lane = threadIdx.x & 63;
  const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // (query, head)
  if (unit >= units) return;
  const int qidx = (int)(unit / H), head = (int)(unit % H);
  const int b = qidx / rows, r = qidx % rows;
  if (n_rows && r >= n_rows[b]) return;
  const float* pp = part + unit * nsplit * PART;
  const float ms = lane < nsplit ? pp[lane * PART + 64] : -INFINITY;
  const float ls = lane < nsplit ? pp[lane * PART + 65] : 0.f;
  float M = ms;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
  const float w = (ms == -INFINITY) ? 0.f : __expf(ms - M);
  float L = ls * w;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) L += __shfl_xor(L, off);
  float acc = 0.f;
  for (int s = 0; s < nsplit; s++) acc = fmaf(__shfl(w, s), pp[s * PART + lane], acc);
  out[row_at(out_rows, b, r) + head * HD + lane] = L > 0.f ? acc / L : 0.f;
}

// Launch the split attention for nq = B * rows queries.  The split length is
// chosen so that about `target` waves cover the chip (256 CUs) while each
// split stays a whole number of U-deep load batches and there are at most 64
// splits; MB_ATTN_WAVES and MB_ATTN_U override the defaults (tuning sweeps).
template <bool BF16, int U>
static void launch_split(mb_ctx* ctx, dim3 grid, const float* q, const Rows& q_rows,
                         const int32_t* pos0, const int32_t* n_rows, int rows,
                         const RingView& ring, int split_len, int nsplit, float* part, float* out,
                         const Rows& out_rows) {
  hipLaunchKernelGGL((k_attn_split<BF16, U>), grid, dim3(256), 0, ctx->stream, q, q_rows, pos0,
                     n_rows, rows, ring.k, ring.v, ring.sp, ring.seq_stride, ring.C, split_len,
                     nsplit, part, out, out_rows);
}

static int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return v && *v ? atoi(v) : dflt;
}

int launch_attn(mb_ctx* ctx, const RingView& ring, int B, int rows, const float* q,
                const Rows& q_rows, const int32_t* pos0, const int32_t* n_rows, int64_t max_valid,
                float* out, const Rows& out_rows) {
  static const int64_t target = env_int("MB_ATTN_WAVES", 8192);
  static const int U = env_int("MB_ATTN_U", 16);
  if (U != 4 && U != 8 && U != 16) return fail(ctx, MB_ERR_ARG, "MB_ATTN_U must be 4, 8 or 16");
  const int gu = (ring.bf16 ? 8 : 4) * U;
  const int C = ring.C;
  if (max_valid > C) max_valid = C;
  if (max_valid < 1) max_valid = 1;
  const int64_t nq = (int64_t)B * rows;
  if (nq == 0) return MB_OK;
  const int64_t units = nq * H;
  const int64_t want = (target + units - 1) / units;
  int64_t split_len = (max_valid + want - 1) / want;
  if (split_len < (max_valid + 63) / 64) split_len = (max_valid + 63) / 64;
  split_len = ((split_len + gu - 1) / gu) * gu;
  const int nsplit = (int)((max_valid + split_len - 1) / split_len);
  if (nq * nsplit > INT32_MAX) return fail(ctx, MB_ERR_ARG, "too many queries in one call");
  float* part = nullptr;
  if (nsplit > 1) {
    part = (float*)scratch(ctx, "attn_part", (size_t)units * nsplit * PART * 4);
    if (!part) return fail(ctx, MB_ERR_NOMEM, "attention partials allocation failed");
  }
  dim3 grid((unsigned)(nq * nsplit), H / 4);
#define MB_SPLIT(BF, UU) \
  launch_split<BF, UU>(ctx, grid, q, q_rows, pos0, n_rows, rows, ring, (int)split_len, nsplit, part, out, out_rows)
  if (ring.bf16) {
    if (U == 4) MB_SPLIT(true, 4); else if (U == 8) MB_SPLIT(true, 8); else MB_SPLIT(true, 16);
  } else {
    if (U == 4) MB_SPLIT(false, 4); else if (U == 8) MB_SPLIT(false, 8); else MB_SPLIT(false, 16);
  }
#undef MB_SPLIT
  MB_HIP(ctx, hipGetLastError());
  if (nsplit > 1) {
    hipLaunchKernelGGL(k_attn_combine, dim3((unsigned)((units + 3) / 4)), dim3(256), 0, ctx->stream,
                       part, nsplit, n_rows, rows, units, out, out_rows);
    MB_HIP(ctx, hipGetLastError());
  }
  return MB_OK;
}

}  // namespace mb
