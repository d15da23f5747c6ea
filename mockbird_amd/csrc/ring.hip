// KV ring kernels for gfx950: RoPE + ring write (append / prefill rows) and
// the split-softmax single-query attention over a wrapping ring.
//
// Ring layout in HBM (per layer, sequence and head, slots contiguous):
//   K[(((layer * max_seqs + seq) * 12 + head) * C + slot) * 64 + dim]
// so one (sequence, head) window is one contiguous run of C * 64 elements and
// a wave streams it with 16-byte loads; the reference's [slot][head*64+dim]
// order (prefill.ts:55-56) is produced only on read-back.
#include <algorithm>

#include "mb_internal.h"
#include "kv_types.h"
#include "rope.h"

namespace mb {

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

// Each thread owns 8 consecutive dims (4 RoPE pairs) of one head of one row:
// 96 threads per row.  It reads q, k, v (2 x 16 B each for fp32 input),
// writes the roped q, the roped K and the raw V into the ring with 16-byte
// stores (bf16: one 16-byte store each), and the head-0 / dims-0 thread
// records the slot's position.  Rows with r >= n_rows[b], negative positions
// or (non-wrapping ring) pos >= C are skipped; the host rejects them first.
// With more than C rows in one call only the last C reach the ring.
template <bool IN_BF16, bool KV_BF16, bool Q_BF16, int NH>
__global__ __launch_bounds__(256) void k_ring_write(
    const void* __restrict__ qkv, Rows qkv_rows, const int32_t* __restrict__ pos0,
    const int32_t* __restrict__ n_rows, int rows_max, int B, void* __restrict__ q_out,
    Rows q_rows, void* __restrict__ ring_k, void* __restrict__ ring_v,
    int32_t* __restrict__ slot_pos, int64_t ring_seq_stride, int C, int wrap,
    const float2* __restrict__ rope_tab) {
  constexpr int D = NH * HD;  // width of each of q, k, v in the fused row
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row_id = t / (NH * 8);
  if (row_id >= (int64_t)B * rows_max) return;
  const int part = (int)(t % (NH * 8)), head = part >> 3, d0 = (part & 7) * 8;
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
  v.window = ctx->cfg.capacity;
  v.wrap = ctx->cfg.wrap;
  v.bf16 = ctx->cfg.kv_dtype == MB_KV_BF16;
  return v;
}

int launch_ring_write(mb_ctx* ctx, const RingView& ring, int B, int rows_max, const void* qkv,
                      int qkv_dtype, const Rows& qkv_rows, const int32_t* pos0,
                      const int32_t* n_rows, void* q_out, int q_dtype, const Rows& q_rows) {
  if (ring.heads != H && ring.heads != 4)
    return fail(ctx, MB_ERR_ARG, "rings of %d heads are not built", ring.heads);
  const int64_t threads = (int64_t)B * rows_max * ring.heads * 8;
  const int64_t blocks = (threads + 255) / 256;
  if (blocks > INT32_MAX) return fail(ctx, MB_ERR_ARG, "too many rows in one call");
  if (blocks == 0) return MB_OK;
  const bool in_bf16 = qkv_dtype == MB_DT_BF16, kv_bf16 = ring.bf16, q_bf16 = q_dtype == MB_DT_BF16;
#define MB_RW(A, Bq, Cq)                                                                          \
  do {                                                                                             \
    if (ring.heads == H)                                                                           \
      hipLaunchKernelGGL((k_ring_write<A, Bq, Cq, H>), dim3((unsigned)blocks), dim3(256), 0,       \
                         ctx->stream, qkv, qkv_rows, pos0, n_rows, rows_max, B, q_out, q_rows,     \
                         ring.k, ring.v, ring.sp, ring.seq_stride, ring.C, ring.wrap, ctx->rope_tab); \
    else                                                                                           \
      hipLaunchKernelGGL((k_ring_write<A, Bq, Cq, 4>), dim3((unsigned)blocks), dim3(256), 0,       \
                         ctx->stream, qkv, qkv_rows, pos0, n_rows, rows_max, B, q_out, q_rows,     \
                         ring.k, ring.v, ring.sp, ring.seq_stride, ring.C, ring.wrap, ctx->rope_tab); \
  } while (0)
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

// Block timeline (measurement builds only, -DMB_BLOCK_TIMELINE=1): each
// k_attn_unit block records {start, end} from the 100 MHz s_memrealtime
// counter and the HW_ID / XCC_ID registers of the CU that ran it, one vector
// store per word from lane 0 of wave 0, for the first kTimelineBlocks blocks of
// every launch (the last launch's stamps survive).  The production build
// compiles none of it.
#ifndef MB_BLOCK_TIMELINE
#define MB_BLOCK_TIMELINE 0
#endif
#if MB_BLOCK_TIMELINE
constexpr int kTimelineBlocks = 8192;
__device__ uint64_t g_block_stamps[4 * kTimelineBlocks];
#endif

// 16-byte streaming load (global_load_dwordx4 ... nt): the K/V window is read
// once per launch, and the non-temporal hint lets the caches stream it.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_stream(const char* p) {
  const u32x4_t v = __builtin_nontemporal_load((const u32x4_t*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// VD (4 or 8) consecutive elements of an fp32 or bf16 row starting at `off`.
template <bool IN_BF16, int VD>
__device__ __forceinline__ void load_n(const void* base, int64_t off, float* out) {
  if (VD == 8) {
    load8<IN_BF16>(base, off, out);
  } else if (IN_BF16) {
    const uint2 v = *(const uint2*)((const uint16_t*)base + off);
    out[0] = bf16_lo(v.x); out[1] = bf16_hi(v.x); out[2] = bf16_lo(v.y); out[3] = bf16_hi(v.y);
  } else {
    const float4 v = *(const float4*)((const float*)base + off);
    out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
  }
}

// 16 bytes of a ring row: 8 bf16 (round to nearest even) or 4 fp32 values.
template <bool KV_BF16>
__device__ __forceinline__ uint4 pack16(const float* x) {
  if (KV_BF16)
    return make_uint4(pack_bf16(x[0], x[1]), pack_bf16(x[2], x[3]), pack_bf16(x[4], x[5]),
                      pack_bf16(x[6], x[7]));
  return make_uint4(__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]),
                    __float_as_uint(x[3]));
}

// One block per (query, head): the live window [0, min(cur + 1, C)) of the
// query at position cur = pos0[b] + r is cut into batches of GU = G * U
// slots, and the block's `nw` waves take them in turn (wave w: batches w,
// w + nw, ...), so the block reads its (sequence, head) run front to back as
// one sequential stream.  The waves fold their online-softmax partials
// through LDS and wave 0 writes the normalised row.  A query attends the
// slots whose stored position p satisfies 0 <= cur - p < C
// (kernels-decode.ts:608-611); they all lie inside physical slots
// [0, min(cur + 1, C)).
//
// Why the batches alternate: a read-only kernel over the same windows (64
// sequences, C = 2048, bf16) reached 0.70 of 8 TB/s when each wave streamed
// its own quarter of the window, and 0.77 when the waves alternated 4-load
// batches; at C = 4096 (full windows) 0.64 against 0.78.  A plain sequential
// read of 4 GiB reached 0.87 on the same GPU.  Fewer, longer streams keep
// the HBM row buffers open.
//
// Lane layout: LR = 64 / VD lanes hold one 64-dim row (VD dims each, one
// 16-byte load), so a wave covers G = VD consecutive slots -- 1 KB of one
// (sequence, head) run -- per load instruction; U loads of K and V are issued
// before any is used.  Scores are reduced across the LR lanes with DPP; each
// lane group keeps its own online-softmax state (max, sum, VD accumulators)
// and the G groups merge with cross-row shuffles at the end of the range.
//
// Liveness: each batch's stored positions are loaded with its K and V rows
// (one dword per lane) and turned into one 64-bit ballot mask, so no load
// waits on another and the per-slot test is a bit lookup.
//
// No barrier is skipped: a block whose query row is beyond n_rows returns as
// a whole before the only __syncthreads.
//
// With APPEND the kernel also does the ring append of ROPE_SPLIT_RING
// (kernels-decode.ts:216-241) for its (sequence, head): `q` is then the fused
// q | k | v row (IN_BF16: bf16 elements), q is roped in registers (and stored
// to q_out when given), and the wave whose batches hold slot cur mod C (cur
// in a non-wrapping ring) ropes k, stores K and V there before its loop --
// the head-0 block also records the slot's position -- and feeds the new row
// to the batch that covers the slot from registers, so the attention sees it
// without reading it back.  Rows 1 only.
// The fused fp32 form keeps 3 waves per SIMD (at most 168 VGPRs): with
// fewer, the local head's launches at 256 voices (3072 one-wave blocks) no
// longer fit the chip in one round.  The bf16 forms get 4 from their
// 1024-thread blocks already.
//
// EARLY (launches with few waves per CU, bf16 4-load batches only): each
// batch issues the next batch's K rows and stored positions as soon as its
// own scores are formed, and the next V rows after its P V, so a wave keeps
// a K half-batch in flight under its softmax.  With 12 waves per CU (64
// sequences, C = 2048) that extra depth cost 0.9 %; with 7.5 (32 sequences,
// C = 4096) it gained 2.4 %.
//
// PARTS (few units, the one-to-eight-voice decode step): each of a unit's nwp
// waves is a one-wave block of its own, so a unit's window is read on up to
// nwp CUs instead of one, and each wave stores its online-softmax state --
// acc[64], max, sum -- to out[(unit * nwp + wave) * PART] instead of folding
// through LDS; the next projection merges them as it reads its input
// (k_gemv_k's PIN form).
template <bool KV_BF16, int U, int MAXNW, bool APPEND, bool IN_BF16, bool EARLY = false,
          bool PARTS = false>
__global__ __launch_bounds__(64 * MAXNW, !KV_BF16 && APPEND ? 3 : 1) void k_attn_unit(
    const void* __restrict__ q, Rows q_rows, const int32_t* __restrict__ pos0,
    const int32_t* __restrict__ n_rows, int rows, void* __restrict__ ring_k,
    void* __restrict__ ring_v, int32_t* __restrict__ slot_pos, int64_t ring_seq_stride, int C,
    int wrap, const float2* __restrict__ rope_tab, float* __restrict__ q_out, Rows qo_rows,
    float* __restrict__ out, Rows out_rows, int nwp) {
  constexpr int VD = KV_BF16 ? 8 : 4;
  constexpr int LR = 64 / VD;
  constexpr int G = VD;
  constexpr int GU = G * U;
  static_assert(GU <= 64, "one stored position per lane covers a batch");
  constexpr int ROWB = HD * (KV_BF16 ? 2 : 4);  // bytes of one slot's 64-dim row
  __shared__ float fold[MAXNW][PART];
  const int lane = threadIdx.x & 63;
  const int wave = PARTS ? (int)blockIdx.x % nwp : (int)threadIdx.x >> 6;
  const int nw = PARTS ? nwp : (int)blockDim.x >> 6;
  const int unit = PARTS ? (int)blockIdx.x / nwp : (int)blockIdx.x;
#if MB_BLOCK_TIMELINE
  const uint64_t t_begin = __builtin_amdgcn_s_memrealtime();
#endif
  const int qidx = unit / H, head = unit % H;
  const int b = qidx / rows, r = qidx % rows;
  if (n_rows && r >= n_rows[b]) return;  // uniform per block
  const int g = lane / LR, sub = lane % LR;
  const int64_t cur = (int64_t)pos0[b] + r;
  const int nvalid = cur < 0 ? 0 : (int)(cur + 1 < C ? cur + 1 : C);
  // the block's waves take the window's batches in turn: wave w reads batches
  // w, w + nw, w + 2 nw, ..., so the block streams its (sequence, head) run
  // front to back as one sequential read
  const int s0 = wave * GU, step = nw * GU, s1 = nvalid;

  const int64_t kv_off = (int64_t)b * ring_seq_stride + (int64_t)head * C * HD + sub * VD;
  const char* kbase = (const char*)ring_k + kv_off * (KV_BF16 ? 2 : 4);
  const char* vbase = (const char*)ring_v + kv_off * (KV_BF16 ? 2 : 4);
  const int32_t* sp = slot_pos + (int64_t)b * C;

  // One batch = GU slots [base, base + GU): lane (g, sub) loads the K and V
  // rows of slots base + u * G + g (u < U) as 16-byte pieces, and lane l < GU
  // also loads the stored position of slot base + l, so one ballot gives the
  // whole batch's liveness with no round trip of its own.  Slots past the
  // wave's range read as empty, and their K/V loads are clamped to `base`.
  uint4 kr[U], vr[U];
  int32_t spl = -1;
  // The first batch is issued in two halves from the prologue: its K rows
  // and stored positions before the RoPE rotation waits for q, its V rows
  // after it.  Those loads are unconditional, each slot clamped to the last
  // one of the window (slot 0 for an empty window, which every ring has),
  // so the compiler counts the same loads on every path and its wait for q
  // leaves them in flight (loads retire in issue order).  Lanes past the
  // window are masked in the liveness ballot.
  const int last = s1 > 0 ? s1 - 1 : 0;
  auto issue_k0 = [&]() {
    spl = sp[min(s0 + lane, last)];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int slot = s0 + u * G + g;
      kr[u] = load_stream(kbase + (int64_t)(slot < s1 ? slot : last) * ROWB);
    }
  };
  auto issue_v0 = [&]() {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int slot = s0 + u * G + g;
      vr[u] = load_stream(vbase + (int64_t)(slot < s1 ? slot : last) * ROWB);
    }
  };
  auto issue = [&](int base) {
    spl = (lane < GU && base + lane < s1) ? sp[base + lane] : -1;
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int slot = base + u * G + g;
      const int sl = slot < s1 ? slot : base;
      kr[u] = load_stream(kbase + (int64_t)sl * ROWB);
      vr[u] = load_stream(vbase + (int64_t)sl * ROWB);
    }
  };
  auto issue_kn = [&](int base) {
    spl = (lane < GU && base + lane < s1) ? sp[base + lane] : -1;
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int slot = base + u * G + g;
      kr[u] = load_stream(kbase + (int64_t)(slot < s1 ? slot : base) * ROWB);
    }
  };
  auto issue_vn = [&](int base) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int slot = base + u * G + g;
      vr[u] = load_stream(vbase + (int64_t)(slot < s1 ? slot : base) * ROWB);
    }
  };

  float qv[VD];
  // The appended row: its slot and whether this wave's range holds it.  The
  // owning wave ropes k, stores K and V into the slot before its loop and
  // keeps the two packed rows to feed the batch that covers the slot.
  int slot_new = -1;
  bool owner = false;
  uint4 knew = make_uint4(0, 0, 0, 0), vnew = make_uint4(0, 0, 0, 0);
  if (APPEND) {
    const int64_t roff = row_at(q_rows, b, r) + head * HD + sub * VD;
    float qi[VD], qo[VD], cs[VD / 2], sn[VD / 2];
    load_n<IN_BF16, VD>(q, roff, qi);
    const bool have = cur >= 0 && cur <= INT32_MAX && (wrap || cur < C);
    const int32_t pos = (int32_t)(have ? cur : 0);
    if (have) {
      slot_new = wrap ? (int)(cur % C) : (int)cur;
      owner = slot_new < s1 && (slot_new / GU) % nw == wave;
    }
    // table entries of pos, clamped (a position beyond the table is
    // evaluated after the K rows are issued, as rope_cs does it)
    const int32_t tpos = pos < kRopeTab ? pos : kRopeTab - 1;
#pragma unroll
    for (int j = 0; j < VD / 2; j++) {
      const float2 t = rope_tab[(int64_t)tpos * 32 + (sub * VD >> 1) + j];
      cs[j] = t.x;
      sn[j] = t.y;
    }
    issue_k0();
    if (pos >= kRopeTab) {  // uniform
#pragma unroll
      for (int j = 0; j < VD / 2; j++) rope_cs(rope_tab, pos, (sub * VD >> 1) + j, cs[j], sn[j]);
    }
#pragma unroll
    for (int j = 0; j < VD / 2; j++) rope_pair(qi[2 * j], qi[2 * j + 1], cs[j], sn[j], qo[2 * j], qo[2 * j + 1]);
    if (q_out && wave == 0 && g == 0) {
      float* op = q_out + row_at(qo_rows, b, r) + head * HD + sub * VD;
#pragma unroll
      for (int i = 0; i < VD; i += 4) *(float4*)(op + i) = make_float4(qo[i], qo[i + 1], qo[i + 2], qo[i + 3]);
    }
#pragma unroll
    for (int i = 0; i < VD; i++) qv[i] = qo[i] * 0.125f;
    issue_v0();
    if (owner) {  // wave-uniform
      float ki[VD], vi[VD], ko[VD];
      load_n<IN_BF16, VD>(q, roff + D, ki);
      load_n<IN_BF16, VD>(q, roff + 2 * D, vi);
#pragma unroll
      for (int j = 0; j < VD / 2; j++)
        rope_pair(ki[2 * j], ki[2 * j + 1], cs[j], sn[j], ko[2 * j], ko[2 * j + 1]);
      knew = pack16<KV_BF16>(ko);
      vnew = pack16<KV_BF16>(vi);
      if (g == 0) {
        *(uint4*)((char*)ring_k + (kv_off + (int64_t)slot_new * HD) * (KV_BF16 ? 2 : 4)) = knew;
        *(uint4*)((char*)ring_v + (kv_off + (int64_t)slot_new * HD) * (KV_BF16 ? 2 : 4)) = vnew;
        if (head == 0 && sub == 0) slot_pos[(int64_t)b * C + slot_new] = (int32_t)cur;
      }
    }
  } else {
    const float* qp = (const float*)q + row_at(q_rows, b, r) + head * HD + sub * VD;
    float4 qt[VD / 4];
#pragma unroll
    for (int i = 0; i < VD / 4; i++) qt[i] = *(const float4*)(qp + 4 * i);
    issue_k0();
    issue_v0();
#pragma unroll
    for (int i = 0; i < VD / 4; i++) {
      // 0.125 = 2^-3: pre-scaling q is exact
      qv[4 * i] = qt[i].x * 0.125f; qv[4 * i + 1] = qt[i].y * 0.125f;
      qv[4 * i + 2] = qt[i].z * 0.125f; qv[4 * i + 3] = qt[i].w * 0.125f;
    }
  }

  float m = -INFINITY, l = 0.f, acc[VD];
#pragma unroll
  for (int i = 0; i < VD; i++) acc[i] = 0.f;

  for (int base = s0; base < s1; base += step) {
    const int64_t dlt = cur - (int64_t)spl;
    const uint64_t live = __ballot(lane < GU && base + lane < s1 && spl >= 0 && dlt >= 0 && dlt < C);
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; u++) ok[u] = (live >> (u * G + g)) & 1ull;
    // the new row joins the batch that covers its slot (its loaded copy of
    // the slot may predate the store above)
    if (APPEND && owner && slot_new >= base && slot_new < base + GU) {  // wave-uniform
#pragma unroll
      for (int u = 0; u < U; u++) {
        if (base + u * G + g == slot_new) {
          kr[u] = knew;
          vr[u] = vnew;
          ok[u] = true;
        }
      }
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
    const bool more = base + step < s1;
    if (EARLY && more) issue_kn(base + step);  // this batch's K rows are consumed
    if (mx != -INFINITY) {  // else nothing live yet in this lane group
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
    if (EARLY) {
      if (more) issue_vn(base + step);
    } else if (more) {
      issue(base + step);
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
  if constexpr (PARTS) {
    if (g == 0) {
      float* pp = out + ((int64_t)unit * nwp + wave) * PART;
#pragma unroll
      for (int i = 0; i < VD; i += 4)
        *(float4*)(pp + sub * VD + i) = make_float4(acc[i], acc[i + 1], acc[i + 2], acc[i + 3]);
      if (sub == 0) *(float2*)(pp + 64) = make_float2(m, l);
    }
    return;
  }
  if (g == 0) {
#pragma unroll
    for (int i = 0; i < VD; i++) fold[wave][sub * VD + i] = acc[i];
    if (sub == 0) {
      fold[wave][64] = m;
      fold[wave][65] = l;
    }
  }
  __syncthreads();
  if (wave != 0) return;
  // fold the waves: lane w first holds wave w's (max, sum), then every lane
  // (= dim) sums its dim over the waves
  const float ms = lane < nw ? fold[lane][64] : -INFINITY;
  const float ls = lane < nw ? fold[lane][65] : 0.f;
  float M = ms;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
  const float w = (ms == -INFINITY) ? 0.f : __expf(ms - M);
  float L = ls * w;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) L += __shfl_xor(L, off);
  float o = 0.f;
  for (int s = 0; s < nw; s++) o = fmaf(__shfl(w, s), fold[s][lane], o);
  out[row_at(out_rows, b, r) + head * HD + lane] = L > 0.f ? o / L : 0.f;
#if MB_BLOCK_TIMELINE
  if (lane == 0 && blockIdx.x < kTimelineBlocks) {
    uint32_t hw, xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    const uint64_t t_end = __builtin_amdgcn_s_memrealtime();
    uint64_t* st = g_block_stamps + 4 * blockIdx.x;
    st[0] = t_begin;
    st[1] = t_end;
    st[2] = hw;
    st[3] = xcc;
  }
#endif
}

// Fused append + attention for windows of at most kShortWindow slots in an
// fp32 non-wrapping ring (the local head's 17-slot ring): k_attn_unit's
// one-wave path with each wave its own (query, head) -- four heads per
// 256-thread block, so 256 voices are 768 blocks instead of 3072 one-wave
// blocks -- and no cross-wave fold.  The window fits one batch (GU = 20
// slots: lane group g of 16 lanes holds slots g, g + 4, ..., g + 16), the
// computation per lane group and the group merge are k_attn_unit's, and the
// slots past the window enter as p = 0 terms there, so the outputs are the
// same bits k_attn_unit gives (its 48-slot batch adds only more zero terms).
constexpr int kShortWindow = 20;
template <bool IN_BF16>
__global__ __launch_bounds__(256) void k_attn_short(
    const void* __restrict__ qkv, Rows q_rows, const int32_t* __restrict__ pos0, int nunits,
    float* __restrict__ ring_k, float* __restrict__ ring_v, int32_t* __restrict__ slot_pos,
    int64_t ring_seq_stride, int C, const float2* __restrict__ rope_tab,
    float* __restrict__ q_out, Rows qo_rows, float* __restrict__ out, Rows out_rows,
    int pos_const) {
  constexpr int VD = 4, LR = 16, G = 4, U = kShortWindow / G, GU = G * U;
  constexpr int ROWB = HD * 4;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int unit = blockIdx.x * 4 + wave;
  if (unit >= nunits) return;  // per wave: no barrier below
  const int b = unit / H, head = unit % H;
  const int g = lane / LR, sub = lane % LR;
  // pos_const >= 0: every query sits at that position (the local head's
  // step), known without a load, so the window's loads issue at once
  const int64_t cur = pos_const >= 0 ? (int64_t)pos_const : (int64_t)pos0[b];
  const int nvalid = cur < 0 ? 0 : (int)(cur + 1 < C ? cur + 1 : C);
  const int64_t kv_off = (int64_t)b * ring_seq_stride + (int64_t)head * C * HD + sub * VD;
  const char* kbase = (const char*)(ring_k + kv_off);
  const char* vbase = (const char*)(ring_v + kv_off);
  const int32_t* sp = slot_pos + (int64_t)b * C;

  // Every load is issued up front and unconditionally: the window's K and V
  // rows and stored positions (slots past the window clamped to slot 0, so
  // a short window -- the local head's ring fills one slot per step -- reads
  // no more lines than it holds; they are masked below), the q | k | v row,
  // and the RoPE table entries of the position (clamped; a position beyond
  // the table is evaluated after them, as rope_cs does).  With no branch
  // around a load the compiler waits once, for all of them.
  uint4 kr[U], vr[U];
  const int32_t spl = sp[lane < nvalid ? lane : 0];
#pragma unroll
  for (int u = 0; u < U; u++) {
    const int slot = u * G + g;
    const int sl = slot < nvalid ? slot : 0;
    kr[u] = load_stream(kbase + (int64_t)sl * ROWB);
    vr[u] = load_stream(vbase + (int64_t)sl * ROWB);
  }

  const int64_t roff = row_at(q_rows, b, 0) + head * HD + sub * VD;
  float qi[VD], qo[VD], cs[VD / 2], sn[VD / 2], qv[VD], ki[VD], vi[VD];
  load_n<IN_BF16, VD>(qkv, roff, qi);
  load_n<IN_BF16, VD>(qkv, roff + D, ki);
  load_n<IN_BF16, VD>(qkv, roff + 2 * D, vi);
  const bool have = cur >= 0 && cur < C;
  const int32_t pos = (int32_t)(have ? cur : 0);
  const int slot_new = have ? (int)cur : -1;
  const int32_t tpos = pos < kRopeTab ? pos : kRopeTab - 1;
#pragma unroll
  for (int j = 0; j < VD / 2; j++) {
    const float2 t = rope_tab[(int64_t)tpos * 32 + (sub * VD >> 1) + j];
    cs[j] = t.x;
    sn[j] = t.y;
  }
  if (pos >= kRopeTab) {  // uniform
#pragma unroll
    for (int j = 0; j < VD / 2; j++) rope_cs(rope_tab, pos, (sub * VD >> 1) + j, cs[j], sn[j]);
  }
#pragma unroll
  for (int j = 0; j < VD / 2; j++) rope_pair(qi[2 * j], qi[2 * j + 1], cs[j], sn[j], qo[2 * j], qo[2 * j + 1]);
  if (q_out && g == 0) {
    float* op = q_out + row_at(qo_rows, b, 0) + head * HD + sub * VD;
    *(float4*)op = make_float4(qo[0], qo[1], qo[2], qo[3]);
  }
#pragma unroll
  for (int i = 0; i < VD; i++) qv[i] = qo[i] * 0.125f;
  uint4 knew = make_uint4(0, 0, 0, 0), vnew = make_uint4(0, 0, 0, 0);
  if (slot_new >= 0) {  // wave-uniform
    float ko[VD];
#pragma unroll
    for (int j = 0; j < VD / 2; j++)
      rope_pair(ki[2 * j], ki[2 * j + 1], cs[j], sn[j], ko[2 * j], ko[2 * j + 1]);
    knew = pack16<false>(ko);
    vnew = pack16<false>(vi);
    if (g == 0) {
      *(uint4*)(ring_k + kv_off + (int64_t)slot_new * HD) = knew;
      *(uint4*)(ring_v + kv_off + (int64_t)slot_new * HD) = vnew;
      if (head == 0 && sub == 0) slot_pos[(int64_t)b * C + slot_new] = (int32_t)cur;
    }
  }

  const int64_t dlt = cur - (int64_t)spl;
  const uint64_t live = __ballot(lane < GU && lane < nvalid && spl >= 0 && dlt >= 0 && dlt < C);
  float sc[U], mx = -INFINITY;
#pragma unroll
  for (int u = 0; u < U; u++) {
    bool ok = (live >> (u * G + g)) & 1ull;
    if (u * G + g == slot_new) {  // the new row, from registers
      kr[u] = knew;
      vr[u] = vnew;
      ok = true;
    }
    float kf[VD];
    unpack<false>(kr[u], kf);
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < VD; i++) dot = fmaf(qv[i], kf[i], dot);
    dot = group_sum<LR>(dot);
    sc[u] = ok ? dot : -INFINITY;
    mx = fmaxf(mx, sc[u]);
  }
  float m = -INFINITY, l = 0.f, acc[VD];
#pragma unroll
  for (int i = 0; i < VD; i++) acc[i] = 0.f;
  if (mx != -INFINITY) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const float p = __expf(sc[u] - mx);
      l += p;
      float vf[VD];
      unpack<false>(vr[u], vf);
#pragma unroll
      for (int i = 0; i < VD; i++) acc[i] = fmaf(p, vf[i], acc[i]);
    }
    m = mx;
  }
#pragma unroll
  for (int off = LR; off < 64; off <<= 1) {
    const float mo = __shfl_xor(m, off);
    const float lo = __shfl_xor(l, off);
    float ao[VD];
#pragma unroll
    for (int i = 0; i < VD; i++) ao[i] = __shfl_xor(acc[i], off);
    merge_state<VD>(m, l, acc, mo, lo, ao);
  }
  if (g == 0) {
    float* op = out + row_at(out_rows, b, 0) + head * HD + sub * VD;
    *(float4*)op = l > 0.f ? make_float4(acc[0] / l, acc[1] / l, acc[2] / l, acc[3] / l)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

// Waves per block for a window of up to `max_valid` slots: one wave per
// `per_wave` slots (180 bf16, 256 fp32) up to 4 waves, and beyond that one
// wave per 820 slots, at most MAXNW.  With alternating batches, measured on
// one MI355X with the fused launch (fractions of 8 TB/s, same GPU per row):
//   - 64 sequences, C = 2048, mixed windows, bf16, 4-load batches: 4 waves
//     0.76, 5 waves 0.72, 6 waves 0.65, 3 waves 0.72, 2 waves 0.68, 8 waves
//     0.68; 8-load batches at 4 waves 0.72 (127 VGPRs against 94: fewer
//     waves resident);
//   - 256 voices, C = 1024, windows 215-550, bf16, 8-load batches: 4 waves
//     0.71, 3 waves 0.70, 6 waves 0.64; 4-load batches 0.69-0.70;
//   - 32 sequences, C = 4096, full windows, bf16, 4-load batches: 5 waves
//     0.71, 2 waves 0.46; 8-load batches 0.70 against 0.75 (same GPU);
//   - 64 sequences, C = 2048, fp32, 12-load batches: 4 waves 0.78 (8-load
//     0.77).
// Windows up to this many slots run the bf16 kernel with 8-load batches.
constexpr int kAttnShortWindow = 1024;
static int unit_waves(int64_t max_valid, int per_wave, int maxnw) {
  const int64_t short_rule = std::min<int64_t>(4, (max_valid + per_wave - 1) / per_wave);
  const int64_t long_rule = (max_valid + 819) / 820;
  return (int)std::min<int64_t>(maxnw, std::max(short_rule, long_rule));
}

template <bool APPEND, bool IN_BF16>
static int launch_unit(mb_ctx* ctx, const RingView& ring, int B, int rows, const void* q,
                       const Rows& q_rows, const int32_t* pos0, const int32_t* n_rows,
                       int64_t max_valid, float* q_out, const Rows& qo_rows, float* out,
                       const Rows& out_rows, int pos_const = -1) {
  if (ring.heads != H || ring.window != ring.C)
    return fail(ctx, MB_ERR_ARG, "single-query decode attention runs on the model's 12-head rings");
  const int C = ring.C;
  if (max_valid > C) max_valid = C;
  if (max_valid < 1) max_valid = 1;
  const int64_t nq = (int64_t)B * rows;
  if (nq == 0) return MB_OK;
  if (nq * H > INT32_MAX) return fail(ctx, MB_ERR_ARG, "too many queries in one call");
  if (APPEND && rows == 1 && !ring.bf16 && !ring.wrap && C <= kShortWindow) {
    const int nunits = (int)(nq * H);
    hipLaunchKernelGGL(k_attn_short<IN_BF16>, dim3((unsigned)((nunits + 3) / 4)), dim3(256), 0,
                       ctx->stream, q, q_rows, pos0, nunits, (float*)ring.k, (float*)ring.v,
                       ring.sp, ring.seq_stride, C, ctx->rope_tab, q_out, qo_rows, out, out_rows,
                       pos_const);
    MB_HIP(ctx, hipGetLastError());
    return MB_OK;
  }
  const dim3 grid((unsigned)(nq * H));
  // Few blocks (one or a few voices) leave most of the chip idle, and each
  // wave's batches are a chain of load round trips: there, enough waves to
  // take the whole window in one batch each.
  const bool few = nq * H <= 128;
  auto short_waves = [&](int nw, int gu, int maxnw) {
    return few ? std::max<int>(nw, (int)std::min<int64_t>(maxnw, (max_valid + gu - 1) / gu)) : nw;
  };
  if (ring.bf16) {
    constexpr int MAXNW = 16;
    const int64_t cus = ctx->cus_per_xcd > 0 ? (int64_t)ctx->xcds * ctx->cus_per_xcd : 256;
    const int nw = short_waves(unit_waves(max_valid, 180, MAXNW), max_valid <= kAttnShortWindow ? 64 : 32, MAXNW);
    // short windows take 8-load batches, longer ones 4-load batches
    if (max_valid <= kAttnShortWindow)
      hipLaunchKernelGGL((k_attn_unit<true, 8, MAXNW, APPEND, IN_BF16>), grid, dim3(64 * nw), 0,
                         ctx->stream, q, q_rows, pos0, n_rows, rows, ring.k, ring.v, ring.sp,
                         ring.seq_stride, C, ring.wrap, ctx->rope_tab, q_out, qo_rows, out, out_rows, 0);
    else if (nq * H * nw <= 8 * cus)  // at most 8 waves per CU: deeper loads
      hipLaunchKernelGGL((k_attn_unit<true, 4, MAXNW, APPEND, IN_BF16, true>), grid, dim3(64 * nw),
                         0, ctx->stream, q, q_rows, pos0, n_rows, rows, ring.k, ring.v, ring.sp,
                         ring.seq_stride, C, ring.wrap, ctx->rope_tab, q_out, qo_rows, out, out_rows, 0);
    else
      hipLaunchKernelGGL((k_attn_unit<true, 4, MAXNW, APPEND, IN_BF16>), grid, dim3(64 * nw), 0,
                         ctx->stream, q, q_rows, pos0, n_rows, rows, ring.k, ring.v, ring.sp,
                         ring.seq_stride, C, ring.wrap, ctx->rope_tab, q_out, qo_rows, out, out_rows, 0);
  } else {
    constexpr int U = 12, MAXNW = 8;
    const int nw = short_waves(unit_waves(max_valid, 256, MAXNW), 4 * U, MAXNW);
    hipLaunchKernelGGL((k_attn_unit<false, U, MAXNW, APPEND, IN_BF16>), grid, dim3(64 * nw), 0,
                       ctx->stream, q, q_rows, pos0, n_rows, rows, ring.k, ring.v, ring.sp,
                       ring.seq_stride, C, ring.wrap, ctx->rope_tab, q_out, qo_rows, out, out_rows, 0);
  }
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

int launch_attn(mb_ctx* ctx, const RingView& ring, int B, int rows, const float* q,
                const Rows& q_rows, const int32_t* pos0, const int32_t* n_rows, int64_t max_valid,
                float* out, const Rows& out_rows) {
  return launch_unit<false, false>(ctx, ring, B, rows, q, q_rows, pos0, n_rows, max_valid, nullptr,
                                   Rows{}, out, out_rows);
}

// The appended decode step of B <= kPartsMaxSeqs sequences as per-wave
// partials (k_attn_unit's PARTS form): fp32 q | k | v rows, one row each.
// `part` holds B * 12 * nw_out * PART floats; nw_out is at most 16.
int launch_append_attn_parts(mb_ctx* ctx, const RingView& ring, int B, const float* qkv,
                             const int32_t* pos, int64_t max_valid, float* part, int& nw_out) {
  if (ring.heads != H || ring.window != ring.C)
    return fail(ctx, MB_ERR_ARG, "single-query decode attention runs on the model's 12-head rings");
  if (B < 1 || B > kPartsMaxSeqs) return fail(ctx, MB_ERR_ARG, "partials take 1..%d sequences", kPartsMaxSeqs);
  const int C = ring.C;
  if (max_valid > C) max_valid = C;
  if (max_valid < 1) max_valid = 1;
  const int nunits = B * H;
  const Rows qkv_rows = dense_rows(QKV, 1);
  if (ring.bf16) {
    constexpr int U = 8, MAXNW = 16;
    const int nw = (int)std::min<int64_t>(MAXNW, std::max<int64_t>(unit_waves(max_valid, 180, MAXNW),
                                                                  (max_valid + 63) / 64));
    hipLaunchKernelGGL((k_attn_unit<true, U, MAXNW, true, false, false, true>),
                       dim3((unsigned)(nunits * nw)), dim3(64), 0, ctx->stream, qkv, qkv_rows, pos,
                       nullptr, 1, ring.k, ring.v, ring.sp, ring.seq_stride, C, ring.wrap,
                       ctx->rope_tab, nullptr, Rows{}, part, Rows{}, nw);
    nw_out = nw;
  } else {
    constexpr int U = 12, MAXNW = 8;
    const int nw = (int)std::min<int64_t>(MAXNW, std::max<int64_t>(unit_waves(max_valid, 256, MAXNW),
                                                                  (max_valid + 4 * U - 1) / (4 * U)));
    hipLaunchKernelGGL((k_attn_unit<false, U, MAXNW, true, false, false, true>),
                       dim3((unsigned)(nunits * nw)), dim3(64), 0, ctx->stream, qkv, qkv_rows, pos,
                       nullptr, 1, ring.k, ring.v, ring.sp, ring.seq_stride, C, ring.wrap,
                       ctx->rope_tab, nullptr, Rows{}, part, Rows{}, nw);
    nw_out = nw;
  }
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

int launch_append_attn(mb_ctx* ctx, const RingView& ring, int B, const void* qkv, int qkv_dtype,
                       const Rows& qkv_rows, const int32_t* pos, int64_t max_valid, float* q_out,
                       const Rows& qo_rows, float* out, const Rows& out_rows, int pos_const) {
  if (qkv_dtype == MB_DT_BF16)
    return launch_unit<true, true>(ctx, ring, B, 1, qkv, qkv_rows, pos, nullptr, max_valid, q_out,
                                   qo_rows, out, out_rows, pos_const);
  return launch_unit<true, false>(ctx, ring, B, 1, qkv, qkv_rows, pos, nullptr, max_valid, q_out,
                                  qo_rows, out, out_rows, pos_const);
}

}  // namespace mb

#if MB_BLOCK_TIMELINE
// Copies the stamps of the first n blocks ({start, end, HW_ID, XCC_ID} per
// block) of the last decode-attention launch to host memory.  Exported by the
// timeline build only.
extern "C" int mb_probe_block_stamps(uint64_t* host, int n) {
  if (!host || n < 0 || n > mb::kTimelineBlocks) return -1;
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(mb::g_block_stamps), sizeof(uint64_t) * 4 * n,
                                  0, hipMemcpyDeviceToHost);
}
#endif
