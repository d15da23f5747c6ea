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
#include <type_traits>

#include "kv_types.h"
#include "lds_dma.h"
#include "mb_internal.h"
#include "rope.h"

namespace mb {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int KT = 64;    // slots per K/V tile
constexpr int QT = 64;    // query rows per workgroup
constexpr int FPAD = 68;  // fp32 LDS row stride (272 B)

// Workgroup -> (sequence, head, query tile).  Query tile t of a causal
// prefill costs about t + 1 K/V tiles, so the work is numbered latest tile
// first, all (sequence, head) pairs of one tile before the next: every XCD
// gets an equal share of every tile length and the longest start first.
// (With the tile index as the fastest grid coordinate, an 8-tile grid would
// send all of tile t to one XCD.)
//
// The dispatcher deals consecutive workgroups round-robin to the nxcd XCDs
// (workgroup L to XCD L % nxcd, as that XCD's (L / nxcd)-th) and, within an
// XCD, round-robin to its cpx CUs: when a launch fits at once, a CU holds
// the XCD's workgroups c, c + cpx, c + 2 cpx, ...  Handing out the work in
// rounds of cpx, every second full round in reverse (a snake), pairs the
// long tiles with short ones on each CU.  Work item g = nxcd * j + x stays
// on XCD x, so a (sequence, head) pair's tiles share one L2 whenever the
// pair count is a multiple of nxcd.  cpx = 0 hands out the work in order.
// The launcher keeps the workgroup count below 2^31, so the numbering is
// done in 32-bit unsigned arithmetic (a 64-bit division by a run-time value
// is a long scalar and vector sequence, run by every wave before its first
// load).
__device__ __forceinline__ void work_item(int& b, int& h, int& qtile, int nxcd, int cpx) {
  const uint32_t L = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  const uint32_t pairs = gridDim.y * gridDim.z;
  uint32_t g = L;
  if (cpx > 0) {
    const uint32_t total = pairs * gridDim.x, ux = (uint32_t)nxcd, uc = (uint32_t)cpx;
    const uint32_t x = L % ux, i = L / ux, nx = (total - x + ux - 1) / ux;
    const uint32_t r = i / uc, c = i % uc;
    const uint32_t j = ((r & 1) && (r + 1) * uc <= nx) ? r * uc + (uc - 1 - c) : i;
    g = ux * j + x;
  }
  qtile = (int)(gridDim.x - 1 - g / pairs);
  const uint32_t hb = g % pairs;
  h = (int)(hb % gridDim.y);
  b = (int)(hb / gridDim.y);
}

__device__ __forceinline__ bool live_slot(int32_t p, int64_t cur, int C) {
  const int64_t d = cur - p;
  return p >= 0 && d >= 0 && d < C;
}


// ---------------------------------------------------------------- bf16 MMA

// Q bf16 [B][rows_max][768] (roped), K/V bf16 ring, fp32 output.
//
// One workgroup = 128 query rows of one (sequence, head).  With 4 waves
// (the launch's choice) each wave owns 32 of them as two 16-query column
// blocks, so every K or V^T fragment read from LDS feeds two MFMAs; with 8,
// one block of 16.  Both products use v_mfma_f32_16x16x32_bf16:
//  - scores: S^T[16 slots][16 queries] += K[16 slots][32 dims] Q^T[32 dims][16 queries];
//  - P V:    O^T[16 dims][16 queries] += V^T[16 dims][32 slots] P^T[32 slots][16 queries].
// For P V, lane l (g = l/16) must hold P^T for 8 slots of one query; the score
// accumulators give it slots sb*16 + 4g + j (j < 4) of blocks sb = 2c and
// 2c + 1, and the MFMA's k order is free, so those 8 slots are its k range.
//
// K/V tiles of 64 slots reach LDS without passing through registers
// (global_load_lds_dwordx4: lane L of a load lands at the uniform LDS base +
// 16 L), three buffers deep, two tiles ahead of the one being computed.  Rows
// are stored in their natural [slot][dim] order with the 16-byte chunks of
// row s XOR-swizzled by s mod 8, so the 16 rows a fragment read touches
// spread over the banks.  V^T fragments come from the natural layout through
// ds_read_b64_tr_b16: within each 16-lane group, lane r points at 4
// consecutive dims of slot s0 + r/4, and lane i receives dim i of slots
// s0 .. s0 + 3 -- four k values of the A operand; two such reads make one.
//
// Every wave issues the same number of loads per tile (its 1 KB pieces of K
// and V, and the tile's 64 stored positions, which all waves write alike),
// with every lane active -- slots past the causal end are clamped to the last
// one and ignored by the compute -- so `vmcnt` counts tiles exactly.  Per tile
// each wave classifies the slots against its queries with two ballots: all in
// the future of every query (the causal upper triangle: skipped), all live
// for every query (no per-slot test), or mixed (the window rule per slot and
// query, against relative positions the wave reads back from its own LDS row).
//
// Where the time goes (16 sequences x 512 rows, 12 heads, ~16 us): the
// workgroups start over ~1.4 us, every one loads its q rows and first tile
// at once (~1.9 us with HBM near peak), and the longest query tiles then run
// ~10 us of tile loop on SIMDs that issue ~60 % of the time.  A wave's tile
// is a dependent chain (scores -> softmax -> P V); taken out of copies of an
// earlier form of the kernel, neither product's MFMAs cost time, the softmax
// did.  Software-pipelining the next tile's scores under this tile's softmax
// needs ~210 registers (2 waves per SIMD) and was slower, as were 8 waves of
// 16 queries, an order that keeps a sequence's query tiles on one XCD, and
// skipping the all-future half of a diagonal tile (its branches cost more
// than the work saved).
constexpr int BQ = 128;  // query rows per workgroup of the bf16 kernel
constexpr int kFlashWaves = 4;  // waves per workgroup of the bf16 kernel
constexpr int NBUF = 3;  // K/V tile buffers
constexpr float kScoreLog2 = 0.125f * 1.4426950408889634f;  // 1/sqrt(64) * log2(e)
constexpr int32_t kRelEmpty = INT32_MAX;  // relative position of an empty slot

typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4_t;

// Maximum over the four lanes of a column, with plain v_max_f32: fmaxf
// wraps both values that come out of each cross-lane swap in a canonicalising
// max (four more instructions per column); the plain instruction returns the
// same maximum for every input but signalling NaNs, which no score is.
__device__ __forceinline__ float col_max_plain(float x) {
  return col_reduce(x, [](float u, float v) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(u), "v"(v));
    return r;
  });
}

// Element offset of (slot row, 8-dim chunk x) in a swizzled 64 x 64 tile.
__device__ __forceinline__ int swz(int row, int x) { return row * HD + ((x ^ (row & 7)) << 3); }

template <int NW>
__global__ __launch_bounds__(64 * NW, 3 * NW / 4) void k_flash_bf16(
    const uint16_t* __restrict__ q, Rows q_rows, const int32_t* __restrict__ pos0,
    const int32_t* __restrict__ n_rows, const uint16_t* __restrict__ ring_k,
    const uint16_t* __restrict__ ring_v, const int32_t* __restrict__ slot_pos,
    int64_t ring_seq_stride, int C, int W, float* __restrict__ out, Rows out_rows, int nxcd,
    int cpx) {
  constexpr int QB = BQ / (16 * NW);  // 16-query blocks per wave
  constexpr int WQ = 16 * QB;         // queries per wave
  constexpr int PIECES = KT / (8 * NW);  // 1 KB pieces of K (and of V) per wave per tile
  constexpr int LOADS = 2 * PIECES + 1;  // loads per wave per tile
  static_assert(QB >= 1 && PIECES >= 1, "wave count");
  __shared__ __align__(16) uint16_t Ks[NBUF][KT * HD];  // [slot][dim], chunks swizzled
  __shared__ __align__(16) uint16_t Vs[NBUF][KT * HD];  // [slot][dim], chunks swizzled
  __shared__ __align__(16) int32_t Ps[NBUF][KT];         // stored position per slot
  __shared__ __align__(16) int32_t Rl[NW][KT];           // per wave: relative positions
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qcol = lane & 15, grp = lane >> 4;
  int b, h, qtile;
  work_item(b, h, qtile, nxcd, cpx);
  const int n = n_rows[b];
  if (qtile * BQ >= n) return;  // uniform per workgroup, before any barrier
  const int64_t p0 = pos0[b];
  const int rw = qtile * BQ + wave * WQ;  // this wave's first query row
  const bool wave_rows = rw < n;
  const int rlast = min(qtile * BQ + BQ, n) - 1;
  const int64_t kv_end64 = p0 + rlast + 1;
  const int kv_end = kv_end64 < C ? (int)kv_end64 : C;

  // B operands of the score MFMA: Q[row][32*kc + 8*grp + 0..7] times
  // 1/sqrt(64) * log2(e), rounded to bf16 once here, so the MFMA yields the
  // scores in log2 units and the softmax needs no per-score scaling.  (The
  // extra rounding of q is a relative 2^-9 per element; the probabilities
  // are rounded to bf16 for P V anyway.)
  bf16x8_t qb[QB][2];
#pragma unroll
  for (int qi = 0; qi < QB; qi++) {
    const int r = rw + qi * 16 + qcol;
#pragma unroll
    for (int kc = 0; kc < 2; kc++) {
      uint4 raw = make_uint4(0, 0, 0, 0);
      if (r < n) raw = *(const uint4*)(q + row_at(q_rows, b, r) + h * HD + kc * 32 + grp * 8);
      const bf16x8_t v = __builtin_bit_cast(bf16x8_t, raw);
#pragma unroll
      for (int e = 0; e < 8; e++) qb[qi][kc][e] = (__bf16)((float)v[e] * kScoreLog2);
    }
  }
  // Window test in 32 bits.  Stored positions are at most INT32_MAX (the ring
  // write stores no larger one).  Relative to ref = min(p0 + qtile*BQ,
  // INT32_MAX), a slot at p has rel = p - ref (an int32) and the query at row
  // offset c within the workgroup has crel = c + ex, where ex = the part of
  // the first query's position above INT32_MAX (0 in practice; clamped at 2^30,
  // beyond every window).  crel - rel is then the true distance cur - p
  // whenever that is >= 0, exactly, as an unsigned 32-bit number, and a huge
  // one when p is in the future, so the window rule 0 <= cur - p < W is one
  // unsigned compare.  An empty slot (or one past the causal end) has rel =
  // INT32_MAX, which fails it for every query.
  const int64_t first = p0 + (int64_t)qtile * BQ;
  const int32_t ref = first < INT32_MAX ? (int32_t)first : INT32_MAX;
  const int32_t ex = (int32_t)min(first - ref, (int64_t)1 << 30);
  const int crel_lo = wave * WQ + ex, crel_hi = min(rw + WQ - 1, n - 1) - qtile * BQ + ex;
  const int lane_lim = kv_end - lane;  // t0 >= lane_lim: this lane's slot is past the end
  int crel[QB];
#pragma unroll
  for (int qi = 0; qi < QB; qi++) crel[qi] = crel_lo + qi * 16 + qcol;
  const uint16_t* kb = ring_k + (int64_t)b * ring_seq_stride + (int64_t)h * C * HD;
  const uint16_t* vb = ring_v + (int64_t)b * ring_seq_stride + (int64_t)h * C * HD;
  const int32_t* sp = slot_pos + (int64_t)b * C;

  // Tile t0 -> buffer bb: wave w loads its KT / NW rows of K and of V as
  // 1 KB pieces (lane L: row 8 (PIECES w + p) + L/8, LDS chunk L mod 8 =
  // global chunk (L mod 8) ^ (row mod 8)), and the 64 stored positions (every
  // wave writes them alike, so each issues the same count of loads).  A whole
  // tile is read from base + t0 * 64 at fixed per-lane offsets; the last,
  // partial tile clamps each lane's slot to the last one instead.
  int prow[PIECES], pchunk[PIECES];
  uint32_t poff[PIECES];
#pragma unroll
  for (int piece = 0; piece < PIECES; piece++) {
    prow[piece] = 8 * (PIECES * wave + piece) + (lane >> 3);
    pchunk[piece] = (lane & 7) ^ (prow[piece] & 7);
    poff[piece] = (uint32_t)(prow[piece] * HD + pchunk[piece] * 8) * 2u;
  }
  auto issue = [&](int t0, int bb) {
    if (t0 + KT <= kv_end) {  // uniform
#pragma unroll
      for (int piece = 0; piece < PIECES; piece++) {
        const int loff = 8 * (PIECES * wave + piece) * HD;
        dma16(kb + (int64_t)t0 * HD, poff[piece], lds_addr(&Ks[bb][loff]));
        dma16(vb + (int64_t)t0 * HD, poff[piece], lds_addr(&Vs[bb][loff]));
      }
      dma4(sp + t0, (uint32_t)lane * 4u, lds_addr(&Ps[bb][0]));
    } else {
#pragma unroll
      for (int piece = 0; piece < PIECES; piece++) {
        const int loff = 8 * (PIECES * wave + piece) * HD;
        const int slot = min(t0 + prow[piece], kv_end - 1);
        const uint32_t off = (uint32_t)(slot * HD + pchunk[piece] * 8) * 2u;
        dma16(kb, off, lds_addr(&Ks[bb][loff]));
        dma16(vb, off, lds_addr(&Vs[bb][loff]));
      }
      dma4(sp, (uint32_t)min(t0 + lane, kv_end - 1) * 4u, lds_addr(&Ps[bb][0]));
    }
  };

  f32x4_t acc[QB][4], lsum[QB];
  // Per query column: the running maximum m (log2 units) enters as the
  // score MFMA's accumulator input moff = -m (0 while m = -inf), so the
  // products come out as t = score - m, the exponent's argument.  lim is
  // the rescale threshold on t: -inf while m = -inf, then 8.
  f32x4_t moff[QB];
  float lim[QB];
#pragma unroll
  for (int qi = 0; qi < QB; qi++) {
#pragma unroll
    for (int d = 0; d < 4; d++) acc[qi][d] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    lsum[qi] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    moff[qi] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    lim[qi] = -INFINITY;
  }
  bf16x8_t ones;
#pragma unroll
  for (int i = 0; i < 8; i++) ones[i] = (__bf16)1.f;
  // P V: lane r of each 16-lane group points at dims 16d + 4(r mod 4) .. + 3
  // of slot 32c + 4 grp + r/4 (and 16 slots later for the second half),
  // which the transposed read turns into V^T[16d + r][those 4 slots]
  const int trow = grp * 4 + (qcol >> 2), tdim = (qcol & 3) * 4;

  // One tile: wait for its loads, publish it, refill the buffer read two
  // tiles ago, then scores, softmax and P V.  FIRST = the wave's first tile
  // (tile 0), which needs no rescale: acc and the weight sum are still zero.
  auto step = [&](int t0, auto bufc, auto first) {
    constexpr int buf = decltype(bufc)::value;  // a constant: LDS offsets fold into the reads
    constexpr bool FIRST = decltype(first)::value;
    // this tile's loads are done once at most the next tile's are
    // outstanding (vmcnt counts in issue order)
    if (!FIRST) {
      if (t0 + KT < kv_end)
        MB_WAIT_VMCNT(LOADS);
      else
        MB_WAIT_VMCNT(0);
    }
    // every wave's part of this tile is in LDS, and every wave is done with
    // the buffer the next issue overwrites (read two tiles ago)
    __syncthreads();
    if (FIRST && KT < kv_end) issue(KT, 1);  // uniform per workgroup
    if (t0 + 2 * KT < kv_end) issue(t0 + 2 * KT, (buf + NBUF - 1) % NBUF);
    if (!wave_rows) return;
    // The slot positions, then (with registers to spare: two query blocks
    // per wave) the K fragments (A of the score MFMA = K[slot sb*16 +
    // qcol][dims 32 kc + 8 grp ..]), issued before the classification so
    // their LDS latency runs under it; the empty asm keeps the compiler from
    // sinking them below the skip branch.
    const int32_t praw = Ps[buf][lane];
    auto kfrag = [&](int sb, int kc) {
      return *(const bf16x8_t*)&Ks[buf][swz(sb * 16 + qcol, kc * 4 + grp)];
    };
    bf16x8_t ka[4][2];
    if constexpr (QB > 1) {
#pragma unroll
      for (int sb = 0; sb < 4; sb++)
#pragma unroll
        for (int kc = 0; kc < 2; kc++) ka[sb][kc] = kfrag(sb, kc);
      asm volatile("" ::: "memory");
    }
    // Per slot (lane): not after every query of this wave (else it is in
    // the causal upper triangle: a tile of such slots only is skipped), and
    // not live for every one of them (`partial`; rel <= crel_lo <= crel_hi
    // makes the unsigned difference exact).  Only the 16-slot blocks holding
    // a partial slot apply the per-slot window test.
    const int32_t rel_l = praw < 0 || t0 >= lane_lim ? kRelEmpty : praw - ref;
    if (__ballot(rel_l <= crel_hi) == 0) return;
    // (every lane is active here, so the complement of a ballot is the
    // ballot of the complement)
    const uint64_t partial =
        ~(__ballot(rel_l <= crel_lo) & __ballot((uint32_t)crel_hi - (uint32_t)rel_l < (uint32_t)W));

    // S^T blocks: rows = slots sb*16 + grp*4 + j, column = query qi*16 + qcol;
    // t = score - m in log2 units (the accumulator starts at -m)
    f32x4_t s[QB][4];
#pragma unroll
    for (int sb = 0; sb < 4; sb++)
#pragma unroll
      for (int qi = 0; qi < QB; qi++) {
        s[qi][sb] = moff[qi];
#pragma unroll
        for (int kc = 0; kc < 2; kc++)
          s[qi][sb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(QB > 1 ? ka[sb][kc] : kfrag(sb, kc),
                                                              qb[qi][kc], s[qi][sb], 0, 0, 0);
      }
    // The A operand of P V for 32-slot chunk c and dim block d; with
    // registers to spare they are read now, so their LDS latency runs under
    // the softmax.
    auto vfrag = [&](int c, int d) {
      const int dim = d * 16 + tdim;
      const int e0 = swz(c * 32 + trow, dim >> 3) + (dim & 7);
      const int e1 = swz(c * 32 + 16 + trow, dim >> 3) + (dim & 7);
      const bf16x4_t lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t*)&Vs[buf][e0]);
      const bf16x4_t hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t*)&Vs[buf][e1]);
      return bf16x8_t{lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
    };
    bf16x8_t va[2][4];
    if constexpr (QB > 1) {
#pragma unroll
      for (int c = 0; c < 2; c++)
#pragma unroll
        for (int d = 0; d < 4; d++) va[c][d] = vfrag(c, d);
    }
    if (partial) {  // uniform
      // the wave's own row of relative positions: lane l's four score
      // elements of block sb stand for slots sb*16 + 4*grp + j
      Rl[wave][lane] = rel_l;
#pragma unroll
      for (int sb = 0; sb < 4; sb++) {
        if ((partial >> (16 * sb)) & 0xFFFFu) {  // uniform
          const int4 pv = *(const int4*)&Rl[wave][sb * 16 + grp * 4];
          const int32_t pj[4] = {pv.x, pv.y, pv.z, pv.w};
#pragma unroll
          for (int j = 0; j < 4; j++)
#pragma unroll
            for (int qi = 0; qi < QB; qi++)
              if ((uint32_t)(crel[qi] - pj[j]) >= (uint32_t)W) s[qi][sb][j] = -INFINITY;
        }
      }
    }
    // Online softmax in log2 units.  The running maximum m only moves when a
    // tile's maximum exceeds it by more than 8 (the conditional rescaling of
    // FlashAttention-3): the weights 2^t then stay <= 256, and the rescale of
    // the accumulators, a wave-uniform branch taken for all query blocks at
    // once, is rare after the first tiles.  The test needs only each lane's
    // own maximum (a column moves iff one of its four lanes exceeds lim); the
    // column maximum is formed on the rare branch.  The result is the same
    // softmax: acc and the weight sum always share one m.
    float xm[QB];       // this lane's maximum of t
    uint64_t grow = 0;  // lanes whose maximum passes the threshold
#pragma unroll
    for (int qi = 0; qi < QB; qi++) {
      float x = -INFINITY;
#pragma unroll
      for (int sb = 0; sb < 4; sb++)
#pragma unroll
        for (int j = 0; j < 4; j++) x = fmaxf(x, s[qi][sb][j]);
      xm[qi] = x;
      grow |= __ballot(x > lim[qi]);
    }
    if (grow) {  // uniform
#pragma unroll
      for (int qi = 0; qi < QB; qi++) {
        const float xt = col_max_plain(xm[qi]);  // column maximum of t
        if (xt > lim[qi]) {  // uniform per column
          if constexpr (!FIRST) {
            // exp2(m_old - m_new); 0 while m_old = -inf (acc is still zero)
            const float scale = lim[qi] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(-xt);
#pragma unroll
            for (int d = 0; d < 4; d++) acc[qi][d] *= scale;
            lsum[qi] *= scale;
          }
#pragma unroll
          for (int sb = 0; sb < 4; sb++) s[qi][sb] -= xt;
          moff[qi] -= xt;
          lim[qi] = 8.f;
        }
      }
    }
    bf16x8_t pb[QB][2];
#pragma unroll
    for (int qi = 0; qi < QB; qi++)
#pragma unroll
      for (int c = 0; c < 2; c++)
#pragma unroll
        for (int e = 0; e < 8; e++)
          pb[qi][c][e] = (__bf16)__builtin_amdgcn_exp2f(s[qi][2 * c + (e >> 2)][e & 3]);
    // O^T[d-block] += V^T[d-block rows][32 slots of chunk c] P^T[those
    // slots][queries].  The weight sum is one more MFMA with an all-ones A,
    // so it adds the same rounded weights the products use.
#pragma unroll
    for (int c = 0; c < 2; c++) {
#pragma unroll
      for (int d = 0; d < 4; d++) {
        const bf16x8_t a = QB > 1 ? va[c][d] : vfrag(c, d);
#pragma unroll
        for (int qi = 0; qi < QB; qi++)
          acc[qi][d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb[qi][c], acc[qi][d], 0, 0, 0);
      }
#pragma unroll
      for (int qi = 0; qi < QB; qi++)
        lsum[qi] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pb[qi][c], lsum[qi], 0, 0, 0);
    }
  };
  // the first tile and q, then every later tile two tiles ahead of its use
  // (kv_end >= 1: the workgroup has rows)
  using std::integral_constant;
  issue(0, 0);
  MB_WAIT_VMCNT(0);
  step(0, integral_constant<int, 0>{}, std::true_type{});
  for (int t0 = KT; t0 < kv_end; t0 += NBUF * KT) {
    static_assert(NBUF == 3, "the loop is unrolled by the buffer count");
    step(t0, integral_constant<int, 1>{}, std::false_type{});
    if (t0 + KT >= kv_end) break;
    step(t0 + KT, integral_constant<int, 2>{}, std::false_type{});
    if (t0 + 2 * KT >= kv_end) break;
    step(t0 + 2 * KT, integral_constant<int, 0>{}, std::false_type{});
  }
  const int buf = ((kv_end + KT - 1) / KT) % NBUF;  // the buffer a next tile would fill
  // The output goes through LDS so that every store writes whole rows.
  // After the last tile's barrier no wave touches two of the three K/V
  // buffers again (the one before the last tile, and the one the next tile
  // would have filled: no load is in flight), so each wave stages its WQ x
  // 64 fp32 block in a quarter of their 32 KB without waiting for the
  // others, 16-byte chunks of row r XOR-swizzled by r mod 16 (conflict-free
  // both ways), and reads it back 16 lanes per row.  The stores are
  // non-temporal: this kernel never reads the rows again, and rows kept out
  // of the L2 leave nothing to write back when the kernel ends (16
  // sequences x 512 rows: 18.9 us with 64-byte pieces through the L2, 16.9
  // us whole rows non-temporal; non-temporal 64-byte pieces gain as much
  // there but lose 4 us at 64 sequences).
  static_assert(BQ * HD * 4 == 4 * KT * HD * 2 && NW % 4 == 0, "output stage");
  float* stage;
  {
    const int f = (wave / (NW / 4)) >> 1;            // which free buffer
    const int fb = f == 0 ? buf : (buf == NBUF - 1 ? 0 : buf + 1);
    uint16_t* region = (wave / (NW / 4)) & 1 ? &Vs[fb][0] : &Ks[fb][0];
    stage = (float*)region + (wave % (NW / 4)) * WQ * HD;
  }
#pragma unroll
  for (int qi = 0; qi < QB; qi++) {
    const float l = lsum[qi][0];
    const float inv = l > 0.f ? __builtin_amdgcn_rcpf(l) : 0.f;
#pragma unroll
    for (int d = 0; d < 4; d++)
      *(f32x4_t*)&stage[(qi * 16 + qcol) * HD + (((4 * d + grp) ^ qcol) << 2)] = acc[qi][d] * inv;
  }
  // Lane (grp, c = lane mod 16) stores chunk c of rows 4 i + grp.  The
  // swizzle (4 i + grp) mod 16 repeats every 4 rows-of-four, so four LDS
  // offsets serve all WQ / 4 reads.
  const int64_t rs = out_rows.row_stride;
  float* ob = out + row_at(out_rows, b, rw) + h * HD + grp * rs + qcol * 4;
  int soff[4];
#pragma unroll
  for (int i = 0; i < 4; i++) soff[i] = (i * 4 + grp) * HD + ((qcol ^ (i * 4 + grp)) << 2);
  auto row_out = [&](int i) {
    return *(const f32x4_t*)&stage[soff[i & 3] + (i >> 2) * 16 * HD];
  };
  if (rw + WQ <= n) {  // uniform: every row of the wave is a query row
#pragma unroll
    for (int i = 0; i < WQ / 4; i++) __builtin_nontemporal_store(row_out(i), (f32x4_t*)(ob + i * 4 * rs));
  } else {
#pragma unroll
    for (int i = 0; i < WQ / 4; i++)
      if (rw + i * 4 + grp < n) __builtin_nontemporal_store(row_out(i), (f32x4_t*)(ob + i * 4 * rs));
  }
}
#undef MB_WAIT_VMCNT

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
    int64_t ring_seq_stride, int C, int W, float* __restrict__ out, Rows out_rows) {
  __shared__ float Ks[KT * FPAD];  // [slot][dim]
  __shared__ float Vs[KT * FPAD];  // [slot][dim]
  __shared__ int32_t Ps[KT];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qcol = lane & 15, grp = lane >> 4;
  int b, h, qtile;
  work_item(b, h, qtile, 8, 0);
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
        const bool ok = live_slot(Ps[sb * 16 + grp * 4 + j], cur, W);
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

// ------------------------------------------------ short chunks, long windows

// Attention of a short chunk of consecutive queries (up to 16 * QB rows per
// sequence, fp32) against a long window: the codec's stages append 4..32
// positions per frame and attend over windows of 500..3248.  A workgroup is
// one (sequence, head); its NW waves take the slot range's 16-slot groups in
// turn (wave w: groups w, w + NW, ...), so the workgroup reads its
// (sequence, head) run front to back as one stream (against each wave
// streaming a contiguous run: 64 voices 1.214 -> 1.198 ms, 256 voices 2.266
// -> 2.248 ms per codec frame, same GPU, alternating), and each wave computes
// every query of the chunk against its groups, reading K and V straight from
// HBM into MFMA operands (no LDS staging).  A wave's first group is issued
// before the chunk's rows are written when it holds none of their slots
// (else after), and is in flight while its q rows are loaded and split
// (64 voices 1.158 -> 1.150 ms per codec frame, 256 voices level).  Scores
// are S^T[16 slots][16 queries]; the P V output block
// d holds dims 4i + d in row i, so in the step for slot 4g + j (g = lane/16)
// a lane feeds 4 contiguous dims of that V row and its own score element j.
//  - fp32 rings: v_mfma_f32_16x16x4f32; lane l feeds K[slot l%16][16g + kc]
//    and Q[query l%16][16g + kc] in step kc (16 contiguous K dims per lane).
//  - bf16 rings: v_mfma_f32_16x16x32_bf16 for the scores (lane l feeds 8
//    contiguous K dims 32c + 8g.. of its slot) and v_mfma_f32_16x16x16bf16_1k
//    for P V (lane l feeds 4 slots 4g..4g+3 of dim 4(l%16) + d, packed from
//    its four 8-byte V loads).  K and V are exact in bf16; q and P are split
//    into a bf16 high part and a bf16 remainder, two MFMAs each, so the
//    products keep about 16 bits (the scores and weights agree with the fp32
//    path to ~1e-5 relative) at an eighth of the fp32 MFMA time.
// Partials (max, sum, 64 dims per query) fold across the waves through LDS.
// Liveness is the window rule: slot position p (empty slots never live) is
// visible to a query at cur iff 0 <= cur - p < W.
template <bool KV_BF16, int QB, int NW>
__global__ __launch_bounds__(64 * NW) void k_attn_window(
    const float* __restrict__ qkv, Rows qkv_rows, const int32_t* __restrict__ pos0,
    const int32_t* __restrict__ n_rows, void* __restrict__ ring_k, void* __restrict__ ring_v,
    int32_t* __restrict__ slot_pos, int64_t ring_seq_stride, int C, int W, int wrap,
    const float2* __restrict__ rope_tab, float* __restrict__ out, Rows out_rows) {
  constexpr int NQ = 16 * QB;
  __shared__ float red_ml[NW][2][NQ];        // per wave: max (log2 units), sum
  __shared__ float red_acc[NW][NQ][HD + 1];  // per wave: unnormalised output
  __shared__ __align__(16) float q_l[NQ][HD];  // the chunk's roped q rows (this head)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int qc = lane & 15, g = lane >> 4;
  const int h = blockIdx.x, b = blockIdx.y;
  const int n = n_rows[b];
  const int64_t p0 = pos0[b];
  const int64_t end64 = p0 + n;
  const int kv_end = end64 < C ? (int)end64 : C;
  const int groups = (kv_end + 15) >> 4;

  constexpr int E = KV_BF16 ? 2 : 4;
  const char* kb = (const char*)ring_k + ((int64_t)b * ring_seq_stride + (int64_t)h * C * HD) * E;
  const char* vb = (const char*)ring_v + ((int64_t)b * ring_seq_stride + (int64_t)h * C * HD) * E;
  const int32_t* sp = slot_pos + (int64_t)b * C;

  // One 16-slot group's loads, as raw registers: K of the lane's slot
  // s0 + qc, V (4 dims) and the stored positions of slots s0 + 4g + j.  Every
  // index is clamped into the window so the loads carry no branch, and the
  // loop issues group gi + 1's loads before computing group gi: the loads of
  // one group stay in flight under the MFMAs of the one before.
  struct Raw {
    uint4 k[KV_BF16 ? 2 : 4];
    uint4 v[KV_BF16 ? 2 : 4];  // bf16: slots j = 0..3 as 2 x uint2 per uint4
    int32_t p[4];
  };
  auto load_group = [&](int gi, Raw& r) {
    const int s0 = gi * 16;
    const int ks = min(s0 + qc, kv_end - 1);
    if constexpr (KV_BF16) {
#pragma unroll
      for (int c = 0; c < 2; c++) r.k[c] = *(const uint4*)(kb + ((int64_t)ks * HD + c * 32 + g * 8) * 2);
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) r.k[i] = *(const uint4*)(kb + ((int64_t)ks * HD + g * 16 + 4 * i) * 4);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int sl = s0 + 4 * g + j;
      const int vs = min(sl, kv_end - 1);
      if constexpr (KV_BF16) {
        const uint2 w = *(const uint2*)(vb + ((int64_t)vs * HD + 4 * qc) * 2);
        if (j & 1) { r.v[j >> 1].z = w.x; r.v[j >> 1].w = w.y; }
        else { r.v[j >> 1].x = w.x; r.v[j >> 1].y = w.y; }
      } else {
        r.v[j] = *(const uint4*)(vb + ((int64_t)vs * HD + 4 * qc) * 4);
      }
      r.p[j] = sp[vs];
    }
  };

  // The wave's first group is issued before the chunk's rows are written
  // when it holds none of the slots they go to (the slots of rows
  // max(0, n - C) .. n - 1, at p0 + r mod C): the other slots' K, V and
  // positions are not written by this launch, so the loads see what they
  // would see after the barrier.  A group that may hold a written slot loads
  // after the barrier.
  Raw cur, nxt;
  bool early = false;
  if (wave < groups && p0 >= 0) {
    const int lo = wave * 16, hi = min(lo + 16, kv_end);
    const int wr0 = n > C ? n - C : 0;
    const int len = n - wr0;
    bool hit = true;
    if (len <= 0) {
      hit = false;
    } else if (len < C) {
      const int64_t first = p0 + wr0;
      const int start = wrap ? (int)(first % C) : (int)min(first, (int64_t)C);
      const int end = start + len;  // the range [start, end) taken mod C
      hit = end <= C ? (start < hi && lo < end) : (start < hi || lo < end - C);
    }
    early = !hit;
    if (early) load_group(wave, cur);
  }

  // The chunk's rows enter the ring first, as k_ring_write writes them but
  // for this head only: thread (r, d0) ropes q and k of row r's dims d0 ..
  // d0 + 7 at position p0 + r, stores K and V at slot pos mod C (only the
  // last C rows of a call longer than C) and keeps q in LDS; every head's
  // workgroup records the slots' positions (the same values), so each reads
  // only what it wrote itself once the barrier below has passed.
  {
    const int Dw = (int)gridDim.x * HD;  // width of each of q, k, v in a fused row
    for (int t = threadIdx.x; t < NQ * 8; t += 64 * NW) {
      const int r = t >> 3, d0 = (t & 7) * 8;
      const int64_t p64 = p0 + r;
      const bool ok = r < n && p64 >= 0 && p64 <= INT32_MAX && (wrap || p64 < C);
      float qo[8], ko[8], vv[8];
      if (ok) {
        const int32_t pos = (int32_t)p64;
        float qi[8], ki[8];
        const int64_t roff = row_at(qkv_rows, b, r) + h * HD + d0;
        load8<false>(qkv, roff, qi);
        load8<false>(qkv, roff + Dw, ki);
        load8<false>(qkv, roff + 2 * Dw, vv);
#pragma unroll
        for (int j = 0; j < 4; j++) {
          float c, sn;
          rope_cs(rope_tab, pos, (d0 >> 1) + j, c, sn);
          rope_pair(qi[2 * j], qi[2 * j + 1], c, sn, qo[2 * j], qo[2 * j + 1]);
          rope_pair(ki[2 * j], ki[2 * j + 1], c, sn, ko[2 * j], ko[2 * j + 1]);
        }
        if (!(n > C && r < n - C)) {
          const int slot = wrap ? (int)(p64 % C) : (int)p64;
          const int64_t koff = (int64_t)b * ring_seq_stride + ((int64_t)h * C + slot) * HD + d0;
          store8<KV_BF16>(ring_k, koff, ko);
          store8<KV_BF16>(ring_v, koff, vv);
          if (d0 == 0) slot_pos[(int64_t)b * C + slot] = pos;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; e++) qo[e] = 0.f;
      }
      *(float4*)&q_l[r][d0] = make_float4(qo[0], qo[1], qo[2], qo[3]);
      *(float4*)&q_l[r][d0 + 4] = make_float4(qo[4], qo[5], qo[6], qo[7]);
    }
  }
  __threadfence_block();
  __syncthreads();  // the rows are in the ring and q in LDS for every wave

  // the wave's first group is in flight while q is split
  if (wave < groups && !early) load_group(wave, cur);
  // Positions relative to the sequence's first query, clamped so the window
  // test is one unsigned compare; an empty slot and a query past n are
  // outside every window.
  constexpr int32_t kFar = 1 << 30;
  int32_t crel[QB];
  // fp32: dims 16g .. 16g+15; bf16: dims 32c + 8g .. +7 for c = 0, 1
  float qv[QB][16];
#pragma unroll
  for (int qb = 0; qb < QB; qb++) {
    const int r = qb * 16 + qc;
    crel[qb] = r < n ? r : -kFar;
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      const int dim = KV_BF16 ? (i >> 3) * 32 + g * 8 + (i & 7) : g * 16 + i;
      const float4 t = r < n ? *(const float4*)&q_l[r][dim] : make_float4(0.f, 0.f, 0.f, 0.f);
      qv[qb][i] = t.x; qv[qb][i + 1] = t.y; qv[qb][i + 2] = t.z; qv[qb][i + 3] = t.w;
    }
  }
  bf16x8_t qh[QB][2], ql[QB][2];
  if constexpr (KV_BF16) {
#pragma unroll
    for (int qb = 0; qb < QB; qb++)
#pragma unroll
      for (int c = 0; c < 2; c++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const float x = qv[qb][c * 8 + e];
          const __bf16 hi = (__bf16)x;
          qh[qb][c][e] = hi;
          ql[qb][c][e] = (__bf16)(x - (float)hi);
        }
  }
  f32x4_t acc[QB][4];
#pragma unroll
  for (int qb = 0; qb < QB; qb++)
#pragma unroll
    for (int d = 0; d < 4; d++) acc[qb][d] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m[QB], l[QB];
#pragma unroll
  for (int qb = 0; qb < QB; qb++) {
    m[qb] = -INFINITY;
    l[qb] = 0.f;
  }

  for (int gi = wave; gi < groups; gi += NW) {
    load_group(gi + NW < groups ? gi + NW : gi, nxt);  // past the wave's last group: a reload, unused
    const int s0 = gi * 16;
    float kf[16];
    bf16x8_t kh[2];
    float vf[4][4];
    uint2 vw[4];
    if constexpr (KV_BF16) {
#pragma unroll
      for (int c = 0; c < 2; c++) kh[c] = __builtin_bit_cast(bf16x8_t, cur.k[c]);
#pragma unroll
      for (int j = 0; j < 4; j++)
        vw[j] = (j & 1) ? make_uint2(cur.v[j >> 1].z, cur.v[j >> 1].w)
                        : make_uint2(cur.v[j >> 1].x, cur.v[j >> 1].y);
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        kf[4 * i] = __uint_as_float(cur.k[i].x); kf[4 * i + 1] = __uint_as_float(cur.k[i].y);
        kf[4 * i + 2] = __uint_as_float(cur.k[i].z); kf[4 * i + 3] = __uint_as_float(cur.k[i].w);
      }
#pragma unroll
      for (int j = 0; j < 4; j++) {
        vf[j][0] = __uint_as_float(cur.v[j].x); vf[j][1] = __uint_as_float(cur.v[j].y);
        vf[j][2] = __uint_as_float(cur.v[j].z); vf[j][3] = __uint_as_float(cur.v[j].w);
      }
    }
    int32_t pj[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int sl = s0 + 4 * g + j;
      const int32_t p = sl < kv_end ? cur.p[j] : -1;
      const int64_t d = (int64_t)p - p0;
      pj[j] = p < 0 ? kFar : (int32_t)(d < -kFar ? -kFar : d > kFar ? kFar : d);
    }
    // bf16 P V operands: for block d, slots 4g..4g+3 of dim 4qc + d
    i16x4_t va[4];
    if constexpr (KV_BF16) {
#pragma unroll
      for (int d = 0; d < 4; d++) {
        const uint32_t sel = (d & 1) ? 0x07060302u : 0x05040100u;
        const int w = d >> 1;
        const uint32_t lo = __builtin_amdgcn_perm(w ? vw[1].y : vw[1].x, w ? vw[0].y : vw[0].x, sel);
        const uint32_t hi = __builtin_amdgcn_perm(w ? vw[3].y : vw[3].x, w ? vw[2].y : vw[2].x, sel);
        va[d] = __builtin_bit_cast(i16x4_t, make_uint2(lo, hi));
      }
    }
#pragma unroll
    for (int qb = 0; qb < QB; qb++) {
      f32x4_t sc = {0.f, 0.f, 0.f, 0.f};
      if constexpr (KV_BF16) {
#pragma unroll
        for (int c = 0; c < 2; c++) {
          sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh[c], qh[qb][c], sc, 0, 0, 0);
          sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh[c], ql[qb][c], sc, 0, 0, 0);
        }
      } else {
#pragma unroll
        for (int kc = 0; kc < 16; kc++)
          sc = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[kc], qv[qb][kc], sc, 0, 0, 0);
      }
      float t[4];
      float mt = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        t[j] = (unsigned)(crel[qb] - pj[j]) < (unsigned)W ? sc[j] * kScoreLog2 : -INFINITY;
        mt = fmaxf(mt, t[j]);
      }
      mt = col_max(mt);
      // conditional rescale (the running max moves only by more than 8)
      const bool grow = mt > m[qb] + 8.f;
      if (__ballot(grow)) {
        const float mn = grow ? mt : m[qb];
        const float scale = grow ? __builtin_amdgcn_exp2f(m[qb] - mn) : 1.f;
        m[qb] = mn;
        l[qb] *= scale;
#pragma unroll
        for (int d = 0; d < 4; d++) acc[qb][d] *= scale;
      }
      const float mu = m[qb] == -INFINITY ? 0.f : m[qb];
      float pw[4], ls = 0.f;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        pw[j] = __builtin_amdgcn_exp2f(t[j] - mu);
        ls += pw[j];
      }
      l[qb] += col_sum(ls);
      if constexpr (KV_BF16) {
        i16x4_t ph, pl;
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const __bf16 hi = (__bf16)pw[j];
          ph[j] = __builtin_bit_cast(short, hi);
          pl[j] = __builtin_bit_cast(short, (__bf16)(pw[j] - (float)hi));
        }
#pragma unroll
        for (int d = 0; d < 4; d++) {
          acc[qb][d] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va[d], ph, acc[qb][d], 0, 0, 0);
          acc[qb][d] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va[d], pl, acc[qb][d], 0, 0, 0);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
          for (int d = 0; d < 4; d++)
            acc[qb][d] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[j][d], pw[j], acc[qb][d], 0, 0, 0);
      }
    }
    cur = nxt;
  }

  // fold the waves: lane (qc, g) holds dims 4((g*4) + r) + d of query qb*16 + qc
#pragma unroll
  for (int qb = 0; qb < QB; qb++) {
    if (g == 0) {
      red_ml[wave][0][qb * 16 + qc] = m[qb];
      red_ml[wave][1][qb * 16 + qc] = l[qb];
    }
#pragma unroll
    for (int d = 0; d < 4; d++)
#pragma unroll
      for (int r = 0; r < 4; r++) red_acc[wave][qb * 16 + qc][4 * (4 * g + r) + d] = acc[qb][d][r];
  }
  __syncthreads();
  for (int t = threadIdx.x; t < NQ * HD; t += 64 * NW) {
    const int qi = t / HD, dim = t % HD;
    if (qi >= n) continue;
    float M = -INFINITY;
    for (int w = 0; w < NW; w++) M = fmaxf(M, red_ml[w][0][qi]);
    float L = 0.f, o = 0.f;
    if (M != -INFINITY) {
      for (int w = 0; w < NW; w++) {
        const float mw = red_ml[w][0][qi];
        const float wt = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
        L += wt * red_ml[w][1][qi];
        o += wt * red_acc[w][qi][dim];
      }
    }
    out[row_at(out_rows, b, qi) + h * HD + dim] = L > 0.f ? o / L : 0.f;
  }
}

// Chunks of up to 32 consecutive rows per sequence (the codec's stages):
// each row's K/V enters the ring and its query attends the window in one
// launch; rows_max bounds n_rows.
int launch_window_attention(mb_ctx* ctx, const RingView& ring, int B, int rows_max,
                            const float* qkv, const Rows& qkv_rows, const int32_t* pos0,
                            const int32_t* n_rows, float* out, const Rows& out_rows) {
  if (rows_max < 1 || rows_max > 32)
    return fail(ctx, MB_ERR_ARG, "window attention takes 1..32 rows per sequence, not %d", rows_max);
  if (B > 65535) return fail(ctx, MB_ERR_ARG, "at most 65535 sequences per call");
  if (B == 0) return MB_OK;
  constexpr int NW = 8;
  const dim3 grid((unsigned)ring.heads, (unsigned)B);
#define MB_WIN(BF, QB)                                                                            \
  hipLaunchKernelGGL((k_attn_window<BF, QB, NW>), grid, dim3(64 * NW), 0, ctx->stream, qkv,      \
                     qkv_rows, pos0, n_rows, ring.k, ring.v, ring.sp, ring.seq_stride, ring.C,   \
                     ring.window, ring.wrap, ctx->rope_tab, out, out_rows)
  if (ring.bf16) {
    if (rows_max <= 16) MB_WIN(true, 1); else MB_WIN(true, 2);
  } else {
    if (rows_max <= 16) MB_WIN(false, 1); else MB_WIN(false, 2);
  }
#undef MB_WIN
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

int launch_prefill_attention(mb_ctx* ctx, const RingView& ring, int B, int rows_max,
                             const void* q, int q_dtype, const Rows& q_rows, const int32_t* pos0,
                             const int32_t* n_rows, float* out, const Rows& out_rows) {
  if (q_dtype == MB_DT_BF16 && !ring.bf16)
    return fail(ctx, MB_ERR_ARG, "bf16 queries need a bf16 ring (the bf16 MFMA path)");
  if (B > 65535) return fail(ctx, MB_ERR_ARG, "at most 65535 sequences per prefill call");
  if (B == 0 || rows_max == 0) return MB_OK;
  if ((int64_t)((rows_max + QT - 1) / QT) * ring.heads * B >= INT32_MAX)
    return fail(ctx, MB_ERR_ARG, "too many query tiles in one prefill call");
  const unsigned nh = (unsigned)ring.heads;
  dim3 grid((unsigned)((rows_max + QT - 1) / QT), nh, (unsigned)B);
  if (q_dtype == MB_DT_BF16)
    hipLaunchKernelGGL(k_flash_bf16<kFlashWaves>,
                       dim3((unsigned)((rows_max + BQ - 1) / BQ), nh, (unsigned)B),
                       dim3(64 * kFlashWaves), 0, ctx->stream, (const uint16_t*)q, q_rows,
                       pos0, n_rows, (const uint16_t*)ring.k, (const uint16_t*)ring.v, ring.sp,
                       ring.seq_stride, ring.C, ring.window, out, out_rows, ctx->xcds,
                       ctx->cus_per_xcd);
  else if (ring.bf16)
    hipLaunchKernelGGL(k_flash_f32<true>, grid, dim3(256), 0, ctx->stream, (const float*)q, q_rows,
                       pos0, n_rows, ring.k, ring.v, ring.sp, ring.seq_stride, ring.C, ring.window,
                       out, out_rows);
  else
    hipLaunchKernelGGL(k_flash_f32<false>, grid, dim3(256), 0, ctx->stream, (const float*)q,
                       q_rows, pos0, n_rows, ring.k, ring.v, ring.sp, ring.seq_stride, ring.C,
                       ring.window, out, out_rows);
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

}  // namespace mb
