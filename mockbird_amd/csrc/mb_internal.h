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

namespace mb {

struct CodecState;
void codec_free(mb_ctx* ctx);

// The 16 audio-embedding tables (or heads), passed by value to kernels.
struct AudioTables {
  const float* t[NVQ];
};

// Device pointers of one d=768 transformer layer ([K, N] row-major matrices),
// plus the LayerNorm-folded forms of the two projections that follow a
// LayerNorm (W' = diag(gamma) W, c = column sums of W', d = beta W; W'
// column-block-major) and column-block-major copies of the other two, which
// the streaming kernel reads at decode sizes, and k-major copies of all four
// (the folded ones folded), which the GEMV kernel reads at up to kGemvMaxM rows.
// In bf16-KV contexts the four column-block-major forms also have split-bf16
// copies (launch_split_w), which decode-sized projections read there.
struct LayerW {
  const float *ln1_w, *ln1_b, *attn_w, *attn_b, *proj_w, *proj_b;
  const float *ln2_w, *ln2_b, *fc_in_w, *fc_in_b, *fc_out_w, *fc_out_b;
  const float *attn_wg, *attn_c, *attn_d, *fc_in_wg, *fc_in_c, *fc_in_d;
  const float *proj_wt, *fc_out_wt;
  // k-major copies: fp32 with the LayerNorm gamma folded in, or, with bf16
  // weight storage, bf16 and unscaled (the kernels apply gamma to the rows)
  const void *attn_wk, *fc_in_wk, *proj_wk, *fc_out_wk;
  const void *attn_wx, *fc_in_wx, *proj_wx, *fc_out_wx;  // null in fp32-KV contexts
};

// Every weight a model call needs, resolved from the uploaded tensors.
struct ModelW {
  std::vector<LayerW> layers;
  const float *lnf_w, *lnf_b, *wte;
  AudioTables audio_emb;
  LayerW local;
  const float *local_lnf_w, *local_lnf_b, *text_head;
  AudioTables audio_heads;
  // the audio heads with the local ln_f folded in (column-block-major and k-major;
  // split-bf16 in bf16-KV contexts, else null)
  AudioTables head_wg, head_c, head_d;
  const void* head_wk[NVQ];  // as LayerW's k-major copies
  const void* head_wx[NVQ];
};

// Projections with fewer rows than this run with their LayerNorm folded in.
constexpr int kFoldMaxM = 1024;

}  // namespace mb

struct mb_ctx {
  mb_config cfg{};
  int device = 0;
  // XCDs of the device and CUs per XCD (hipDeviceAttributeNumberOfXccs,
  // MultiprocessorCount / that); cus_per_xcd stays 0 when unknown
  int xcds = 8;
  int cus_per_xcd = 0;
  // mb_set_weight_storage: the decoder's projection weights rounded to bf16
  // and read as bf16 by the decode-sized kernels
  bool w_bf16 = false;
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
  mb::ModelW model{};
  bool model_ok = false;       // `model` resolved since the last upload
  int32_t end_id = 7;          // audio_end_token_id
  int32_t assistant_id = 9;    // audio_assistant_slot_token_id
  double penalty = 1.2;        // audio_repetition_penalty (a JS number in the reference)
  bool penalty_f32 = false;    // MB_PENALTY_F32: the penalty applied in f32

  // Local head state: a 17-slot fp32 cache per sequence, the per-channel
  // repetition history, the last frame's codes and continue flags.
  float* local_k = nullptr;
  float* local_v = nullptr;
  int32_t* local_sp = nullptr;
  int32_t* local_pos = nullptr;  // [17][max_seqs], row s filled with s
  uint32_t* seen = nullptr;      // [max_seqs][16][32]
  int32_t* tokens = nullptr;     // [max_seqs][16]
  int32_t* cont = nullptr;       // [max_seqs]
  std::map<std::string, mb::Scratch> scratch;
  // Bumped whenever a buffer a captured graph may point at moves (scratch
  // reallocation, weight upload, first-use local-head state).
  uint64_t graph_gen = 0;
  // The captured frame of mb_decode_frames_dev and what it was captured for.
  hipGraphExec_t frame_exec = nullptr;
  hipStream_t capture_stream = nullptr;
  uint64_t frame_key[8] = {};
  // While mb_decode_frames_dev enqueues a frame: the sequences still alive
  // (a stopped sequence stays stopped); null for the per-call entry points.
  int32_t* frame_alive = nullptr;
  int64_t device_bytes = 0;
  std::atomic<int> cancel{0};
  // The codec decoder's rings, buffers and resolved weights (codec.hip);
  // codec_ok is cleared by every upload.
  mb::CodecState* codec = nullptr;
  bool codec_ok = false;
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

// Makes the context's device current for one entry point and gives the
// caller's current device back when it returns, so a context created for
// device d works from a thread whose current device is another one.
struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int device) {
    int cur = -1;
    if (device >= 0 && hipGetDevice(&cur) == hipSuccess && cur != device &&
        hipSetDevice(device) == hipSuccess)
      prev = cur;
  }
  ~DeviceGuard() {
    if (prev >= 0) (void)hipSetDevice(prev);
  }
  DeviceGuard(const DeviceGuard&) = delete;
  DeviceGuard& operator=(const DeviceGuard&) = delete;
};
#define MB_DEVICE_GUARD(ctx) mb::DeviceGuard mb_device_guard_((ctx) ? (ctx)->device : -1)

// Device scratch named `name` of at least `bytes`, kept between calls.
void* scratch(mb_ctx* ctx, const char* name, size_t bytes);

// The uploaded tensor `name` if its dims are `dims`; otherwise null, and the
// first problem is recorded in `missing` ("weight not uploaded: ...").
const DeviceTensor* find(mb_ctx* ctx, const std::string& name, std::initializer_list<int64_t> dims,
                         std::string& missing);
// A device tensor owned by the context under an internal ('#') name, freed
// with the uploaded weights; reallocated only when its size changes.
float* internal_tensor(mb_ctx* ctx, const std::string& name, int64_t numel);
// Frees the internal tensor `name` (after the context's stream drains), if any.
void drop_internal(mb_ctx* ctx, const std::string& name);

inline size_t kv_elem_bytes(const mb_ctx* ctx) { return ctx->cfg.kv_dtype == MB_KV_BF16 ? 2 : 4; }

// Element offset of (layer, seq, head=0, slot=0, dim=0) in ring_k / ring_v.
inline int64_t ring_base(const mb_ctx* ctx, int layer, int seq) {
  return ((int64_t)layer * ctx->cfg.max_seqs + seq) * H * (int64_t)ctx->cfg.capacity * HD;
}
inline int64_t slot_base(const mb_ctx* ctx, int layer, int seq) {
  return ((int64_t)layer * ctx->cfg.max_seqs + seq) * (int64_t)ctx->cfg.capacity;
}

// A ring as the kernels see it: sequence 0's K/V/slot positions for one
// layer (or for the local head's 17-slot cache).
// C is the slot count (slot = pos mod C); `window` is how far back a query
// sees: slot p is live for a query at cur iff 0 <= cur - p < window.  The
// model's rings use window = C.  The codec's rings add slack slots beyond
// their window so that appending a chunk of positions before attending to
// it never overwrites a position an earlier query of the chunk still sees.
struct RingView {
  void* k = nullptr;
  void* v = nullptr;
  int32_t* sp = nullptr;
  int64_t seq_stride = 0;  // K/V elements between consecutive sequences
  int C = 0;
  int window = 0;
  int heads = H;
  int wrap = 1;
  bool bf16 = false;
};
RingView global_ring(const mb_ctx* ctx, int layer);

// Row addressing of a batched [B][rows] operand: row r of sequence b starts
// at element row_off ? (row_off[b] + r) * row_stride : b * seq_stride + r * row_stride
// (row_off packs ragged sequences back to back).
struct Rows {
  int64_t row_stride = 0;
  int64_t seq_stride = 0;
  const int32_t* row_off = nullptr;
};
inline Rows dense_rows(int64_t row_stride, int rows_max) {
  Rows r;
  r.row_stride = row_stride;
  r.seq_stride = row_stride * rows_max;
  return r;
}
__host__ __device__ inline int64_t row_at(const Rows& R, int b, int r) {
  return R.row_off ? ((int64_t)R.row_off[b] + r) * R.row_stride
                   : (int64_t)b * R.seq_stride + (int64_t)r * R.row_stride;
}

// Kernel launchers (ring.hip, prefill.hip).
int launch_ring_write(mb_ctx* ctx, const RingView& ring, int B, int rows_max, const void* qkv,
                      int qkv_dtype, const Rows& qkv_rows, const int32_t* pos0,
                      const int32_t* n_rows, void* q_out, int q_dtype, const Rows& q_rows);
// Decode steps of at most this many sequences, with bf16 weight storage,
// run their attention as per-wave partials merged by the O projection
// (launch_append_attn_parts, launch_gemv_k_parts).
constexpr int kPartsMaxSeqs = 8;
int launch_append_attn_parts(mb_ctx* ctx, const RingView& ring, int B, const float* qkv,
                             const int32_t* pos, int64_t max_valid, float* part, int& nw_out);
int launch_gemv_k_parts(mb_ctx* ctx, int epi, const float* part, int nwp, const uint16_t* Wk,
                        int N, const float* bias, float* Cm, int64_t ldc, int M);
int launch_attn(mb_ctx* ctx, const RingView& ring, int B, int rows, const float* q,
                const Rows& q_rows, const int32_t* pos0, const int32_t* n_rows, int64_t max_valid,
                float* out, const Rows& out_rows);
// Ring append fused into the decode attention: one row per sequence, qkv
// [B] fused rows at pos[b]; q_out (roped q) may be null.
// pos_const >= 0: every row sits at that position (pos is then not read
// where the kernel can skip it: the short-window fp32 ring of the local head).
int launch_append_attn(mb_ctx* ctx, const RingView& ring, int B, const void* qkv, int qkv_dtype,
                       const Rows& qkv_rows, const int32_t* pos, int64_t max_valid, float* q_out,
                       const Rows& qo_rows, float* out, const Rows& out_rows, int pos_const = -1);
int launch_prefill_attention(mb_ctx* ctx, const RingView& ring, int B, int rows_max,
                             const void* q, int q_dtype, const Rows& q_rows, const int32_t* pos0,
                             const int32_t* n_rows, float* out, const Rows& out_rows);
// Chunks of up to 32 consecutive rows per sequence against long windows
// (the codec's stages), out of the causal windowed rule: qkv holds the fused
// fp32 rows (q | k | v, ring.heads x 64 each); every row is roped and written
// into the ring as launch_ring_write writes it, then its query attends.
int launch_window_attention(mb_ctx* ctx, const RingView& ring, int B, int rows_max,
                            const float* qkv, const Rows& qkv_rows, const int32_t* pos0,
                            const int32_t* n_rows, float* out, const Rows& out_rows);
int launch_fill_i32(mb_ctx* ctx, int32_t* p, int64_t n, int32_t value);
int launch_fill_kv(mb_ctx* ctx, void* p, int64_t n, float value);

// gemm.hip.  EPI_SCALE_ADD (the codec's layer scale) reads the `bias`
// argument as a per-column scale s and stores C + s * (A W); EPI_GELU_ERF
// applies the exact (erf) GELU after the bias.
enum { EPI_STORE = 0, EPI_GELU = 1, EPI_ADD = 2, EPI_SCALE_ADD = 3, EPI_GELU_ERF = 4 };
// W is [K][N] row-major, or with w_tiled the column-block-major copy from
// launch_tile_w ([N / 64][K][64]; only where gemm_streams(M, N), else
// MB_ERR_STATE).
// `part` (optional, part_cap floats) takes the streaming kernel's split-K
// partials in place of the context's growable scratch; a split that needs
// more is MB_ERR_ARG.  M <= kGemvMaxM rows take the GEMV kernel, which needs
// no scratch.
constexpr int kGemvMaxM = 8;
int launch_gemm(mb_ctx* ctx, int epi, const float* A, int64_t lda, const float* W, int N, int K,
                const float* bias, float* Cm, int64_t ldc, int M, bool w_tiled = false,
                float* part = nullptr, size_t part_cap = 0);
// Floats of split-K partials launch_gemm writes for an M x N x K projection
// (0: no split).
size_t gemm_partial_floats(int M, int N, int K);
// noalloc.hip: resolve the static split-K scratch array's address on the
// context's (current) device, once per device.
int noalloc_init(mb_ctx* ctx);
int launch_tile_w(mb_ctx* ctx, const float* W, int K, int N, float* Wt);
// Wk[n][k] = gamma[k] W[k][n] (gamma null: 1), the k-major copy launch_gemv_k
// reads; with gamma it holds the values launch_fold_ln's Wg holds.
int launch_kmajor_w(mb_ctx* ctx, const float* W, int K, int N, const float* gamma, float* Wk);
// C = epi(A Wk^T + bias) for M <= kGemvMaxM rows on a k-major weight copy;
// with lnc (and lnd) the rows are the raw residual stream and the LayerNorm
// is folded in (c, d from launch_fold_ln, Wk from launch_kmajor_w with gamma).
// With `pick` (one row, K = 768, a folded LayerNorm, EPI_STORE) the row is
// not read from A: the launch makes the previous audio channel's greedy
// choice itself and takes that code's embedding row (PickIn, pick.h).
struct PickIn;
int launch_gemv_k(mb_ctx* ctx, int epi, const float* A, int64_t lda, const float* Wk, int N, int K,
                  const float* bias, float* Cm, int64_t ldc, int M, const float* lnc,
                  const float* lnd, const PickIn* pick = nullptr);

// LayerNorm folded into the projection after it: Wg, c, d from
// launch_fold_ln (Wg column-block-major, as launch_tile_w writes it);
// launch_gemm_ln returns MB_ERR_STATE where the streaming
// kernel does not take M x N (gemm_streams false), and the caller then runs
// the LayerNorm and launch_gemm apart.
bool gemm_streams(int M, int N);
int launch_fold_ln(mb_ctx* ctx, const float* W, int K, int N, const float* gamma,
                   const float* beta, float* Wg, float* c, float* d);
int launch_gemm_ln(mb_ctx* ctx, int epi, const float* x, int64_t ldx, const float* Wg, int N,
                   int K, const float* c, const float* d, const float* bias, float* Cm,
                   int64_t ldc, int M);
// Split-bf16 projections (bf16-KV contexts): Wx, 2 K N bf16 values, holds
// each weight of an fp32 W -- column-block-major [N / 64][K][64] (tiled:
// launch_tile_w, launch_fold_ln's Wg) or row-major [K][N] -- as a bf16 high
// part and a bf16 remainder, and
// launch_gemm_x3 computes C = epi(A W + bias) with every product as three
// bf16 products summed in fp32 (within about 2^-16 of the fp32 product).
// Takes kGemvMaxM < M with gemm_streams(M, N), else MB_ERR_STATE; with lnc
// (and lnd) A is the raw residual stream and the LayerNorm is folded in, as
// for launch_gemm_ln.  K a multiple of 128.
int launch_split_w(mb_ctx* ctx, const float* Wt, int K, int N, void* Wx, bool tiled = true);
int launch_gemm_x3(mb_ctx* ctx, int epi, const float* A, int64_t lda, const void* Wx, int N,
                   int K, const float* bias, float* Cm, int64_t ldc, int M, const float* lnc,
                   const float* lnd);

// bf16 weight storage (mb_set_weight_storage).  launch_round_bf16: Wr =
// bf16(W) kept as fp32 (round to nearest even), the weights every other copy
// derives from.  launch_kmajor_w16: Wk16[n][k] = bf16(W[k][n]).
// launch_gemv_k16: launch_gemv_k on that copy; with lnc the LayerNorm is
// folded in with gamma applied to the rows on the fly (c, d from
// launch_fold_ln over Wr with gamma, W itself unscaled).  launch_split_w1:
// the high halves of launch_split_w's layout (Wr is bf16-exact: no
// remainder), which launch_gemm_x2 reads, two bf16 products per product;
// gamma as for launch_gemv_k16 (only with lnc).
int launch_round_bf16(mb_ctx* ctx, const float* W, int64_t n, float* Wr);
int launch_kmajor_w16(mb_ctx* ctx, const float* W, int K, int N, uint16_t* Wk);
int launch_gemv_k16(mb_ctx* ctx, int epi, const float* A, int64_t lda, const uint16_t* Wk,
                    int N, int K, const float* bias, float* Cm, int64_t ldc, int M,
                    const float* lnc, const float* lnd, const float* gamma,
                    const PickIn* pick = nullptr);
int launch_split_w1(mb_ctx* ctx, const float* Wt, int K, int N, void* Wx, bool tiled = true);
int launch_gemm_x2(mb_ctx* ctx, int epi, const float* A, int64_t lda, const void* Wx1, int N,
                   int K, const float* bias, float* Cm, int64_t ldc, int M, const float* lnc,
                   const float* lnd, const float* gamma);

// layers.hip
int launch_layernorm(mb_ctx* ctx, const float* x, int64_t ldx, const int32_t* src_row, int M,
                     const float* w, const float* b, float* y, int64_t ldy, int width = D);
// x[row] = the row's embedding sum, the row being ids[row] (17 ids) or, with
// ids null, the frame row [assistant_id, codes[row][0..15]].
int launch_embed_rows(mb_ctx* ctx, const int32_t* ids, int M, const float* wte, int vocab,
                      const AudioTables& audio, float* x, const int32_t* codes = nullptr,
                      int assistant_id = 0);
int launch_embed_local(mb_ctx* ctx, int step, int B, const float* wte, int assistant_id,
                       const AudioTables& audio, const int32_t* tokens, float* x);
// With x non-null, text_decide also writes wte[assistant_id] to x[b] (step
// 1's input) and argmax_penalty writes next_emb[winner] (the next step's);
// with te non-null text_decide writes its two dot products (end, assistant)
// to te[b][2].
int launch_text_decide(mb_ctx* ctx, const float* h, int B, const float* head, int vocab, int end_id,
                       int assistant_id, const int32_t* alive, int32_t* cont,
                       const float* wte = nullptr, float* x = nullptr, double* te = nullptr);
int launch_argmax_penalty(mb_ctx* ctx, const float* logits, int B, int ch, int rec0,
                          double penalty, bool penalty_f32, uint32_t* seen, const int32_t* cont,
                          int32_t* tokens, const float* next_emb = nullptr, float* x = nullptr);
int launch_frame_rows(mb_ctx* ctx, const int32_t* tokens, int B, int assistant_id, int32_t* rows17);
int launch_frame_emit(mb_ctx* ctx, const int32_t* tokens, const int32_t* cont, int B,
                      int32_t* frame_idx, int32_t* codes, int32_t* cont_out, int32_t* pos,
                      int32_t* alive);

}  // namespace mb
