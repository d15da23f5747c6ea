// The streaming codec decoder on gfx950, batched over voices.
//
// The reference runs the decoder one position at a time: per frame the RVQ
// front, then for each of the four stages and each of its layers, every
// position in turn through LayerNorm -> qkv GEMV -> RoPE + ring write ->
// attention -> out GEMV -> layer-scale add -> LayerNorm -> FFN (exact GELU)
// -> layer-scale add (codec.ts:470-765).  Here one launch covers all voices
// and all of a stage's positions in a frame (4, 8, 16 or 32 per voice):
//
//  - the projections are one GEMM each over B x positions rows, with the
//    layer-scale residual add and the GELU fused into their epilogues;
//  - a layer appends the frame's positions to its ring and then attends to
//    them in one pass over the window, in one launch (k_attn_window: each
//    (voice, head) workgroup ropes and stores its head's new rows, then its
//    waves take the window's slot groups in turn, all of the chunk's queries
//    per wave).  Position i of the chunk
//    must not see i + 1 ..; the window rule (stored position <= cur) gives
//    that, and each ring holds its window plus one frame of positions, so an
//    append never overwrites a position that an earlier query of the same
//    chunk still sees (the reference's ring of exactly `context` slots is
//    only ever one position ahead of its query).  The visible set of every
//    query is therefore the reference's;
//  - the two interleaves (the RVQ front's x4 and the x2 sub-pixel upsample
//    between stages) and the head's channel split are column permutations
//    of the projection that produces them, applied once to the weights, so
//    no data-movement kernel runs for them.
//
// Ring layout per codec layer: K/V [voice][head][slot][64] (contiguous per
// (voice, head), as the model's rings), slot_pos [voice][slot].
#include <cstring>
#include <vector>

#include "kv_types.h"
#include "mb_internal.h"

namespace mb {

namespace {

constexpr int kD = 256;        // codec model width
constexpr int kHeads = 4;      // heads of 64
constexpr int kFfn = 1024;     // FFN width
constexpr int kRvq = 512;      // RVQ accumulator width
constexpr int kRvqOut = 768;   // RVQ output projection width (4 positions x 192)
constexpr int kEntry = 8;      // codebook entry width
constexpr int kStages = 4;
constexpr int kMaxPos = 32;    // positions per frame in the last stage
constexpr int kSamples = 3840; // samples per frame per channel
constexpr int kLatent = 240;   // last stage's output width
constexpr int kDecoderIndex[kStages] = {1, 3, 5, 7};

struct CodecLayerW {
  const float *ln1_w, *ln1_b, *qkv, *o, *ln2_w, *ln2_b, *f1, *f2, *s1, *s2;
  // norm1 folded into qkv and norm2 into f1 (launch_fold_ln): W', c, d
  const float *qkv_g, *qkv_c, *qkv_d, *f1_g, *f1_c, *f1_d;
  // bf16 rings: split-bf16 copies of the folded qkv / f1 and of o / f2
  // (launch_split_w) for the frames whose rows the streaming kernel takes
  const void *qkv_x = nullptr, *o_x = nullptr, *f1_x = nullptr, *f2_x = nullptr;
};

struct CodecStageW {
  const float* in_proj = nullptr;   // [192 | 384][256]
  const float* out_proj = nullptr;  // [256][768 | 256], columns permuted
  std::vector<CodecLayerW> layers;
};

}  // namespace

struct CodecState {
  mb_codec_config cfg{};
  int n_layers = 0;
  int layer0[kStages] = {};  // first layer (numbered across stages) of each stage
  int slots[kStages] = {};   // ring slots of each stage: context + positions per frame
  std::vector<int64_t> kv_off, sp_off;  // per layer: element offsets in ring_k/v, slot_pos
  void* ring_k = nullptr;
  void* ring_v = nullptr;
  int32_t* slot_pos = nullptr;
  int32_t* pos = nullptr;   // [4][max_voices]: the next absolute position of each stage
  int32_t* nrow = nullptr;  // [4][max_voices]: positions per frame of each stage
  float *acc = nullptr, *x = nullptr, *h = nullptr, *qkv = nullptr, *att = nullptr,
        *ffn = nullptr, *wide = nullptr;
  int32_t* frame = nullptr;  // the frame a decode call is at (device counter)
  std::vector<void*> owned;
  // one captured frame of mb_codec_decode_dev and what it was captured for
  hipGraphExec_t exec = nullptr;
  uint64_t key[6] = {};
  // resolved weights
  const float *rvq_w = nullptr, *rvq_b = nullptr, *rvq_book = nullptr, *rvq_out = nullptr,
              *rvq_out_b = nullptr;
  CodecStageW stages[kStages];
};

namespace {

__host__ __device__ constexpr int positions(int s) { return 4 << s; }

// ------------------------------------------------------------------ kernels

// acc[b][n] = sum_k (W_k[n] . codebook_k[code_k] + b_k[n]) in quantiser
// order, each dot over the 8 entry values in order (RVQ_ACCUM,
// kernels-decode.ts:537-558).  A code outside [0, 1024) adds no codebook row.
// `frame` is the device frame counter: codes of the current frame start at
// codes + frame * B * 16.
__global__ __launch_bounds__(256) void k_rvq_accum(const int32_t* __restrict__ codes_all,
                                                   const int32_t* __restrict__ frame, int B,
                                                   const float* __restrict__ w,
                                                   const float* __restrict__ bias,
                                                   const float* __restrict__ book,
                                                   float* __restrict__ acc) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= (int64_t)B * kRvq) return;
  const int b = (int)(t / kRvq), n = (int)(t % kRvq);
  const int32_t* codes = codes_all + (int64_t)*frame * B * NVQ;
  float a = 0.f;
  for (int k = 0; k < NVQ; k++) {
    const int32_t code = codes[(int64_t)b * NVQ + k];
    float dot = 0.f;
    if (code >= 0 && code < CODES) {
      const float* wr = w + ((int64_t)k * kRvq + n) * kEntry;
      const float* e = book + ((int64_t)k * CODES + code) * kEntry;
#pragma unroll
      for (int j = 0; j < kEntry; j++) dot = dot + wr[j] * e[j];
    }
    a = (a + dot) + bias[k * kRvq + n];
  }
  acc[t] = a;
}

// dst[k][j] = 0 if map[j] < 0, else src[map[j]][k] (TRANSPOSE) or
// src[k][map[j]]: the column permutations folded into the projections.
template <bool TRANSPOSE>
__global__ __launch_bounds__(256) void k_gather_cols(const float* __restrict__ src, int K,
                                                     int n_src, const int32_t* __restrict__ map,
                                                     int n_dst, float* __restrict__ dst) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= (int64_t)K * n_dst) return;
  const int k = (int)(t / n_dst), j = (int)(t % n_dst);
  const int m = map[j];
  dst[t] = m < 0 ? 0.f : TRANSPOSE ? src[(int64_t)m * K + k] : src[(int64_t)k * n_src + m];
}

// pcm[b][c][f * 3840 + t * 120 + j] = latent[b * 32 + t][c * 120 + j]: the
// last stage's output columns are already (channel, sample) ordered, so the
// head (CODEC_HEAD, kernels-decode.ts:747-768) is this copy.
__global__ __launch_bounds__(256) void k_codec_head(const float* __restrict__ latent, int B,
                                                    const int32_t* __restrict__ frame, int64_t T,
                                                    float* __restrict__ pcm) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= (int64_t)B * 2 * kSamples) return;
  const int f = *frame;
  const int b = (int)(t / (2 * kSamples));
  const int rest = (int)(t % (2 * kSamples));
  const int c = rest / kSamples, i = rest % kSamples, pos = i / 120, j = i % 120;
  pcm[((int64_t)b * 2 + c) * T + (int64_t)f * kSamples + i] =
      latent[((int64_t)b * kMaxPos + pos) * kD + c * 120 + j];
}

// The end of a frame: every stage's positions advance by its positions per
// frame for voices b < B (pos [4][V]; each stage's layers read only their
// own stage's positions, so all four move here, once the frame's last stage
// has run), and the frame counter by one.
__global__ void k_frame_advance(int32_t* __restrict__ pos, int V, int B, int32_t* __restrict__ frame) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < B) {
#pragma unroll
    for (int s = 0; s < kStages; s++) pos[(int64_t)s * V + i] += positions(s);
  }
  if (i == 0) *frame += 1;
}

// ------------------------------------------------------------------ helpers

RingView codec_ring(const mb_ctx* ctx, const CodecState& cs, int layer, int stage) {
  const size_t e = cs.cfg.kv_dtype == MB_KV_BF16 ? 2 : 4;
  RingView v;
  v.k = (char*)cs.ring_k + cs.kv_off[layer] * e;
  v.v = (char*)cs.ring_v + cs.kv_off[layer] * e;
  v.sp = cs.slot_pos + cs.sp_off[layer];
  v.C = cs.slots[stage];
  v.window = cs.cfg.context[stage];
  v.heads = kHeads;
  v.seq_stride = (int64_t)kHeads * v.C * HD;
  v.wrap = 1;
  v.bf16 = cs.cfg.kv_dtype == MB_KV_BF16;
  (void)ctx;
  return v;
}

int cancelled(mb_ctx* ctx) {
  if (ctx->cancel.load()) return fail(ctx, MB_ERR_CANCELLED, "cancelled");
  return MB_OK;
}

void* dev_alloc(mb_ctx* ctx, CodecState& cs, size_t bytes) {
  void* p = nullptr;
  if (hipMalloc(&p, bytes) != hipSuccess) return nullptr;
  cs.owned.push_back(p);
  ctx->device_bytes += (int64_t)bytes;
  return p;
}

// Internal tensor `name` = the projection `src` with its output columns
// gathered through `map` (negative: a zero column); `transpose` reads src as
// [n_src][K] (a graph weight stored output-major) instead of [K][n_src].
int gather_cols(mb_ctx* ctx, const std::string& name, const float* src, int K, int n_src,
                const std::vector<int32_t>& map, bool transpose, const float** out) {
  const int n_dst = (int)map.size();
  float* dst = internal_tensor(ctx, name, (int64_t)K * n_dst);
  int32_t* dmap = (int32_t*)internal_tensor(ctx, name + ".map", n_dst);
  if (!dst || !dmap) return fail(ctx, MB_ERR_NOMEM, "codec weight %s", name.c_str());
  MB_HIP(ctx, hipMemcpyAsync(dmap, map.data(), map.size() * 4, hipMemcpyHostToDevice, ctx->stream));
  const unsigned grid = (unsigned)(((int64_t)K * n_dst + 255) / 256);
  if (transpose)
    hipLaunchKernelGGL(k_gather_cols<true>, dim3(grid), dim3(256), 0, ctx->stream, src, K, n_src,
                       dmap, n_dst, dst);
  else
    hipLaunchKernelGGL(k_gather_cols<false>, dim3(grid), dim3(256), 0, ctx->stream, src, K, n_src,
                       dmap, n_dst, dst);
  MB_HIP(ctx, hipGetLastError());
  // the map is read by the launch just queued; keep it until the stream passes it
  MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
  *out = dst;
  return MB_OK;
}

// One of two accepted shapes (a 1x1 convolution may carry its trailing 1).
const float* get2(mb_ctx* ctx, const std::string& n, std::initializer_list<int64_t> a,
                  std::initializer_list<int64_t> b, std::string& missing) {
  std::string ignore;
  const DeviceTensor* t = find(ctx, n, a, ignore);
  if (!t) t = find(ctx, n, b, missing);
  return t ? t->ptr : nullptr;
}

// Resolve every codec weight once per upload and build the permuted
// projections (the reference resolves its blocks the same way, by name and
// shape, and throws when one is missing: decodeWeights.ts:69-156).
int codec_resolve(mb_ctx* ctx) {
  if (ctx->codec_ok) return MB_OK;
  CodecState& cs = *ctx->codec;
  std::string missing;
  auto get = [&](const std::string& n, std::initializer_list<int64_t> d) {
    const DeviceTensor* t = find(ctx, n, d, missing);
    return t ? (const float*)t->ptr : nullptr;
  };
  const float *conv[NVQ], *cbias[NVQ], *book[NVQ];
  for (int k = 0; k < NVQ; k++) {
    const std::string p = "model.quantizer.quantizers." + std::to_string(k) + ".";
    conv[k] = get2(ctx, p + "out_proj.weight", {kRvq, kEntry}, {kRvq, kEntry, 1}, missing);
    cbias[k] = get(p + "out_proj.bias", {kRvq});
    book[k] = get(p + "codebook.weight", {CODES, kEntry});
  }
  const float* out_w = get2(ctx, "model.quantizer.output_proj.weight", {kRvqOut, kRvq},
                            {kRvqOut, kRvq, 1}, missing);
  const float* out_b = get("model.quantizer.output_proj.bias", {kRvqOut});
  const float* stage_out[kStages] = {};
  for (int s = 0; s < kStages; s++) {
    const std::string p = "model.decoder." + std::to_string(kDecoderIndex[s]) + ".";
    CodecStageW& st = cs.stages[s];
    st.in_proj = get(p + "input_proj.weight", {s == 0 ? 192 : 384, kD});
    stage_out[s] = get(p + "output_proj.weight", {kD, s == kStages - 1 ? kLatent : kRvqOut});
    st.layers.assign(cs.cfg.layers[s], CodecLayerW{});
    for (int i = 0; i < cs.cfg.layers[s]; i++) {
      const std::string l = p + "transformer.layers." + std::to_string(i) + ".";
      CodecLayerW& w = st.layers[i];
      w.qkv = get(l + "self_attn.in_proj.weight", {kD, 3 * kD});
      w.o = get(l + "self_attn.out_proj.weight", {kD, kD});
      w.f1 = get(l + "ffn.0.weight", {kD, kFfn});
      w.f2 = get(l + "ffn.2.weight", {kFfn, kD});
      w.ln1_w = get(l + "norm1.weight", {kD});
      w.ln1_b = get(l + "norm1.bias", {kD});
      w.ln2_w = get(l + "norm2.weight", {kD});
      w.ln2_b = get(l + "norm2.bias", {kD});
      w.s1 = get(l + "layer_scale_1.scale", {kD});
      w.s2 = get(l + "layer_scale_2.scale", {kD});
    }
  }
  if (!missing.empty()) return fail(ctx, MB_ERR_STATE, "codec %s", missing.c_str());

  // norm1 / norm2 folded into the projections after them, for the frames
  // whose rows the streaming kernel takes
  auto fold = [&](const std::string& name, const float* W, int N, const float* gamma,
                  const float* beta, const float*& wg, const float*& c, const float*& d) {
    float* pw = internal_tensor(ctx, name + ".w", (int64_t)kD * N);
    float* pc = internal_tensor(ctx, name + ".c", N);
    float* pd = internal_tensor(ctx, name + ".d", N);
    if (!pw || !pc || !pd) return fail(ctx, MB_ERR_NOMEM, "codec folded weights (%s)", name.c_str());
    wg = pw;
    c = pc;
    d = pd;
    return launch_fold_ln(ctx, W, kD, N, gamma, beta, pw, pc, pd);
  };
  for (int s = 0; s < kStages; s++)
    for (int i = 0; i < cs.cfg.layers[s]; i++) {
      CodecLayerW& w = cs.stages[s].layers[i];
      const std::string key = "#codec/s" + std::to_string(s) + "l" + std::to_string(i);
      int frc = fold(key + ".qkv", w.qkv, 3 * kD, w.ln1_w, w.ln1_b, w.qkv_g, w.qkv_c, w.qkv_d);
      if (!frc) frc = fold(key + ".f1", w.f1, kFfn, w.ln2_w, w.ln2_b, w.f1_g, w.f1_c, w.f1_d);
      if (!frc && cs.cfg.kv_dtype == MB_KV_BF16) {
        auto split = [&](const std::string& name, const float* W, int K, int N, bool tiled,
                         const void*& wx) {
          float* p = internal_tensor(ctx, name, (int64_t)K * N);  // 2 K N bf16
          if (!p) return fail(ctx, MB_ERR_NOMEM, "codec split weights (%s)", name.c_str());
          wx = p;
          return launch_split_w(ctx, W, K, N, p, tiled);
        };
        frc = split(key + ".qkv.x", w.qkv_g, kD, 3 * kD, true, w.qkv_x);
        if (!frc) frc = split(key + ".f1.x", w.f1_g, kD, kFfn, true, w.f1_x);
        if (!frc) frc = split(key + ".o.x", w.o, kD, kD, false, w.o_x);
        if (!frc) frc = split(key + ".f2.x", w.f2, kFfn, kD, false, w.f2_x);
      }
      if (frc) return frc;
    }

  // the per-quantiser tensors side by side: W [16][512][8], b [16][512], codebooks [16][1024][8]
  float* rw = internal_tensor(ctx, "#codec/rvq_w", (int64_t)NVQ * kRvq * kEntry);
  float* rb = internal_tensor(ctx, "#codec/rvq_b", (int64_t)NVQ * kRvq);
  float* rk = internal_tensor(ctx, "#codec/rvq_book", (int64_t)NVQ * CODES * kEntry);
  if (!rw || !rb || !rk) return fail(ctx, MB_ERR_NOMEM, "codec RVQ tables");
  for (int k = 0; k < NVQ; k++) {
    MB_HIP(ctx, hipMemcpyAsync(rw + (int64_t)k * kRvq * kEntry, conv[k], kRvq * kEntry * 4,
                               hipMemcpyDeviceToDevice, ctx->stream));
    MB_HIP(ctx, hipMemcpyAsync(rb + (int64_t)k * kRvq, cbias[k], kRvq * 4, hipMemcpyDeviceToDevice,
                               ctx->stream));
    MB_HIP(ctx, hipMemcpyAsync(rk + (int64_t)k * CODES * kEntry, book[k], CODES * kEntry * 4,
                               hipMemcpyDeviceToDevice, ctx->stream));
  }
  cs.rvq_w = rw;
  cs.rvq_b = rb;
  cs.rvq_book = rk;

  int rc;
  // RVQ output projection, [768][512] output-major in the graph: transposed
  // to [512][768] with output column s*192 + m taking channel 4m + s, so the
  // GEMM's row is the x4-interleaved [4][192] block (RVQ_PROJECT,
  // kernels-decode.ts:562-574: dst[(n & 3) * 192 + (n >> 2)] = g[n]).
  std::vector<int32_t> map(kRvqOut);
  for (int j = 0; j < kRvqOut; j++) map[j] = 4 * (j % 192) + j / 192;
  if ((rc = gather_cols(ctx, "#codec/rvq_out", out_w, kRvq, kRvqOut, map, true, &cs.rvq_out)))
    return rc;
  {
    std::vector<int32_t> bmap = map;
    if ((rc = gather_cols(ctx, "#codec/rvq_out_b", out_b, 1, kRvqOut, bmap, false, &cs.rvq_out_b)))
      return rc;
  }
  // stage outputs: for s < 3 column r*384 + m takes column 2m + r (the x2
  // upsample new[2t + r][m] = old[t][2m + r], UPSAMPLE2 kernels-decode.ts:
  // 722-745, becomes "row t is rows 2t and 2t + 1"); the last stage's column
  // c*120 + j takes latent column 2j + c (CODEC_HEAD: audio[c][t*120 + j] =
  // latent[t][2j + c]), padded with zero columns to 256.
  for (int s = 0; s < kStages; s++) {
    const bool last = s == kStages - 1;
    std::vector<int32_t> m(last ? kD : kRvqOut);
    for (int j = 0; j < (int)m.size(); j++) {
      if (last) m[j] = j < kLatent ? 2 * (j % 120) + j / 120 : -1;
      else m[j] = 2 * (j % 384) + j / 384;
    }
    if ((rc = gather_cols(ctx, "#codec/out" + std::to_string(s), stage_out[s], kD,
                          last ? kLatent : kRvqOut, m, false, &cs.stages[s].out_proj)))
      return rc;
  }
  MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
  ctx->codec_ok = true;
  return MB_OK;
}

// One frame for voices b < B: the frame *cs.frame of codes [n][B][16]
// (device) -> that frame of pcm [B][2][T], then the counter advances.  Every
// launch is on the context's stream and reads the frame index from the
// device, so the same launches serve every frame (one captured graph).
int codec_frame(mb_ctx* ctx, int B, const int32_t* codes, float* pcm, int64_t T) {
  CodecState& cs = *ctx->codec;
  const int V = cs.cfg.max_voices;
  int rc;
  hipLaunchKernelGGL(k_rvq_accum, dim3((unsigned)(((int64_t)B * kRvq + 255) / 256)), dim3(256), 0,
                     ctx->stream, codes, cs.frame, B, cs.rvq_w, cs.rvq_b, cs.rvq_book, cs.acc);
  MB_HIP(ctx, hipGetLastError());
  if ((rc = launch_gemm(ctx, EPI_STORE, cs.acc, kRvq, cs.rvq_out, kRvqOut, kRvq, cs.rvq_out_b,
                        cs.wide, kRvqOut, B)))
    return rc;
  int in_w = 192;
  for (int s = 0; s < kStages; s++) {
    const int n = positions(s), M = B * n;
    const CodecStageW& st = cs.stages[s];
    int32_t* pos = cs.pos + (int64_t)s * V;
    const int32_t* nrow = cs.nrow + (int64_t)s * V;
    if ((rc = launch_gemm(ctx, EPI_STORE, cs.wide, in_w, st.in_proj, kD, in_w, nullptr, cs.x, kD, M)))
      return rc;
    for (int i = 0; i < cs.cfg.layers[s]; i++) {
      const CodecLayerW& w = st.layers[i];
      const RingView ring = codec_ring(ctx, cs, cs.layer0[s] + i, s);
      // With bf16 rings every projection above kGemvMaxM rows takes the
      // split-bf16 products, norm1 / norm2 folded into them.  With fp32 rings
      // they are folded where the streaming kernel takes the rows, else run
      // apart.
      const bool fold_qkv = gemm_streams(M, 3 * kD), fold_f1 = gemm_streams(M, kFfn);
      const bool x3 = w.qkv_x && M > kGemvMaxM;
      auto qkv_proj = [&]() {
        if (x3)
          return launch_gemm_x3(ctx, EPI_STORE, cs.x, kD, w.qkv_x, 3 * kD, kD, nullptr, cs.qkv,
                                3 * kD, M, w.qkv_c, w.qkv_d);
        if (fold_qkv)
          return launch_gemm_ln(ctx, EPI_STORE, cs.x, kD, w.qkv_g, 3 * kD, kD, w.qkv_c, w.qkv_d,
                                nullptr, cs.qkv, 3 * kD, M);
        int r = launch_layernorm(ctx, cs.x, kD, nullptr, M, w.ln1_w, w.ln1_b, cs.h, kD, kD);
        return r ? r : launch_gemm(ctx, EPI_STORE, cs.h, kD, w.qkv, 3 * kD, kD, nullptr, cs.qkv, 3 * kD, M);
      };
      auto f1_proj = [&]() {
        if (x3)
          return launch_gemm_x3(ctx, EPI_GELU_ERF, cs.x, kD, w.f1_x, kFfn, kD, nullptr, cs.ffn,
                                kFfn, M, w.f1_c, w.f1_d);
        if (fold_f1)
          return launch_gemm_ln(ctx, EPI_GELU_ERF, cs.x, kD, w.f1_g, kFfn, kD, w.f1_c, w.f1_d,
                                nullptr, cs.ffn, kFfn, M);
        int r = launch_layernorm(ctx, cs.x, kD, nullptr, M, w.ln2_w, w.ln2_b, cs.h, kD, kD);
        return r ? r : launch_gemm(ctx, EPI_GELU_ERF, cs.h, kD, w.f1, kFfn, kD, nullptr, cs.ffn, kFfn, M);
      };
      if ((rc = qkv_proj()) ||
          (rc = launch_window_attention(ctx, ring, B, n, cs.qkv, dense_rows(3 * kD, n), pos, nrow,
                                        cs.att, dense_rows(kD, n))) ||
          (rc = x3 ? launch_gemm_x3(ctx, EPI_SCALE_ADD, cs.att, kD, w.o_x, kD, kD, w.s1, cs.x, kD,
                                      M, nullptr, nullptr)
                     : launch_gemm(ctx, EPI_SCALE_ADD, cs.att, kD, w.o, kD, kD, w.s1, cs.x, kD, M)) ||
          (rc = f1_proj()) ||
          (rc = x3 ? launch_gemm_x3(ctx, EPI_SCALE_ADD, cs.ffn, kFfn, w.f2_x, kD, kFfn, w.s2, cs.x,
                                      kD, M, nullptr, nullptr)
                     : launch_gemm(ctx, EPI_SCALE_ADD, cs.ffn, kFfn, w.f2, kD, kFfn, w.s2, cs.x, kD, M)))
        return rc;
    }
    const int out_w = s == kStages - 1 ? kD : kRvqOut;
    if ((rc = launch_gemm(ctx, EPI_STORE, cs.x, kD, st.out_proj, out_w, kD, nullptr, cs.wide, out_w, M)))
      return rc;
    in_w = 384;
  }
  hipLaunchKernelGGL(k_codec_head, dim3((unsigned)(((int64_t)B * 2 * kSamples + 255) / 256)),
                     dim3(256), 0, ctx->stream, cs.wide, B, cs.frame, T, pcm);
  hipLaunchKernelGGL(k_frame_advance, dim3((unsigned)((B + 255) / 256)), dim3(256), 0, ctx->stream,
                     cs.pos, V, B, cs.frame);
  MB_HIP(ctx, hipGetLastError());
  return MB_OK;
}

int check_codec(mb_ctx* ctx, int B, int n_frames) {
  if (!ctx->codec) return fail(ctx, MB_ERR_STATE, "codec not initialised (mb_codec_init)");
  if (B < 0 || B > ctx->codec->cfg.max_voices)
    return fail(ctx, MB_ERR_ARG, "B %d out of [0, max_voices %d]", B, ctx->codec->cfg.max_voices);
  if (n_frames < 0) return fail(ctx, MB_ERR_ARG, "n_frames %d < 0", n_frames);
  return codec_resolve(ctx);
}

}  // namespace

// Called from entry points that already run on the context's device.
void codec_free(mb_ctx* ctx) {
  if (!ctx->codec) return;
  if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
  if (ctx->codec->exec) (void)hipGraphExecDestroy(ctx->codec->exec);
  for (void* p : ctx->codec->owned) (void)hipFree(p);
  delete ctx->codec;
  ctx->codec = nullptr;
  ctx->codec_ok = false;
}

}  // namespace mb

using namespace mb;

extern "C" int mb_codec_init(mb_ctx* ctx, const mb_codec_config* cfg) {
  MB_DEVICE_GUARD(ctx);
  if (!ctx || !cfg) return MB_ERR_ARG;
  if (cfg->max_voices < 1 || cfg->max_voices > 65535)
    return fail(ctx, MB_ERR_ARG, "codec max_voices %d out of [1, 65535]", cfg->max_voices);
  if (cfg->kv_dtype != MB_KV_F32 && cfg->kv_dtype != MB_KV_BF16)
    return fail(ctx, MB_ERR_ARG, "codec kv_dtype %d", cfg->kv_dtype);
  for (int s = 0; s < kStages; s++) {
    if (cfg->layers[s] < 1 || cfg->layers[s] > 16)
      return fail(ctx, MB_ERR_ARG, "codec stage %d: %d layers out of [1, 16]", s, cfg->layers[s]);
    if (cfg->context[s] < 1 || cfg->context[s] + positions(s) > (1 << 20))
      return fail(ctx, MB_ERR_ARG, "codec stage %d: context %d out of range", s, cfg->context[s]);
  }
  codec_free(ctx);
  CodecState* cs = new CodecState();
  ctx->codec = cs;
  cs->cfg = *cfg;
  const int V = cfg->max_voices;
  const size_t e = cfg->kv_dtype == MB_KV_BF16 ? 2 : 4;
  int64_t kv = 0, sp = 0;
  for (int s = 0; s < kStages; s++) {
    cs->layer0[s] = cs->n_layers;
    cs->slots[s] = cfg->context[s] + positions(s);
    for (int i = 0; i < cfg->layers[s]; i++) {
      cs->kv_off.push_back(kv);
      cs->sp_off.push_back(sp);
      kv += (int64_t)V * kHeads * cs->slots[s] * HD;
      sp += (int64_t)V * cs->slots[s];
      cs->n_layers++;
    }
  }
  const int64_t rows = (int64_t)V * kMaxPos;
  cs->ring_k = dev_alloc(ctx, *cs, (size_t)kv * e);
  cs->ring_v = dev_alloc(ctx, *cs, (size_t)kv * e);
  cs->slot_pos = (int32_t*)dev_alloc(ctx, *cs, (size_t)sp * 4);
  cs->pos = (int32_t*)dev_alloc(ctx, *cs, (size_t)kStages * V * 4);
  cs->nrow = (int32_t*)dev_alloc(ctx, *cs, (size_t)kStages * V * 4);
  cs->frame = (int32_t*)dev_alloc(ctx, *cs, 4);
  cs->acc = (float*)dev_alloc(ctx, *cs, (size_t)V * kRvq * 4);
  cs->x = (float*)dev_alloc(ctx, *cs, (size_t)rows * kD * 4);
  cs->h = (float*)dev_alloc(ctx, *cs, (size_t)rows * kD * 4);
  cs->qkv = (float*)dev_alloc(ctx, *cs, (size_t)rows * 3 * kD * 4);
  cs->att = (float*)dev_alloc(ctx, *cs, (size_t)rows * kD * 4);
  cs->ffn = (float*)dev_alloc(ctx, *cs, (size_t)rows * kFfn * 4);
  cs->wide = (float*)dev_alloc(ctx, *cs, (size_t)rows * kRvqOut * 4);
  for (void* p : {cs->ring_k, cs->ring_v, (void*)cs->slot_pos, (void*)cs->pos, (void*)cs->nrow,
                  (void*)cs->frame,
                  (void*)cs->acc, (void*)cs->x, (void*)cs->h, (void*)cs->qkv,
                  (void*)cs->att, (void*)cs->ffn, (void*)cs->wide})
    if (!p) {
      codec_free(ctx);
      return fail(ctx, MB_ERR_NOMEM, "codec rings and buffers for %d voices", V);
    }
  int rc;
  for (int s = 0; s < kStages; s++)
    if ((rc = launch_fill_i32(ctx, cs->nrow + (int64_t)s * V, V, positions(s)))) return rc;
  ctx->codec_ok = false;
  return mb_codec_reset(ctx, -1, nullptr);
}

extern "C" int mb_codec_reset(mb_ctx* ctx, int n, const int32_t* voices) {
  MB_DEVICE_GUARD(ctx);
  if (!ctx) return MB_ERR_ARG;
  if (!ctx->codec) return fail(ctx, MB_ERR_STATE, "codec not initialised (mb_codec_init)");
  CodecState& cs = *ctx->codec;
  const int V = cs.cfg.max_voices;
  int rc;
  if (n < 0) {
    int64_t sp = 0;
    for (int s = 0; s < kStages; s++) sp += (int64_t)cs.cfg.layers[s] * V * cs.slots[s];
    if ((rc = launch_fill_i32(ctx, cs.slot_pos, sp, -1))) return rc;
    if ((rc = launch_fill_i32(ctx, cs.pos, (int64_t)kStages * V, 0))) return rc;
  } else {
    if (n > 0 && !voices) return fail(ctx, MB_ERR_ARG, "mb_codec_reset: voices is NULL");
    for (int i = 0; i < n; i++)
      if (voices[i] < 0 || voices[i] >= V)
        return fail(ctx, MB_ERR_ARG, "voice %d out of [0, %d)", voices[i], V);
    for (int i = 0; i < n; i++) {
      const int b = voices[i];
      for (int s = 0; s < kStages; s++) {
        for (int l = 0; l < cs.cfg.layers[s]; l++)
          if ((rc = launch_fill_i32(ctx, cs.slot_pos + cs.sp_off[cs.layer0[s] + l] +
                                             (int64_t)b * cs.slots[s],
                                    cs.slots[s], -1)))
            return rc;
        if ((rc = launch_fill_i32(ctx, cs.pos + (int64_t)s * V + b, 1, 0))) return rc;
      }
    }
  }
  MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return MB_OK;
}

extern "C" int mb_codec_decode_dev(mb_ctx* ctx, int B, int n_frames, const int32_t* codes,
                                   float* pcm) {
  MB_DEVICE_GUARD(ctx);
  if (!ctx) return MB_ERR_ARG;
  int rc = check_codec(ctx, B, n_frames);
  if (rc) return rc;
  if (B == 0 || n_frames == 0) return MB_OK;
  if (!codes || !pcm) return fail(ctx, MB_ERR_ARG, "mb_codec_decode_dev: null pointer");
  CodecState& cs = *ctx->codec;
  const int64_t T = (int64_t)n_frames * kSamples;
  if ((rc = cancelled(ctx))) return rc;
  if ((rc = launch_fill_i32(ctx, cs.frame, 1, 0))) return rc;
  // Frame 0 runs eagerly (it sizes every scratch buffer a frame touches, so
  // nothing is allocated during the capture); the next frames replay it
  // from a HIP graph, captured once per (B, codes, pcm, T) and buffer set.
  if ((rc = codec_frame(ctx, B, codes, pcm, T))) return rc;
  if (n_frames == 1) return MB_OK;
  const uint64_t key[6] = {(uint64_t)B, (uint64_t)(uintptr_t)codes, (uint64_t)(uintptr_t)pcm,
                           (uint64_t)T, ctx->graph_gen, 1};
  if (!cs.exec || memcmp(key, cs.key, sizeof key) != 0) {
    if (cs.exec) {
      MB_HIP(ctx, hipGraphExecDestroy(cs.exec));
      cs.exec = nullptr;
    }
    if (!ctx->capture_stream)
      MB_HIP(ctx, hipStreamCreateWithFlags(&ctx->capture_stream, hipStreamNonBlocking));
    hipStream_t saved = ctx->stream;
    const hipError_t eb = hipStreamBeginCapture(ctx->capture_stream, hipStreamCaptureModeThreadLocal);
    if (eb != hipSuccess) return hip_fail(ctx, eb, "hipStreamBeginCapture");
    ctx->stream = ctx->capture_stream;
    rc = codec_frame(ctx, B, codes, pcm, T);
    hipGraph_t graph = nullptr;
    const hipError_t e = hipStreamEndCapture(ctx->stream, &graph);
    ctx->stream = saved;
    if (rc || e != hipSuccess || ctx->graph_gen != key[4]) {
      if (graph) (void)hipGraphDestroy(graph);
      if (rc) return rc;
      if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamEndCapture");
      return fail(ctx, MB_ERR_STATE, "a buffer moved while the codec frame was captured");
    }
    const hipError_t ei = hipGraphInstantiate(&cs.exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (ei != hipSuccess) {
      cs.exec = nullptr;
      return hip_fail(ctx, ei, "hipGraphInstantiate");
    }
    memcpy(cs.key, key, sizeof key);
  }
  for (int f = 1; f < n_frames; f++) {
    if ((rc = cancelled(ctx))) return rc;
    MB_HIP(ctx, hipGraphLaunch(cs.exec, ctx->stream));
  }
  return MB_OK;
}

extern "C" int mb_codec_decode(mb_ctx* ctx, int B, int n_frames, const int32_t* codes, float* pcm) {
  MB_DEVICE_GUARD(ctx);
  if (!ctx) return MB_ERR_ARG;
  int rc = check_codec(ctx, B, n_frames);
  if (rc) return rc;
  if (B == 0 || n_frames == 0) return MB_OK;
  if (!codes || !pcm) return fail(ctx, MB_ERR_ARG, "mb_codec_decode: null pointer");
  const int64_t nc = (int64_t)n_frames * B * NVQ;
  for (int64_t i = 0; i < nc; i++)
    if (codes[i] < 0 || codes[i] >= CODES)
      return fail(ctx, MB_ERR_ARG, "code %d at %lld out of [0, %d)", codes[i], (long long)i, CODES);
  const int64_t T = (int64_t)n_frames * kSamples;
  const size_t pcm_bytes = (size_t)B * 2 * T * 4;
  int32_t* dc = (int32_t*)scratch(ctx, "codec_codes", (size_t)nc * 4);
  float* dp = (float*)scratch(ctx, "codec_pcm", pcm_bytes);
  if (!dc || !dp) return fail(ctx, MB_ERR_NOMEM, "codec staging for %d frames", n_frames);
  MB_HIP(ctx, hipMemcpyAsync(dc, codes, (size_t)nc * 4, hipMemcpyHostToDevice, ctx->stream));
  if ((rc = mb_codec_decode_dev(ctx, B, n_frames, dc, dp))) return rc;
  MB_HIP(ctx, hipMemcpyAsync(pcm, dp, pcm_bytes, hipMemcpyDeviceToHost, ctx->stream));
  MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return MB_OK;
}

extern "C" int mb_codec_read_ring(mb_ctx* ctx, int layer, int voice, float* k, float* v,
                                  int32_t* slot_pos, int32_t* slots) {
  MB_DEVICE_GUARD(ctx);
  if (!ctx) return MB_ERR_ARG;
  if (!ctx->codec) return fail(ctx, MB_ERR_STATE, "codec not initialised (mb_codec_init)");
  CodecState& cs = *ctx->codec;
  if (layer < 0 || layer >= cs.n_layers)
    return fail(ctx, MB_ERR_ARG, "codec layer %d out of [0, %d)", layer, cs.n_layers);
  if (voice < 0 || voice >= cs.cfg.max_voices)
    return fail(ctx, MB_ERR_ARG, "voice %d out of [0, %d)", voice, cs.cfg.max_voices);
  int s = 0;
  while (s + 1 < kStages && layer >= cs.layer0[s + 1]) s++;
  const int C = cs.slots[s];
  if (slots) *slots = C;
  MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
  const RingView ring = codec_ring(ctx, cs, layer, s);
  const bool bf16 = ring.bf16;
  const size_t e = bf16 ? 2 : 4;
  std::vector<uint8_t> host((size_t)kHeads * C * HD * e);
  for (int which = 0; which < 2; which++) {
    float* out = which ? v : k;
    if (!out) continue;
    const char* src = (const char*)(which ? ring.v : ring.k) + (size_t)voice * ring.seq_stride * e;
    MB_HIP(ctx, hipMemcpy(host.data(), src, host.size(), hipMemcpyDeviceToHost));
    for (int h = 0; h < kHeads; h++)
      for (int sl = 0; sl < C; sl++)
        for (int d = 0; d < HD; d++) {
          const size_t i = ((size_t)h * C + sl) * HD + d;
          float val;
          if (bf16) {
            uint16_t b16;
            std::memcpy(&b16, host.data() + i * 2, 2);
            const uint32_t w = (uint32_t)b16 << 16;
            std::memcpy(&val, &w, 4);
          } else {
            std::memcpy(&val, host.data() + i * 4, 4);
          }
          out[(size_t)sl * kD + h * HD + d] = val;
        }
  }
  if (slot_pos)
    MB_HIP(ctx, hipMemcpy(slot_pos, ring.sp + (int64_t)voice * C, (size_t)C * 4,
                          hipMemcpyDeviceToHost));
  return MB_OK;
}
