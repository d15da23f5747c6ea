// The decoder around the ring: global prefill, one global decode step, and
// the 17-step local frame head, each a sequence of launches on the context's
// stream (LN -> QKV GEMM -> RoPE + ring write -> attention -> O GEMM (+x) ->
// LN -> fc_in GEMM (+GELU) -> fc_out GEMM (+x) per layer; ref-decode.mjs:
// 175-272 and decode.ts:474-620 give the order, including that each layer's
// MLP follows its own attention).
#include <cmath>
#include <cstring>

#include "mb_internal.h"
#include "pick.h"

namespace mb {

namespace {

int resolve_layer(mb_ctx* ctx, const std::string& p, LayerW& w, std::string& missing) {
  auto get = [&](const char* n, std::initializer_list<int64_t> d) {
    const DeviceTensor* t = find(ctx, p + n, d, missing);
    return t ? (const float*)t->ptr : nullptr;
  };
  w.ln1_w = get("ln_1.weight", {D});
  w.ln1_b = get("ln_1.bias", {D});
  w.attn_w = get("attn.c_attn.weight", {D, QKV});
  w.attn_b = get("attn.c_attn.bias", {QKV});
  w.proj_w = get("attn.c_proj.weight", {D, D});
  w.proj_b = get("attn.c_proj.bias", {D});
  w.ln2_w = get("ln_2.weight", {D});
  w.ln2_b = get("ln_2.bias", {D});
  w.fc_in_w = get("mlp.fc_in.weight", {D, FFN});
  w.fc_in_b = get("mlp.fc_in.bias", {FFN});
  w.fc_out_w = get("mlp.fc_out.weight", {FFN, D});
  w.fc_out_b = get("mlp.fc_out.bias", {D});
  return missing.empty() ? MB_OK : MB_ERR_STATE;
}

// LayerNorm (gamma, beta) folded into the [K][N] projection W after it.
int fold(mb_ctx* ctx, const std::string& name, const float* W, int K, int N, const float* gamma,
         const float* beta, const float*& wg, const float*& c, const float*& d) {
  float* pw = internal_tensor(ctx, name + ".w", (int64_t)K * N);
  float* pc = internal_tensor(ctx, name + ".c", N);
  float* pd = internal_tensor(ctx, name + ".d", N);
  if (!pw || !pc || !pd) return fail(ctx, MB_ERR_NOMEM, "folded weight allocation failed (%s)", name.c_str());
  wg = pw;
  c = pc;
  d = pd;
  return launch_fold_ln(ctx, W, K, N, gamma, beta, pw, pc, pd);
}

// A column-block-major copy of the [K][N] projection W (launch_tile_w).
int tile(mb_ctx* ctx, const std::string& name, const float* W, int K, int N, const float*& wt) {
  float* p = internal_tensor(ctx, name, (int64_t)K * N);
  if (!p) return fail(ctx, MB_ERR_NOMEM, "tiled weight allocation failed (%s)", name.c_str());
  wt = p;
  return launch_tile_w(ctx, W, K, N, p);
}

// The k-major copy the GEMV kernels read of the [K][N] projection W:
// Wk[n][k] = gamma[k] W[k][n] in fp32 (launch_kmajor_w; gamma null: the
// plain transpose), or with bf16 weight storage bf16(W[k][n]) with no gamma
// (the kernel applies it to the rows).
int kmajor(mb_ctx* ctx, const std::string& name, const float* W, int K, int N, const float* gamma,
           const void*& wk) {
  const int64_t n = (int64_t)K * N;
  float* p = internal_tensor(ctx, name, ctx->w_bf16 ? (n + 1) / 2 : n);
  if (!p) return fail(ctx, MB_ERR_NOMEM, "k-major weight allocation failed (%s)", name.c_str());
  wk = p;
  if (ctx->w_bf16) return launch_kmajor_w16(ctx, W, K, N, (uint16_t*)p);
  return launch_kmajor_w(ctx, W, K, N, gamma, p);
}

// The split-bf16 copy of a [K][N] projection for bf16-KV contexts (null in
// fp32-KV contexts): of the column-block-major Wt (launch_split_w, gamma
// already folded in where the LayerNorm is), or with bf16 weight storage
// the high halves alone (launch_split_w1) of the row-major, unscaled W.
int split(mb_ctx* ctx, const std::string& name, const float* Wt, const float* W, int K, int N,
          const void*& wx) {
  wx = nullptr;
  if (ctx->cfg.kv_dtype != MB_KV_BF16) return MB_OK;
  const int64_t n = (int64_t)K * N;  // 2 K N bf16, or K N with bf16 storage
  float* p = internal_tensor(ctx, name, ctx->w_bf16 ? (n + 1) / 2 : n);
  if (!p) return fail(ctx, MB_ERR_NOMEM, "split weight allocation failed (%s)", name.c_str());
  wx = p;
  if (ctx->w_bf16) return launch_split_w1(ctx, W, K, N, p, false);
  return launch_split_w(ctx, Wt, K, N, p);
}

// With bf16 weight storage: W <- bf16(W) in a copy of its own (the uploaded
// tensor is left as it is), from which every other copy derives.  With fp32
// storage the copy a bf16 period left behind is freed.
int round_w(mb_ctx* ctx, const std::string& name, const float*& W, int64_t n) {
  if (!ctx->w_bf16) {
    drop_internal(ctx, name);
    return MB_OK;
  }
  float* p = internal_tensor(ctx, name, n);
  if (!p) return fail(ctx, MB_ERR_NOMEM, "rounded weight allocation failed (%s)", name.c_str());
  const int rc = launch_round_bf16(ctx, W, n, p);
  W = p;
  return rc;
}

int fold_layer(mb_ctx* ctx, const std::string& key, LayerW& w) {
  int rc;
  if ((rc = round_w(ctx, key + ".attn.r", w.attn_w, (int64_t)D * QKV)) ||
      (rc = round_w(ctx, key + ".proj.r", w.proj_w, (int64_t)D * D)) ||
      (rc = round_w(ctx, key + ".fc_in.r", w.fc_in_w, (int64_t)D * FFN)) ||
      (rc = round_w(ctx, key + ".fc_out.r", w.fc_out_w, (int64_t)FFN * D)))
    return rc;
  if ((rc = fold(ctx, key + ".attn", w.attn_w, D, QKV, w.ln1_w, w.ln1_b, w.attn_wg, w.attn_c,
                 w.attn_d)))
    return rc;
  if ((rc = tile(ctx, key + ".proj.t", w.proj_w, D, D, w.proj_wt))) return rc;
  if ((rc = tile(ctx, key + ".fc_out.t", w.fc_out_w, FFN, D, w.fc_out_wt))) return rc;
  if ((rc = kmajor(ctx, key + ".attn.k", w.attn_w, D, QKV, w.ln1_w, w.attn_wk))) return rc;
  if ((rc = kmajor(ctx, key + ".fc_in.k", w.fc_in_w, D, FFN, w.ln2_w, w.fc_in_wk))) return rc;
  if ((rc = kmajor(ctx, key + ".proj.k", w.proj_w, D, D, nullptr, w.proj_wk))) return rc;
  if ((rc = kmajor(ctx, key + ".fc_out.k", w.fc_out_w, FFN, D, nullptr, w.fc_out_wk))) return rc;
  if ((rc = fold(ctx, key + ".fc_in", w.fc_in_w, D, FFN, w.ln2_w, w.ln2_b, w.fc_in_wg, w.fc_in_c,
                 w.fc_in_d)))
    return rc;
  if ((rc = split(ctx, key + ".attn.x", w.attn_wg, w.attn_w, D, QKV, w.attn_wx)) ||
      (rc = split(ctx, key + ".fc_in.x", w.fc_in_wg, w.fc_in_w, D, FFN, w.fc_in_wx)) ||
      (rc = split(ctx, key + ".proj.x", w.proj_wt, w.proj_w, D, D, w.proj_wx)))
    return rc;
  return split(ctx, key + ".fc_out.x", w.fc_out_wt, w.fc_out_w, FFN, D, w.fc_out_wx);
}

// The decode-sized projections: the GEMV kernel (k-major copy) and the
// split-bf16 kernel, in the form the context's weight storage calls for.
// `gamma` is the folded LayerNorm's (used with lnc under bf16 storage).
int proj_gemv(mb_ctx* ctx, int epi, const float* A, int64_t lda, const void* wk, int N, int K,
              const float* bias, float* C, int64_t ldc, int M, const float* lnc, const float* lnd,
              const float* gamma, const PickIn* pick = nullptr) {
  if (ctx->w_bf16)
    return launch_gemv_k16(ctx, epi, A, lda, (const uint16_t*)wk, N, K, bias, C, ldc, M, lnc, lnd,
                           lnc ? gamma : nullptr, pick);
  return launch_gemv_k(ctx, epi, A, lda, (const float*)wk, N, K, bias, C, ldc, M, lnc, lnd, pick);
}
int proj_split(mb_ctx* ctx, int epi, const float* A, int64_t lda, const void* wx, int N, int K,
               const float* bias, float* C, int64_t ldc, int M, const float* lnc, const float* lnd,
               const float* gamma) {
  if (ctx->w_bf16)
    return launch_gemm_x2(ctx, epi, A, lda, wx, N, K, bias, C, ldc, M, lnc, lnd,
                          lnc ? gamma : nullptr);
  return launch_gemm_x3(ctx, epi, A, lda, wx, N, K, bias, C, ldc, M, lnc, lnd);
}

// Resolve every weight once per upload (gpu.ts:339-343 throws "weight not
// uploaded" the same way).  `local` selects the local-head half.
int resolve(mb_ctx* ctx, bool global, bool local) {
  if (ctx->model_ok) return MB_OK;
  std::string missing;
  ModelW& m = ctx->model;
  const int64_t V = ctx->cfg.vocab;
  if (V < 10) return fail(ctx, MB_ERR_STATE, "mb_config.vocab must cover the text ids (>= 10)");
  auto get = [&](const std::string& n, std::initializer_list<int64_t> d) {
    const DeviceTensor* t = find(ctx, n, d, missing);
    return t ? (const float*)t->ptr : nullptr;
  };
  m.wte = get("core.model.transformer.wte.weight", {V, D});
  for (int k = 0; k < NVQ; k++)
    m.audio_emb.t[k] = get("core.model.audio_embeddings." + std::to_string(k) + ".weight", {CODES, D});
  if (global) {
    m.layers.assign(ctx->cfg.n_layers, LayerW{});
    for (int l = 0; l < ctx->cfg.n_layers; l++)
      resolve_layer(ctx, "core.model.transformer.h." + std::to_string(l) + ".", m.layers[l], missing);
    m.lnf_w = get("core.model.transformer.ln_f.weight", {D});
    m.lnf_b = get("core.model.transformer.ln_f.bias", {D});
  }
  if (local) {
    resolve_layer(ctx, "model.local_transformer.h.0.", m.local, missing);
    m.local_lnf_w = get("model.local_transformer.ln_f.weight", {D});
    m.local_lnf_b = get("model.local_transformer.ln_f.bias", {D});
    m.text_head = get("model.text_lm_head.weight", {D, V});
    for (int k = 0; k < NVQ; k++)
      m.audio_heads.t[k] = get("model.audio_lm_heads." + std::to_string(k) + ".weight", {D, CODES});
  }
  if (!missing.empty()) return fail(ctx, MB_ERR_STATE, "%s", missing.c_str());
  if (global && local) {
    int rc;
    for (size_t l = 0; l < m.layers.size(); l++)
      if ((rc = fold_layer(ctx, "#fold/h" + std::to_string(l), m.layers[l]))) return rc;
    if ((rc = fold_layer(ctx, "#fold/local", m.local))) return rc;
    for (int k = 0; k < NVQ; k++) {
      const std::string p = "#fold/head" + std::to_string(k);
      if ((rc = round_w(ctx, p + ".r", m.audio_heads.t[k], (int64_t)D * CODES)) ||
          (rc = fold(ctx, p, m.audio_heads.t[k], D, CODES, m.local_lnf_w, m.local_lnf_b,
                     m.head_wg.t[k], m.head_c.t[k], m.head_d.t[k])) ||
          (rc = kmajor(ctx, p + ".k", m.audio_heads.t[k], D, CODES, m.local_lnf_w, m.head_wk[k])) ||
          (rc = split(ctx, p + ".x", m.head_wg.t[k], m.audio_heads.t[k], D, CODES, m.head_wx[k])))
        return rc;
    }
    ctx->model_ok = true;
  }
  return MB_OK;
}

int need_model(mb_ctx* ctx) {
  if (ctx->model_ok) return MB_OK;
  return resolve(ctx, true, true);
}

struct Act {
  float *x, *norm, *qkv, *q, *att, *ffn, *logits;
};

int activations(mb_ctx* ctx, int64_t M, Act& a) {
  a.x = (float*)scratch(ctx, "act_x", (size_t)M * D * 4);
  a.norm = (float*)scratch(ctx, "act_norm", (size_t)M * D * 4);
  a.qkv = (float*)scratch(ctx, "act_qkv", (size_t)M * QKV * 4);
  a.q = (float*)scratch(ctx, "act_q", (size_t)M * D * 4);
  a.att = (float*)scratch(ctx, "act_att", (size_t)M * D * 4);
  a.ffn = (float*)scratch(ctx, "act_ffn", (size_t)M * FFN * 4);
  a.logits = (float*)scratch(ctx, "act_logits", (size_t)M * CODES * 4);
  if (!a.x || !a.norm || !a.qkv || !a.q || !a.att || !a.ffn || !a.logits)
    return fail(ctx, MB_ERR_NOMEM, "activation allocation failed (%lld rows)", (long long)M);
  return MB_OK;
}

int cancelled(mb_ctx* ctx) {
  if (ctx->cancel.load()) return fail(ctx, MB_ERR_CANCELLED, "cancelled");
  return MB_OK;
}

// One d=768 layer over M rows held in a.x.  Rows belong to B sequences with
// n_rows[b] rows at positions pos0[b] + r (packed by `packed` when prefill is
// set, else one row per sequence).  With `pick` (one row) the QKV projection
// makes the previous channel's code choice and writes a.x itself.
int run_layer(mb_ctx* ctx, const LayerW& w, const RingView& ring, int B, int rows_max, int64_t M,
              const int32_t* pos0, const int32_t* n_rows, const int32_t* row_off, bool prefill,
              int64_t max_valid, Act& a, int pos_const = -1, const PickIn* pick = nullptr) {
  int rc;
  // decode-sized M: each LayerNorm is folded into the projection after it;
  // up to kGemvMaxM rows the projections read the k-major copies
  const bool folded = M < kFoldMaxM;
  const bool gemv = M <= kGemvMaxM;
  // bf16-KV contexts: every projection above kGemvMaxM rows as split-bf16
  // products, the LayerNorm folded in (the streaming kernel at decode sizes,
  // the tiled one at prefill sizes)
  const bool x3 = !gemv && w.attn_wx;
  if (pick && !(gemv && M == 1))
    return fail(ctx, MB_ERR_STATE, "the code choice rides on a one-row projection (M %lld)",
                (long long)M);
  if (gemv) {
    if ((rc = proj_gemv(ctx, EPI_STORE, a.x, D, w.attn_wk, QKV, D, w.attn_b, a.qkv, QKV,
                        (int)M, w.attn_c, w.attn_d, w.ln1_w, pick)))
      return rc;
  } else if (x3) {
    if ((rc = proj_split(ctx, EPI_STORE, a.x, D, w.attn_wx, QKV, D, w.attn_b, a.qkv, QKV,
                         (int)M, w.attn_c, w.attn_d, w.ln1_w)))
      return rc;
  } else if (folded) {
    if ((rc = launch_gemm_ln(ctx, EPI_STORE, a.x, D, w.attn_wg, QKV, D, w.attn_c, w.attn_d,
                             w.attn_b, a.qkv, QKV, (int)M)))
      return rc;
  } else {
    if ((rc = launch_layernorm(ctx, a.x, D, nullptr, (int)M, w.ln1_w, w.ln1_b, a.norm, D))) return rc;
    if ((rc = launch_gemm(ctx, EPI_STORE, a.norm, D, w.attn_w, QKV, D, w.attn_b, a.qkv, QKV, (int)M)))
      return rc;
  }
  // The decode step of up to kPartsMaxSeqs sequences with bf16 weights (the
  // global layers; the local head's attention is k_attn_short): the
  // attention as per-wave partials merged by the O projection.
  const bool parts = !prefill && gemv && ctx->w_bf16 && pos_const < 0 && B <= kPartsMaxSeqs &&
                     ring.heads == H && ring.window == ring.C;
  float* part = nullptr;
  int nwp = 0;
  if (parts) {
    part = (float*)scratch(ctx, "attn_parts", (size_t)B * H * 16 * PART * sizeof(float));
    if (!part) return fail(ctx, MB_ERR_NOMEM, "attention partials");
  }
  Rows qkv_rows, q_rows;
  if (prefill) {
    qkv_rows.row_stride = QKV;
    qkv_rows.row_off = row_off;
    q_rows.row_stride = D;
    q_rows.row_off = row_off;
  } else {
    qkv_rows = dense_rows(QKV, 1);
    q_rows = dense_rows(D, 1);
  }
  if (prefill) {
    if ((rc = launch_ring_write(ctx, ring, B, rows_max, a.qkv, MB_DT_F32, qkv_rows, pos0, n_rows,
                                a.q, MB_DT_F32, q_rows)))
      return rc;
    rc = launch_prefill_attention(ctx, ring, B, rows_max, a.q, MB_DT_F32, q_rows, pos0, n_rows,
                                  a.att, q_rows);
  } else if (parts) {
    // a few sequences: the attention's waves spread over one-wave blocks and
    // leave their partial states, which the O projection merges as it reads
    rc = launch_append_attn_parts(ctx, ring, B, a.qkv, pos0, max_valid, part, nwp);
  } else {
    // one launch appends this row's K/V and attends the ring including it
    rc = launch_append_attn(ctx, ring, B, a.qkv, MB_DT_F32, qkv_rows, pos0, max_valid, nullptr,
                            Rows{}, a.att, q_rows, pos_const);
  }
  if (rc) return rc;
  // decode sizes read the column-block-major copies of O and fc_out
  const bool tiled = gemm_streams((int)M, D);
  if ((rc = parts ? launch_gemv_k_parts(ctx, EPI_ADD, part, nwp, (const uint16_t*)w.proj_wk, D,
                                        w.proj_b, a.x, D, (int)M)
           : gemv ? proj_gemv(ctx, EPI_ADD, a.att, D, w.proj_wk, D, D, w.proj_b, a.x, D, (int)M,
                             nullptr, nullptr, nullptr)
           : x3 ? proj_split(ctx, EPI_ADD, a.att, D, w.proj_wx, D, D, w.proj_b, a.x, D, (int)M,
                             nullptr, nullptr, nullptr)
                : launch_gemm(ctx, EPI_ADD, a.att, D, tiled ? w.proj_wt : w.proj_w, D, D, w.proj_b,
                              a.x, D, (int)M, tiled)))
    return rc;
  if (gemv) {
    if ((rc = proj_gemv(ctx, EPI_GELU, a.x, D, w.fc_in_wk, FFN, D, w.fc_in_b, a.ffn, FFN,
                        (int)M, w.fc_in_c, w.fc_in_d, w.ln2_w)))
      return rc;
  } else if (x3) {
    if ((rc = proj_split(ctx, EPI_GELU, a.x, D, w.fc_in_wx, FFN, D, w.fc_in_b, a.ffn, FFN,
                         (int)M, w.fc_in_c, w.fc_in_d, w.ln2_w)))
      return rc;
  } else if (folded) {
    if ((rc = launch_gemm_ln(ctx, EPI_GELU, a.x, D, w.fc_in_wg, FFN, D, w.fc_in_c, w.fc_in_d,
                             w.fc_in_b, a.ffn, FFN, (int)M)))
      return rc;
  } else {
    if ((rc = launch_layernorm(ctx, a.x, D, nullptr, (int)M, w.ln2_w, w.ln2_b, a.norm, D))) return rc;
    if ((rc = launch_gemm(ctx, EPI_GELU, a.norm, D, w.fc_in_w, FFN, D, w.fc_in_b, a.ffn, FFN, (int)M)))
      return rc;
  }
  if (gemv)
    return proj_gemv(ctx, EPI_ADD, a.ffn, FFN, w.fc_out_wk, D, FFN, w.fc_out_b, a.x, D, (int)M,
                     nullptr, nullptr, nullptr);
  if (x3)
    return proj_split(ctx, EPI_ADD, a.ffn, FFN, w.fc_out_wx, D, FFN, w.fc_out_b, a.x, D, (int)M,
                      nullptr, nullptr, nullptr);
  return launch_gemm(ctx, EPI_ADD, a.ffn, FFN, tiled ? w.fc_out_wt : w.fc_out_w, D, FFN, w.fc_out_b,
                     a.x, D, (int)M, tiled);
}

// Local-head state, allocated on first use: every local slot empty, seen
// masks clear, local positions [17][max_seqs] = step.
int local_state(mb_ctx* ctx) {
  if (ctx->local_k) return MB_OK;
  const int64_t S = ctx->cfg.max_seqs;
  const size_t kv = (size_t)S * H * ROW * HD * 4;
  MB_HIP(ctx, hipMalloc(&ctx->local_k, kv));
  MB_HIP(ctx, hipMalloc(&ctx->local_v, kv));
  MB_HIP(ctx, hipMalloc(&ctx->local_sp, (size_t)S * ROW * 4));
  MB_HIP(ctx, hipMalloc(&ctx->local_pos, (size_t)S * ROW * 4));
  MB_HIP(ctx, hipMalloc(&ctx->seen, (size_t)S * NVQ * 32 * 4));
  MB_HIP(ctx, hipMalloc(&ctx->tokens, (size_t)S * NVQ * 4));
  MB_HIP(ctx, hipMalloc(&ctx->cont, (size_t)S * 4));
  ctx->device_bytes += (int64_t)(2 * kv + S * ROW * 8 + S * NVQ * 32 * 4 + S * NVQ * 4 + S * 4);
  ctx->graph_gen++;
  int rc;
  // the local cache is fp32 whatever the global rings hold: clear it as words
  if ((rc = launch_fill_i32(ctx, (int32_t*)ctx->local_k, (int64_t)kv / 4, 0))) return rc;
  if ((rc = launch_fill_i32(ctx, (int32_t*)ctx->local_v, (int64_t)kv / 4, 0))) return rc;
  if ((rc = launch_fill_i32(ctx, ctx->local_sp, S * ROW, -1))) return rc;
  for (int s = 0; s < ROW; s++)
    if ((rc = launch_fill_i32(ctx, ctx->local_pos + (int64_t)s * S, S, s))) return rc;
  if ((rc = launch_fill_i32(ctx, (int32_t*)ctx->seen, S * NVQ * 32, 0))) return rc;
  if ((rc = launch_fill_i32(ctx, ctx->tokens, S * NVQ, 0))) return rc;
  return launch_fill_i32(ctx, ctx->cont, S, 0);
}

RingView local_ring(mb_ctx* ctx) {
  RingView v;
  v.k = ctx->local_k;
  v.v = ctx->local_v;
  v.sp = ctx->local_sp;
  v.seq_stride = (int64_t)H * ROW * HD;
  v.C = ROW;
  v.window = ROW;
  v.wrap = 0;
  v.bf16 = false;
  return v;
}

int check_ids(mb_ctx* ctx, const int32_t* ids, int64_t rows) {
  for (int64_t r = 0; r < rows; r++) {
    const int32_t* id = ids + r * ROW;
    if (id[0] < 0 || id[0] >= ctx->cfg.vocab)
      return fail(ctx, MB_ERR_ARG, "row %lld: text id %d outside [0, %d)", (long long)r, id[0],
                  ctx->cfg.vocab);
    for (int k = 1; k < ROW; k++)
      if (id[k] < 0 || id[k] > PAD)
        return fail(ctx, MB_ERR_ARG, "row %lld: audio id %d outside [0, 1024]", (long long)r, id[k]);
  }
  return MB_OK;
}

// Global decode step on device buffers (rows17, pos, hidden all device);
// with rows17 null the rows are the frame rows of the codes in ctx->tokens.
int decode_step(mb_ctx* ctx, int B, const int32_t* rows17, const int32_t* pos, int64_t max_pos,
                float* hidden) {
  int rc;
  Act a;
  if ((rc = activations(ctx, B, a))) return rc;
  const ModelW& m = ctx->model;
  if ((rc = launch_embed_rows(ctx, rows17, B, m.wte, ctx->cfg.vocab, m.audio_emb, a.x,
                              rows17 ? nullptr : ctx->tokens, ctx->assistant_id)))
    return rc;
  for (int l = 0; l < ctx->cfg.n_layers; l++) {
    if ((rc = cancelled(ctx))) return rc;
    if ((rc = run_layer(ctx, m.layers[l], global_ring(ctx, l), B, 1, B, pos, nullptr, nullptr, false,
                        max_pos + 1, a)))
      return rc;
  }
  return launch_layernorm(ctx, a.x, D, nullptr, B, m.lnf_w, m.lnf_b, hidden, D);
}

// What a teacher-forced run of the local head (mb_local_logits) reads and
// writes: the codes fed to steps 2..16 ([B][16]), and where the text
// decision's two dot products ([B][2]) and every channel's audio-head logits
// ([B][16][1024]) go.
struct LogitsProbe {
  const int32_t* forced = nullptr;
  double* text2 = nullptr;
  float* logits = nullptr;
  int32_t* cont = nullptr;  // the decision's flag (not the context's)
};

// Local-head steps 0 .. last_step on device buffers.  With `pick` each step
// ends in its greedy choice (the text decision at step 0, a code per channel
// after it); without it the steps only run the layer and ln_f, embedding the
// codes already held in ctx->tokens, and the last step's ln_f output is left in
// a.norm (DecodeRunner.nextFrameSteps, decode.ts:970-1030).  With `probe`
// (no pick) the steps embed probe->forced instead and end in the same heads
// the picking frame evaluates, written to the probe's outputs.
int local_steps(mb_ctx* ctx, int B, const float* hidden, int last_step, bool pick, Act& a,
                const LogitsProbe* probe = nullptr) {
  int rc;
  if ((rc = local_state(ctx))) return rc;
  if ((rc = activations(ctx, B, a))) return rc;
  const ModelW& m = ctx->model;
  const RingView ring = local_ring(ctx);
  const int64_t S = ctx->cfg.max_seqs;
  const bool heads = pick || probe;
  // One voice: the code choice of every channel but the last is made by the
  // next step's QKV projection (PickIn), not by a launch of its own; the
  // last channel's argmax launch records them all in the seen sets.
  const bool fuse = pick && B == 1;
  PickIn pending{};
  bool have_pending = false;
  for (int step = 0; step <= last_step; step++) {
    if ((rc = cancelled(ctx))) return rc;
    // picking, the previous step's decision kernel already wrote this step's
    // input row (wte[assistant_id], then the previous channel's code)
    if (step == 0)
      MB_HIP(ctx, hipMemcpyAsync(a.x, hidden, (size_t)B * D * 4, hipMemcpyDeviceToDevice, ctx->stream));
    else if (!pick && (rc = launch_embed_local(ctx, step, B, m.wte, ctx->assistant_id,
                                               m.audio_emb, probe ? probe->forced : ctx->tokens,
                                               a.x)))
      return rc;
    // (every voice's local step sits at position `step`)
    if ((rc = run_layer(ctx, m.local, ring, B, 1, B, ctx->local_pos + (int64_t)step * S, nullptr,
                        nullptr, false, step + 1, a, step, have_pending ? &pending : nullptr)))
      return rc;
    have_pending = false;
    // the audio heads take ln_f folded in (decode-sized B); the text decision
    // and the step probe read ln_f itself
    const bool folded_head = heads && step > 0 && B < kFoldMaxM;
    if (!folded_head &&
        (rc = launch_layernorm(ctx, a.x, D, nullptr, B, m.local_lnf_w, m.local_lnf_b, a.norm, D)))
      return rc;
    if (!heads) continue;
    const bool embed_next = pick && step < last_step;
    if (step == 0) {
      rc = launch_text_decide(ctx, a.norm, B, m.text_head, ctx->cfg.vocab, ctx->end_id,
                              ctx->assistant_id, pick ? ctx->frame_alive : nullptr,
                              pick ? ctx->cont : probe->cont, m.wte, embed_next ? a.x : nullptr,
                              probe ? probe->text2 : nullptr);
    } else {
      const int ch = step - 1;
      float* lg = pick ? a.logits : probe->logits + (int64_t)ch * CODES;
      const int64_t ldl = pick ? CODES : (int64_t)NVQ * CODES;
      if (folded_head && B <= kGemvMaxM)
        rc = proj_gemv(ctx, EPI_STORE, a.x, D, m.head_wk[ch], CODES, D, nullptr, lg, ldl, B,
                       m.head_c.t[ch], m.head_d.t[ch], m.local_lnf_w);
      else if (folded_head && m.head_wx[ch] && gemm_streams(B, CODES))
        rc = proj_split(ctx, EPI_STORE, a.x, D, m.head_wx[ch], CODES, D, nullptr, lg, ldl, B,
                        m.head_c.t[ch], m.head_d.t[ch], m.local_lnf_w);
      else if (folded_head)
        rc = launch_gemm_ln(ctx, EPI_STORE, a.x, D, m.head_wg.t[ch], CODES, D, m.head_c.t[ch],
                            m.head_d.t[ch], nullptr, lg, ldl, B);
      else
        rc = launch_gemm(ctx, EPI_STORE, a.norm, D, m.audio_heads.t[ch], CODES, D, nullptr, lg, ldl,
                         B);
      if (rc) return rc;
      if (pick && fuse && embed_next) {
        pending = PickIn{a.logits, ctx->seen, ctx->tokens, m.audio_emb.t[ch], a.x, ctx->penalty,
                         ch, (int)ctx->penalty_f32};
        have_pending = true;
      } else if (pick) {
        rc = launch_argmax_penalty(ctx, a.logits, B, ch, fuse ? 0 : ch, ctx->penalty,
                                   ctx->penalty_f32, ctx->seen, ctx->cont, ctx->tokens,
                                   embed_next ? m.audio_emb.t[ch] : nullptr,
                                   embed_next ? a.x : nullptr);
      }
    }
    if (rc) return rc;
  }
  return MB_OK;
}

// The 17-step local head on device buffers; codes/cont/rows17_out optional.
int local_frame(mb_ctx* ctx, int B, const float* hidden, int32_t* codes, int32_t* cont,
                int32_t* rows17_out) {
  Act a;
  int rc = local_steps(ctx, B, hidden, ROW - 1, true, a);
  if (rc) return rc;
  if (codes)
    MB_HIP(ctx, hipMemcpyAsync(codes, ctx->tokens, (size_t)B * NVQ * 4, hipMemcpyDeviceToDevice,
                               ctx->stream));
  if (cont)
    MB_HIP(ctx, hipMemcpyAsync(cont, ctx->cont, (size_t)B * 4, hipMemcpyDeviceToDevice, ctx->stream));
  if (rows17_out) return launch_frame_rows(ctx, ctx->tokens, B, ctx->assistant_id, rows17_out);
  return MB_OK;
}

int check_b(mb_ctx* ctx, int B) {
  if (!ctx) return MB_ERR_ARG;
  if (B < 0 || B > ctx->cfg.max_seqs)
    return fail(ctx, MB_ERR_ARG, "B %d out of [0, %d]", B, ctx->cfg.max_seqs);
  return MB_OK;
}

}  // namespace

}  // namespace mb

using namespace mb;

extern "C" {

int mb_set_local_head(mb_ctx* ctx, int32_t audio_end_id, int32_t assistant_id, double penalty) {
  if (!ctx) return MB_ERR_ARG;
  if (audio_end_id < 0 || assistant_id < 0 || audio_end_id >= ctx->cfg.vocab ||
      assistant_id >= ctx->cfg.vocab || !(penalty > 0.0) || !(penalty < INFINITY))
    return fail(ctx, MB_ERR_ARG, "local head settings out of range");
  // the captured frame graph holds these values as kernel arguments
  if (audio_end_id != ctx->end_id || assistant_id != ctx->assistant_id || penalty != ctx->penalty)
    ctx->graph_gen++;
  ctx->end_id = audio_end_id;
  ctx->assistant_id = assistant_id;
  ctx->penalty = penalty;
  return MB_OK;
}

int mb_set_penalty_precision(mb_ctx* ctx, int32_t precision) {
  if (!ctx) return MB_ERR_ARG;
  if (precision != MB_PENALTY_F64 && precision != MB_PENALTY_F32)
    return fail(ctx, MB_ERR_ARG, "penalty precision must be MB_PENALTY_F64 or MB_PENALTY_F32");
  const bool f32 = precision == MB_PENALTY_F32;
  if (f32 != ctx->penalty_f32) ctx->graph_gen++;  // a kernel argument of the frame graph
  ctx->penalty_f32 = f32;
  return MB_OK;
}

int mb_set_weight_storage(mb_ctx* ctx, int32_t storage) {
  if (!ctx) return MB_ERR_ARG;
  if (storage != MB_W_F32 && storage != MB_W_BF16)
    return fail(ctx, MB_ERR_ARG, "weight storage must be MB_W_F32 or MB_W_BF16");
  const bool bf16 = storage == MB_W_BF16;
  if (bf16 != ctx->w_bf16) {
    ctx->w_bf16 = bf16;
    ctx->model_ok = false;  // the copies are derived again, from the uploads
    ctx->graph_gen++;
  }
  return MB_OK;
}

int mb_clear_seen(mb_ctx* ctx, int n, const int32_t* seq_ids) {
  MB_DEVICE_GUARD(ctx);
  int rc = check_b(ctx, 0);
  if (rc) return rc;
  if ((rc = local_state(ctx))) return rc;
  if (n < 0) {
    rc = launch_fill_i32(ctx, (int32_t*)ctx->seen, (int64_t)ctx->cfg.max_seqs * NVQ * 32, 0);
    if (rc) return rc;
  } else {
    if (n > 0 && !seq_ids) return fail(ctx, MB_ERR_ARG, "mb_clear_seen: seq_ids is null");
    for (int i = 0; i < n; i++) {
      if (seq_ids[i] < 0 || seq_ids[i] >= ctx->cfg.max_seqs)
        return fail(ctx, MB_ERR_ARG, "mb_clear_seen: sequence %d out of range", seq_ids[i]);
      rc = launch_fill_i32(ctx, (int32_t*)ctx->seen + (int64_t)seq_ids[i] * NVQ * 32, NVQ * 32, 0);
      if (rc) return rc;
    }
  }
  MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return MB_OK;
}

}  // extern "C"

namespace mb {
namespace {

// Global prefill through the first `layer_count` layers; ln_f of each
// sequence's last row goes to last_hidden [B][768] and, when all_hidden is
// set, ln_f of every row to all_hidden[B][rows_max][768] (rows past n_rows[b]
// are zeroed).
int prefill(mb_ctx* ctx, int B, int rows_max, const int32_t* ids, const int32_t* n_rows,
            int layer_count, float* last_hidden, float* all_hidden) {
  int rc = check_b(ctx, B);
  if (rc) return rc;
  if (B == 0) return MB_OK;
  if (layer_count < 1 || layer_count > ctx->cfg.n_layers)
    return fail(ctx, MB_ERR_ARG, "layer_count %d out of [1, %d]", layer_count, ctx->cfg.n_layers);
  if (!ids || !n_rows || (!last_hidden && !all_hidden)) return fail(ctx, MB_ERR_ARG, "null pointer");
  if (rows_max < 1 || rows_max > ctx->cfg.max_rows)
    return fail(ctx, MB_ERR_ARG, "rows_max %d out of [1, %d]", rows_max, ctx->cfg.max_rows);
  if ((rc = need_model(ctx))) return rc;
  std::vector<int32_t> off(B), last(B), zeros(B, 0);
  int64_t M = 0;
  for (int b = 0; b < B; b++) {
    if (n_rows[b] < 1 || n_rows[b] > rows_max)
      return fail(ctx, MB_ERR_ARG, "prefill called with %d rows for sequence %d", n_rows[b], b);
    if (n_rows[b] > ctx->cfg.capacity)
      return fail(ctx, MB_ERR_RANGE, "prompt of %d rows exceeds the KV ring (%d slots)", n_rows[b],
                  ctx->cfg.capacity);
    off[b] = (int32_t)M;
    M += n_rows[b];
    last[b] = (int32_t)(M - 1);
  }
  std::vector<int32_t> packed((size_t)M * ROW);
  for (int b = 0; b < B; b++)
    memcpy(packed.data() + (size_t)off[b] * ROW, ids + (size_t)b * rows_max * ROW,
           (size_t)n_rows[b] * ROW * 4);
  if ((rc = check_ids(ctx, packed.data(), M))) return rc;
  Act a;
  if ((rc = activations(ctx, M, a))) return rc;
  int32_t* d_ids = (int32_t*)scratch(ctx, "prefill_ids", (size_t)M * ROW * 4);
  int32_t* d_meta = (int32_t*)scratch(ctx, "prefill_meta", (size_t)B * 4 * 4);
  float* d_hidden = (float*)scratch(ctx, "hidden", (size_t)B * D * 4);
  if (!d_ids || !d_meta || !d_hidden) return fail(ctx, MB_ERR_NOMEM, "staging allocation failed");
  int32_t* d_off = d_meta;
  int32_t* d_n = d_meta + B;
  int32_t* d_pos0 = d_meta + 2 * B;
  int32_t* d_last = d_meta + 3 * B;
  MB_HIP(ctx, hipMemcpyAsync(d_ids, packed.data(), (size_t)M * ROW * 4, hipMemcpyHostToDevice, ctx->stream));
  MB_HIP(ctx, hipMemcpyAsync(d_off, off.data(), (size_t)B * 4, hipMemcpyHostToDevice, ctx->stream));
  MB_HIP(ctx, hipMemcpyAsync(d_n, n_rows, (size_t)B * 4, hipMemcpyHostToDevice, ctx->stream));
  MB_HIP(ctx, hipMemcpyAsync(d_pos0, zeros.data(), (size_t)B * 4, hipMemcpyHostToDevice, ctx->stream));
  MB_HIP(ctx, hipMemcpyAsync(d_last, last.data(), (size_t)B * 4, hipMemcpyHostToDevice, ctx->stream));
  // a fresh utterance per sequence: every slot of its rings forgets its position
  for (int l = 0; l < ctx->cfg.n_layers; l++)
    if ((rc = launch_fill_i32(ctx, ctx->slot_pos + slot_base(ctx, l, 0), (int64_t)B * ctx->cfg.capacity, -1)))
      return rc;
  const ModelW& m = ctx->model;
  if ((rc = launch_embed_rows(ctx, d_ids, (int)M, m.wte, ctx->cfg.vocab, m.audio_emb, a.x))) return rc;
  for (int l = 0; l < layer_count; l++) {
    if ((rc = cancelled(ctx))) return rc;
    if ((rc = run_layer(ctx, m.layers[l], global_ring(ctx, l), B, rows_max, M, d_pos0, d_n, d_off,
                        true, ctx->cfg.capacity, a)))
      return rc;
  }
  if (last_hidden) {
    if ((rc = launch_layernorm(ctx, a.x, D, d_last, B, m.lnf_w, m.lnf_b, d_hidden, D))) return rc;
    MB_HIP(ctx, hipMemcpyAsync(last_hidden, d_hidden, (size_t)B * D * 4, hipMemcpyDeviceToHost,
                               ctx->stream));
  }
  std::vector<float> rows;
  if (all_hidden) {
    if ((rc = launch_layernorm(ctx, a.x, D, nullptr, (int)M, m.lnf_w, m.lnf_b, a.norm, D))) return rc;
    rows.resize((size_t)M * D);
    MB_HIP(ctx, hipMemcpyAsync(rows.data(), a.norm, rows.size() * 4, hipMemcpyDeviceToHost,
                               ctx->stream));
  }
  MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
  if (all_hidden) {
    memset(all_hidden, 0, (size_t)B * rows_max * D * 4);
    for (int b = 0; b < B; b++)
      memcpy(all_hidden + (size_t)b * rows_max * D, rows.data() + (size_t)off[b] * D,
             (size_t)n_rows[b] * D * 4);
  }
  return MB_OK;
}

}  // namespace
}  // namespace mb

extern "C" {

int mb_prefill(mb_ctx* ctx, int B, int rows_max, const int32_t* ids, const int32_t* n_rows,
               float* last_hidden) {
  MB_DEVICE_GUARD(ctx);
  if (ctx && !last_hidden) return fail(ctx, MB_ERR_ARG, "null pointer");
  return prefill(ctx, B, rows_max, ids, n_rows, ctx ? ctx->cfg.n_layers : 0, last_hidden, nullptr);
}

int mb_prefill_rows(mb_ctx* ctx, int B, int rows_max, const int32_t* ids, const int32_t* n_rows,
                    int layer_count, float* hidden) {
  MB_DEVICE_GUARD(ctx);
  if (ctx && !hidden) return fail(ctx, MB_ERR_ARG, "null pointer");
  if (ctx && layer_count <= 0) layer_count = ctx->cfg.n_layers;
  return prefill(ctx, B, rows_max, ids, n_rows, layer_count, nullptr, hidden);
}

int mb_decode_step(mb_ctx* ctx, int B, const int32_t* rows17, const int32_t* pos, float* hidden) {
  MB_DEVICE_GUARD(ctx);
  int rc = check_b(ctx, B);
  if (rc) return rc;
  if (B == 0) return MB_OK;
  if (!rows17 || !pos || !hidden) return fail(ctx, MB_ERR_ARG, "null pointer");
  if ((rc = need_model(ctx))) return rc;
  if ((rc = check_ids(ctx, rows17, B))) return rc;
  int64_t max_pos = 0;
  for (int b = 0; b < B; b++) {
    if (pos[b] < 0) return fail(ctx, MB_ERR_ARG, "sequence %d: negative position %d", b, pos[b]);
    if (!ctx->cfg.wrap && pos[b] >= ctx->cfg.capacity)
      return fail(ctx, MB_ERR_RANGE,
                  "decode position %d exceeds the KV ring (%d slots); it must be sized "
                  "prefill_rows + max_new_frames",
                  pos[b], ctx->cfg.capacity);
    if (pos[b] > max_pos) max_pos = pos[b];
  }
  int32_t* d_rows = (int32_t*)scratch(ctx, "step_rows", (size_t)B * ROW * 4);
  int32_t* d_pos = (int32_t*)scratch(ctx, "step_pos", (size_t)B * 4);
  float* d_hidden = (float*)scratch(ctx, "hidden", (size_t)B * D * 4);
  if (!d_rows || !d_pos || !d_hidden) return fail(ctx, MB_ERR_NOMEM, "staging allocation failed");
  MB_HIP(ctx, hipMemcpyAsync(d_rows, rows17, (size_t)B * ROW * 4, hipMemcpyHostToDevice, ctx->stream));
  MB_HIP(ctx, hipMemcpyAsync(d_pos, pos, (size_t)B * 4, hipMemcpyHostToDevice, ctx->stream));
  if ((rc = decode_step(ctx, B, d_rows, d_pos, max_pos, d_hidden))) return rc;
  MB_HIP(ctx, hipMemcpyAsync(hidden, d_hidden, (size_t)B * D * 4, hipMemcpyDeviceToHost, ctx->stream));
  MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return MB_OK;
}

int mb_local_frame(mb_ctx* ctx, int B, const float* hidden, int32_t* codes, int32_t* cont) {
  MB_DEVICE_GUARD(ctx);
  int rc = check_b(ctx, B);
  if (rc) return rc;
  if (B == 0) return MB_OK;
  if (!hidden || !codes || !cont) return fail(ctx, MB_ERR_ARG, "null pointer");
  if ((rc = need_model(ctx))) return rc;
  float* d_hidden = (float*)scratch(ctx, "hidden", (size_t)B * D * 4);
  int32_t* d_out = (int32_t*)scratch(ctx, "frame_out", (size_t)B * (NVQ + 1) * 4);
  if (!d_hidden || !d_out) return fail(ctx, MB_ERR_NOMEM, "staging allocation failed");
  MB_HIP(ctx, hipMemcpyAsync(d_hidden, hidden, (size_t)B * D * 4, hipMemcpyHostToDevice, ctx->stream));
  if ((rc = local_frame(ctx, B, d_hidden, d_out, d_out + (size_t)B * NVQ, nullptr))) return rc;
  MB_HIP(ctx, hipMemcpyAsync(codes, d_out, (size_t)B * NVQ * 4, hipMemcpyDeviceToHost, ctx->stream));
  MB_HIP(ctx, hipMemcpyAsync(cont, d_out + (size_t)B * NVQ, (size_t)B * 4, hipMemcpyDeviceToHost, ctx->stream));
  MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return MB_OK;
}

int mb_local_steps(mb_ctx* ctx, int B, const float* hidden, int max_step, float* out) {
  MB_DEVICE_GUARD(ctx);
  int rc = check_b(ctx, B);
  if (rc) return rc;
  if (B == 0) return MB_OK;
  if (!hidden || !out) return fail(ctx, MB_ERR_ARG, "null pointer");
  if (max_step < 0 || max_step >= ROW)
    return fail(ctx, MB_ERR_ARG, "max_step %d out of [0, %d)", max_step, ROW);
  if ((rc = need_model(ctx))) return rc;
  float* d_hidden = (float*)scratch(ctx, "hidden", (size_t)B * D * 4);
  if (!d_hidden) return fail(ctx, MB_ERR_NOMEM, "staging allocation failed");
  MB_HIP(ctx, hipMemcpyAsync(d_hidden, hidden, (size_t)B * D * 4, hipMemcpyHostToDevice, ctx->stream));
  Act a;
  if ((rc = local_steps(ctx, B, d_hidden, max_step, false, a))) return rc;
  MB_HIP(ctx, hipMemcpyAsync(out, a.norm, (size_t)B * D * 4, hipMemcpyDeviceToHost, ctx->stream));
  MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return MB_OK;
}

int mb_local_logits(mb_ctx* ctx, int B, const float* hidden, const int32_t* codes, double* text2,
                    float* logits) {
  MB_DEVICE_GUARD(ctx);
  int rc = check_b(ctx, B);
  if (rc) return rc;
  if (B == 0) return MB_OK;
  if (!hidden || !codes || !text2 || !logits) return fail(ctx, MB_ERR_ARG, "null pointer");
  for (int64_t i = 0; i < (int64_t)B * NVQ; i++)
    if (codes[i] < 0 || codes[i] >= CODES)
      return fail(ctx, MB_ERR_ARG, "code %d outside [0, %d)", codes[i], CODES);
  if ((rc = need_model(ctx))) return rc;
  float* d_hidden = (float*)scratch(ctx, "hidden", (size_t)B * D * 4);
  int32_t* d_codes = (int32_t*)scratch(ctx, "probe_codes", (size_t)B * (NVQ + 1) * 4);
  double* d_text = (double*)scratch(ctx, "probe_text", (size_t)B * 2 * 8);
  float* d_logits = (float*)scratch(ctx, "probe_logits", (size_t)B * NVQ * CODES * 4);
  if (!d_hidden || !d_codes || !d_text || !d_logits)
    return fail(ctx, MB_ERR_NOMEM, "staging allocation failed");
  MB_HIP(ctx, hipMemcpyAsync(d_hidden, hidden, (size_t)B * D * 4, hipMemcpyHostToDevice, ctx->stream));
  MB_HIP(ctx, hipMemcpyAsync(d_codes, codes, (size_t)B * NVQ * 4, hipMemcpyHostToDevice, ctx->stream));
  LogitsProbe probe;
  probe.forced = d_codes;
  probe.cont = d_codes + (int64_t)B * NVQ;
  probe.text2 = d_text;
  probe.logits = d_logits;
  Act a;
  if ((rc = local_steps(ctx, B, d_hidden, ROW - 1, false, a, &probe))) return rc;
  MB_HIP(ctx, hipMemcpyAsync(text2, d_text, (size_t)B * 2 * 8, hipMemcpyDeviceToHost, ctx->stream));
  MB_HIP(ctx, hipMemcpyAsync(logits, d_logits, (size_t)B * NVQ * CODES * 4, hipMemcpyDeviceToHost,
                             ctx->stream));
  MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return MB_OK;
}

int mb_decode_step_dev(mb_ctx* ctx, int B, const int32_t* rows17, const int32_t* pos,
                       int32_t max_pos, float* hidden) {
  MB_DEVICE_GUARD(ctx);
  int rc = check_b(ctx, B);
  if (rc) return rc;
  if (B == 0) return MB_OK;
  if (!rows17 || !pos || !hidden) return fail(ctx, MB_ERR_ARG, "null pointer");
  if (max_pos < 0) return fail(ctx, MB_ERR_ARG, "max_pos %d is negative", max_pos);
  if ((rc = need_model(ctx))) return rc;
  return decode_step(ctx, B, rows17, pos, max_pos, hidden);
}

}  // extern "C"

namespace mb {
namespace {

// One device-resident frame: local head on `hidden` -> codes, global decode
// step of their frame rows (embedded from the codes) at pos -> `hidden`,
// then the frame's codes and flags to the outputs and pos += cont.
int enqueue_frame(mb_ctx* ctx, int B, float* hidden, int32_t* pos, int32_t max_pos,
                  int32_t* frame_idx, int32_t* alive, int32_t* codes, int32_t* cont) {
  ctx->frame_alive = alive;
  int rc = local_frame(ctx, B, hidden, nullptr, nullptr, nullptr);
  ctx->frame_alive = nullptr;
  if (rc) return rc;
  if ((rc = decode_step(ctx, B, nullptr, pos, max_pos, hidden))) return rc;
  return launch_frame_emit(ctx, ctx->tokens, ctx->cont, B, frame_idx, codes, cont, pos, alive);
}

}  // namespace
}  // namespace mb

extern "C" {

int mb_decode_frames_dev(mb_ctx* ctx, int B, int n_frames, float* hidden, int32_t* pos,
                         int32_t max_pos, int32_t* codes, int32_t* cont) {
  MB_DEVICE_GUARD(ctx);
  int rc = check_b(ctx, B);
  if (rc) return rc;
  if (n_frames < 0) return fail(ctx, MB_ERR_ARG, "n_frames %d is negative", n_frames);
  if (B == 0 || n_frames == 0) return MB_OK;
  if (!hidden || !pos || !codes || !cont) return fail(ctx, MB_ERR_ARG, "null pointer");
  if (max_pos < 0) return fail(ctx, MB_ERR_ARG, "max_pos %d is negative", max_pos);
  if (!ctx->cfg.wrap && max_pos >= ctx->cfg.capacity)
    return fail(ctx, MB_ERR_RANGE, "decode position %d exceeds the KV ring (%d slots)", max_pos,
                ctx->cfg.capacity);
  if ((rc = need_model(ctx))) return rc;
  if ((rc = cancelled(ctx))) return rc;
  int32_t* fidx = (int32_t*)scratch(ctx, "frame_idx", 4);
  int32_t* alive = (int32_t*)scratch(ctx, "frame_alive", (size_t)B * 4);
  if (!fidx || !alive) return fail(ctx, MB_ERR_NOMEM, "frame staging allocation failed");
  if ((rc = launch_fill_i32(ctx, fidx, 1, 0))) return rc;
  if ((rc = launch_fill_i32(ctx, alive, B, 1))) return rc;
  // Frame 0 runs eagerly: it sizes every scratch buffer the frame touches, so
  // nothing is allocated while the next frame is captured.
  if ((rc = enqueue_frame(ctx, B, hidden, pos, max_pos, fidx, alive, codes, cont))) return rc;
  if (n_frames == 1) return MB_OK;
  const uint64_t key[8] = {(uint64_t)B, (uint64_t)max_pos, (uint64_t)(uintptr_t)hidden,
                           (uint64_t)(uintptr_t)pos, (uint64_t)(uintptr_t)codes,
                           (uint64_t)(uintptr_t)cont, ctx->graph_gen, 1};
  if (!ctx->frame_exec || memcmp(key, ctx->frame_key, sizeof key) != 0) {
    if (ctx->frame_exec) {
      MB_HIP(ctx, hipGraphExecDestroy(ctx->frame_exec));
      ctx->frame_exec = nullptr;
    }
    if (!ctx->capture_stream)
      MB_HIP(ctx, hipStreamCreateWithFlags(&ctx->capture_stream, hipStreamNonBlocking));
    hipStream_t saved = ctx->stream;
    const hipError_t eb = hipStreamBeginCapture(ctx->capture_stream, hipStreamCaptureModeThreadLocal);
    if (eb != hipSuccess) return hip_fail(ctx, eb, "hipStreamBeginCapture");
    ctx->stream = ctx->capture_stream;
    rc = enqueue_frame(ctx, B, hidden, pos, max_pos, fidx, alive, codes, cont);
    hipGraph_t graph = nullptr;
    const hipError_t e = hipStreamEndCapture(ctx->stream, &graph);
    ctx->stream = saved;
    if (rc || e != hipSuccess || ctx->graph_gen != key[6]) {
      if (graph) (void)hipGraphDestroy(graph);
      if (rc) return rc;
      if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamEndCapture");
      return fail(ctx, MB_ERR_STATE, "a buffer moved while the frame was captured");
    }
    const hipError_t ei = hipGraphInstantiate(&ctx->frame_exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (ei != hipSuccess) {
      ctx->frame_exec = nullptr;
      return hip_fail(ctx, ei, "hipGraphInstantiate");
    }
    memcpy(ctx->frame_key, key, sizeof key);
  }
  for (int f = 1; f < n_frames; f++) {
    if ((rc = cancelled(ctx))) return rc;
    MB_HIP(ctx, hipGraphLaunch(ctx->frame_exec, ctx->stream));
  }
  return MB_OK;
}

int mb_decode_frames(mb_ctx* ctx, int B, int n_frames, float* hidden, int32_t* pos,
                     int32_t* codes, int32_t* cont) {
  MB_DEVICE_GUARD(ctx);
  int rc = check_b(ctx, B);
  if (rc) return rc;
  if (n_frames < 0) return fail(ctx, MB_ERR_ARG, "n_frames %d is negative", n_frames);
  if (B == 0 || n_frames == 0) return MB_OK;
  if (!hidden || !pos || !codes || !cont) return fail(ctx, MB_ERR_ARG, "null pointer");
  int64_t max_pos = 0;
  for (int b = 0; b < B; b++) {
    if (pos[b] < 0) return fail(ctx, MB_ERR_ARG, "sequence %d: negative position %d", b, pos[b]);
    if ((int64_t)pos[b] + n_frames - 1 > max_pos) max_pos = (int64_t)pos[b] + n_frames - 1;
  }
  if (max_pos > INT32_MAX) return fail(ctx, MB_ERR_ARG, "positions overflow int32");
  float* d_hidden = (float*)scratch(ctx, "frames_hidden", (size_t)B * D * 4);
  int32_t* d_pos = (int32_t*)scratch(ctx, "frames_pos", (size_t)B * 4);
  int32_t* d_codes = (int32_t*)scratch(ctx, "frames_codes", (size_t)n_frames * B * NVQ * 4);
  int32_t* d_cont = (int32_t*)scratch(ctx, "frames_cont", (size_t)n_frames * B * 4);
  if (!d_hidden || !d_pos || !d_codes || !d_cont)
    return fail(ctx, MB_ERR_NOMEM, "staging allocation failed");
  MB_HIP(ctx, hipMemcpyAsync(d_hidden, hidden, (size_t)B * D * 4, hipMemcpyHostToDevice, ctx->stream));
  MB_HIP(ctx, hipMemcpyAsync(d_pos, pos, (size_t)B * 4, hipMemcpyHostToDevice, ctx->stream));
  if ((rc = mb_decode_frames_dev(ctx, B, n_frames, d_hidden, d_pos, (int32_t)max_pos, d_codes,
                                 d_cont))) {
    (void)hipStreamSynchronize(ctx->stream);
    return rc;
  }
  MB_HIP(ctx, hipMemcpyAsync(hidden, d_hidden, (size_t)B * D * 4, hipMemcpyDeviceToHost, ctx->stream));
  MB_HIP(ctx, hipMemcpyAsync(pos, d_pos, (size_t)B * 4, hipMemcpyDeviceToHost, ctx->stream));
  MB_HIP(ctx, hipMemcpyAsync(codes, d_codes, (size_t)n_frames * B * NVQ * 4, hipMemcpyDeviceToHost,
                             ctx->stream));
  MB_HIP(ctx, hipMemcpyAsync(cont, d_cont, (size_t)n_frames * B * 4, hipMemcpyDeviceToHost,
                             ctx->stream));
  MB_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return MB_OK;
}

int mb_local_frame_dev(mb_ctx* ctx, int B, const float* hidden, int32_t* codes, int32_t* cont,
                       int32_t* rows17_out) {
  MB_DEVICE_GUARD(ctx);
  int rc = check_b(ctx, B);
  if (rc) return rc;
  if (B == 0) return MB_OK;
  if (!hidden) return fail(ctx, MB_ERR_ARG, "null pointer");
  if ((rc = need_model(ctx))) return rc;
  return local_frame(ctx, B, hidden, codes, cont, rows17_out);
}

}  // extern "C"
