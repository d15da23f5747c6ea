/*
 * mockbird_hip.h -- C ABI of the MI355X (gfx950) decoder hot path for
 * MOSS-TTS-Nano: KV ring append with RoPE on K, ring-aware single-query decode
 * attention, causal prefill attention, and the QKV/O projections around them.
 *
 * This is the drop-in boundary.  The host engine (GpuTtsEngine / PrefillRunner /
 * DecodeRunner in the reference, src/lib/tts/engine/gpu.ts:65-92,
 * prefill.ts:114-674, decode.ts:201-1046) binds these entry points through a
 * thin N-API addon; every signature uses plain pointers and sizes.
 *
 * Conventions
 *  - Every call returns MB_OK (0) or an MB_ERR_* code; mb_last_error(ctx)
 *    returns the message of the last failing call on that context.
 *  - Host-pointer calls (no suffix) copy in, run on the context's stream and
 *    synchronise before returning, like the reference's submit + mapAsync.
 *  - `_dev` calls take device pointers, enqueue on the context's stream and
 *    return without synchronising (for callers that keep data in HBM).
 *  - Every call runs on the context's device (mb_config.device) and leaves
 *    the calling thread's current HIP device as it found it.
 *  - Sequences ("voices") are addressed 0 .. max_seqs-1; a batched call with
 *    B sequences works on sequences 0 .. B-1.
 *  - Fused QKV rows are [2304] = q | k | v, each 768 wide, head-major
 *    (head*64 + dim) as the exported graph lays them out (kernels-batch.ts:1-15).
 *  - Ring semantics (kernels-decode.ts:679-714 and :590-667): a row at
 *    absolute position pos is written to slot pos mod capacity, the slot
 *    records pos, and a query at position cur sees exactly the slots whose
 *    stored position p satisfies 0 <= cur - p < capacity.  With
 *    mb_config.wrap == 0 the reference's non-wrapping global ring is kept
 *    instead: slot == pos and pos >= capacity is MB_ERR_RANGE
 *    (decode.ts:719-724).
 *  - Attention scale is 0.125 (1/sqrt(64)); RoPE pairs (2i, 2i+1) at
 *    frequency 10000^(-2i/64), out[2i] = x[2i] cos - x[2i+1] sin,
 *    out[2i+1] = x[2i+1] cos + x[2i] sin (kernels-decode.ts:204-241).
 *
 * Not thread-safe per context: calls on one context must not overlap.
 */
#ifndef MOCKBIRD_HIP_H
#define MOCKBIRD_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MB_ABI_VERSION 2

enum {
  MB_OK = 0,
  MB_ERR_ARG = 1,       /* bad argument (null pointer, size out of range, unknown name) */
  MB_ERR_RANGE = 2,     /* position does not fit a non-wrapping ring (decode.ts:719-724) */
  MB_ERR_HIP = 3,       /* a HIP runtime call failed */
  MB_ERR_STATE = 4,     /* call out of order (e.g. a weight is missing) */
  MB_ERR_CANCELLED = 5, /* mb_cancel() was observed between layers */
  MB_ERR_NOMEM = 6      /* device allocation failed */
};

enum { MB_KV_F32 = 0, MB_KV_BF16 = 1 };
enum { MB_DT_F32 = 0, MB_DT_BF16 = 1 };
/* Epilogues of mb_linear_dev. */
enum { MB_EPI_STORE = 0, MB_EPI_GELU = 1, MB_EPI_ADD = 2, MB_EPI_SCALE_ADD = 3, MB_EPI_GELU_ERF = 4 };

typedef struct mb_config {
  int32_t n_layers;   /* global transformer layers (12) */
  int32_t vocab;      /* rows of the text embedding / columns of the text head */
  int32_t capacity;   /* KV ring slots per sequence and layer (C) */
  int32_t max_seqs;   /* sequences (voices) the context holds rings for */
  int32_t max_rows;   /* most prompt rows one prefill call may carry per sequence */
  int32_t kv_dtype;   /* MB_KV_F32 or MB_KV_BF16 (round-to-nearest-even on store) */
  int32_t wrap;       /* 1: slot = pos mod C; 0: the reference's non-wrapping ring */
  int32_t device;     /* HIP device ordinal */
} mb_config;

typedef struct mb_ctx mb_ctx;

/* ---------------------------------------------------------------- context */

int mb_abi_version(void);

/* Create a context: allocates the rings (every slot empty) and activations.
 * Replaces the device + buffer set-up of createGpuEngineFor (gpu.ts:316-388)
 * and the PrefillRunner / DecodeRunner constructors (prefill.ts:128-167,
 * decode.ts:255-290). */
int mb_create(const mb_config* cfg, mb_ctx** out);
/* Free everything (gpu.ts:283-291 dispose). */
void mb_destroy(mb_ctx* ctx);
const char* mb_last_error(const mb_ctx* ctx);
/* Launch every later call on `hip_stream` (a hipStream_t; NULL is HIP's
 * default stream).  A new context launches on a stream of its own, which
 * mb_get_stream() returns until this is called. */
int mb_set_stream(mb_ctx* ctx, void* hip_stream);
void* mb_get_stream(mb_ctx* ctx);
int mb_synchronize(mb_ctx* ctx);
/* Device bytes held by the context (rings + activations + weights). */
int64_t mb_device_bytes(const mb_ctx* ctx);

/* Copy one fp32 tensor in by name (uploadWeights, weights.ts:44-119).  Names
 * follow the exported graph: core.model.transformer.h.{i}.{ln_1,ln_2}.{weight,
 * bias}, .attn.c_attn.{weight,bias} [768,2304], .attn.c_proj.* [768,768],
 * .mlp.fc_in.* [768,3072], .mlp.fc_out.* [3072,768],
 * core.model.transformer.ln_f.*, core.model.transformer.wte.weight
 * [vocab,768], core.model.audio_embeddings.{k}.weight [1024,768],
 * model.local_transformer.h.0.* and model.local_transformer.ln_f.* (same
 * shapes), model.text_lm_head.weight [768,vocab],
 * model.audio_lm_heads.{k}.weight [768,1024].  Matrices are [K, N] row-major
 * as in the graph (no transposition, doc section 9.1). */
int mb_upload_tensor(mb_ctx* ctx, const char* name, const float* data, const int64_t* dims,
                     int ndims);

/* Request cancellation: the next layer boundary of a running or later model
 * call returns MB_ERR_CANCELLED (the reference polls isCancelled() per frame,
 * runtime.ts:506, :541).  mb_cancel(ctx, 0) clears the request. */
int mb_cancel(mb_ctx* ctx, int on);

/* ------------------------------------------------------------------- ring */

/* Empty the rings of `n` sequences (seq_ids; n < 0 means every sequence) on
 * every layer: all slots forget their position (engine.reset, gpu.ts:237-242,
 * codec.ts:279-282). */
int mb_ring_reset(mb_ctx* ctx, int n, const int32_t* seq_ids);

/* Fill K and V of slots [0, n_slots) of (layer, seq) with `sentinel` (rounded
 * to bf16 for bf16 rings) without touching slot positions: the warm-up
 * read-back probe of PrefillRunner.poisonKv (prefill.ts:610-620). */
int mb_ring_poison(mb_ctx* ctx, int layer, int seq, int n_slots, float sentinel);

/* Read slots [slot0, slot0+n) of (layer, seq) into the reference layout:
 * k, v [n][768] fp32 (head*64 + dim; bf16 widened exactly) and slot_pos[n]
 * (absolute position or -1).  Any output may be NULL.  Replaces
 * PrefillRunner.readLayerCache (prefill.ts:661-673). */
int mb_read_ring(mb_ctx* ctx, int layer, int seq, int slot0, int n, float* k, float* v,
                 int32_t* slot_pos);

/* The inverse of mb_read_ring: store k, v [n][768] fp32 (rounded to nearest
 * even bf16 for bf16 rings) and slot_pos[n] into slots [slot0, slot0+n) of
 * (layer, seq).  A NULL input leaves that part of the slots as it is.  Every
 * position must be -1 (empty) or one the ring itself puts in that slot (pos
 * mod C; pos itself on a non-wrapping ring), else MB_ERR_ARG and nothing is
 * written.  With mb_read_ring it dumps and reloads a prefilled cache, as the
 * reference's oracle does with its prefill cache file
 * (tools/onnx-probe/ref-decode.mjs:327-372). */
int mb_write_ring(mb_ctx* ctx, int layer, int seq, int slot0, int n, const float* k,
                  const float* v, const int32_t* slot_pos);

/* Append one row per sequence b < B at absolute position pos[b]: q is roped
 * into q_out[b][768], K = rope(k) and V = v are stored at slot pos mod C of
 * `layer`, and the slot records pos.  qkv is [B][2304].
 * Replaces ROPE_SPLIT_RING (kernels-decode.ts:216-241, dispatched at
 * decode.ts:527-535) with the wrap rule of ROPE_SPLIT_CODEC (:679-714). */
int mb_ring_append(mb_ctx* ctx, int layer, int B, const float* qkv, const int32_t* pos,
                   float* q_out);

/* Write n_rows[b] consecutive rows per sequence, starting at pos0[b]:
 * qkv [B][rows_max][2304] -> roped q_out [B][rows_max][768] plus K/V into the
 * ring.  The prefill form of the append: ROPE_SPLIT_CACHE
 * (kernels-batch.ts:194-234, prefill.ts:424-432) with pos0 = 0. */
int mb_ring_write_rows(mb_ctx* ctx, int layer, int B, int rows_max, const float* qkv,
                       const int32_t* pos0, const int32_t* n_rows, float* q_out);

/* Single-query decode attention for sequences b < B: q[b][768] (roped) at
 * position pos[b] over the live slots of `layer`; out[b][768].
 * Replaces ATTEND_RING (kernels-decode.ts:254-327, decode.ts:536-552) with the
 * live-slot mask of ATTEND_RING_CODEC (kernels-decode.ts:590-667). */
int mb_decode_attention(mb_ctx* ctx, int layer, int B, const float* q, const int32_t* pos,
                        float* out);

/* mb_ring_append followed by mb_decode_attention in one launch: the row of
 * sequence b at pos[b] is appended (K = rope(k), V = v at slot pos mod C, the
 * slot records pos) and its roped q attends the ring including that row;
 * out[b][768] receives the attention output and q_out[b][768] (may be NULL)
 * the roped q.  Results equal the two calls in sequence.  Replaces the
 * ROPE_SPLIT_RING + ATTEND_RING pair of one decode layer
 * (kernels-decode.ts:216-327, dispatched decode.ts:527-552). */
int mb_append_attend(mb_ctx* ctx, int layer, int B, const float* qkv, const int32_t* pos,
                     float* q_out, float* out);

/* Causal prefill attention: q [B][rows_max][768] (roped) for rows r < n_rows[b]
 * at positions pos0[b] + r, each attending the live slots of `layer` whose
 * position is <= its own; out [B][rows_max][768].  Replaces ATTENTION_SCORES /
 * _SOFTMAX / _APPLY (kernels-batch.ts:246-350, prefill.ts:434-462). */
int mb_prefill_attention(mb_ctx* ctx, int layer, int B, int rows_max, const float* q,
                         const int32_t* pos0, const int32_t* n_rows, float* out);

/* ---- device-pointer forms (enqueue only; shapes and meaning as above) ----
 * qkv_dtype / q_dtype select MB_DT_F32 or MB_DT_BF16 inputs; row strides are
 * in elements.  max_pos bounds every pos (pass capacity - 1 or larger when
 * unknown): it sizes the attention split without reading device memory. */
int mb_ring_append_dev(mb_ctx* ctx, int layer, int B, const void* qkv, int qkv_dtype,
                       int64_t qkv_stride, const int32_t* pos, float* q_out, int64_t q_stride);
int mb_ring_write_rows_dev(mb_ctx* ctx, int layer, int B, int rows_max, const void* qkv,
                           int qkv_dtype, const int32_t* pos0, const int32_t* n_rows, void* q_out,
                           int q_dtype);
int mb_decode_attention_dev(mb_ctx* ctx, int layer, int B, const float* q, int64_t q_stride,
                            const int32_t* pos, int32_t max_pos, float* out, int64_t out_stride);
int mb_prefill_attention_dev(mb_ctx* ctx, int layer, int B, int rows_max, const void* q,
                             int q_dtype, const int32_t* pos0, const int32_t* n_rows, float* out);
int mb_append_attend_dev(mb_ctx* ctx, int layer, int B, const void* qkv, int qkv_dtype,
                         int64_t qkv_stride, const int32_t* pos, int32_t max_pos, float* q_out,
                         int64_t q_stride, float* out, int64_t out_stride);

/* Kernel-level projection on device pointers (row a7):
 *   C[M][N] = epi(A[M][K] * W[K][N] + bias[N])
 * W row-major [K, N] as the exported graph stores its MatMul initialisers;
 * bias may be NULL; epi MB_EPI_STORE writes, MB_EPI_GELU applies gelu-tanh,
 * MB_EPI_ADD adds into C (the residual), MB_EPI_GELU_ERF applies the exact
 * (erf) GELU, and MB_EPI_SCALE_ADD reads `bias` as a per-column scale s and
 * stores C + s * (A W) (the codec's layer scale).  fp32 products and
 * accumulation.  Needs N % 64 == 0, K % 64 == 0, lda and ldc multiples of 4
 * and 16-byte aligned pointers.  Replaces GEMM_NT (kernels-batch.ts:156-184,
 * called prefill.ts:404-422, :464-482), GEMV / GEMV_NOB (kernels-decode.ts:
 * 127-166, called decode.ts:517-526, :553-562, codec.ts:536-735) with the
 * GELU_TANH / GELU_ERF / ADD_RESIDUAL / LAYER_SCALE_ADD passes that follow
 * them (kernels-decode.ts:330-415) fused in. */
int mb_linear_dev(mb_ctx* ctx, int M, int N, int K, const float* A, int64_t lda, const float* W,
                  const float* bias, float* C, int64_t ldc, int epi);

/* The projection of mb_linear_dev at the precision bf16-KV model contexts
 * run their projections in (above 8 rows): each fp32 product a w is taken as
 * ah wh + ah wl + al wh, with ah = bf16(a) and al = bf16(a - ah) (likewise
 * w), three bf16 MFMA products summed in fp32 -- within about 2^-16 |a w| of
 * the fp32 product, for a fifth of the matrix-core time.
 * mb_split_weights_dev writes a row-major [K, N] W in that kernel's operand
 * order to Wx (2 K N bf16 = 4 K N bytes, 16-byte aligned; N % 64 == 0,
 * K % 32 == 0); mb_linear_split_dev computes C[M][N] = epi(A W + bias) from
 * it, with mb_linear_dev's epilogues.  It takes M > 8: below 1024 rows (or
 * at most 512 tiles of 64 x 64) a streaming kernel that needs K % 128 == 0,
 * above that a kernel tiled 32-128 rows x 128 columns over all of k that
 * needs N % 128 == 0; M <= 8 returns MB_ERR_STATE.
 * Replaces the same GEMM_NT / GEMV passes as mb_linear_dev (kernels-batch.ts:
 * 156-184, kernels-decode.ts:127-166).  Enqueue only. */
int mb_split_weights_dev(mb_ctx* ctx, const float* W, int K, int N, void* Wx);
int mb_linear_split_dev(mb_ctx* ctx, int M, int N, int K, const float* A, int64_t lda,
                        const void* Wx, const float* bias, float* C, int64_t ldc, int epi);

/* mb_linear_dev that allocates nothing.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, kernels and results as mb_linear_dev; the split-K partials that
 * mb_linear_dev keeps in the context's growable scratch live in a static
 * 4 MiB device array per GPU instead (resolved by mb_create, held until the
 * process ends).  That size covers every split the kernel chooses; a shape
 * needing more returns MB_ERR_ARG.  Every call on one GPU shares that GPU's
 * array, so calls that overlap on one GPU race.  Enqueue only. */
int mb_linear_noalloc_dev(mb_ctx* ctx, int M, int N, int K, const float* A, int64_t lda,
                          const float* W, const float* bias, float* C, int64_t ldc, int epi);

/* ------------------------------------------------------------------ model
 * The decoder around the rings, fp32 weights uploaded with mb_upload_tensor.
 * Row ids are int32 [17]: text id in column 0 (< vocab), audio codes in
 * columns 1..16 (< 1024, or 1024 = pad), as promptRows.ts:1-44 lays them out. */

/* Local-head settings (LocalHeadSettings, gpu.ts:59-63): the text-head
 * columns of audio_end and assistant_slot (7, 9) and the repetition penalty
 * (1.2).  Those are also the defaults.  The penalty is a double: the
 * reference applies the JS number generation_defaults.audio_repetition_penalty
 * (mossTtsRuntime.js:506-521, policy.ts:273-290), and a penalised score can
 * fall between s / 1.2 and s / 1.2f.  A change invalidates the captured
 * frame graph of mb_decode_frames_dev. */
int mb_set_local_head(mb_ctx* ctx, int32_t audio_end_id, int32_t assistant_id, double penalty);

/* Arithmetic of the repetition penalty in the greedy choice.  The reference
 * has two: its CPU path (the frame loop of mossTtsRuntime.js:1965-2141 over
 * local_cached_step, the app's greedy path since the published model ships
 * no local_greedy_frame graph) penalises and compares JS numbers, doubles
 * (argmaxWithRepetitionPenalty, mossTtsRuntime.js:506-521; policy.ts:273-290);
 * its WGSL engine passes the penalty as float bits (decode.ts:908) and
 * multiplies or divides and compares in f32 (ARGMAX_PENALTY,
 * kernels-decode.ts:454-461).  A penalised score can fall between s / 1.2
 * and s / 1.2f, so the two can pick different codes.
 *   MB_PENALTY_F64 (the default): the CPU path's doubles.
 *   MB_PENALTY_F32: the WGSL engine's f32 arithmetic (the penalty rounded to
 *   f32, a correctly rounded f32 multiply or divide; WGSL only bounds its f32
 *   division to 2.5 ulp, so bit parity with a given WebGPU driver is not
 *   claimed).
 * A change invalidates the captured frame graph of mb_decode_frames_dev. */
#define MB_PENALTY_F64 0
#define MB_PENALTY_F32 1
int mb_set_penalty_precision(mb_ctx* ctx, int32_t precision);

/* Weight storage of the decoder's projections (c_attn, c_proj, fc_in, fc_out
 * of every layer, the local layer's, and the 16 audio heads): MB_W_F32 (the
 * default, the reference's fp32 weights) or MB_W_BF16.  With MB_W_BF16 each
 * of those weights is rounded to bf16 once (round to nearest even) when the
 * model is resolved, and the decode-sized kernels read the bf16 copies --
 * half the weight bytes; products and sums stay fp32, so the results are
 * those of the fp32 path on the rounded weights.  Embeddings and the text
 * head stay fp32.  The bf16 re-export of the model weights that
 * docs/moss-tts-runtime-analysis.md:408-411 plans (the reference's own
 * "f16 re-export", a separate, independent win) is what this stands for;
 * the uploaded tensors are left as they are, and a later call switches back
 * (the rounded copies are then freed).  Re-derives the weight copies on the
 * next model call and invalidates the captured frame graph. */
#define MB_W_F32 0
#define MB_W_BF16 1
int mb_set_weight_storage(mb_ctx* ctx, int32_t storage);

/* Global prefill of sequences b < B: ids [B][rows_max][17], n_rows[b] rows at
 * positions 0 .. n_rows[b]-1 (n_rows[b] <= capacity).  Each sequence's rings
 * are emptied first (a new utterance), every layer's K/V is written from
 * slot 0, and last_hidden[b][768] receives ln_f of the sequence's last row.
 * Replaces GpuTtsEngine.prefill / PrefillRunner.run (gpu.ts:173-192,
 * prefill.ts:325-603). */
int mb_prefill(mb_ctx* ctx, int B, int rows_max, const int32_t* ids, const int32_t* n_rows,
               float* last_hidden);

/* mb_prefill returning ln_f of every row: hidden [B][rows_max][768], rows
 * r >= n_rows[b] zeroed.  PrefillRunner.run reads back the whole [rows, 768]
 * hidden block the same way (prefill.ts:325-603, compared row by row in
 * tests/gpu/prefill.test.mjs:104-149).  layer_count (<= 0: every layer) runs
 * only the first layers before ln_f, as run()'s layerCount argument does for
 * single-layer conformance (prefill.ts:320-331); the other layers' rings are
 * left empty. */
int mb_prefill_rows(mb_ctx* ctx, int B, int rows_max, const int32_t* ids, const int32_t* n_rows,
                    int layer_count, float* hidden);

/* One global decode step for sequences b < B: embed rows17[b][17], run every
 * layer at position pos[b] (appending K/V to each layer's ring) and write
 * ln_f into hidden[b][768].  Replaces GpuTtsEngine.decodeStep /
 * DecodeRunner.globalStep (gpu.ts:244-258, decode.ts:712-775). */
int mb_decode_step(mb_ctx* ctx, int B, const int32_t* rows17, const int32_t* pos, float* hidden);

/* The 17-step local frame head for sequences b < B from the global hidden
 * state hidden[b][768]: cont[b] = 1 when the text head chooses the
 * assistant slot over audio_end, then 16 greedy codes with the repetition
 * penalty on each channel's history (codes[b][16]).  A sequence that stops
 * keeps its history unchanged.  Replaces GpuTtsEngine.nextFrame /
 * DecodeRunner.nextFrame (gpu.ts:268-272, decode.ts:788-939). */
int mb_local_frame(mb_ctx* ctx, int B, const float* hidden, int32_t* codes, int32_t* cont);

/* Run local-head steps 0 .. max_step (< 17) without their greedy choices and
 * return the last step's ln_f output out[b][768]; steps >= 2 embed the codes
 * of the previous frame.  The conformance probe
 * DecodeRunner.nextFrameSteps (decode.ts:970-1030). */
int mb_local_steps(mb_ctx* ctx, int B, const float* hidden, int max_step, float* out);

/* The 17-step local frame head teacher-forced with codes[b][16] (each in
 * [0, 1024)): step 0 runs on hidden[b][768], step 1 on wte[assistant_id], step
 * s >= 2 on the embedding of codes[b][s - 2] on channel s - 2, exactly as the
 * greedy frame would have run had it chosen those codes.  text2[b][2]
 * receives step 0's text-head dot products (audio_end, assistant) as the
 * continue decision compares them, and logits[b][16][1024] each channel's
 * audio-head logits before the repetition penalty, as the greedy choice reads
 * them.  The repetition history, the last frame's codes and the captured
 * frame graph are left untouched.  The logits buffer the reference's
 * ARGMAX_PENALTY reads (decode.ts:879-927, kernels-decode.ts:428-478), made
 * visible for parity checks. */
int mb_local_logits(mb_ctx* ctx, int B, const float* hidden, const int32_t* codes, double* text2,
                    float* logits);

/* Forget the repetition history of `n` sequences (n < 0: all) -- the
 * clearSeen part of engine.reset (decode.ts:276-280, gpu.ts:237-242). */
int mb_clear_seen(mb_ctx* ctx, int n, const int32_t* seq_ids);

/* Device-pointer forms.  mb_decode_step_dev takes rows17 [B][17], pos [B]
 * (every pos <= max_pos) and hidden [B][768] in device memory;
 * mb_local_frame_dev writes codes [B][16], cont [B] and, when rows17_out is
 * not NULL, the next frame rows [assistant_id, codes...] (buildFrameRow,
 * policy.ts:83-88), all in device memory (any output may be NULL). */
int mb_decode_step_dev(mb_ctx* ctx, int B, const int32_t* rows17, const int32_t* pos,
                       int32_t max_pos, float* hidden);
int mb_local_frame_dev(mb_ctx* ctx, int B, const float* hidden, int32_t* codes, int32_t* cont,
                       int32_t* rows17_out);

/* The frame loop on the device: n_frames greedy frames for sequences b < B.
 * Each frame is DecodeRunner.nextFrame on hidden (decode.ts:788-939), then
 * the global decode step of its frame row [assistant_id, codes] at pos[b]
 * (GpuTtsEngine.decodeStep, gpu.ts:244-257), whose ln_f output replaces
 * hidden; pos[b] then advances by one if sequence b continued (the runtime's
 * loop, runtime.ts:528-561).  codes [n_frames][B][16] and cont
 * [n_frames][B] receive every frame.  Every sequence starts the call alive;
 * one that stops stays stopped for the rest of the call, keeps its position,
 * and its later frames carry cont = 0 with codes to be ignored.
 * All pointers are device memory; max_pos bounds every position the call
 * reaches (pos[b] + n_frames - 1).  The first frame runs as ordinary
 * launches and the next ones replay it from a HIP graph, captured once and
 * kept while B, max_pos, the pointers and the context's buffers stay the
 * same, so the host issues one graph launch per frame.  Enqueue only. */
int mb_decode_frames_dev(mb_ctx* ctx, int B, int n_frames, float* hidden, int32_t* pos,
                         int32_t max_pos, int32_t* codes, int32_t* cont);

/* Host-pointer form of mb_decode_frames_dev: hidden [B][768] and pos [B] are
 * read, and on return hold the state after the last frame (the hidden state
 * and position the next frame starts from); codes [n_frames][B][16] and cont
 * [n_frames][B] receive every frame.  Synchronises before returning.  The
 * whole of WgpuTtsRuntime's frame loop (runtime.ts:539-561: nextFrame, then
 * decodeStep at prompt_rows + step) for many voices in one call. */
int mb_decode_frames(mb_ctx* ctx, int B, int n_frames, float* hidden, int32_t* pos,
                     int32_t* codes, int32_t* cont);

/* ------------------------------------------------------------ the codec
 *
 * The streaming codec decoder (codec.ts:1-30): 16 RVQ codes per 12.5 Hz
 * frame -> 3840 stereo samples at 48 kHz, for up to max_voices independent
 * voices per call.  Per frame: the RVQ front (16 codebook gathers through
 * the per-quantiser 1x1 convolutions, then the [768,512] output projection,
 * interleaved x4 into 4 positions of 192), four transformer stages of
 * d = 256 (4 heads of 64) over 4, 8, 16, 32 positions, each with its own
 * wrapping ring per layer keyed by absolute position (the window rule of
 * ATTEND_RING_CODEC, kernels-decode.ts:590-667), an x2 sub-pixel upsample
 * between stages, and the head that lays the 240-wide latent out as PCM.
 *
 * Weights are uploaded with mb_upload_tensor under these names ([K, N]
 * row-major as the graph's MatMul initialisers hold them, which the
 * reference finds by shape and offset order, decodeWeights.ts:69-156):
 *   model.quantizer.quantizers.{k}.out_proj.weight   [512, 8] (or [512, 8, 1])
 *   model.quantizer.quantizers.{k}.out_proj.bias     [512]
 *   model.quantizer.quantizers.{k}.codebook.weight   [1024, 8]
 *   model.quantizer.output_proj.weight               [768, 512] (or [768, 512, 1])
 *   model.quantizer.output_proj.bias                 [768]
 * and for stage s = 0..3, ds = 1, 3, 5, 7, layer i:
 *   model.decoder.{ds}.input_proj.weight             [192 | 384, 256]
 *   model.decoder.{ds}.output_proj.weight            [256, 768] (s < 3) | [256, 240]
 *   model.decoder.{ds}.transformer.layers.{i}.self_attn.in_proj.weight   [256, 768]
 *   model.decoder.{ds}.transformer.layers.{i}.self_attn.out_proj.weight  [256, 256]
 *   model.decoder.{ds}.transformer.layers.{i}.ffn.0.weight               [256, 1024]
 *   model.decoder.{ds}.transformer.layers.{i}.ffn.2.weight               [1024, 256]
 *   model.decoder.{ds}.transformer.layers.{i}.norm1.weight / .bias        [256]
 *   model.decoder.{ds}.transformer.layers.{i}.norm2.weight / .bias        [256]
 *   model.decoder.{ds}.transformer.layers.{i}.layer_scale_1.scale         [256]
 *   model.decoder.{ds}.transformer.layers.{i}.layer_scale_2.scale         [256]
 */
typedef struct mb_codec_config {
  int32_t max_voices; /* voices decoded together (rings and buffers sized for them) */
  int32_t kv_dtype;   /* MB_KV_F32 or MB_KV_BF16 for the codec rings */
  int32_t layers[4];  /* transformer layers per stage: 4, 2, 2, 4 */
  int32_t context[4]; /* ring window per stage in positions: 500, 1696, 2480, 3248 */
} mb_codec_config;

/* Allocate the codec's rings and buffers on this context (again: frees the
 * previous ones).  Every voice starts empty at position 0 of every stage.
 * Replaces the CodecRunner constructor (codec.ts:198-262). */
int mb_codec_init(mb_ctx* ctx, const mb_codec_config* cfg);

/* A fresh utterance for `n` voices (n < 0: all): every ring slot reads as
 * empty and every stage restarts at position 0 (CodecRunner.resetRings,
 * codec.ts:265-269). */
int mb_codec_reset(mb_ctx* ctx, int n, const int32_t* voices);

/* Decode n_frames frames for voices b < B, continuing each voice's rings:
 * codes [n_frames][B][16] in [0, 1024) -> pcm [B][2][n_frames * 3840]
 * (per voice, left channel then right, frames in order).  Host pointers;
 * synchronises before returning.  Replaces CodecRunner.decodeFrames
 * (codec.ts:766-813) for many voices at once. */
int mb_codec_decode(mb_ctx* ctx, int B, int n_frames, const int32_t* codes, float* pcm);

/* Device-pointer form of mb_codec_decode (codes and pcm in device memory;
 * a code outside [0, 1024) contributes no codebook row).  The first frame
 * runs as ordinary launches and the next ones replay it from a HIP graph,
 * captured once and kept while B, the pointers and the context's buffers
 * stay the same.  Enqueue only. */
int mb_codec_decode_dev(mb_ctx* ctx, int B, int n_frames, const int32_t* codes, float* pcm);

/* Parity read-back of one codec layer's ring for one voice (layers numbered
 * across stages, 0 .. sum(layers) - 1): k and v [slots][256] in the
 * reference's [slot][head * 64 + dim] order, slot_pos [slots]; *slots
 * receives the ring's slot count (its window plus the stage's positions per
 * frame, so that a frame's positions are appended before they are
 * attended).  Any output may be NULL.  Synchronises. */
int mb_codec_read_ring(mb_ctx* ctx, int layer, int voice, float* k, float* v, int32_t* slot_pos,
                       int32_t* slots);

#ifdef __cplusplus
}
#endif

#endif /* MOCKBIRD_HIP_H */
