// MultiVoiceEngine: many concurrent voices on one GPU, one ring per voice and
// layer.  Each voice follows the single-voice engine's semantics (gpu.ts:65-92);
// the batch only shares launches.  Rings wrap by default (slot = pos mod C,
// FIFO eviction), the codec ring's rule (kernels-decode.ts:590-714).
import { HIDDEN, kvDtypeCode, loadNative, N_VQ, orDefault, ROW_WIDTH } from "./native.mjs";
import { packPromptRows } from "./prefill.mjs";
import { CODEC_SHAPE, resolveCodecTensors, resolveEngineTensors } from "./weights.mjs";

const SAMPLES_PER_FRAME = 3840;

export class MultiVoiceEngine {
  constructor(native, handle, maxVoices, capacity, maxRows) {
    this.native = native;
    this.handle = handle;
    this.maxVoices = maxVoices;
    this.capacity = capacity;
    this.maxRows = maxRows;
    this.voices = 0;
    this.hidden = null;
    this.positions = null;
    this.stopped = null;
    this.hasCodec = false;
    this.disposed = false;
  }

  /**
   * Prefill one prompt per voice (voices 0 .. prompts.length-1); returns the
   * last-row hidden state of each.  Every voice starts a new utterance.
   */
  async prefill(prompts) {
    const B = prompts.length;
    if (B < 1 || B > this.maxVoices) throw new Error(`prefill of ${B} voices (max ${this.maxVoices})`);
    const n = Int32Array.from(prompts, (p) => p.length);
    const rowsMax = Math.max(...n);
    if (Math.min(...n) < 1) throw new Error("prefill called with no rows");
    const ids = new Int32Array(B * rowsMax * ROW_WIDTH).fill(1024);
    prompts.forEach((p, b) => ids.set(packPromptRows(p), b * rowsMax * ROW_WIDTH));
    this.native.clearSeen(this.handle, null);
    const flat = await this.native.prefillAsync(this.handle, B, rowsMax, ids, n);
    this.voices = B;
    this.hidden = flat;
    this.positions = n.slice();
    this.stopped = new Uint8Array(B);
    return Array.from({ length: B }, (_, b) => flat.slice(b * HIDDEN, (b + 1) * HIDDEN));
  }

  /**
   * Generate `nFrames` frames for every voice on the device (local head, then
   * the global step of the frame row, per frame).  Returns per voice the
   * frames produced until it chose audio_end (then `stopped[b]` is true).
   */
  async generate(nFrames) {
    const B = this.voices;
    if (!B) throw new Error("generate before prefill");
    const { codes, cont } = await this.native.decodeFramesAsync(this.handle, B, nFrames, this.hidden,
      this.positions);
    const frames = Array.from({ length: B }, () => []);
    for (let f = 0; f < nFrames; f += 1) {
      for (let b = 0; b < B; b += 1) {
        if (this.stopped[b]) continue;
        if (!cont[f * B + b]) {
          this.stopped[b] = 1;
          continue;
        }
        const o = (f * B + b) * N_VQ;
        frames[b].push(Array.from(codes.subarray(o, o + N_VQ)));
      }
    }
    return { frames, stopped: Array.from(this.stopped, (s) => s === 1) };
  }

  /** One local-head frame per voice from the given hidden states (null = stop). */
  async nextFrames(hidden) {
    const B = hidden.length;
    const flat = new Float32Array(B * HIDDEN);
    hidden.forEach((h, b) => flat.set(h, b * HIDDEN));
    const r = await this.native.localFrameAsync(this.handle, B, flat);
    return Array.from({ length: B }, (_, b) =>
      r.cont[b] ? Array.from(r.codes.subarray(b * N_VQ, (b + 1) * N_VQ)) : null,
    );
  }

  /** One global step per voice: rows[b] appended at positions[b]. */
  async decodeSteps(rows, positions) {
    const B = rows.length;
    const flat = new Int32Array(B * ROW_WIDTH).fill(1024);
    rows.forEach((r, b) => flat.set(r.subarray ? r.subarray(0, ROW_WIDTH) : r.slice(0, ROW_WIDTH), b * ROW_WIDTH));
    const out = await this.native.decodeStepAsync(this.handle, B, flat, Int32Array.from(positions));
    return Array.from({ length: B }, (_, b) => out.slice(b * HIDDEN, (b + 1) * HIDDEN));
  }

  /**
   * Codec: n frames for voices 0 .. B-1 at once, codes[f][b] = 16 codes of
   * voice b's frame f; returns per voice [left, right] Float32Arrays of
   * n * 3840 samples, continuing each voice's codec rings.
   */
  async decodeAudio(codes) {
    if (!this.hasCodec) throw new Error("decodeAudio: the engine was created without codec weights");
    const n = codes.length;
    if (!n) return [];
    const B = codes[0].length;
    if (B < 1 || B > this.maxVoices) throw new Error(`decodeAudio of ${B} voices (max ${this.maxVoices})`);
    const flat = new Int32Array(n * B * N_VQ);
    for (let f = 0; f < n; f += 1) {
      if (codes[f].length !== B) throw new Error(`frame ${f} has ${codes[f].length} voices, expected ${B}`);
      for (let b = 0; b < B; b += 1) flat.set(codes[f][b].slice(0, N_VQ), (f * B + b) * N_VQ);
    }
    const pcm = await this.native.codecDecodeAsync(this.handle, B, n, flat);
    const T = n * SAMPLES_PER_FRAME;
    return Array.from({ length: B }, (_, b) => [
      pcm.slice((2 * b) * T, (2 * b + 1) * T),
      pcm.slice((2 * b + 1) * T, (2 * b + 2) * T),
    ]);
  }

  /** Empty the rings and repetition history of some voices (all when omitted). */
  reset(voices) {
    const ids = voices ? Int32Array.from(voices) : null;
    this.native.ringReset(this.handle, ids);
    this.native.clearSeen(this.handle, ids);
    if (this.hasCodec) this.native.codecReset(this.handle, ids);
  }

  /** Frees the context; throws MB_ERR_BUSY (and stays usable) while an *Async call is in flight. */
  dispose() {
    if (this.disposed) return;
    this.native.destroy(this.handle);
    this.disposed = true;
  }
}

/**
 * A context for `maxVoices` voices: options {localHead, maxVoices, capacity
 * (1024), maxRows (capacity), kvDtype ("bf16"), weightDtype ("f32" | "bf16"),
 * penaltyPrecision ("f64" | "f32"), wrap (true), device (0),
 * codecShape, codecKvDtype ("bf16")}; a `codec` table sets up the codec for
 * every voice (decodeAudio).
 */
export async function createMultiVoiceEngine(tables, log, options) {
  const native = loadNative();
  const { tensors, vocab, layers } = resolveEngineTensors(tables);
  const capacity = orDefault(options.capacity, 1024);
  const maxRows = orDefault(options.maxRows, capacity);
  const handle = native.create({
    nLayers: layers,
    vocab,
    capacity,
    maxSeqs: options.maxVoices,
    maxRows,
    kvDtype: kvDtypeCode(native, orDefault(options.kvDtype, "bf16")),
    wrap: orDefault(options.wrap, true),
    device: orDefault(options.device, 0),
  });
  try {
    for (const t of tensors) native.uploadTensor(handle, t.name, t.data, t.dims);
    const s = options.localHead;
    if (options.weightDtype) native.setWeightStorage(handle, options.weightDtype);
    if (options.penaltyPrecision) native.setPenaltyPrecision(handle, options.penaltyPrecision);
    native.setLocalHead(handle, s.audioEndTokenId, s.audioAssistantSlotTokenId, s.repetitionPenalty);
    let hasCodec = false;
    if (tables.codec) {
      const shape = orDefault(options.codecShape, CODEC_SHAPE);
      for (const t of resolveCodecTensors(tables.codec, shape)) {
        native.uploadTensor(handle, t.name, t.data, t.dims);
      }
      native.codecInit(handle, {
        maxVoices: options.maxVoices,
        kvDtype: kvDtypeCode(native, orDefault(options.codecKvDtype, "bf16")),
        layers: shape.layersPerStage,
        context: shape.contextPerStage,
      });
      hasCodec = true;
    }
    if (log) log(`multi-voice engine: ${options.maxVoices} voices, ${layers} layers, ring ${capacity}`);
    const engine = new MultiVoiceEngine(native, handle, options.maxVoices, capacity, maxRows);
    engine.hasCodec = hasCodec;
    return engine;
  } catch (error) {
    native.destroy(handle);
    throw error;
  }
}
