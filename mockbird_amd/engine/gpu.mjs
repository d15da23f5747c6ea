// The GpuTtsEngine of the reference (src/lib/tts/engine/gpu.ts:65-92), backed
// by the HIP library through the N-API addon.  Method names, argument meaning
// and error behaviour follow gpu.ts so WgpuTtsRuntime (runtime.ts:357-561)
// can drive it unchanged: prefill -> nextFrame -> decodeStep -> ... -> reset.
//
// The codec (decodeFrames) runs when the engine is created with a codec
// weight table; the clone encoder (encodeWaveform) is not part of this
// library.  A missing stage throws EngineNotImplemented, which is how the
// reference itself reports one (gpu.ts:28-36, :279-281).
import { kvDtypeCode, loadNative, N_VQ, orDefault, ROW_WIDTH } from "./native.mjs";
import { DecodeRunner } from "./decode.mjs";
import { PrefillRunner, packPromptRows } from "./prefill.mjs";
import { CODEC_SHAPE, resolveCodecTensors, resolveEngineTensors } from "./weights.mjs";

export class EngineNotImplemented extends Error {
  constructor(step) {
    super(`HIP engine: "${step}" is not implemented by this library.`);
    this.name = "EngineNotImplemented";
  }
}

const SAMPLES_PER_FRAME = 3840;
const SAMPLE_RATE = 48000;
const CHANNELS = 2;
const AUDIO_START = 6;
/** -1.5 * 2^13: exact in fp32 and in bf16, so it reads back unchanged from either ring. */
const KV_SENTINEL = -12288;

/** buildFrameRow / frameRowFrom (policy.ts:83-88, promptRows.ts:39-44). */
export function frameRowFrom(assistantSlot, frame) {
  const row = new Int32Array(ROW_WIDTH).fill(1024);
  row[0] = assistantSlot;
  row.set(frame.slice(0, ROW_WIDTH - 1), 1);
  return row;
}

/**
 * The largest decode-vs-prefill gap warm-up accepts.  With fp32 K/V both
 * paths multiply in fp32 (1e-3).  With bf16 K/V the prefill path's causal
 * attention rounds q and the softmax weights to bf16 for its matrix products
 * while the decode step keeps them in fp32, so the two agree to the bf16
 * bar (2e-2).  Either bar is taken relative to the hidden state's largest
 * magnitude once that exceeds 1, as real weights give hidden states of tens.
 */
function warmupTolerance(kvBf16, hidden) {
  let scale = 1;
  for (let i = 0; i < hidden.length; i += 1) scale = Math.max(scale, Math.abs(hidden[i]));
  return (kvBf16 ? 2e-2 : 1e-3) * scale;
}

/** max |a - b| over two equally long arrays */
function maxAbsDiff(a, b) {
  let m = 0;
  for (let i = 0; i < a.length; i += 1) m = Math.max(m, Math.abs(a[i] - b[i]));
  return m;
}

/**
 * One engine = one context holding one voice.  All per-utterance state is
 * the `utterance` record: how many rows its ring holds (the position the next
 * decode step appends at) and the hidden state of its latest global step.
 * `null` between reset() and the next prefill.
 */
class HipTtsEngineImpl {
  constructor(native, handle, info, settings, maxSlots, maxRows, layers) {
    Object.assign(this, { native, handle, info, settings, layerCount: layers, maxSlots });
    this.sampleRate = SAMPLE_RATE;
    this.channels = CHANNELS;
    this.samplesPerFrame = SAMPLES_PER_FRAME;
    this.prefillRunner = new PrefillRunner(native, handle, maxSlots, maxRows);
    this.decoder = new DecodeRunner(native, handle, maxSlots, settings);
    this.utterance = null;
    this.hasCodec = false;
    this.kvBf16 = false;
    this.disposed = false;
  }

  get deviceInfo() {
    return this.info;
  }

  /** rows in the global KV ring: the position the next decode step appends at */
  get position() {
    return this.utterance ? this.utterance.rows : 0;
  }

  async prefill(input) {
    const ids = packPromptRows(input.inputIds);
    const rows = ids.length / ROW_WIDTH;
    const hidden = await this.native.prefillAsync(this.handle, 1, rows, ids, Int32Array.of(rows));
    this.utterance = { rows, hidden };
    return hidden;
  }

  async decodeStep(input) {
    const u = this.utterance;
    if (u === null) throw new Error("decodeStep before prefill");
    const at = orDefault(input.position, u.rows);
    const hidden = await this.decoder.globalStep(input.row, at);
    u.rows = at + 1;
    u.hidden = hidden;
    return hidden;
  }

  nextFrame(hidden) {
    return this.decoder.nextFrame(hidden);
  }

  /**
   * Bring-up self-test of this library's path, then a clean state.
   *  1. Layer 0's first four slots are poisoned and a two-row prompt is
   *     prefilled: slots 0-1 must now hold K/V and slots 2-3 must still read
   *     the sentinel (the read-back path works, and the prefill wrote exactly
   *     its rows).
   *  2. The prefill's hidden state must be finite and non-zero.
   *  3. The same two rows as a one-row prefill plus one decode step at
   *     position 1 must give the same hidden state: the decode path (fused
   *     ring append + decode attention) agrees with the prefill path (ring
   *     write + causal prefill attention).
   * The failure messages are the reference's where its warm-up checks the
   * same condition (gpu.ts:201-234).
   */
  async warmup() {
    const row = new Int32Array(ROW_WIDTH).fill(1024);
    row[0] = AUDIO_START;
    const prompt = [Array.from(row), Array.from(row)];
    const probeSlots = Math.min(4, this.maxSlots);
    this.native.ringPoison(this.handle, 0, 0, probeSlots, KV_SENTINEL);
    const t0 = Date.now();
    const both = await this.prefill({ inputIds: prompt, attentionMask: [[1, 1]] });
    const prefillMs = Date.now() - t0;
    if (both.some((x) => !Number.isFinite(x))) {
      throw new Error("warmup produced a non-finite hidden state — a kernel wrote garbage");
    }
    if (both.every((x) => x === 0)) {
      throw new Error("warmup produced an all-zero hidden state — nothing was computed");
    }
    const ring = this.native.readRing(this.handle, 0, 0, 0, probeSlots);
    const untouched = ring.key.subarray(prompt.length * 768);
    if (untouched.length && !untouched.every((x) => x === KV_SENTINEL)) {
      throw new Error("warmup read-back is broken: the KV sentinel was not visible");
    }
    const written = (a) => a.subarray(0, prompt.length * 768).some((x) => x !== 0 && x !== KV_SENTINEL);
    if (!written(ring.key) || !written(ring.value)) {
      throw new Error(
        "warmup left the layer-0 KV cache empty (read-back verified: the sentinel was visible)",
      );
    }
    await this.prefill({ inputIds: prompt.slice(0, 1), attentionMask: [[1]] });
    const stepped = await this.decodeStep({ row, position: 1 });
    const gap = maxAbsDiff(stepped, both);
    if (!(gap < warmupTolerance(this.kvBf16, both))) {
      throw new Error(`warmup: the decode step disagrees with the prefill of the same rows (max |diff| ${gap})`);
    }
    this.reset();
    return { prefillMs, layers: this.layerCount, rows: prompt.length };
  }

  /** A fresh utterance: empty ring, repetition history and codec rings (gpu.ts:237-242). */
  reset() {
    this.utterance = null;
    this.native.ringReset(this.handle, null);
    this.decoder.clearSeen();
    if (this.hasCodec) this.native.codecReset(this.handle, null);
  }

  /**
   * Codes -> 48 kHz stereo, continuing the codec rings
   * (CodecRunner.decodeFrames, codec.ts:766-813): one Float32Array per
   * channel, 3840 samples per frame.  A missing code reads as 0, as there.
   */
  async decodeFrames(frames) {
    if (frames.length === 0) return [];
    if (!this.hasCodec) throw new EngineNotImplemented("codec decoder (no codec weights given)");
    const codes = new Int32Array(frames.length * N_VQ);
    frames.forEach((frame, f) => {
      for (let k = 0; k < N_VQ; k += 1) codes[f * N_VQ + k] = orDefault(frame[k], 0);
    });
    const pcm = await this.native.codecDecodeAsync(this.handle, 1, frames.length, codes);
    const half = pcm.length / 2;
    return [pcm.subarray(0, half), pcm.subarray(half)];
  }

  encodeWaveform(_waveform, _length) {
    throw new EngineNotImplemented("clone encoder (codec encode convs)");
  }

  /**
   * Frees the context.  While an *Async call is in flight destroy throws
   * MB_ERR_BUSY and the engine stays usable: await the call, then dispose
   * again.
   */
  dispose() {
    if (this.disposed) return;
    this.native.destroy(this.handle);
    this.disposed = true;
    this.utterance = null;
    this.prefillRunner.dispose();
  }
}

/**
 * Bring up a context, upload the weights and return a warmed-up engine
 * (createGpuEngineFor, gpu.ts:316-388).  `tables` = {global, local[, codec]}
 * WeightTables; options: {localHead, maxSlots (570), maxRows (= maxSlots),
 * layers (12: the count the model must resolve to), kvDtype ("f32" | "bf16"),
 * weightDtype ("f32" | "bf16": projection weights rounded to and read as
 * bf16, mb_set_weight_storage), penaltyPrecision ("f64": the reference CPU
 * path's doubles, the default | "f32": its WGSL engine's arithmetic,
 * mb_set_penalty_precision),
 * wrap (false: the reference's non-wrapping ring), device (0), codecShape
 * ({layersPerStage, contextPerStage}, the real shape by default),
 * codecKvDtype ("f32")}.  With a codec table the codec decoder is set up
 * for one voice (decodeFrames).
 */
export async function createGpuEngineFor(tables, log, options) {
  const native = loadNative();
  const { tensors, vocab, layers } = resolveEngineTensors(tables);
  const expected = orDefault(options.layers, 12);
  if (layers !== expected) {
    throw new Error(`expected ${expected} transformer layers, resolved ${layers}`);
  }
  const maxSlots = orDefault(options.maxSlots, 570);
  const maxRows = orDefault(options.maxRows, maxSlots);
  const handle = native.create({
    nLayers: layers,
    vocab,
    capacity: maxSlots,
    maxSeqs: 1,
    maxRows,
    kvDtype: kvDtypeCode(native, options.kvDtype),
    wrap: orDefault(options.wrap, false),
    device: orDefault(options.device, 0),
  });
  try {
    if (options.weightDtype) native.setWeightStorage(handle, options.weightDtype);
    if (options.penaltyPrecision) native.setPenaltyPrecision(handle, options.penaltyPrecision);
    let bytes = 0;
    for (const t of tensors) {
      native.uploadTensor(handle, t.name, t.data, t.dims);
      bytes += t.data.byteLength;
    }
    log(`weights: ${tensors.length} tensors (${(bytes / 1e6).toFixed(0)} MB of GPU memory)`);
    let codecShape = null;
    if (tables.codec) {
      codecShape = orDefault(options.codecShape, CODEC_SHAPE);
      const codecTensors = resolveCodecTensors(tables.codec, codecShape);
      for (const t of codecTensors) native.uploadTensor(handle, t.name, t.data, t.dims);
      native.codecInit(handle, {
        maxVoices: 1,
        kvDtype: kvDtypeCode(native, options.codecKvDtype),
        layers: codecShape.layersPerStage,
        context: codecShape.contextPerStage,
      });
      log(`codec: ${codecTensors.length} tensors, stages ${codecShape.layersPerStage.join("/")}`);
    }
    const info = { adapterName: "MI355X (gfx950, HIP)", deviceBytes: native.deviceBytes(handle) };
    const engine = new HipTtsEngineImpl(native, handle, info, options.localHead, maxSlots, maxRows,
      layers);
    engine.hasCodec = codecShape !== null;
    engine.kvBf16 = options.kvDtype === "bf16";
    log(`engine ready: ${layers} layers, KV ring ${maxSlots} slots, vocab ${vocab}`);
    const warm = await engine.warmup();
    log(`warmup: 1 prefill over ${warm.rows} rows in ${warm.prefillMs} ms`);
    return engine;
  } catch (error) {
    native.destroy(handle);
    throw error;
  }
}

/** Kept for callers that only want the "not wired" signal (gpu.ts:391-395). */
export function createGpuEngine() {
  throw new EngineNotImplemented("device init (await createGpuEngineFor with parsed weight tables)");
}
