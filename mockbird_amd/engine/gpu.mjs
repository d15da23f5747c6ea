// The GpuTtsEngine of the reference (src/lib/tts/engine/gpu.ts:65-92), backed
// by the HIP library through the N-API addon.  Method names, argument meaning
// and error behaviour follow gpu.ts so WgpuTtsRuntime (runtime.ts:357-561)
// can drive it unchanged: prefill -> nextFrame -> decodeStep -> ... -> reset.
//
// The codec (decodeFrames) runs when the engine is created with a codec
// weight table; the clone encoder (encodeWaveform) is not part of this
// library.  A missing stage throws EngineNotImplemented, which is how the
// reference itself reports one (gpu.ts:28-36, :279-281).
import { HIDDEN, kvDtypeCode, loadNative, N_VQ, orDefault, ROW_WIDTH } from "./native.mjs";
import { DecodeRunner } from "./decode.mjs";
import { PrefillRunner, stageRows } from "./prefill.mjs";
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

/** buildFrameRow / frameRowFrom (policy.ts:83-88, promptRows.ts:39-44). */
export function frameRowFrom(assistantSlot, frame) {
  const row = new Int32Array(ROW_WIDTH).fill(1024);
  row[0] = assistantSlot;
  for (let k = 0; k < Math.min(frame.length, ROW_WIDTH - 1); k += 1) row[k + 1] = frame[k];
  return row;
}

class HipTtsEngineImpl {
  constructor(native, handle, info, settings, maxSlots, maxRows, layers) {
    this.sampleRate = SAMPLE_RATE;
    this.channels = CHANNELS;
    this.samplesPerFrame = SAMPLES_PER_FRAME;
    this.native = native;
    this.handle = handle;
    this.info = info;
    this.settings = settings;
    this.layerCount = layers;
    this.prefillRunner = new PrefillRunner(native, handle, maxSlots, maxRows);
    this.decoder = new DecodeRunner(native, handle, maxSlots, settings);
    /** rows currently in the global KV cache (== the next sequence position) */
    this.pastValidLength = 0;
    this.lastHidden = null;
    this.hasCodec = false;
    this.disposed = false;
  }

  get deviceInfo() {
    return this.info;
  }

  /** rows in the global KV cache -- the decode step appends at this position */
  get position() {
    return this.pastValidLength;
  }

  async prefill(input) {
    const rows = input.inputIds.length;
    if (rows === 0) throw new Error("prefill called with no rows");
    this.prefillRunner.stageIds(stageRows(input.inputIds));
    const hidden = await this.prefillRunner.run(rows, null, null, this.decoder.maxSlotCount);
    this.pastValidLength = rows;
    this.lastHidden = hidden.slice((rows - 1) * HIDDEN, rows * HIDDEN);
    return this.lastHidden;
  }

  /**
   * Warm-up (gpu.ts:196-235): prove the read-back path with a poisoned cache,
   * run one two-row prefill, check the hidden state is finite and non-zero and
   * that layer 0's cache was written, then reset.
   */
  async warmup() {
    const row = new Array(ROW_WIDTH).fill(1024);
    row[0] = 6; // audio_start_token_id
    const rows = [row, row];
    await this.prefillRunner.poisonKv(rows.length);
    const poison = await this.prefillRunner.readLayerCache(0, rows.length);
    if (!poison.key.every((value) => value === -12345.5)) {
      throw new Error("warmup read-back is broken: the KV sentinel was not visible");
    }
    const started = Date.now();
    const hidden = await this.prefill({ inputIds: rows, attentionMask: [[1, 1]] });
    const elapsed = Date.now() - started;
    for (const value of hidden) {
      if (!Number.isFinite(value)) {
        throw new Error("warmup produced a non-finite hidden state — a kernel wrote garbage");
      }
    }
    if (!hidden.some((value) => value !== 0)) {
      throw new Error("warmup produced an all-zero hidden state — nothing was computed");
    }
    const cache = await this.prefillRunner.readLayerCache(0, rows.length);
    if (!cache.key.some((value) => value !== 0) || !cache.value.some((value) => value !== 0)) {
      throw new Error(
        "warmup left the layer-0 KV cache empty (read-back verified: the sentinel was visible)",
      );
    }
    this.reset();
    return { prefillMs: elapsed, layers: this.layerCount, rows: rows.length };
  }

  /** A fresh utterance: drop the KV ring and the repetition history (gpu.ts:237-242). */
  reset() {
    this.pastValidLength = 0;
    this.lastHidden = null;
    this.decoder.clearSeen();
    this.native.ringReset(this.handle, null);
    if (this.hasCodec) this.native.codecReset(this.handle, null);
  }

  async decodeStep(input) {
    if (!this.lastHidden) throw new Error("decodeStep before prefill");
    const position = orDefault(input.position, this.pastValidLength);
    const hidden = await this.decoder.globalStep(input.row, position);
    this.pastValidLength = position + 1;
    this.lastHidden = hidden;
    return hidden;
  }

  async nextFrame(hidden) {
    const frame = await this.decoder.nextFrame(hidden);
    if (frame) this.lastHidden = hidden;
    return frame;
  }

  /**
   * Codes -> 48 kHz stereo, continuing the codec rings
   * (CodecRunner.decodeFrames, codec.ts:766-813): one Float32Array per
   * channel, 3840 samples per frame.  A missing code reads as 0, as there.
   */
  async decodeFrames(frames) {
    if (!frames.length) return [];
    if (!this.hasCodec) throw new EngineNotImplemented("codec decoder (no codec weights given)");
    const n = frames.length;
    const codes = new Int32Array(n * N_VQ);
    for (let f = 0; f < n; f += 1) {
      for (let k = 0; k < N_VQ; k += 1) codes[f * N_VQ + k] = orDefault(frames[f][k], 0);
    }
    const pcm = this.native.codecDecode(this.handle, 1, n, codes);
    const T = n * SAMPLES_PER_FRAME;
    return [pcm.slice(0, T), pcm.slice(T, 2 * T)];
  }

  encodeWaveform(_waveform, _length) {
    throw new EngineNotImplemented("clone encoder (codec encode convs)");
  }

  dispose() {
    if (this.disposed) return;
    this.disposed = true;
    this.decoder.dispose();
    this.prefillRunner.dispose();
    this.native.destroy(this.handle);
  }
}

/**
 * Bring up a context, upload the weights and return a warmed-up engine
 * (createGpuEngineFor, gpu.ts:316-388).  `tables` = {global, local[, codec]}
 * WeightTables; options: {localHead, maxSlots (570), maxRows (= maxSlots),
 * layers (12: the count the model must resolve to), kvDtype ("f32" | "bf16"),
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
    const engine = new HipTtsEngineImpl(native, handle, info, options.localHead, maxSlots, maxRows, layers);
    engine.hasCodec = codecShape !== null;
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
