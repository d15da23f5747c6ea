// PrefillRunner: the global prefill over a prompt of 17-wide rows, mirroring
// the reference's PrefillRunner (src/lib/tts/engine/prefill.ts:114-674) method
// by method.  The rings and weights live in the native context (one mb_ctx per
// engine); the decode runner shares that context the way the reference's
// DecodeRunner shares `buffers.kv` (gpu.ts:149-160).
import { AUDIO_PAD_ID, HIDDEN, ROW_WIDTH } from "./native.mjs";

export const PREFILL_SHAPES = { HIDDEN, QKV: 3 * HIDDEN, FFN: 4 * HIDDEN, HEADS: 12, HEAD_DIM: 64 };

export class PrefillRunner {
  /**
   * @param native   the addon (loadNative())
   * @param handle   the context both runners use
   * @param maxSlots global KV ring slots (the context's capacity)
   * @param maxRows  most rows one prefill may carry
   */
  constructor(native, handle, maxSlots, maxRows) {
    this.native = native;
    this.handle = handle;
    this.maxSlots = maxSlots;
    this.maxRows = maxRows;
    this.staged = null;
    // The reference exposes its buffer set; here the shared ring is the context.
    this.buffers = { kv: handle };
  }

  /** Stage prompt ids [rows, 17] (u32) for the next run() (prefill.ts:641-649). */
  stageIds(ids) {
    if (ids.length % ROW_WIDTH !== 0) {
      throw new Error(`stageIds: ${ids.length} ids is not a whole number of ${ROW_WIDTH}-wide rows`);
    }
    this.staged = Int32Array.from(ids, (v) => v | 0);
  }

  /**
   * Run `layerCount` layers over the staged rows at positions 0 .. rows-1,
   * writing every layer's K/V from slot 0, and return ln_f of every row,
   * [rows, 768] (prefill.ts:325-603; `layerCount` is the single-layer
   * conformance switch of :320-324).  `layers` and `embed` are accepted for
   * signature parity: the context resolved the weights by name at upload.
   */
  async run(rows, _layers, _embed, _maxSlots, layerCount) {
    if (!this.staged || this.staged.length < rows * ROW_WIDTH) {
      throw new Error(`prefill: ${rows} rows requested but fewer ids were staged`);
    }
    if (rows < 1) throw new Error("prefill called with no rows");
    if (rows > this.maxRows) {
      throw new Error(`prefill: ${rows} rows exceed the runner's ${this.maxRows}-row buffers`);
    }
    const ids = this.staged.subarray(0, rows * ROW_WIDTH);
    const count = layerCount === undefined ? 0 : layerCount;
    return this.native.prefillAsync(this.handle, 1, rows, ids, Int32Array.of(rows), count, true);
  }

  /**
   * Write the sentinel into K and V of the first `rows` slots of layer 0, so
   * the warm-up can tell "nothing was written" from "read back from the wrong
   * place" (prefill.ts:610-620).
   */
  async poisonKv(rows, sentinel = -12345.5) {
    this.native.ringPoison(this.handle, 0, 0, rows, sentinel);
  }

  /** K/V of `rows` slots of one layer, [rows, 768] each (prefill.ts:661-673). */
  async readLayerCache(layer, rows) {
    const r = this.native.readRing(this.handle, layer, 0, 0, rows);
    return { key: r.key, value: r.value };
  }

  dispose() {
    this.staged = null;
  }
}

/**
 * A prompt of rows (number arrays: text id, then up to 16 codes) as one
 * Int32Array of 17-wide rows; columns a row leaves out are the audio pad
 * (the reference pads the same way, gpu.ts:176-181).  Throws on an empty
 * prompt with the reference's message.
 */
export function packPromptRows(inputIds) {
  if (inputIds.length === 0) throw new Error("prefill called with no rows");
  const out = new Int32Array(inputIds.length * ROW_WIDTH).fill(AUDIO_PAD_ID);
  let at = 0;
  for (const row of inputIds) {
    out.set(row.length > ROW_WIDTH ? row.slice(0, ROW_WIDTH) : row, at);
    at += ROW_WIDTH;
  }
  return out;
}
