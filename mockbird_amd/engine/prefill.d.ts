import type { Native, NativeHandle } from "./native";

export const PREFILL_SHAPES: { HIDDEN: 768; QKV: 2304; FFN: 3072; HEADS: 12; HEAD_DIM: 64 };

export class PrefillRunner {
  constructor(native: Native, handle: NativeHandle, maxSlots: number, maxRows: number);
  readonly buffers: { kv: NativeHandle };
  stageIds(ids: Uint32Array): void;
  run(rows: number, layers: unknown, embed: unknown, maxSlots: number, layerCount?: number): Promise<Float32Array>;
  poisonKv(rows: number, sentinel?: number): Promise<void>;
  readLayerCache(layer: number, rows: number): Promise<{ key: Float32Array; value: Float32Array }>;
  dispose(): void;
}

/** A prompt as 17-wide Int32 rows, missing columns padded with 1024; throws on no rows. */
export function packPromptRows(inputIds: number[][]): Int32Array;
