/** Handle of one mb_ctx (rings, weights and activations on one GPU). */
export type NativeHandle = { readonly __mbContext: unique symbol };

export type NativeConfig = {
  nLayers?: number;
  vocab?: number;
  capacity?: number;
  maxSeqs?: number;
  maxRows?: number;
  kvDtype?: number;
  wrap?: boolean | number;
  device?: number;
};

/** An Error thrown by the addon: `code` names the MB_ERR_* status. */
export interface NativeError extends Error {
  code: string;
  status: number;
}

export interface Native {
  readonly KV: { F32: number; BF16: number };
  abiVersion(): number;
  create(config: NativeConfig): NativeHandle;
  destroy(h: NativeHandle): void;
  deviceBytes(h: NativeHandle): number;
  uploadTensor(h: NativeHandle, name: string, data: Float32Array, dims: number[]): void;
  cancel(h: NativeHandle, on?: boolean): void;
  setLocalHead(h: NativeHandle, audioEnd: number, assistant: number, penalty: number): void;
  setWeightStorage(h: NativeHandle, storage: "f32" | "bf16"): void;
  /** The repetition penalty's arithmetic: "f64" (the reference CPU path) or "f32" (its WGSL engine). */
  setPenaltyPrecision(h: NativeHandle, precision: "f64" | "f32"): void;
  ringReset(h: NativeHandle, seqIds: Int32Array | null): void;
  clearSeen(h: NativeHandle, seqIds: Int32Array | null): void;
  ringPoison(h: NativeHandle, layer: number, seq: number, nSlots: number, sentinel: number): void;
  readRing(
    h: NativeHandle,
    layer: number,
    seq: number,
    slot0: number,
    n: number,
  ): { key: Float32Array; value: Float32Array; slotPos: Int32Array };
  writeRing(
    h: NativeHandle,
    layer: number,
    seq: number,
    slot0: number,
    n: number,
    key: Float32Array | null,
    value: Float32Array | null,
    slotPos: Int32Array | null,
  ): void;
  ringAppend(h: NativeHandle, layer: number, B: number, qkv: Float32Array, pos: Int32Array): Float32Array;
  ringWriteRows(
    h: NativeHandle,
    layer: number,
    B: number,
    rowsMax: number,
    qkv: Float32Array,
    pos0: Int32Array,
    nRows: Int32Array,
  ): Float32Array;
  decodeAttention(h: NativeHandle, layer: number, B: number, q: Float32Array, pos: Int32Array): Float32Array;
  prefillAttention(
    h: NativeHandle,
    layer: number,
    B: number,
    rowsMax: number,
    q: Float32Array,
    pos0: Int32Array,
    nRows: Int32Array,
  ): Float32Array;
  prefill(
    h: NativeHandle,
    B: number,
    rowsMax: number,
    ids: Int32Array,
    nRows: Int32Array,
    layerCount?: number,
    allRows?: boolean,
  ): Float32Array;
  decodeStep(h: NativeHandle, B: number, rows17: Int32Array, pos: Int32Array): Float32Array;
  localFrame(h: NativeHandle, B: number, hidden: Float32Array): { codes: Int32Array; cont: Int32Array };
  localSteps(h: NativeHandle, B: number, hidden: Float32Array, maxStep: number): Float32Array;
  decodeFrames(
    h: NativeHandle,
    B: number,
    nFrames: number,
    hidden: Float32Array,
    pos: Int32Array,
  ): { codes: Int32Array; cont: Int32Array };
  codecInit(
    h: NativeHandle,
    config?: { maxVoices?: number; kvDtype?: number; layers?: number[]; context?: number[] },
  ): void;
  codecReset(h: NativeHandle, voices: Int32Array | null): void;
  /** codes [nFrames][B][16] -> pcm [B][2][nFrames * 3840] */
  codecDecode(h: NativeHandle, B: number, nFrames: number, codes: Int32Array): Float32Array;
  /**
   * The same calls run on a libuv worker thread: each returns a Promise of
   * what its synchronous form returns.  While one is in flight every other
   * call on the handle throws an Error with code "MB_ERR_BUSY".
   */
  prefillAsync(
    h: NativeHandle,
    B: number,
    rowsMax: number,
    ids: Int32Array,
    nRows: Int32Array,
    layerCount?: number,
    allRows?: boolean,
  ): Promise<Float32Array>;
  decodeStepAsync(h: NativeHandle, B: number, rows17: Int32Array, pos: Int32Array): Promise<Float32Array>;
  localFrameAsync(h: NativeHandle, B: number, hidden: Float32Array): Promise<{ codes: Int32Array; cont: Int32Array }>;
  decodeFramesAsync(
    h: NativeHandle,
    B: number,
    nFrames: number,
    hidden: Float32Array,
    pos: Int32Array,
  ): Promise<{ codes: Int32Array; cont: Int32Array }>;
  codecDecodeAsync(h: NativeHandle, B: number, nFrames: number, codes: Int32Array): Promise<Float32Array>;
  lastError(h: NativeHandle): string;
}

export function loadNative(): Native;
export function kvDtypeCode(native: Native, name?: "f32" | "bf16"): number;
export const ROW_WIDTH: 17;
export const N_VQ: 16;
export const HIDDEN: 768;
export const AUDIO_PAD_ID: 1024;
