import type { CodecShape, WeightTable } from "./weights";

export class EngineNotImplemented extends Error {
  constructor(step: string);
}

export type PrefillInput = { inputIds: number[][]; attentionMask: number[][] };
export type DecodeStepInput = { row: Int32Array; position: number };
export type LocalHeadSettings = {
  audioEndTokenId: number;
  audioAssistantSlotTokenId: number;
  repetitionPenalty: number;
};

/** The reference's engine interface (gpu.ts:65-92). */
export interface GpuTtsEngine {
  readonly sampleRate: number;
  readonly channels: number;
  readonly samplesPerFrame: number;
  prefill(input: PrefillInput): Promise<Float32Array>;
  decodeStep(input: DecodeStepInput): Promise<Float32Array>;
  nextFrame(hidden: Float32Array): Promise<number[] | null>;
  decodeFrames(frames: number[][]): Promise<Float32Array[]>;
  reset(): void;
  encodeWaveform(waveform: Float32Array, length: number): Promise<number[][]>;
  dispose(): void;
}

export type EngineWeights = { global: WeightTable; local: WeightTable; codec?: WeightTable };

export type EngineOptions = {
  localHead: LocalHeadSettings;
  maxSlots?: number;
  maxRows?: number;
  /** transformer layers the weights must resolve to (12) */
  layers?: number;
  kvDtype?: "f32" | "bf16";
  /** projection weights rounded to and read as bf16 (mb_set_weight_storage) */
  weightDtype?: "f32" | "bf16";
  /** Repetition-penalty arithmetic: "f64" (default, the reference CPU path) or "f32" (its WGSL engine). */
  penaltyPrecision?: "f64" | "f32";
  /** false (default): the reference's non-wrapping global ring */
  wrap?: boolean;
  device?: number;
  /** the codec's layers and ring windows per stage (4/2/2/4, 500/1696/2480/3248) */
  codecShape?: CodecShape;
  codecKvDtype?: "f32" | "bf16";
};

export function createGpuEngineFor(
  tables: EngineWeights,
  log: (message: string) => void,
  options: EngineOptions,
): Promise<GpuTtsEngine & { readonly position: number; warmup(): Promise<{ prefillMs: number; layers: number; rows: number }> }>;
export function createGpuEngine(): GpuTtsEngine;
export function frameRowFrom(assistantSlot: number, frame: number[]): Int32Array;
