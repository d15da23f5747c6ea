import type { EngineWeights, LocalHeadSettings } from "./gpu";
import type { CodecShape } from "./weights";

export class MultiVoiceEngine {
  readonly maxVoices: number;
  readonly capacity: number;
  prefill(prompts: number[][][]): Promise<Float32Array[]>;
  generate(nFrames: number): Promise<{ frames: number[][][]; stopped: boolean[] }>;
  nextFrames(hidden: Float32Array[]): Promise<(number[] | null)[]>;
  decodeSteps(rows: Int32Array[], positions: number[]): Promise<Float32Array[]>;
  /** codes[f][b] = 16 codes of voice b's frame f -> per voice [left, right] */
  decodeAudio(codes: number[][][]): Promise<Float32Array[][]>;
  reset(voices?: number[]): void;
  dispose(): void;
}

export type MultiVoiceOptions = {
  localHead: LocalHeadSettings;
  maxVoices: number;
  capacity?: number;
  maxRows?: number;
  kvDtype?: "f32" | "bf16";
  /** projection weights rounded to and read as bf16 (mb_set_weight_storage) */
  weightDtype?: "f32" | "bf16";
  /** Repetition-penalty arithmetic: "f64" (default, the reference CPU path) or "f32" (its WGSL engine). */
  penaltyPrecision?: "f64" | "f32";
  wrap?: boolean;
  device?: number;
  codecShape?: CodecShape;
  codecKvDtype?: "f32" | "bf16";
};

export function createMultiVoiceEngine(
  tables: EngineWeights,
  log: ((message: string) => void) | null,
  options: MultiVoiceOptions,
): Promise<MultiVoiceEngine>;
