import type { LocalHeadSettings } from "./gpu";
import type { Native, NativeHandle } from "./native";

export class DecodeRunner {
  constructor(native: Native, handle: NativeHandle, maxSlots: number, settings: LocalHeadSettings);
  clearSeen(): void;
  globalStep(row: Int32Array, position: number, layers?: unknown, lnF?: unknown, embed?: unknown): Promise<Float32Array>;
  nextFrame(hidden: Float32Array, embed?: unknown): Promise<number[] | null>;
  nextFrameSteps(hidden: Float32Array, embed: unknown, maxStep: number): Promise<Float32Array>;
  readonly maxSlotCount: number;
  dispose(): void;
}
