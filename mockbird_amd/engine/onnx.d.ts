import type { WeightTable } from "./weights";

/** A WeightTable over an .onnx graph's bytes and its external-data sidecar (onnxWeights.ts:124-240). */
export function openOnnx(model: Uint8Array, sidecar: Uint8Array): WeightTable;
/** openOnnx over files. */
export function loadOnnxTable(onnxPath: string, dataPath: string): WeightTable;
