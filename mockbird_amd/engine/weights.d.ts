export type Tensor = {
  name: string;
  dims: number[];
  data: Float32Array;
  source?: "external" | "inline-constant" | "inline-raw" | "alias";
  offset?: number;
};

/** The reference's WeightTable (onnxWeights.ts:68-76). */
export type WeightTable = {
  get(name: string): Tensor;
  has(name: string): boolean;
  names(): string[];
  size: number;
  byShape(dims: string): Float32Array[];
};

export function loadSidecarTable(manifestPath: string): WeightTable;
export function tableOf(tensors: Map<string, Tensor>): WeightTable;
export function countLayers(table: WeightTable): number;
export function resolveEngineTensors(tables: { global: WeightTable; local: WeightTable }): {
  tensors: { name: string; dims: number[]; data: Float32Array }[];
  vocab: number;
  layers: number;
};

/** Layers and ring windows (positions) per codec stage. */
export type CodecShape = { layersPerStage: number[]; contextPerStage: number[] };
export const CODEC_SHAPE: CodecShape;
export function resolveCodecTensors(
  table: WeightTable,
  shape?: CodecShape,
): { name: string; dims: number[]; data: Float32Array }[];
