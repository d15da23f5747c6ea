// GPU driver of the ONNX load path: opens hand-built global / local .onnx
// graphs (external data in .data sidecars, an inline Constant, an Identity
// alias, anonymous projections) with loadOnnxTable, brings the engine up
// with createGpuEngineFor on those tables (onnxWeights.ts:124-240 feeding
// gpu.ts:316-388), runs one voice through prefill and the reference runtime's
// frame loop, and prints one JSON object for the Python test to check.
//
//   node engine_onnx_run.mjs <dir>   (dir holds global.onnx/.data, local.onnx/.data, case.json)
import fs from "fs";
import path from "path";

import { createGpuEngineFor, frameRowFrom } from "../../mockbird_amd/engine/gpu.mjs";
import { loadOnnxTable } from "../../mockbird_amd/engine/onnx.mjs";

const dir = process.argv[2];
const spec = JSON.parse(fs.readFileSync(path.join(dir, "case.json"), "utf8"));
const open = (n) => loadOnnxTable(path.join(dir, `${n}.onnx`), path.join(dir, `${n}.data`));
const tables = { global: open("global"), local: open("local") };
const localHead = { audioEndTokenId: 7, audioAssistantSlotTokenId: 9, repetitionPenalty: 1.2 };
const log = (m) => console.error(m);

async function main() {
  const engine = await createGpuEngineFor(tables, log, {
    localHead,
    maxSlots: spec.maxSlots,
    layers: spec.layers,
  });
  const prompt = spec.prompt;
  engine.reset();
  let hidden = await engine.prefill({ inputIds: prompt, attentionMask: [prompt.map(() => 1)] });
  const res = { prefillHidden: Array.from(hidden), frames: [], hiddens: [] };
  for (let step = 0; step < spec.frames; step += 1) {
    const frame = await engine.nextFrame(hidden);
    if (!frame) break;
    res.frames.push(frame);
    hidden = await engine.decodeStep({ row: frameRowFrom(9, frame), position: prompt.length + step });
    res.hiddens.push(Array.from(hidden));
  }
  res.sources = {
    alias: tables.global.get("core.model.transformer.h.1.ln_1.weight").source,
    constant: tables.global.get("core.model.transformer.ln_f.bias").source,
  };
  engine.dispose();
  console.log(JSON.stringify(res));
}

main().catch((e) => {
  console.error(e.stack || String(e));
  process.exit(1);
});
