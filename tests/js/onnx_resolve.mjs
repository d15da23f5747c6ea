// Opens hand-built .onnx graphs with external-data sidecars through the
// engine's loader and resolves them as the engine does; writes every
// resolved tensor (f32, in resolution order) to <dir>/resolved.bin and an
// index to stdout.
//
//   node onnx_resolve.mjs <dir>   (dir holds global.onnx/.data, local.onnx/.data)
import fs from "fs";
import path from "path";

import { loadOnnxTable } from "../../mockbird_amd/engine/onnx.mjs";
import { resolveEngineTensors } from "../../mockbird_amd/engine/weights.mjs";

const dir = process.argv[2];
const open = (n) => loadOnnxTable(path.join(dir, `${n}.onnx`), path.join(dir, `${n}.data`));
const tables = { global: open("global"), local: open("local") };
const { tensors, vocab, layers } = resolveEngineTensors(tables);
const parts = tensors.map((t) => Buffer.from(t.data.buffer, t.data.byteOffset, t.data.byteLength));
fs.writeFileSync(path.join(dir, "resolved.bin"), Buffer.concat(parts));
const g = tables.global;
console.log(JSON.stringify({
  vocab,
  layers,
  index: tensors.map((t) => [t.name, t.dims, t.data.length]),
  sources: {
    alias: g.get("core.model.transformer.h.1.ln_1.weight").source,
    constant: g.get("core.model.transformer.ln_f.bias").source,
    external: g.get("core.model.transformer.wte.weight").source,
  },
  globalSize: g.size,
}));
