// CPU-side checks of the JavaScript host: the addon loads and exports every
// binding, the engine modules import, weight tables resolve anonymous
// projections by shape and offset order (as prefill.ts:78-107 and
// decodeWeights.ts:24-51 do), and argument errors surface as exceptions
// before any device call.  Prints one JSON object.
import { loadNative } from "../../mockbird_amd/engine/native.mjs";
import { createGpuEngine, EngineNotImplemented, frameRowFrom } from "../../mockbird_amd/engine/gpu.mjs";
import { resolveCodecTensors, resolveEngineTensors, tableOf } from "../../mockbird_amd/engine/weights.mjs";
import { packPromptRows } from "../../mockbird_amd/engine/prefill.mjs";

const out = {};
const native = loadNative();
out.exports = Object.keys(native).sort();
out.abi = native.abiVersion();

// two tiny tables: two global layers (vocab 16) with every projection but
// layer 0's c_attn anonymous, and a local head whose matrices are all anonymous
let offset = 0;
let tag = 1;
out.tags = {};
const add = (map, name, dims) => {
  const n = dims.reduce((a, b) => a * b, 1);
  map.set(name, { name, dims, data: new Float32Array(n).fill(tag), offset });
  out.tags[name] = tag;
  tag += 1;
  offset += n * 4;
};
const layer = (map, p, anon) => {
  add(map, `${p}ln_1.weight`, [768]);
  add(map, `${p}ln_1.bias`, [768]);
  add(map, anon ? `onnx::MatMul_${tag}` : `${p}attn.c_attn.weight`, [768, 2304]);
  add(map, `${p}attn.c_attn.bias`, [2304]);
  add(map, `onnx::MatMul_${tag}`, [768, 768]);
  add(map, `${p}attn.c_proj.bias`, [768]);
  add(map, `${p}ln_2.weight`, [768]);
  add(map, `${p}ln_2.bias`, [768]);
  add(map, `onnx::MatMul_${tag}`, [768, 3072]);
  add(map, `${p}mlp.fc_in.bias`, [3072]);
  add(map, `onnx::MatMul_${tag}`, [3072, 768]);
  add(map, `${p}mlp.fc_out.bias`, [768]);
};
const g = new Map();
layer(g, "core.model.transformer.h.0.", false);
layer(g, "core.model.transformer.h.1.", true);
add(g, "core.model.transformer.ln_f.weight", [768]);
add(g, "core.model.transformer.ln_f.bias", [768]);
add(g, "core.model.transformer.wte.weight", [16, 768]);
for (let k = 0; k < 16; k += 1) add(g, `core.model.audio_embeddings.${k}.weight`, [1024, 768]);
const l = new Map();
offset = 0;
layer(l, "model.local_transformer.h.0.", true);
add(l, "model.local_transformer.ln_f.weight", [768]);
add(l, "model.local_transformer.ln_f.bias", [768]);
add(l, "onnx::MatMul_text", [768, 16]);
for (let k = 0; k < 16; k += 1) add(l, `onnx::MatMul_audio_${k}`, [768, 1024]);
const global = tableOf(g);
const local = tableOf(l);
const r = resolveEngineTensors({ global, local });
out.vocab = r.vocab;
out.layers = r.layers;
out.resolved = r.tensors.map((x) => [x.name, x.dims, x.data[0]]);

// a codec table in the sidecar's order, every projection anonymous: per
// stage the input projection, then per layer in_proj, out_proj, ffn.0, ffn.2
// and the named norms / scales, then the stage output; the RVQ front's 16
// convolutions and output projection are anonymous too
const c = new Map();
offset = 0;
const dec = [1, 3, 5, 7];
const codecLayers = [2, 1, 1, 2];
for (let k = 0; k < 16; k += 1) {
  add(c, `onnx::Conv_rvq_${k}`, [512, 8, 1]);
  add(c, `model.quantizer.quantizers.${k}.out_proj.bias`, [512]);
  add(c, `model.quantizer.quantizers.${k}.codebook.weight`, [1024, 8]);
}
add(c, "onnx::Conv_rvq_out", [768, 512, 1]);
add(c, "model.quantizer.output_proj.bias", [768]);
for (let s = 0; s < 4; s += 1) {
  add(c, `onnx::MatMul_in_${s}`, [s === 0 ? 192 : 384, 256]);
  for (let i = 0; i < codecLayers[s]; i += 1) {
    const p = `model.decoder.${dec[s]}.transformer.layers.${i}.`;
    add(c, `onnx::MatMul_qkv_${s}_${i}`, [256, 768]);
    add(c, `onnx::MatMul_o_${s}_${i}`, [256, 256]);
    add(c, `onnx::MatMul_f0_${s}_${i}`, [256, 1024]);
    add(c, `onnx::MatMul_f2_${s}_${i}`, [1024, 256]);
    for (const n of ["norm1.weight", "norm1.bias", "norm2.weight", "norm2.bias",
                     "layer_scale_1.scale", "layer_scale_2.scale"]) add(c, p + n, [256]);
  }
  add(c, `onnx::MatMul_out_${s}`, [256, s === 3 ? 240 : 768]);
}
out.codec = resolveCodecTensors(tableOf(c), { layersPerStage: codecLayers, contextPerStage: [6, 12, 20, 40] })
  .map((x) => [x.name, x.dims, x.data[0]]);

// staging and frame rows
out.staged = Array.from(packPromptRows([[6], [8, 1, 2, 3]]));
try {
  packPromptRows([]);
} catch (e) {
  out.emptyPrompt = e.message;
}
out.frameRow = Array.from(frameRowFrom(9, [5, 6, 7]));

// errors before any device call
const errs = {};
try {
  native.create({ nLayers: 0 });
} catch (e) {
  errs.badConfig = [e.code, e.message];
}
// malformed configurations: every one is refused with a JS error
errs.createCases = [
  null, 7, "cfg", {}, { nLayers: "12" }, { nLayers: 2.5 }, { nLayers: NaN }, { capacity: -1 },
  { maxSeqs: 1e12 }, { kvDtype: 9 }, { wrap: 3 }, { device: -1 }, { nLayers: 2, capacity: 16 },
].map((cfg) => {
  try {
    const h = native.create(cfg);
    native.destroy(h);  // a GPU host accepts the valid ones
    return "created";
  } catch (e) {
    return e.code || e.name;
  }
});
try {
  native.destroy({});
} catch (e) {
  errs.destroyBad = e.name;
}
try {
  native.prefill({}, 1, 1, new Int32Array(17), Int32Array.of(1));
} catch (e) {
  errs.badHandle = [e.name, e.message];
}
try {
  native.prefillAsync({}, 1, 1, new Int32Array(17), Int32Array.of(1));
} catch (e) {
  errs.badHandleAsync = [e.name, e.message];
}
try {
  createGpuEngine();
} catch (e) {
  errs.notImplemented = [e instanceof EngineNotImplemented, e.name];
}
out.errors = errs;
console.log(JSON.stringify(out));
