// Weight tables and their resolution into the graph names the C library
// uploads by.
//
// A WeightTable has the reference's shape (onnxWeights.ts:68-76): get(name),
// has(name), names(), size and byShape(dims) -- the tensors of one shape in
// sidecar-offset order.  The exported graphs keep their projections as
// anonymous MatMul initialisers, so, as resolveLayerWeights (prefill.ts:78-107)
// and resolveLocalWeights (decodeWeights.ts:24-51) do, a matrix is taken by
// name when the table has that name and otherwise by shape and offset order;
// biases, LayerNorm parameters and embeddings are always taken by name.
import fs from "fs";
import path from "path";

import { HIDDEN, N_VQ, orDefault } from "./native.mjs";

const QKV = 3 * HIDDEN;
const FFN = 4 * HIDDEN;
const CODEBOOK = 1024;

/**
 * A WeightTable over one raw little-endian f32 sidecar and its JSON manifest
 * {"data": "<file>", "tensors": [{"name", "dims", "offset"}]} (offset in bytes).
 * The sidecar is read once; every tensor is a view into it.
 */
export function loadSidecarTable(manifestPath) {
  const manifest = JSON.parse(fs.readFileSync(manifestPath, "utf8"));
  const dataPath = path.resolve(path.dirname(manifestPath), manifest.data);
  const bytes = fs.readFileSync(dataPath);
  if (bytes.byteOffset % 4 !== 0) throw new Error(`${dataPath}: unaligned buffer`);
  const all = new Float32Array(bytes.buffer, bytes.byteOffset, bytes.byteLength >> 2);
  const tensors = new Map();
  for (const t of manifest.tensors) {
    const n = t.dims.reduce((a, b) => a * b, 1);
    if (t.offset % 4 !== 0 || t.offset / 4 + n > all.length) {
      throw new Error(`${manifestPath}: tensor ${t.name} lies outside the sidecar`);
    }
    tensors.set(t.name, {
      name: t.name,
      dims: t.dims.slice(),
      data: all.subarray(t.offset / 4, t.offset / 4 + n),
      source: "external",
      offset: t.offset,
    });
  }
  return tableOf(tensors);
}

/** A WeightTable over a Map name -> {dims, data[, offset]}. */
export function tableOf(tensors) {
  const list = [...tensors.values()].sort((a, b) => orDefault(a.offset, 0) - orDefault(b.offset, 0));
  return {
    get(name) {
      const t = tensors.get(name);
      if (!t) throw new Error(`weight not uploaded: ${name}`);
      return t;
    },
    has(name) {
      return tensors.has(name);
    },
    names() {
      return [...tensors.keys()];
    },
    get size() {
      return tensors.size;
    },
    byShape(dims) {
      return list.filter((t) => t.dims.join("x") === dims).map((t) => t.data);
    },
  };
}

function pickMatrix(table, name, shape, index) {
  if (table.has(name)) {
    const t = table.get(name);
    if (t.dims.join("x") !== shape) {
      throw new Error(`weight has the wrong shape: ${name} is ${t.dims.join("x")}, expected ${shape}`);
    }
    return t.data;
  }
  const list = table.byShape(shape);
  if (!list[index]) throw new Error(`no ${shape} block at index ${index} for ${name}`);
  return list[index];
}

function layerTensors(table, prefix, index, out) {
  const mats = [
    ["attn.c_attn.weight", `${HIDDEN}x${QKV}`, [HIDDEN, QKV]],
    ["attn.c_proj.weight", `${HIDDEN}x${HIDDEN}`, [HIDDEN, HIDDEN]],
    ["mlp.fc_in.weight", `${HIDDEN}x${FFN}`, [HIDDEN, FFN]],
    ["mlp.fc_out.weight", `${FFN}x${HIDDEN}`, [FFN, HIDDEN]],
  ];
  for (const [suffix, shape, dims] of mats) {
    out.push({ name: prefix + suffix, dims, data: pickMatrix(table, prefix + suffix, shape, index) });
  }
  const named = [
    ["ln_1.weight", [HIDDEN]],
    ["ln_1.bias", [HIDDEN]],
    ["attn.c_attn.bias", [QKV]],
    ["attn.c_proj.bias", [HIDDEN]],
    ["ln_2.weight", [HIDDEN]],
    ["ln_2.bias", [HIDDEN]],
    ["mlp.fc_in.bias", [FFN]],
    ["mlp.fc_out.bias", [HIDDEN]],
  ];
  for (const [suffix, dims] of named) {
    out.push({ name: prefix + suffix, dims, data: table.get(prefix + suffix).data });
  }
}

/** Number of global layers: as many as every per-layer matrix shape has blocks. */
export function countLayers(table) {
  let n = 0;
  while (table.has(`core.model.transformer.h.${n}.ln_1.weight`)) n += 1;
  return n;
}

/**
 * Every tensor the library needs, as [{name, dims, data}], resolved from the
 * engine's weight tables {global, local} (EngineWeights, gpu.ts:294-298).
 * Returns the tensors plus the text vocabulary (rows of wte).
 */
export function resolveEngineTensors(tables) {
  const out = [];
  const g = tables.global;
  const layers = countLayers(g);
  for (let i = 0; i < layers; i += 1) layerTensors(g, `core.model.transformer.h.${i}.`, i, out);
  for (const n of ["core.model.transformer.ln_f.weight", "core.model.transformer.ln_f.bias"]) {
    out.push({ name: n, dims: [HIDDEN], data: g.get(n).data });
  }
  const wte = g.get("core.model.transformer.wte.weight");
  const vocab = wte.dims[0];
  out.push({ name: "core.model.transformer.wte.weight", dims: [vocab, HIDDEN], data: wte.data });
  for (let k = 0; k < N_VQ; k += 1) {
    const n = `core.model.audio_embeddings.${k}.weight`;
    out.push({ name: n, dims: [CODEBOOK, HIDDEN], data: g.get(n).data });
  }
  const l = tables.local;
  layerTensors(l, "model.local_transformer.h.0.", 0, out);
  for (const n of ["model.local_transformer.ln_f.weight", "model.local_transformer.ln_f.bias"]) {
    out.push({ name: n, dims: [HIDDEN], data: l.get(n).data });
  }
  out.push({
    name: "model.text_lm_head.weight",
    dims: [HIDDEN, vocab],
    data: pickMatrix(l, "model.text_lm_head.weight", `${HIDDEN}x${vocab}`, 0),
  });
  for (let k = 0; k < N_VQ; k += 1) {
    const n = `model.audio_lm_heads.${k}.weight`;
    out.push({ name: n, dims: [HIDDEN, CODEBOOK], data: pickMatrix(l, n, `${HIDDEN}x${CODEBOOK}`, k) });
  }
  return { tensors: out, vocab, layers };
}

/** The codec's default shape (codec.ts:1-30): layers and ring windows per stage. */
export const CODEC_SHAPE = { layersPerStage: [4, 2, 2, 4], contextPerStage: [500, 1696, 2480, 3248] };

const CODEC_D = 256;
const CODEC_DECODER = [1, 3, 5, 7];

/**
 * The codec's tensors under the names mb_codec_* uploads by, from the codec
 * WeightTable, resolved as resolveCodecWeights does (decodeWeights.ts:69-156):
 * a matrix by name when the table has it, else by shape and offset order --
 * the [256,768] run holds, stage by stage, each layer's attention input and
 * then the stage's output projection (the last stage's is [256,240]); the
 * [256,256], [256,1024] and [1024,256] runs hold one block per layer; stage 1
 * reads [192,256], the others [384,256] in order; the 16 RVQ convolutions are
 * the [512,8,1] run and the output projection the [768,512,1] block.
 * Norms, layer scales, quantiser biases and codebooks are taken by name.
 */
export function resolveCodecTensors(table, shape) {
  const layersPerStage = (shape || CODEC_SHAPE).layersPerStage;
  const out = [];
  const pick = (name, dims, list, index) => {
    const key = dims.join("x");
    if (table.has(name)) {
      const t = table.get(name);
      if (t.dims.join("x") !== key && !(t.dims.length === dims.length + 1 && t.dims[dims.length] === 1 &&
          t.dims.slice(0, dims.length).join("x") === key)) {
        throw new Error(`codec weight has the wrong shape: ${name} is ${t.dims.join("x")}, expected ${key}`);
      }
      return t.data;
    }
    if (!list[index]) throw new Error(`codec: no ${key} block at index ${index} for ${name}`);
    return list[index];
  };
  const named = (name, dims) => out.push({ name, dims, data: table.get(name).data });
  const wide = table.byShape(`${CODEC_D}x768`);
  const convs = table.byShape("512x8x1");
  for (let k = 0; k < N_VQ; k += 1) {
    const p = `model.quantizer.quantizers.${k}.`;
    out.push({ name: p + "out_proj.weight", dims: [512, 8], data: pick(p + "out_proj.weight", [512, 8], convs, k) });
    named(p + "out_proj.bias", [512]);
    named(p + "codebook.weight", [CODEBOOK, 8]);
  }
  out.push({
    name: "model.quantizer.output_proj.weight",
    dims: [768, 512],
    data: pick("model.quantizer.output_proj.weight", [768, 512], table.byShape("768x512x1"), 0),
  });
  named("model.quantizer.output_proj.bias", [768]);
  let cursor = 0;
  let layer = 0;
  const last = layersPerStage.length - 1;
  for (let s = 0; s < layersPerStage.length; s += 1) {
    const p = `model.decoder.${CODEC_DECODER[s]}.`;
    const inW = s === 0 ? 192 : 384;
    out.push({
      name: p + "input_proj.weight",
      dims: [inW, CODEC_D],
      data: pick(p + "input_proj.weight", [inW, CODEC_D], table.byShape(`${inW}x${CODEC_D}`), s === 0 ? 0 : s - 1),
    });
    for (let i = 0; i < layersPerStage[s]; i += 1, layer += 1) {
      const q = `${p}transformer.layers.${i}.`;
      const mats = [
        ["self_attn.in_proj.weight", [CODEC_D, 3 * CODEC_D], wide, cursor],
        ["self_attn.out_proj.weight", [CODEC_D, CODEC_D], table.byShape(`${CODEC_D}x${CODEC_D}`), layer],
        ["ffn.0.weight", [CODEC_D, 1024], table.byShape(`${CODEC_D}x1024`), layer],
        ["ffn.2.weight", [1024, CODEC_D], table.byShape(`1024x${CODEC_D}`), layer],
      ];
      for (const [suffix, dims, list, index] of mats) {
        out.push({ name: q + suffix, dims, data: pick(q + suffix, dims, list, index) });
      }
      cursor += 1;
      for (const n of ["norm1.weight", "norm1.bias", "norm2.weight", "norm2.bias",
                       "layer_scale_1.scale", "layer_scale_2.scale"]) named(q + n, [CODEC_D]);
    }
    const outW = s === last ? 240 : 768;
    const list = s === last ? table.byShape(`${CODEC_D}x240`) : wide;
    out.push({
      name: p + "output_proj.weight",
      dims: [CODEC_D, outW],
      data: pick(p + "output_proj.weight", [CODEC_D, outW], list, s === last ? 0 : cursor),
    });
    if (s !== last) cursor += 1;
  }
  return out;
}
