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
