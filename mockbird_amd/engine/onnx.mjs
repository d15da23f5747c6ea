// Weight tables straight from the published .onnx graphs and their .data
// sidecars (onnxWeights.ts:1-240), with no graph executor: the engine only
// needs the initialisers, as views into the sidecar.
//
// A graph holds its weights three ways, and the table answers for all three:
//   - initialisers with external data: (location, offset, length) into the
//     sidecar -- zero-copy Float32Array views when 4-byte aligned;
//   - Constant nodes whose `value` tensor carries inline raw bytes (copied,
//     since a protobuf payload has no alignment);
//   - Identity nodes that alias one name to another (the exported graph
//     shares LayerNorm scales this way), followed up to 8 hops.
// byShape(dims) lists the external initialisers of one shape in sidecar
// order -- the order the anonymous `onnx::MatMul_*` projections are resolved
// by (prefill.ts:78-107, decodeWeights.ts:24-156).
import fs from "fs";

const FLOAT = 1; // TensorProto.DataType.FLOAT

/** Protobuf fields of `buf` as [number, wireType, value] (varint or bytes). */
function* fields(buf) {
  let i = 0;
  const varint = () => {
    let v = 0;
    let scale = 1;
    for (;;) {
      if (i >= buf.length) throw new Error("truncated protobuf varint");
      const byte = buf[i++];
      v += (byte & 0x7f) * scale;
      if (!(byte & 0x80)) return v;
      scale *= 128;
    }
  };
  while (i < buf.length) {
    const key = varint();
    const no = Math.floor(key / 8);
    const wire = key & 7;
    if (wire === 0) {
      yield [no, wire, varint()];
    } else if (wire === 2) {
      const len = varint();
      if (i + len > buf.length) throw new Error("truncated protobuf field");
      yield [no, wire, buf.subarray(i, i + len)];
      i += len;
    } else if (wire === 1 || wire === 5) {
      const len = wire === 1 ? 8 : 4;
      yield [no, wire, buf.subarray(i, i + len)];
      i += len;
    } else {
      throw new Error(`unsupported protobuf wire type ${wire}`);
    }
  }
}

function text(bytes) {
  return Buffer.from(bytes.buffer, bytes.byteOffset, bytes.byteLength).toString("utf8");
}

/** Packed varints (proto3 repeated int64) or a single unpacked one. */
function pushInts(out, wire, v) {
  if (wire === 0) {
    out.push(v);
    return;
  }
  for (const [, , x] of fields(concatVarints(v))) out.push(x);
}
// re-key a packed run as field-1 varints so fields() can read it
function concatVarints(bytes) {
  const out = [];
  let i = 0;
  while (i < bytes.length) {
    out.push(0x08);
    do {
      out.push(bytes[i]);
    } while (bytes[i++] & 0x80);
  }
  return Uint8Array.from(out);
}

/** A TensorProto: name, dims, data type, inline bytes, external-data keys. */
function tensorProto(buf) {
  const t = { name: "", dims: [], type: 0, raw: null, floats: null, external: {} };
  for (const [no, wire, v] of fields(buf)) {
    if (no === 1) pushInts(t.dims, wire, v);
    else if (no === 2) t.type = v;
    else if (no === 4 && wire === 2) t.floats = v; // packed float_data
    else if (no === 8) t.name = text(v);
    else if (no === 9) t.raw = v;
    else if (no === 13 && wire === 2) {
      let key = "";
      let value = "";
      for (const [k, , w] of fields(v)) {
        if (k === 1) key = text(w);
        else if (k === 2) value = text(w);
      }
      t.external[key] = value;
    }
  }
  return t;
}

/** `bytes` as f32, copied when the payload is not 4-byte aligned. */
function f32(bytes) {
  const n = bytes.byteLength >> 2;
  if (bytes.byteOffset % 4 === 0) return new Float32Array(bytes.buffer, bytes.byteOffset, n);
  return new Float32Array(Uint8Array.from(bytes.subarray(0, 4 * n)).buffer);
}

/**
 * A WeightTable over a model's bytes and its sidecar's bytes (both
 * Uint8Array): get(name) (following Identity aliases), has, names, size,
 * byShape(dims) over the external initialisers in sidecar order.  Only f32
 * tensors are kept (the engine's weights are all f32).
 */
export function openOnnx(model, sidecar) {
  let graph = null;
  for (const [no, , v] of fields(model)) if (no === 7) graph = v;
  if (!graph) throw new Error("model has no GraphProto");
  const tensors = new Map();
  const aliases = new Map();
  const add = (t) => {
    if (!tensors.has(t.name)) tensors.set(t.name, t);
  };
  const inline = (p) => (p.raw && p.raw.byteLength >= 4 ? f32(p.raw) : p.floats ? f32(p.floats) : null);
  for (const [no, , v] of fields(graph)) {
    if (no === 5) {
      const p = tensorProto(v);
      if (p.type !== FLOAT) continue;
      if (p.external.location !== undefined) {
        const offset = Number(p.external.offset || 0);
        const count = p.dims.reduce((a, b) => a * b, 1);
        const length = p.external.length !== undefined ? Number(p.external.length) : 4 * count;
        if (length !== 4 * count || offset + length > sidecar.byteLength) {
          throw new Error(`initialiser ${p.name}: ${length} bytes at ${offset} do not fit the sidecar`);
        }
        add({ name: p.name, dims: p.dims, data: f32(sidecar.subarray(offset, offset + length)),
              source: "external", offset });
      } else {
        const data = inline(p);
        if (data) add({ name: p.name, dims: p.dims, data, source: "inline-raw", offset: -1 });
      }
    } else if (no === 1) {
      let op = "";
      const ins = [];
      const outs = [];
      const values = [];
      for (const [k, , w] of fields(v)) {
        if (k === 1) ins.push(text(w));
        else if (k === 2) outs.push(text(w));
        else if (k === 4) op = text(w);
        else if (k === 5) {
          let attr = "";
          let t = null;
          for (const [x, , y] of fields(w)) {
            if (x === 1) attr = text(y);
            else if (x === 5) t = y;
          }
          if (attr === "value" && t) values.push(t);
        }
      }
      if (op === "Identity" && ins.length === 1 && outs.length === 1) aliases.set(outs[0], ins[0]);
      if (op === "Constant") {
        for (const bytes of values) {
          const p = tensorProto(bytes);
          const data = p.type === FLOAT ? inline(p) : null;
          if (!data) continue;
          for (const o of outs) add({ name: o, dims: p.dims, data, source: "inline-constant", offset: -1 });
        }
      }
    }
  }
  const resolve = (name) => {
    let cur = name;
    for (let hop = 0; hop < 8; hop += 1) {
      if (tensors.has(cur)) return cur;
      const next = aliases.get(cur);
      if (next === undefined) break;
      cur = next;
    }
    return cur;
  };
  for (const [alias, target] of aliases) {
    if (tensors.has(alias)) continue;
    const t = tensors.get(resolve(target));
    if (t) tensors.set(alias, Object.assign({}, t, { name: alias, source: "alias" }));
  }
  const external = [...tensors.values()]
    .filter((t) => t.source === "external")
    .sort((a, b) => a.offset - b.offset);
  return {
    get(name) {
      const t = tensors.get(resolve(name));
      if (!t) throw new Error(`weight not uploaded: ${name}`);
      return t;
    },
    has(name) {
      return tensors.has(resolve(name));
    },
    names() {
      return [...tensors.keys()];
    },
    get size() {
      return tensors.size;
    },
    byShape(dims) {
      return external.filter((t) => t.dims.join("x") === dims).map((t) => t.data);
    },
  };
}

/** openOnnx over files: the .onnx graph and its external-data sidecar. */
export function loadOnnxTable(onnxPath, dataPath) {
  const model = fs.readFileSync(onnxPath);
  const data = fs.readFileSync(dataPath);
  return openOnnx(new Uint8Array(model.buffer, model.byteOffset, model.byteLength),
                  new Uint8Array(data.buffer, data.byteOffset, data.byteLength));
}
