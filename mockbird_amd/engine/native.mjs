// Loads the N-API binding of libmockbird_hip.so (built in-tree by
// `python -m mockbird_amd.build`).  There is no other backend: a missing or
// unloadable addon is an error, never a silent fallback.
import { createRequire } from "module";
import path from "path";
import { fileURLToPath } from "url";

const require = createRequire(import.meta.url);
const here = path.dirname(fileURLToPath(import.meta.url));

let cached = null;

/**
 * The addon's exports (create, prefill, decodeStep, localFrame, ...).
 * MB_HIP_ADDON names another build of the same addon (the host-sanitized one).
 */
export function loadNative() {
  if (cached) return cached;
  const file = process.env.MB_HIP_ADDON || path.join(here, "mockbird_hip.node");
  try {
    cached = require(file);
  } catch (error) {
    throw new Error(
      `${file} is not built or cannot load (build it with \`python -m mockbird_amd.build\`): ` +
        error.message,
    );
  }
  return cached;
}

/** Row width of the model's input rows: text id + 16 audio codes. */
export const ROW_WIDTH = 17;
export const N_VQ = 16;
export const HIDDEN = 768;
export const AUDIO_PAD_ID = 1024;

/** KV storage types of a context. */
export function kvDtypeCode(native, name) {
  if (name === undefined || name === "f32") return native.KV.F32;
  if (name === "bf16") return native.KV.BF16;
  throw new Error(`unknown kvDtype ${name} (expected "f32" or "bf16")`);
}

/** `value` unless it is undefined or null (Node 12 has no `??`). */
export function orDefault(value, fallback) {
  return value === undefined || value === null ? fallback : value;
}
