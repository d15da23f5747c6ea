// GPU driver of the JavaScript host: runs the reference runtime's loop
// (runtime.ts:523-561: reset, prefill, then nextFrame -> decodeStep per
// frame) through GpuTtsEngine, then the batched MultiVoiceEngine, and prints
// one JSON object with every result for the Python test to check.
//
//   node engine_run.mjs <dir>   (dir holds global.json, local.json, case.json)
import fs from "fs";
import path from "path";

import { createGpuEngineFor, frameRowFrom } from "../../mockbird_amd/engine/gpu.mjs";
import { createMultiVoiceEngine } from "../../mockbird_amd/engine/multivoice.mjs";
import { loadSidecarTable } from "../../mockbird_amd/engine/weights.mjs";

const dir = process.argv[2];
const spec = JSON.parse(fs.readFileSync(path.join(dir, "case.json"), "utf8"));
const tables = {
  global: loadSidecarTable(path.join(dir, "global.json")),
  local: loadSidecarTable(path.join(dir, "local.json")),
  codec: loadSidecarTable(path.join(dir, "codec.json")),
};
const codecShape = { layersPerStage: spec.codec.layers, contextPerStage: spec.codec.context };
const localHead = { audioEndTokenId: 7, audioAssistantSlotTokenId: 9, repetitionPenalty: 1.2 };
const out = { log: [] };
const log = (m) => {
  out.log.push(m);
  console.error(m);
};

async function single() {
  const engine = await createGpuEngineFor(tables, log, {
    localHead,
    maxSlots: spec.maxSlots,
    layers: spec.layers,
    codecShape,
  });
  const prompt = spec.prompts[0];
  engine.reset();
  let hidden = await engine.prefill({ inputIds: prompt, attentionMask: [prompt.map(() => 1)] });
  const res = { prefillHidden: Array.from(hidden), frames: [], hiddens: [] };
  const cache = await engine.prefillRunner.readLayerCache(0, prompt.length);
  res.layer0Key = Array.from(cache.key.subarray(0, 4 * 768));
  for (let step = 0; step < spec.frames; step += 1) {
    const frame = await engine.nextFrame(hidden);
    if (!frame) {
      res.stopped = step;
      break;
    }
    res.frames.push(frame);
    hidden = await engine.decodeStep({ row: frameRowFrom(9, frame), position: prompt.length + step });
    res.hiddens.push(Array.from(hidden));
  }
  res.position = engine.position;
  // the engine's calls run off the JS thread: the event loop keeps turning
  // while a prefill runs, and another call on the busy context is refused
  let ticks = 0;
  let running = true;
  const spin = () => {
    if (!running) return;
    ticks += 1;
    setImmediate(spin);
  };
  setImmediate(spin);
  const pending = engine.prefill({ inputIds: prompt, attentionMask: [prompt.map(() => 1)] });
  let busy = null;
  try {
    engine.native.readRing(engine.handle, 0, 0, 0, 1);
  } catch (e) {
    busy = e.code;
  }
  // dispose while the prefill is in flight is refused and leaves the engine usable
  let disposeBusy = null;
  try {
    engine.dispose();
  } catch (e) {
    disposeBusy = e.code;
  }
  await pending;
  running = false;
  res.async = { ticks, busy, disposeBusy, disposedEarly: engine.disposed };
  // the codec: the voice's code frames over two calls (the rings carry over)
  const codes = spec.codec.single;
  const a = await engine.decodeFrames(codes.slice(0, 2));
  const b = await engine.decodeFrames(codes.slice(2));
  res.pcm = [0, 1].map((c) => Array.from(a[c]).concat(Array.from(b[c])));
  // the reference's ring never wraps: a position past it throws (decode.ts:719-724)
  try {
    await engine.decodeStep({ row: frameRowFrom(9, res.frames[0]), position: spec.maxSlots });
    res.rangeError = null;
  } catch (e) {
    res.rangeError = [e.code, e.message];
  }
  engine.reset();
  try {
    await engine.decodeStep({ row: frameRowFrom(9, res.frames[0]), position: 0 });
    res.beforePrefill = null;
  } catch (e) {
    res.beforePrefill = e.message;
  }
  engine.dispose();
  return res;
}

async function multi() {
  const engine = await createMultiVoiceEngine(tables, log, {
    localHead,
    maxVoices: spec.prompts.length,
    capacity: spec.maxSlots,
    kvDtype: "f32",
    codecShape,
    codecKvDtype: "f32",
  });
  const hidden = await engine.prefill(spec.prompts);
  const gen = await engine.generate(spec.frames);
  const audio = await engine.decodeAudio(spec.codec.multi);
  engine.dispose();
  return {
    prefillHidden: hidden.map((h) => Array.from(h)),
    frames: gen.frames,
    stopped: gen.stopped,
    pcm: audio.map((ch) => ch.map((x) => Array.from(x))),
  };
}

// Engines with bf16 K/V rings, fp32 and bf16 weights: creation runs the
// warm-up (its decode-vs-prefill check then compares fp32 decode attention
// with the bf16 prefill path), then the prompt's prefill and one frame.
async function bf16Variants() {
  const res = [];
  for (const weightDtype of ["f32", "bf16"]) {
    const engine = await createGpuEngineFor({ global: tables.global, local: tables.local }, log, {
      localHead,
      maxSlots: spec.maxSlots,
      layers: spec.layers,
      kvDtype: "bf16",
      weightDtype,
      penaltyPrecision: weightDtype === "bf16" ? "f32" : "f64",
    });
    const prompt = spec.prompts[0];
    const hidden = await engine.prefill({ inputIds: prompt, attentionMask: [prompt.map(() => 1)] });
    const frame = await engine.nextFrame(hidden);
    engine.dispose();
    res.push({ weightDtype, prefillHidden: Array.from(hidden), frame });
  }
  return res;
}

// Node 12 has no top-level await
(async () => {
  out.single = await single();
  out.multi = await multi();
  out.bf16 = await bf16Variants();
  console.log(JSON.stringify(out));
})().catch((error) => {
  console.error(error && error.stack ? error.stack : error);
  process.exit(1);
});
