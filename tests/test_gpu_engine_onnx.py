"""Row f3 on the GPU: weights that reach the engine as hand-encoded .onnx
graphs with .data sidecars (the published graphs' form) load through
loadOnnxTable into createGpuEngineFor (onnxWeights.ts:124-240 feeding
gpu.ts:316-388), and the engine's prefill and frame loop then match the
oracle run on the weights the graphs were written from.

The graphs hold their weights the three ways the published ones do
(external initialisers, an inline Constant, an Identity alias sharing a
LayerNorm scale) with the projections under anonymous onnx::MatMul_* names,
so the engine must resolve them by shape and sidecar order.  Bars: prefill
and decode hidden states within 1e-4 (fp32 KV); the codes compared frame by
frame with the oracle teacher-forced by the engine's codes
(tests/frame_check.py; a code may differ only at an oracle near tie within
2.4e-4).
"""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from mockbird_amd import synth
from oracle import oracle
from conftest import say
from frame_check import FrameCheck
from test_engine_onnx import _write

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
L, V, C, FRAMES = 2, 64, 128, 5
BAR = 2.4e-4


def test_onnx_graphs_drive_the_gpu_engine(tmp_path):
    if shutil.which("node") is None:
        pytest.fail("node is not installed")
    w = synth.model_weights(n_layers=L, vocab=V, seed=21, bias_std=0.02, ln_std=0.1)
    w["model.text_lm_head.weight"][:, 9] = w["model.text_lm_head.weight"][:, 7]  # never stops
    # the exported graph shares the LayerNorm scale of layer 1 with layer 0
    w["core.model.transformer.h.1.ln_1.weight"] = w["core.model.transformer.h.0.ln_1.weight"].copy()
    glob = {k: v for k, v in w.items() if not k.startswith("model.")}
    loc = {k: v for k, v in w.items() if k.startswith("model.")}
    anon = {k for k, v in w.items() if v.ndim == 2 and "wte" not in k and "audio_embeddings" not in k}
    _write(str(tmp_path / "global"), glob, anon,
           alias=("core.model.transformer.h.1.ln_1.weight", "core.model.transformer.h.0.ln_1.weight"),
           constant="core.model.transformer.ln_f.bias")
    _write(str(tmp_path / "local"), loc, anon)
    prompt = synth.prompt(77, n_frames=9, n_text=7, vocab=V)
    spec = {"layers": L, "maxSlots": C, "frames": FRAMES, "prompt": prompt.tolist()}
    (tmp_path / "case.json").write_text(json.dumps(spec))
    say("ONNX graphs -> loadOnnxTable -> createGpuEngineFor: prefill + frames")
    r = subprocess.run(["node", os.path.join(ROOT, "tests", "js", "engine_onnx_run.mjs"), str(tmp_path)],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["sources"] == {"alias": "alias", "constant": "inline-constant"}
    assert len(out["frames"]) == FRAMES

    m = oracle.Model(w, n_layers=L, vocab=V)
    st = oracle.ModelState(m, 1, C)
    h = st.prefill_all(0, prompt)[-1]
    assert np.abs(np.array(out["prefillHidden"], np.float32) - h).max() < 1e-4
    chk = FrameCheck(1)
    pos, worst = prompt.shape[0], 0.0
    for f, frame in enumerate(out["frames"]):
        frame = np.array(frame, np.int32)
        text2, logits = m.local_logits(h, frame)
        chk.frame(0, f"onnx frame {f}", frame, True, text2, logits, 1e-4, bar=BAR)
        h = st.decode_step(synth.frame_row(frame)[None], [pos])[0]
        worst = max(worst, float(np.abs(np.array(out["hiddens"][f], np.float32) - h).max()))
        pos += 1
    chk.summary("ONNX engine")
    say(f"  max |hidden diff| after a step: {worst:.2e}")
    assert worst < 1e-4
    assert chk.codes_equal + chk.codes_tied == 16 * FRAMES
