"""The JavaScript host engine on the GPU, through the N-API addon: the
reference runtime's frame loop on GpuTtsEngine and the batched
MultiVoiceEngine, each checked against the oracle on the same seeded model.

The weights travel as sidecar + manifest tables with the projections under
anonymous names, so the engine must resolve them by shape and offset order
as the reference's loaders do.  Bars: hidden states within 1e-4 (fp32 KV),
greedy codes compared frame by frame with the oracle teacher-forced by the
engine's codes (tests/frame_check.py; a code may differ only at an oracle
near tie within 2.4e-4), the non-wrapping ring's range error and the
decode-before-prefill error as the reference throws them.  The engine's
promises are asynchronous: the event loop runs while a prefill is on the
GPU, and a second call on the busy context is refused.
"""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from mockbird_amd import synth
from oracle import oracle
from conftest import rounded_weights, say, write_sidecar
from frame_check import FrameCheck

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
L, V, C, FRAMES = 2, 64, 128, 6
BAR = 2.4e-4
CODEC_LAYERS, CODEC_CONTEXT = (1, 1, 1, 2), (6, 12, 20, 40)


def _tables(w, tmp):
    glob, loc = [], []
    n_anon = 0
    for name, arr in w.items():
        anon = arr.ndim == 2 and not name.endswith("wte.weight") and "audio_embeddings" not in name
        key = f"onnx::MatMul_{n_anon}" if anon else name
        n_anon += anon
        (loc if name.startswith("model.") else glob).append((key, arr))
    write_sidecar(os.path.join(tmp, "global.json"), glob)
    write_sidecar(os.path.join(tmp, "local.json"), loc)


def _codec_table(cw, tmp):
    """The codec weights in the sidecar's order with every projection under an
    anonymous name and the 1x1 convolutions in their graph shape [., ., 1]."""
    entries = []
    for i, (name, arr) in enumerate(cw.items()):
        if name.endswith("out_proj.weight") and name.startswith("model.quantizer") or \
                name == "model.quantizer.output_proj.weight":
            entries.append((f"onnx::Conv_{i}", arr.reshape(arr.shape + (1,))))
        elif arr.ndim == 2 and "codebook" not in name:
            entries.append((f"onnx::MatMul_c{i}", arr))
        else:
            entries.append((name, arr))
    write_sidecar(os.path.join(tmp, "codec.json"), entries)


def _follow(m, prompt, js_frames, js_hiddens, chk, v, label):
    """The oracle teacher-forced by the engine's frames: every frame's codes
    checked by `chk`, then decoded at the next position; returns the oracle's
    prefill hidden and the largest hidden-state difference after a step."""
    st = oracle.ModelState(m, 1, C)
    h = st.prefill_all(0, prompt)[-1]
    h0 = h.copy()
    pos, worst = prompt.shape[0], 0.0
    for f, frame in enumerate(js_frames):
        frame = np.array(frame, np.int32)
        text2, logits = m.local_logits(h, frame)
        chk.frame(v, f"{label} frame {f}", frame, True, text2, logits, 1e-4, bar=BAR)
        h = st.decode_step(synth.frame_row(frame)[None], [pos])[0]
        if js_hiddens is not None:
            worst = max(worst, float(np.abs(np.array(js_hiddens[f], np.float32) - h).max()))
        pos += 1
    return h0, worst


def test_engine_runtime_loop_and_multivoice_match_oracle(tmp_path):
    if shutil.which("node") is None:
        pytest.fail("node is not installed")
    w = synth.model_weights(n_layers=L, vocab=V, seed=11, bias_std=0.02, ln_std=0.1)
    w["model.text_lm_head.weight"][:, 9] = w["model.text_lm_head.weight"][:, 7]  # never stops
    prompts = [synth.prompt(40 + b, n_frames=4 + 5 * b, n_text=6 + b, vocab=V) for b in range(3)]
    _tables(w, str(tmp_path))
    cw = synth.codec_weights(CODEC_LAYERS, seed=12)
    _codec_table(cw, str(tmp_path))
    codes1 = synth.codec_codes(31, 4, 1)
    codes3 = synth.codec_codes(32, 3, 3)
    spec = {"layers": L, "maxSlots": C, "frames": FRAMES, "prompts": [p.tolist() for p in prompts],
            "codec": {"layers": list(CODEC_LAYERS), "context": list(CODEC_CONTEXT),
                      "single": codes1[:, 0].tolist(), "multi": codes3.tolist()}}
    (tmp_path / "case.json").write_text(json.dumps(spec))
    say("JS engine: single-voice runtime loop + 3-voice MultiVoiceEngine")
    r = subprocess.run(["node", os.path.join(ROOT, "tests", "js", "engine_run.mjs"), str(tmp_path)],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert any("warmup" in m for m in out["log"])
    m = oracle.Model(w, n_layers=L, vocab=V)

    s = out["single"]
    chk = FrameCheck(1 + len(prompts))
    h0, worst = _follow(m, prompts[0], s["frames"], s["hiddens"], chk, 0, "single")
    assert np.abs(np.array(s["prefillHidden"], np.float32) - h0).max() < 1e-4
    assert worst < 1e-4
    st = oracle.ModelState(m, 1, C)
    st.prefill_all(0, prompts[0])
    k_ref = st.K[0, 0][:4]
    assert np.abs(np.array(s["layer0Key"], np.float32).reshape(4, 768) - k_ref).max() < 1e-4
    assert len(s["frames"]) == FRAMES and s["position"] == prompts[0].shape[0] + FRAMES
    assert s["rangeError"][0] == "MB_ERR_RANGE" and "exceeds the KV ring" in s["rangeError"][1]
    assert s["beforePrefill"] == "decodeStep before prefill"
    a = s["async"]
    say(f"  event-loop turns during one prefill: {a['ticks']}; overlapping call: {a['busy']}")
    assert a["ticks"] >= 1 and a["busy"] == "MB_ERR_BUSY"
    assert a["disposeBusy"] == "MB_ERR_BUSY" and a["disposedEarly"] is False

    mv = out["multi"]
    for b, p in enumerate(prompts):
        assert not mv["stopped"][b] and len(mv["frames"][b]) == FRAMES
        h0, _ = _follow(m, p, mv["frames"][b], None, chk, 1 + b, f"voice {b}")
        assert np.abs(np.array(mv["prefillHidden"][b], np.float32) - h0).max() < 1e-4, b
    chk.summary("JS engines")
    assert chk.codes_equal + chk.codes_tied == 16 * FRAMES * (1 + len(prompts))

    # the codec through GpuTtsEngine.decodeFrames (one voice, two calls) and
    # MultiVoiceEngine.decodeAudio (3 voices), fp32 rings: within 2e-5 of scale
    ora = oracle.CodecOracle(cw, 1, CODEC_LAYERS, CODEC_CONTEXT)
    want = ora.decode(codes1)[0]
    got = np.array(s["pcm"], np.float32)
    assert got.shape == want.shape
    assert np.abs(got - want).max() <= 2e-5 * np.abs(want).max()
    ora3 = oracle.CodecOracle(cw, 3, CODEC_LAYERS, CODEC_CONTEXT)
    want3 = ora3.decode(codes3)
    got3 = np.array(mv["pcm"], np.float32)
    assert got3.shape == want3.shape
    assert np.abs(got3 - want3).max() <= 2e-5 * np.abs(want3).max()
    say("  codec: decodeFrames and decodeAudio match the oracle")

    # bf16 K/V engines passed their warm-up (creation returned) with fp32 and
    # bf16 weights; their prefill is the oracle's within the bf16 bar, on
    # the bf16-rounded weights for weightDtype "bf16"
    assert [v["weightDtype"] for v in out["bf16"]] == ["f32", "bf16"]
    for v in out["bf16"]:
        wv = w if v["weightDtype"] == "f32" else rounded_weights(w)
        st = oracle.ModelState(oracle.Model(wv, n_layers=L, vocab=V), 1, C, kv_bf16=True)
        h0 = st.prefill_all(0, prompts[0])[-1]
        err = float(np.abs(np.array(v["prefillHidden"], np.float32) - h0).max())
        say(f"  bf16 K/V engine, {v['weightDtype']} weights: prefill within {err:.2e}")
        assert err < 2e-2 and v["frame"] is not None and len(v["frame"]) == 16
