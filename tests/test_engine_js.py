"""The JavaScript host engine on the CPU: the N-API addon loads under Node and
exports every binding, the engine modules import, anonymous projections
resolve by shape and offset order, and argument errors throw before any
device call."""
import json
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ADDON = os.path.join(ROOT, "mockbird_amd", "engine", "mockbird_hip.node")
BINDINGS = {
    "KV", "abiVersion", "cancel", "clearSeen", "create", "decodeAttention", "decodeFrames",
    "decodeStep", "destroy", "deviceBytes", "lastError", "localFrame", "localSteps", "prefill",
    "prefillAttention", "readRing", "writeRing", "ringAppend", "ringPoison", "ringReset", "ringWriteRows",
    "setLocalHead", "setWeightStorage", "setPenaltyPrecision", "uploadTensor", "codecInit", "codecReset", "codecDecode",
    "prefillAsync", "decodeStepAsync", "localFrameAsync", "decodeFramesAsync", "codecDecodeAsync",
}


def _node():
    node = shutil.which("node")
    if node is None:
        pytest.fail("node is not installed; the JavaScript host cannot be checked")
    if not os.path.exists(ADDON):
        pytest.fail("mockbird_hip.node is not built (python -m mockbird_amd.build)")
    return node


@pytest.fixture(scope="module")
def report():
    r = subprocess.run([_node(), os.path.join(ROOT, "tests", "js", "engine_cpu.mjs")],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout.strip().splitlines()[-1])


def test_addon_exports_every_binding(report):
    assert set(report["exports"]) == BINDINGS
    assert report["abi"] == 2


def test_tables_resolve_by_name_then_shape(report):
    tags = report["tags"]
    got = {name: (dims, tag) for name, dims, tag in report["resolved"]}
    assert report["vocab"] == 16 and report["layers"] == 2
    # layer 0's c_attn is named; layer 1's is the second [768,2304] block by offset
    assert got["core.model.transformer.h.0.attn.c_attn.weight"][1] == \
        tags["core.model.transformer.h.0.attn.c_attn.weight"]
    anon = sorted((t, n) for n, t in tags.items() if n.startswith("onnx::MatMul_"))
    assert got["core.model.transformer.h.1.attn.c_attn.weight"][1] == anon[3][0]
    # the local head's text head is its only [768, vocab] block, audio heads in order
    assert got["model.text_lm_head.weight"] == ([768, 16], tags["onnx::MatMul_text"])
    for k in range(16):
        assert got[f"model.audio_lm_heads.{k}.weight"][1] == tags[f"onnx::MatMul_audio_{k}"]
    # biases and LayerNorm parameters come by name
    assert got["model.local_transformer.h.0.mlp.fc_in.bias"][1] == \
        tags["model.local_transformer.h.0.mlp.fc_in.bias"]
    assert len(report["resolved"]) == 2 * 12 + 2 + 1 + 16 + 12 + 2 + 1 + 16


def test_rows_are_padded_with_the_audio_pad(report):
    s = report["staged"]
    assert s[:17] == [6] + [1024] * 16
    assert s[17:34] == [8, 1, 2, 3] + [1024] * 13
    assert report["frameRow"] == [9, 5, 6, 7] + [1024] * 13
    assert report["emptyPrompt"] == "prefill called with no rows"


def test_errors_throw_before_device_calls(report):
    e = report["errors"]
    assert e["badConfig"][0] == "MB_ERR_ARG"
    assert e["badHandle"][0] == "TypeError"
    assert e["badHandleAsync"][0] == "TypeError"  # thrown before a Promise is made
    assert e["notImplemented"] == [True, "EngineNotImplemented"]
    assert e["destroyBad"] == "TypeError"
    # malformed configurations: non-objects and non-numbers are type errors,
    # fractional / non-finite / huge numbers range errors, out-of-range values
    # the library's MB_ERR_ARG; the two valid ones reach the device (no GPU
    # here: MB_ERR_HIP; a GPU host creates and destroys them)
    c = e["createCases"]
    assert c[:3] == ["ERR_INVALID_ARG_TYPE"] * 3 and c[4] == "ERR_INVALID_ARG_TYPE"
    assert c[5] == c[6] == c[8] == "ERR_OUT_OF_RANGE"
    assert c[7] == c[9] == c[10] == c[11] == "MB_ERR_ARG"
    assert c[3] in ("MB_ERR_HIP", "created") and c[12] in ("MB_ERR_HIP", "created")


def test_codec_table_resolves_by_shape_and_order(report):
    """resolveCodecTensors follows resolveCodecWeights (decodeWeights.ts:69-156):
    the [256,768] run alternates layer inputs and stage outputs, the per-layer
    runs go by layer, the RVQ convolutions by quantiser."""
    tags = report["tags"]
    got = {name: (dims, tag) for name, dims, tag in report["codec"]}
    dec = (1, 3, 5, 7)
    layers = (2, 1, 1, 2)
    for k in range(16):
        assert got[f"model.quantizer.quantizers.{k}.out_proj.weight"] == ([512, 8], tags[f"onnx::Conv_rvq_{k}"])
        assert got[f"model.quantizer.quantizers.{k}.codebook.weight"][1] == \
            tags[f"model.quantizer.quantizers.{k}.codebook.weight"]
    assert got["model.quantizer.output_proj.weight"] == ([768, 512], tags["onnx::Conv_rvq_out"])
    for s in range(4):
        p = f"model.decoder.{dec[s]}."
        assert got[p + "input_proj.weight"][1] == tags[f"onnx::MatMul_in_{s}"]
        assert got[p + "output_proj.weight"] == ([256, 240 if s == 3 else 768], tags[f"onnx::MatMul_out_{s}"])
        for i in range(layers[s]):
            q = p + f"transformer.layers.{i}."
            assert got[q + "self_attn.in_proj.weight"][1] == tags[f"onnx::MatMul_qkv_{s}_{i}"]
            assert got[q + "self_attn.out_proj.weight"][1] == tags[f"onnx::MatMul_o_{s}_{i}"]
            assert got[q + "ffn.0.weight"][1] == tags[f"onnx::MatMul_f0_{s}_{i}"]
            assert got[q + "ffn.2.weight"][1] == tags[f"onnx::MatMul_f2_{s}_{i}"]
            assert got[q + "layer_scale_2.scale"][1] == tags[q + "layer_scale_2.scale"]
    assert len(got) == 16 * 3 + 2 + 4 * 2 + sum(layers) * 10
