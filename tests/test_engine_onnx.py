"""The engine's ONNX weight loader (mockbird_amd/engine/onnx.mjs) on
hand-built graphs: the three ways the published graphs hold their weights
(onnxWeights.ts:1-240) -- initialisers with external data in a sidecar,
a Constant node with an inline (unaligned) payload, an Identity alias -- and
anonymous `onnx::MatMul_*` projections resolved by shape and sidecar order.
Every resolved tensor must equal the weight it was written from, bit for bit.

The graphs are encoded here with a minimal protobuf writer (ModelProto field
7 = graph; GraphProto 1 = node, 5 = initializer; NodeProto 1/2 = input/output,
4 = op_type, 5 = attribute; AttributeProto 1 = name, 5 = t; TensorProto 1 =
dims, 2 = data_type, 8 = name, 9 = raw_data, 13 = external_data,
14 = data_location), the ONNX schema's field numbers.
"""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from mockbird_amd import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _varint(n: int) -> bytes:
    out = bytearray()
    while True:
        b = n & 0x7F
        n >>= 7
        out.append(b | (0x80 if n else 0))
        if not n:
            return bytes(out)


def _f(no: int, v) -> bytes:
    if isinstance(v, int):
        return _varint(no << 3) + _varint(v)
    v = v.encode() if isinstance(v, str) else bytes(v)
    return _varint(no << 3 | 2) + _varint(len(v)) + v


def _tensor(name, dims, raw=None, external=None) -> bytes:
    b = b"".join(_f(1, d) for d in dims) + _f(2, 1) + _f(8, name)
    if raw is not None:
        b += _f(9, raw)
    if external is not None:
        for k, v in (("location", external[0]), ("offset", str(external[1])),
                     ("length", str(external[2]))):
            b += _f(13, _f(1, k) + _f(2, v))
        b += _f(14, 1)
    return b


def _node(op, ins, outs, value=None) -> bytes:
    b = b"".join(_f(1, i) for i in ins) + b"".join(_f(2, o) for o in outs) + _f(4, op)
    if value is not None:
        b += _f(5, _f(1, "value") + _f(5, value) + _f(20, 4))
    return b


def _write(path, weights, anon, alias=None, constant=None):
    """weights: name -> array in sidecar order; anon: names stored as onnx::MatMul_*;
    alias: (name, target) as an Identity node; constant: a name stored inline."""
    data = bytearray()
    graph = b""
    n = 0
    for name, a in weights.items():
        if alias and name == alias[0]:
            continue
        a = np.ascontiguousarray(a, "<f4")
        if constant and name == constant:
            graph += _f(1, _node("Constant", [], [name], _tensor("", a.shape, raw=a.tobytes())))
            continue
        key = f"onnx::MatMul_{n}" if name in anon else name
        n += name in anon
        off = len(data)
        data += a.tobytes()
        graph += _f(5, _tensor(key, a.shape, external=(os.path.basename(path) + ".data", off, a.nbytes)))
    if alias:
        graph += _f(1, _node("Identity", [alias[1]], [alias[0]]))
    # a non-float initialiser the loader must skip
    graph += _f(5, _varint(1 << 3) + _varint(3) + _f(2, 7) + _f(8, "some_int64"))
    with open(path + ".onnx", "wb") as f:
        f.write(_f(1, 8) + _f(7, graph))
    with open(path + ".data", "wb") as f:
        f.write(bytes(data))


def test_onnx_tables_resolve_bit_exact(tmp_path):
    node = shutil.which("node")
    if node is None:
        pytest.fail("node is not installed")
    w = synth.model_weights(n_layers=2, vocab=16, seed=3, bias_std=0.1, ln_std=0.1)
    # the exported graph shares the LayerNorm scale of layer 1 with layer 0
    w["core.model.transformer.h.1.ln_1.weight"] = w["core.model.transformer.h.0.ln_1.weight"].copy()
    glob = {k: v for k, v in w.items() if not k.startswith("model.")}
    loc = {k: v for k, v in w.items() if k.startswith("model.")}
    anon = {k for k, v in w.items() if v.ndim == 2 and "wte" not in k and "audio_embeddings" not in k}
    _write(str(tmp_path / "global"), glob, anon,
           alias=("core.model.transformer.h.1.ln_1.weight", "core.model.transformer.h.0.ln_1.weight"),
           constant="core.model.transformer.ln_f.bias")
    _write(str(tmp_path / "local"), loc, anon)
    r = subprocess.run([node, os.path.join(ROOT, "tests", "js", "onnx_resolve.mjs"), str(tmp_path)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-3000:]
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["vocab"] == 16 and out["layers"] == 2
    assert out["sources"] == {"alias": "alias", "constant": "inline-constant", "external": "external"}
    blob = np.fromfile(tmp_path / "resolved.bin", dtype="<f4")
    off = 0
    for name, dims, count in out["index"]:
        got = blob[off:off + count].reshape(dims)
        off += count
        assert np.array_equal(got, w[name]), name
    assert off == blob.size
    assert len(out["index"]) == len(w)
