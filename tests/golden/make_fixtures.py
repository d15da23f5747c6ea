"""Extract the reference's own ORT captures that pin RoPE into a small fixture.

    python tests/golden/make_fixtures.py

Reads /root/reference/tests/fixtures/golden/prefill-{8,195}rows-{ids,layer0-k,
layer0-v} (captured by the reference from moss_tts_prefill.onnx under
onnxruntime-node 1.30.0, see prefill-reference.json) and keeps only the rows
whose prompt ids repeat: layer 0 sees the same input embedding for equal ids,
so those rows carry one un-roped k (and one v) at several positions.  That is
what fixes the RoPE convention (sign, pairing, fp32 angle, inv_freq table)
against the graph without the model weights.  Output: ort_layer0_rope.npz.
"""
import os

import numpy as np

SRC = "/root/reference/tests/fixtures/golden"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ort_layer0_rope.npz")


def main():
    data = {}
    for n in (8, 195):
        ids = np.fromfile(f"{SRC}/prefill-{n}rows-ids.u32", dtype=np.uint32).reshape(n, 17)
        k = np.fromfile(f"{SRC}/prefill-{n}rows-layer0-k.f32", dtype=np.float32).reshape(n, 768)
        v = np.fromfile(f"{SRC}/prefill-{n}rows-layer0-v.f32", dtype=np.float32).reshape(n, 768)
        groups = {}
        for r in range(n):
            groups.setdefault(ids[r].tobytes(), []).append(r)
        rows = sorted(r for g in groups.values() if len(g) > 1 for r in g)
        data[f"rows{n}"] = np.array(rows, np.int32)
        data[f"ids{n}"] = ids[rows]
        data[f"k{n}"] = k[rows]
        data[f"v{n}"] = v[rows]
    np.savez_compressed(OUT, **data)
    print(OUT, {k: v.shape for k, v in data.items()})


if __name__ == "__main__":
    main()
