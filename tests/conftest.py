import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")


def say(msg: str) -> None:
    """Print and flush a progress line (names the case before each GPU step)."""
    print(msg, flush=True)


@pytest.fixture
def rng():
    return np.random.default_rng(0x2F6E2B1)


def write_sidecar(manifest_path: str, tensors) -> None:
    """Write (name, float32 array) pairs as one raw little-endian f32 sidecar
    plus its JSON manifest {"data", "tensors": [{"name", "dims", "offset"}]},
    in the given order (the order anonymous projections are resolved by)."""
    import json

    data_path = manifest_path + ".data"
    entries, off = [], 0
    with open(data_path, "wb") as f:
        for name, arr in tensors:
            a = np.ascontiguousarray(arr, dtype="<f4")
            f.write(a.tobytes())
            entries.append({"name": name, "dims": list(a.shape), "offset": off})
            off += a.nbytes
    with open(manifest_path, "w") as f:
        json.dump({"data": os.path.basename(data_path), "tensors": entries}, f)


BF16_ROUNDED = ("attn.c_attn.weight", "attn.c_proj.weight", "mlp.fc_in.weight", "mlp.fc_out.weight")


def rounded_weights(w):
    """The model as bf16 weight storage holds it: every layer's projection
    matrices and the audio heads rounded to bf16 (round to nearest even),
    everything else as uploaded."""
    from oracle import oracle

    out = dict(w)
    for name, a in w.items():
        if name.endswith(BF16_ROUNDED) or name.startswith("model.audio_lm_heads."):
            out[name] = oracle.bf16_round(a)
    return out
