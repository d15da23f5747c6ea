"""Pin the oracle's RoPE against the reference's own ORT captures.

tests/golden/ort_layer0_rope.npz holds the rows of the reference fixtures
prefill-{8,195}rows-layer0-{k,v}.f32 (ORT 1.30.0 running moss_tts_prefill.onnx)
whose prompt ids repeat.  Layer 0's K/V depend on the row's ids only, so a
group of equal-id rows carries one un-roped k at several positions: K[p] =
R(p) k and V[p] = v.  Rotating the first row of a group back and forward to
every other position with the oracle's RoPE must land on the captured values
to fp32 rounding.  The same check run with the plausible wrong conventions
(opposite sign, half-split pairing, fp64 angle, correctly-rounded inv_freq)
misses by orders of magnitude more, so the fixture discriminates them.
"""
import os

import numpy as np
import pytest

from oracle import oracle

FIX = os.path.join(os.path.dirname(__file__), "golden", "ort_layer0_rope.npz")


def _groups(ids, rows):
    g = {}
    for i in range(ids.shape[0]):
        g.setdefault(ids[i].tobytes(), []).append(i)
    return [v for v in g.values() if len(v) > 1]


def _rot_pairs(x, ang, sign=1.0, interleaved=True):
    """Rotate 64-wide heads by per-pair angles in float64 (test-side model)."""
    x = x.astype(np.float64).reshape(12, 64)
    if interleaved:
        a, b = x[:, 0::2], x[:, 1::2]
    else:
        a, b = x[:, :32], x[:, 32:]
    c, s = np.cos(ang), np.sin(sign * ang)
    oa, ob = a * c - b * s, b * c + a * s
    out = np.empty_like(x)
    if interleaved:
        out[:, 0::2], out[:, 1::2] = oa, ob
    else:
        out[:, :32], out[:, 32:] = oa, ob
    return out.reshape(768)


def _angles(pos, table, fp32=True):
    if fp32:
        return (np.float32(pos) * table.astype(np.float32)).astype(np.float64)
    return pos * table.astype(np.float64)


def _residual(predict):
    d = np.load(FIX)
    worst = 0.0
    for n in (8, 195):
        rows, ids, K = d[f"rows{n}"], d[f"ids{n}"], d[f"k{n}"]
        for grp in _groups(ids, rows):
            i0 = grp[0]
            for j in grp[1:]:
                pred = predict(K[i0], int(rows[i0]), int(rows[j]))
                worst = max(worst, float(np.abs(pred - K[j].astype(np.float64)).max()))
    return worst


def test_fixture_has_repeated_rows():
    d = np.load(FIX)
    assert len(_groups(d["ids195"], d["rows195"])) >= 2
    assert d["rows195"].max() >= 190  # positions up to 194 exercise the fp32 angle


def test_values_are_stored_unrotated():
    """V of equal-id rows is bit-identical at every position: V is not roped
    (kernels-decode.ts:240, ROPE_SPLIT_RING writes v raw)."""
    d = np.load(FIX)
    for n in (8, 195):
        for grp in _groups(d[f"ids{n}"], d[f"rows{n}"]):
            V = d[f"v{n}"][grp]
            assert np.array_equal(V, np.broadcast_to(V[0], V.shape))


def test_oracle_rope_reproduces_ort_keys():
    table = oracle.inv_freq()

    def predict(k_first, p0, p1):
        # undo the capture's rotation at p0 (float64), then re-rotate with the oracle at p1
        k_raw = _rot_pairs(k_first, -_angles(p0, table))
        return oracle.rope(k_raw.astype(np.float32), p1).astype(np.float64)

    err = _residual(predict)
    assert err < 2e-6, err


@pytest.mark.parametrize("name,sign,interleaved,fp32,rounded", [
    ("opposite sign (kernels.test.mjs:240)", -1.0, True, True, False),
    ("half-split pairing", 1.0, False, True, False),
    ("fp64 angle", 1.0, True, False, False),
    ("correctly rounded inv_freq", 1.0, True, True, True),
])
def test_wrong_conventions_miss_the_fixture(name, sign, interleaved, fp32, rounded):
    table = oracle.inv_freq()
    if rounded:
        table = (10000.0 ** (-(2 * np.arange(32)) / 64.0)).astype(np.float32)

    def predict(k_first, p0, p1):
        k_raw = _rot_pairs(k_first, -_angles(p0, table, fp32), sign, interleaved)
        return _rot_pairs(k_raw, _angles(p1, table, fp32), sign, interleaved)

    assert _residual(predict) > 4e-6, name


def test_inv_freq_is_torchs_fp32_table():
    torch = pytest.importorskip("torch")
    t = (1.0 / (10000 ** (torch.arange(0, 64, 2).float() / 64))).numpy()
    assert np.array_equal(t.view(np.uint32), oracle.inv_freq().view(np.uint32))
