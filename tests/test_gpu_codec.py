"""GPU parity of the batched codec decoder (mb_codec_*) against the oracle.

The oracle decodes one voice one position at a time through rings of
exactly `context` slots, as the reference's CodecRunner does
(codec.ts:470-765); the GPU decodes all voices and all of a stage's
positions per launch through rings with one frame of slack slots.  The
visible window of every query is the same, so the PCM must agree:

- fp32 rings: within 2e-5 of the output's scale (fp32 MFMA products against
  the oracle's double sums through up to 12 layers; measured 6e-7);
- bf16 rings: within 1e-3 of the scale (K and V rounded to bf16 on store, in
  the oracle as well; a value the two round differently moves by one bf16
  step; measured 1e-5).

Small windows (6, 12, 20, 40 positions) make every ring wrap within a few
frames; the full-size cases run the real stage shapes (4, 2, 2, 4 layers,
windows 500 / 1696 / 2480 / 3248), for 3 frames and for long runs at the
benchmark's voice counts in which the rings fill and wrap.
"""
import numpy as np
import pytest

import mockbird_amd as mb
from mockbird_amd import synth
from oracle import oracle
from conftest import say

pytestmark = pytest.mark.gpu

SMALL_LAYERS = (2, 1, 1, 2)
SMALL_CTX = (6, 12, 20, 40)


def _ctx():
    return mb.Context(n_layers=1, capacity=16, max_seqs=1, max_rows=16)


def _close(got, want, rel, what):
    scale = float(np.abs(want).max())
    err = float(np.abs(got - want).max())
    assert err <= rel * scale, (what, err, scale)
    return err / scale


@pytest.mark.parametrize("kv", [mb.MB_KV_F32, mb.MB_KV_BF16])
def test_codec_small_windows_wrap(kv):
    """3 voices, 9 frames over two calls; every stage's ring wraps."""
    say(f"codec small windows kv={kv}")
    B = 3
    w = synth.codec_weights(SMALL_LAYERS, seed=11)
    codes = synth.codec_codes(12, 9, B)
    ora = oracle.CodecOracle(w, B, SMALL_LAYERS, SMALL_CTX, kv_bf16=(kv == mb.MB_KV_BF16))
    want = ora.decode(codes)
    with _ctx() as ctx:
        ctx.upload_all(w)
        ctx.codec_init(B, SMALL_LAYERS, SMALL_CTX, kv_dtype=kv)
        got = np.concatenate([ctx.codec_decode(codes[:4]), ctx.codec_decode(codes[4:])], axis=2)
    rel = 2e-5 if kv == mb.MB_KV_F32 else 1e-3
    for b in range(B):
        r = _close(got[b], want[b], rel, f"voice {b}")
        say(f"  voice {b}: max error / scale {r:.2e}")


def test_codec_ring_contents_match_by_position():
    """The rings hold the same K/V per absolute position as the oracle's
    (the GPU's extra slots hold older positions, outside every window)."""
    say("codec ring contents")
    B = 2
    w = synth.codec_weights(SMALL_LAYERS, seed=13)
    codes = synth.codec_codes(14, 5, B)
    ora = oracle.CodecOracle(w, B, SMALL_LAYERS, SMALL_CTX)
    ora.decode(codes)
    with _ctx() as ctx:
        ctx.upload_all(w)
        ctx.codec_init(B, SMALL_LAYERS, SMALL_CTX)
        ctx.codec_decode(codes)
        for layer in range(sum(SMALL_LAYERS)):
            for b in range(B):
                k, v, sp = ctx.codec_read_ring(layer, b)
                ko, vo, spo = ora.layer_ring(layer, b)
                live = {int(p): j for j, p in enumerate(spo) if p >= 0}
                mine = {int(p): j for j, p in enumerate(sp) if p >= 0}
                assert set(live) <= set(mine), (layer, b)
                # the GPU keeps exactly the window plus one frame of positions
                newest = max(mine)
                assert min(mine) >= newest - len(sp) + 1, (layer, b)
                for p, j in live.items():
                    g = mine[p]
                    scale = max(1.0, float(np.abs(ko[j]).max()))
                    assert np.abs(k[g] - ko[j]).max() <= 1e-4 * scale, (layer, b, p)
                    assert np.abs(v[g] - vo[j]).max() <= 1e-4 * scale, (layer, b, p)


def test_codec_reset_one_voice():
    """A voice reset mid-stream decodes exactly like a fresh one while the
    other voice continues exactly where it was (every kernel computes each
    voice's rows from that voice's data alone, so both are bit-identical)."""
    say("codec reset one voice")
    B = 2
    w = synth.codec_weights(SMALL_LAYERS, seed=15)
    codes = synth.codec_codes(16, 6, B)
    with _ctx() as ctx:
        ctx.upload_all(w)
        ctx.codec_init(B, SMALL_LAYERS, SMALL_CTX)
        whole = ctx.codec_decode(codes)
        ctx.codec_reset()
        first = ctx.codec_decode(codes[:3])
        ctx.codec_reset([1])
        nxt = codes[3:].copy()
        nxt[:, 1] = codes[:3, 1]
        more = ctx.codec_decode(nxt)
    assert np.array_equal(first, whole[:, :, :3 * 3840])
    assert np.array_equal(more[0], whole[0][:, 3 * 3840:])
    assert np.array_equal(more[1], whole[1][:, :3 * 3840])


def test_codec_full_size_shapes():
    """The real stage shapes: 4/2/2/4 layers, windows 500/1696/2480/3248, 2 voices, 3 frames."""
    say("codec full size")
    B = 2
    w = synth.codec_weights(mb.CODEC_LAYERS, seed=17)
    codes = synth.codec_codes(18, 3, B)
    ora = oracle.CodecOracle(w, B)
    want = ora.decode(codes)
    with _ctx() as ctx:
        ctx.upload_all(w)
        ctx.codec_init(B)
        got = ctx.codec_decode(codes)
    for b in range(B):
        r = _close(got[b], want[b], 2e-5, f"voice {b}")
        say(f"  voice {b}: max error / scale {r:.2e}")


@pytest.mark.parametrize("B,kv,frames", [(256, mb.MB_KV_BF16, 216), (64, mb.MB_KV_F32, 110)])
def test_codec_full_size_long_run(B, kv, frames):
    """The real stage shapes at the benchmark's voice counts and ring types
    (256 voices with bf16 rings, 64 with fp32 rings), so the projections run
    the row-tiled forms the benchmark times, decoded in calls of 24 frames.
    Over 216 frames every stage's ring fills and wraps (stage 2, the last to
    fill, holds 1696 + 8 slots: 213 frames); over 110 frames stages 1 and 4
    wrap.  The oracle follows three voices in different row tiles; their PCM
    must agree within the bar of the ring type on every call."""
    say(f"codec full size, {B} voices, kv={kv}, {frames} frames")
    watch = [0, B // 2 + 3, B - 1]
    w = synth.codec_weights(mb.CODEC_LAYERS, seed=19)
    codes = synth.codec_codes(20, frames, B)
    ora = oracle.CodecOracle(w, len(watch), kv_bf16=(kv == mb.MB_KV_BF16))
    rel = 2e-5 if kv == mb.MB_KV_F32 else 1e-3
    worst = 0.0
    with _ctx() as ctx:
        ctx.upload_all(w)
        ctx.codec_init(B, kv_dtype=kv)
        for f0 in range(0, frames, 24):
            f1 = min(frames, f0 + 24)
            got = ctx.codec_decode(codes[f0:f1])
            want = ora.decode(np.ascontiguousarray(codes[f0:f1][:, watch]))
            for i, b in enumerate(watch):
                worst = max(worst, _close(got[b], want[i], rel, f"voice {b} frames {f0}-{f1}"))
            assert np.isfinite(got).all()
    say(f"  max error / scale over {len(watch)} voices: {worst:.2e}")


def test_codec_argument_errors():
    say("codec argument errors")
    with _ctx() as ctx:
        with pytest.raises(mb.MbError) as e:
            ctx.codec_decode(np.zeros((1, 1, 16), np.int32))
        assert e.value.code == mb.MB_ERR_STATE  # not initialised
        ctx.codec_init(2, SMALL_LAYERS, SMALL_CTX)
        with pytest.raises(mb.MbError) as e:
            ctx.codec_decode(np.zeros((1, 1, 16), np.int32))
        assert e.value.code == mb.MB_ERR_STATE and "weight not uploaded" in str(e.value)
        ctx.upload_all(synth.codec_weights(SMALL_LAYERS, seed=1))
        bad = np.zeros((1, 1, 16), np.int32)
        bad[0, 0, 5] = 1024
        with pytest.raises(mb.MbError) as e:
            ctx.codec_decode(bad)
        assert e.value.code == mb.MB_ERR_ARG
        with pytest.raises(mb.MbError) as e:
            ctx.codec_decode(np.zeros((1, 3, 16), np.int32))  # B > max_voices
        assert e.value.code == mb.MB_ERR_ARG
