"""Pins of the codec-decoder oracle (oracle/codec_oracle.c).

No fixture of the reference covers the codec with weights that exist here
(its golden PCM statistics come from the published model, which is not in
the container), so the oracle is checked against what the mathematics and
the reference's own definitions fix:

- erf (Abramowitz & Stegun 7.1.26, as GELU_ERF evaluates it) against
  math.erf within the method's published bound 1.5e-7;
- the RVQ front against a direct numpy statement of RVQ_ACCUM / RVQ_PROJECT
  and its x4 interleave (kernels-decode.ts:537-574);
- the whole decoder against an independent float64 numpy decoder that keeps
  every past position (no ring) and masks by the window rule of
  ATTEND_RING_CODEC, runs each stage's positions as one causal block, and
  states the upsample and the head by their reference definitions
  (new[2t + r][m] = old[t][2m + r]; audio[c][t*120 + j] = latent[t][2j + c]).
  Small windows make every ring wrap several times, so a wrong slot,
  eviction or window shows as an O(1) difference;
- the oracle's state across calls: n frames at once equal the same frames
  over several calls.
"""
import math

import numpy as np
import pytest

from mockbird_amd import synth
from oracle import oracle

LAYERS = (2, 1, 1, 2)
CONTEXT = (6, 12, 20, 40)


def test_erf_as_within_its_bound():
    xs = np.linspace(-6.0, 6.0, 4001)
    err = max(abs(oracle.erf_as(x) - math.erf(x)) for x in xs)
    assert err <= 1.5e-7, err
    for x in (-3.0, -0.5, 0.0, 0.7, 4.0):
        want = 0.5 * x * (1.0 + math.erf(x / math.sqrt(2.0)))
        assert abs(oracle.gelu_erf(x) - want) <= 1e-6 * max(1.0, abs(x)), x


def test_rvq_front_matches_its_definition():
    w = synth.codec_weights(LAYERS, seed=3)
    o = oracle.CodecOracle(w, 1, LAYERS, CONTEXT)
    codes = synth.codec_codes(5, 1, 1)[0, 0]
    acc = np.zeros(512)
    for k in range(16):
        p = f"model.quantizer.quantizers.{k}."
        acc += (w[p + "out_proj.weight"].astype(np.float64)
                @ w[p + "codebook.weight"][codes[k]].astype(np.float64)
                + w[p + "out_proj.bias"])
    g = w["model.quantizer.output_proj.weight"].astype(np.float64) @ acc.astype(np.float32) \
        + w["model.quantizer.output_proj.bias"]
    want = g.reshape(192, 4).T  # position s, channel m = g[4m + s]
    got = o.rvq(codes)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


def _rope(x, pos, inv):
    """x [rows][4*64] at positions pos[rows], pairs (2i, 2i+1) rotated by pos*inv[i]."""
    a = (pos[:, None].astype(np.float32) * inv[None, :]).astype(np.float64)
    c, s = np.cos(a), np.sin(a)
    y = x.reshape(x.shape[0], 4, 32, 2)
    out = np.empty_like(y)
    out[..., 0] = y[..., 0] * c[:, None, :] - y[..., 1] * s[:, None, :]
    out[..., 1] = y[..., 1] * c[:, None, :] + y[..., 0] * s[:, None, :]
    return out.reshape(x.shape)


def _ln(x, w, b):
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)
    return (x - m) / np.sqrt(v + 1e-5) * w + b


def _gelu(x):
    from scipy.special import erf
    return 0.5 * x * (1.0 + erf(x / np.sqrt(2.0)))


class NumpyCodec:
    """Float64 decoder with the full history of every layer (no ring)."""

    def __init__(self, w, layers, context):
        self.w = {k: v.astype(np.float64) for k, v in w.items()}
        self.layers, self.context = layers, context
        self.inv = oracle.inv_freq()
        n_l = sum(layers)
        self.Kh = [np.zeros((0, 256)) for _ in range(n_l)]
        self.Vh = [np.zeros((0, 256)) for _ in range(n_l)]
        self.pos = [0, 0, 0, 0]

    def frame(self, codes):
        w = self.w
        acc = np.zeros(512)
        for k in range(16):
            p = f"model.quantizer.quantizers.{k}."
            acc += w[p + "out_proj.weight"] @ w[p + "codebook.weight"][codes[k]] + w[p + "out_proj.bias"]
        g = w["model.quantizer.output_proj.weight"] @ acc + w["model.quantizer.output_proj.bias"]
        x_in = g.reshape(192, 4).T          # [4][192]
        li = 0
        for s in range(4):
            n, W = 4 << s, self.context[s]
            p = f"model.decoder.{(1, 3, 5, 7)[s]}."
            x = x_in @ w[p + "input_proj.weight"]
            pos = self.pos[s] + np.arange(n)
            for i in range(self.layers[s]):
                q = p + f"transformer.layers.{i}."
                h = _ln(x, w[q + "norm1.weight"], w[q + "norm1.bias"])
                qkv = h @ w[q + "self_attn.in_proj.weight"]
                qr = _rope(qkv[:, :256], pos, self.inv)
                kr = _rope(qkv[:, 256:512], pos, self.inv)
                self.Kh[li] = np.concatenate([self.Kh[li], kr])
                self.Vh[li] = np.concatenate([self.Vh[li], qkv[:, 512:]])
                hp = np.arange(self.Kh[li].shape[0])          # position of each history row
                mask = (hp[None, :] <= pos[:, None]) & (pos[:, None] - hp[None, :] < W)
                ctx = np.zeros((n, 256))
                for hd in range(4):
                    sl = slice(hd * 64, hd * 64 + 64)
                    sc = qr[:, sl] @ self.Kh[li][:, sl].T * 0.125
                    sc = np.where(mask, sc, -np.inf)
                    pr = np.exp(sc - sc.max(1, keepdims=True))
                    pr /= pr.sum(1, keepdims=True)
                    ctx[:, sl] = pr @ self.Vh[li][:, sl]
                x = x + w[q + "layer_scale_1.scale"] * (ctx @ w[q + "self_attn.out_proj.weight"])
                h = _ln(x, w[q + "norm2.weight"], w[q + "norm2.bias"])
                f = _gelu(h @ w[q + "ffn.0.weight"])
                x = x + w[q + "layer_scale_2.scale"] * (f @ w[q + "ffn.2.weight"])
                li += 1
            out = x @ w[p + "output_proj.weight"]
            self.pos[s] += n
            if s < 3:
                # new[2t + r][m] = old[t][2m + r]
                x_in = np.stack([out[:, 0::2], out[:, 1::2]], axis=1).reshape(2 * n, 384)
        # audio[c][t*120 + j] = latent[t][2j + c]
        return np.stack([out[:, 0::2].reshape(-1), out[:, 1::2].reshape(-1)])


def test_decoder_matches_a_full_history_restatement():
    w = synth.codec_weights(LAYERS, seed=7)
    codes = synth.codec_codes(8, 7, 2)
    o = oracle.CodecOracle(w, 2, LAYERS, CONTEXT)
    got = o.decode(codes)
    for b in range(2):
        ref = NumpyCodec(w, LAYERS, CONTEXT)
        want = np.concatenate([ref.frame(codes[f, b]) for f in range(codes.shape[0])], axis=1)
        scale = np.abs(want).max()
        err = np.abs(got[b] - want).max()
        assert err <= 2e-5 * scale, (b, err, scale)
    # every stage wrapped: 7 frames x (4, 8, 16, 32) positions > windows (6, 12, 20, 40)
    assert (o.pos[0] == [28, 56, 112, 224]).all()


def test_decoder_state_carries_across_calls():
    w = synth.codec_weights(LAYERS, seed=9)
    codes = synth.codec_codes(10, 5, 2)
    a = oracle.CodecOracle(w, 2, LAYERS, CONTEXT)
    whole = a.decode(codes)
    b = oracle.CodecOracle(w, 2, LAYERS, CONTEXT)
    parts = np.concatenate([b.decode(codes[:2]), b.decode(codes[2:3]), b.decode(codes[3:])], axis=2)
    assert np.array_equal(whole, parts)
    b.reset([1])
    again = b.decode(codes[:2])
    assert np.array_equal(again[1], whole[1][:, :2 * 3840])
