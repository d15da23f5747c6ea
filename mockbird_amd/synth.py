"""Seeded synthetic model weights, prompts and q/k/v streams.

The benchmark configurations use a random-init model with MOSS-TTS-Nano's
shapes (docs/moss-tts-runtime-analysis.md:58-123): matrices and embeddings
N(0, std) from a seed, biases 0, LayerNorm scale 1 and shift 0 (the real
model's LayerNorm scales are all ones, doc:849).  Tests may ask for non-zero
biases and LayerNorm parameters so that an indexing mistake in those shows.

Generator: numpy PCG64 (`np.random.default_rng(seed)`), float32 standard
normals scaled in float32; one independent stream per tensor, derived from
(seed, tensor index), so any subset of tensors is reproducible on its own.
Tensor names are the exported graph's (ref-decode.mjs:40-80), with the
anonymous MatMul initialisers given the names of the layers they feed.
"""
from __future__ import annotations

import numpy as np

D, QKV, FFN, NVQ, CODES, ROW, PAD = 768, 2304, 3072, 16, 1024, 17, 1024
AUDIO_START, AUDIO_END, USER_SLOT, ASSISTANT_SLOT = 6, 7, 8, 9

LAYER_SHAPES = (
    ("ln_1.weight", (D,), "ln_w"), ("ln_1.bias", (D,), "bias"),
    ("attn.c_attn.weight", (D, QKV), "mat"), ("attn.c_attn.bias", (QKV,), "bias"),
    ("attn.c_proj.weight", (D, D), "mat"), ("attn.c_proj.bias", (D,), "bias"),
    ("ln_2.weight", (D,), "ln_w"), ("ln_2.bias", (D,), "bias"),
    ("mlp.fc_in.weight", (D, FFN), "mat"), ("mlp.fc_in.bias", (FFN,), "bias"),
    ("mlp.fc_out.weight", (FFN, D), "mat"), ("mlp.fc_out.bias", (D,), "bias"),
)


def tensor_specs(n_layers: int = 12, vocab: int = 32000):
    """(name, shape, kind) of every tensor of the synthetic model, in a fixed order."""
    specs = []
    for i in range(n_layers):
        specs += [(f"core.model.transformer.h.{i}.{n}", s, k) for n, s, k in LAYER_SHAPES]
    specs += [("core.model.transformer.ln_f.weight", (D,), "ln_w"),
              ("core.model.transformer.ln_f.bias", (D,), "bias"),
              ("core.model.transformer.wte.weight", (vocab, D), "mat")]
    specs += [(f"core.model.audio_embeddings.{k}.weight", (CODES, D), "mat") for k in range(NVQ)]
    specs += [(f"model.local_transformer.h.0.{n}", s, k) for n, s, k in LAYER_SHAPES]
    specs += [("model.local_transformer.ln_f.weight", (D,), "ln_w"),
              ("model.local_transformer.ln_f.bias", (D,), "bias"),
              ("model.text_lm_head.weight", (D, vocab), "mat")]
    specs += [(f"model.audio_lm_heads.{k}.weight", (D, CODES), "mat") for k in range(NVQ)]
    return specs


def model_weights(n_layers: int = 12, vocab: int = 32000, seed: int = 0, std: float = 0.02,
                  bias_std: float = 0.0, ln_std: float = 0.0) -> dict[str, np.ndarray]:
    out = {}
    for idx, (name, shape, kind) in enumerate(tensor_specs(n_layers, vocab)):
        g = np.random.default_rng([seed, idx])
        if kind == "mat":
            a = g.standard_normal(shape, dtype=np.float32) * np.float32(std)
        elif kind == "bias":
            a = (g.standard_normal(shape, dtype=np.float32) * np.float32(bias_std)
                 if bias_std else np.zeros(shape, np.float32))
        else:  # LayerNorm scale
            a = (np.float32(1) + g.standard_normal(shape, dtype=np.float32) * np.float32(ln_std)
                 if ln_std else np.ones(shape, np.float32))
        out[name] = np.ascontiguousarray(a, dtype=np.float32)
    return out


def voice_clone_rows(codes: np.ndarray, text: np.ndarray) -> np.ndarray:
    """buildVoiceCloneRows with empty templates (policy.ts:49-80):
    [audio_start] + one audio row per code frame + [audio_end] + text + [audio_start]."""
    codes = np.asarray(codes, np.int32).reshape(-1, NVQ)
    text = np.asarray(text, np.int32).reshape(-1)
    rows = np.full((codes.shape[0] + text.size + 3, ROW), PAD, np.int32)
    r = 0
    rows[r, 0] = AUDIO_START; r += 1
    for f in range(codes.shape[0]):
        rows[r, 0] = USER_SLOT
        rows[r, 1:] = codes[f]
        r += 1
    rows[r, 0] = AUDIO_END; r += 1
    for t in text:
        rows[r, 0] = t
        r += 1
    rows[r, 0] = AUDIO_START
    return rows


def frame_row(frame) -> np.ndarray:
    """buildFrameRow (policy.ts:83-88): [assistant_slot, codes...]."""
    row = np.full(ROW, PAD, np.int32)
    row[0] = ASSISTANT_SLOT
    row[1:1 + len(frame)] = np.asarray(frame, np.int32)[:NVQ]
    return row


def prompt(seed: int, n_frames: int = 150, n_text: int = 128, vocab: int = 32000) -> np.ndarray:
    """A seeded voice-clone prompt: n_frames code frames U[0,1024), n_text ids U[0,vocab)."""
    g = np.random.default_rng([seed, 0x5EED])
    codes = g.integers(0, CODES, size=(n_frames, NVQ), dtype=np.int32)
    text = g.integers(0, vocab, size=n_text, dtype=np.int32)
    return voice_clone_rows(codes, text)


def qkv_rows(seed, shape) -> np.ndarray:
    """q | k | v rows ~ N(0, 1), float32."""
    g = np.random.default_rng(seed)
    return g.standard_normal(tuple(shape) + (QKV,), dtype=np.float32)


# ------------------------------------------------------------------ the codec
CODEC_D, CODEC_FFN = 256, 1024
CODEC_DECODER_INDEX = (1, 3, 5, 7)


def codec_specs(layers=(4, 2, 2, 4)):
    """(name, shape, kind, scale) of every codec tensor, in a fixed order.  The
    names are the ones include/mockbird_hip.h lists for mb_codec_*; the
    matrices are [K, N] as the graph's MatMul initialisers hold them, except
    the two output-major 1x1 convolutions of the RVQ front."""
    d, f = CODEC_D, CODEC_FFN
    specs = []
    for k in range(NVQ):
        p = f"model.quantizer.quantizers.{k}."
        specs += [(p + "out_proj.weight", (512, 8), "mat", 0.35),
                  (p + "out_proj.bias", (512,), "vec", 0.02),
                  (p + "codebook.weight", (CODES, 8), "mat", 1.0)]
    specs += [("model.quantizer.output_proj.weight", (768, 512), "mat", 512 ** -0.5),
              ("model.quantizer.output_proj.bias", (768,), "vec", 0.02)]
    for s, n_layers in enumerate(layers):
        p = f"model.decoder.{CODEC_DECODER_INDEX[s]}."
        w_in = 192 if s == 0 else 384
        specs.append((p + "input_proj.weight", (w_in, d), "mat", w_in ** -0.5))
        for i in range(n_layers):
            q = p + f"transformer.layers.{i}."
            specs += [(q + "self_attn.in_proj.weight", (d, 3 * d), "mat", d ** -0.5),
                      (q + "self_attn.out_proj.weight", (d, d), "mat", d ** -0.5),
                      (q + "ffn.0.weight", (d, f), "mat", d ** -0.5),
                      (q + "ffn.2.weight", (f, d), "mat", f ** -0.5),
                      (q + "norm1.weight", (d,), "ln_w", 0.1), (q + "norm1.bias", (d,), "vec", 0.05),
                      (q + "norm2.weight", (d,), "ln_w", 0.1), (q + "norm2.bias", (d,), "vec", 0.05),
                      (q + "layer_scale_1.scale", (d,), "scale", 0.2),
                      (q + "layer_scale_2.scale", (d,), "scale", 0.2)]
        specs.append((p + "output_proj.weight", (d, 240 if s == len(layers) - 1 else 768), "mat",
                      d ** -0.5))
    return specs


def codec_weights(layers=(4, 2, 2, 4), seed: int = 0) -> dict[str, np.ndarray]:
    """Seeded random codec weights at the real shapes: matrices N(0, scale),
    LayerNorm scales 1 + N(0, 0.1), shifts and biases small normals, layer
    scales 0.2 (1 + N(0, 0.25)); one stream per tensor from (seed, index)."""
    out = {}
    for idx, (name, shape, kind, sc) in enumerate(codec_specs(layers)):
        g = np.random.default_rng([seed, 0xC0DEC, idx])
        a = g.standard_normal(shape, dtype=np.float32)
        if kind == "ln_w":
            a = np.float32(1) + a * np.float32(sc)
        elif kind == "scale":
            a = np.float32(sc) * (np.float32(1) + a * np.float32(0.25))
        else:
            a = a * np.float32(sc)
        out[name] = np.ascontiguousarray(a, dtype=np.float32)
    return out


def codec_codes(seed: int, n_frames: int, B: int) -> np.ndarray:
    """Seeded code frames [n_frames][B][16] in [0, 1024)."""
    g = np.random.default_rng([seed, 0xC0DE5])
    return g.integers(0, CODES, size=(n_frames, B, NVQ), dtype=np.int32)
