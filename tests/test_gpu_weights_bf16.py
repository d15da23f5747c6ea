"""GPU parity of bf16 weight storage (mb_set_weight_storage(MB_W_BF16)).

With bf16 storage the decoder's projection weights -- c_attn, c_proj,
fc_in, fc_out of every layer and of the local layer, and the 16 audio heads
-- are rounded to bf16 once and read as bf16; products and sums stay fp32.
The oracle is therefore run on the same model with exactly those tensors
rounded to bf16 (round to nearest even, oracle.bf16_round) and everything
else unchanged, and the GPU must match it to the bars of the fp32-storage
tests: hidden states and logits within 1e-4 (fp32 K/V) or 2e-2 (bf16 K/V),
codes exact up to counted near ties.  The model has non-trivial LayerNorm
scales and biases, so the LayerNorm scale that bf16 storage applies to the
rows instead of folding into the weights is exercised.

Voice counts pick the kernels: 3 voices run the GEMV kernel on the bf16
k-major copies (and up to 8 voices the decode attention as per-wave partials
merged by the O projection, over windows of hundreds of slots and a wrapping
ring in the long-window cases), 12 voices the two-product split-bf16 kernel (bf16 K/V) or
the folded fp32 streaming kernel on the rounded weights (fp32 K/V); 64 and
256 voices (bf16 K/V) run the split-bf16 kernel's row-tiled forms that the
benchmark's many-voice frames use.
"""
import numpy as np
import pytest

import mockbird_amd as mb
from mockbird_amd import synth
from oracle import oracle
from conftest import rounded_weights, say
from frame_check import FrameCheck

pytestmark = pytest.mark.gpu

TOL = {mb.MB_KV_F32: 1e-4, mb.MB_KV_BF16: 2e-2}


def _prompts(B, V):
    prompts = [synth.prompt(20 + b, n_frames=3 + 4 * b, n_text=4 + b % 5, vocab=V) for b in range(B)]
    n = np.array([p.shape[0] for p in prompts], np.int32)
    ids = np.full((B, n.max(), 17), 1024, np.int32)
    ids[:, :, 0] = 0
    for b, p in enumerate(prompts):
        ids[b, :n[b]] = p
    return ids, n


@pytest.mark.parametrize("kv,B", [(mb.MB_KV_F32, 3), (mb.MB_KV_F32, 12), (mb.MB_KV_BF16, 3),
                                  (mb.MB_KV_BF16, 12)])
def test_bf16_weights_prefill_decode_frames(kv, B):
    say(f"bf16 weights: kv={kv} voices={B}")
    L, V, C = 2, 64, 128
    w = synth.model_weights(n_layers=L, vocab=V, seed=11, bias_std=0.02, ln_std=0.1)
    m = oracle.Model(rounded_weights(w), n_layers=L, vocab=V)
    m_f32 = oracle.Model(w, n_layers=L, vocab=V)
    ids, n = _prompts(B, V)
    st = oracle.ModelState(m, B, C, kv_bf16=(kv == mb.MB_KV_BF16))
    chk = FrameCheck(B)
    with mb.Context(n_layers=L, capacity=C, max_seqs=B, max_rows=96, kv_dtype=kv, vocab=V) as ctx:
        ctx.upload_all(w)
        ctx.set_weight_storage(mb.MB_W_BF16)
        h = ctx.prefill(ids, n)
        h_or = st.prefill(ids, n)
        assert np.abs(h - h_or).max() < TOL[kv]
        if kv == mb.MB_KV_F32:
            # the storage took effect: the unrounded model is much further away
            st32 = oracle.ModelState(m_f32, B, C)
            far = float(np.abs(h - st32.prefill(ids, n)).max())
            assert far > 10 * float(np.abs(h - h_or).max()), far
        pos = n.copy()
        for f in range(5):
            codes, cont = ctx.local_frame(h)
            g_text, g_logits = ctx.local_logits(h, codes)
            for b in range(B):
                o_text, o_logits = m.local_logits(h_or[b], codes[b])
                chk.frame(b, f"frame {f} voice {b}", codes[b], cont[b], o_text, o_logits, TOL[kv],
                          g_text[b], g_logits[b])
            rows = np.stack([synth.frame_row(codes[b]) for b in range(B)])
            h = ctx.decode_step(rows, pos)
            h_or = st.decode_step(rows, pos)
            assert np.abs(h - h_or).max() < TOL[kv], f
            pos = pos + 1
    chk.summary(f"bf16 weights kv={kv} voices={B}")
    assert chk.codes_equal + chk.codes_tied >= 16 * 5  # at least one voice went on every frame


@pytest.mark.parametrize("kv,C,lens", [
    (mb.MB_KV_BF16, 1024, (600,)),
    (mb.MB_KV_F32, 1024, (560, 300, 64, 129, 200)),
    (mb.MB_KV_BF16, 256, (253, 250, 120, 255, 40)),
])
def test_bf16_weights_few_voices_long_windows(kv, C, lens):
    """Up to 8 voices with bf16 weights: the global layers' decode attention
    leaves per-wave partial states and the O projection merges them.
    Windows of hundreds of slots spread each (voice, head) over several waves
    (up to 16 on a bf16 ring, 8 on fp32), the short voices of a launch get
    waves with no live slot, and the 256-slot ring wraps during the frames
    (voices at 253 and 255 cross position 256)."""
    B = len(lens)
    say(f"bf16 weights, few voices, long windows: kv={kv} C={C} lens={lens}")
    L, V = 2, 64
    w = synth.model_weights(n_layers=L, vocab=V, seed=13, bias_std=0.02, ln_std=0.1)
    # every voice goes on (assistant column = audio_end column), so every
    # frame's codes are compared
    w["model.text_lm_head.weight"][:, 9] = w["model.text_lm_head.weight"][:, 7]
    m = oracle.Model(rounded_weights(w), n_layers=L, vocab=V)
    prompts = [synth.prompt(40 + b, n_frames=n - 3 - (4 + b), n_text=4 + b, vocab=V)
               for b, n in enumerate(lens)]
    n = np.array([p.shape[0] for p in prompts], np.int32)
    assert tuple(n) == lens
    ids = np.full((B, n.max(), 17), 1024, np.int32)
    ids[:, :, 0] = 0
    for b, p in enumerate(prompts):
        ids[b, :n[b]] = p
    st = oracle.ModelState(m, B, C, kv_bf16=(kv == mb.MB_KV_BF16))
    chk = FrameCheck(B)
    frames = 5
    with mb.Context(n_layers=L, capacity=C, max_seqs=B, max_rows=int(n.max()), kv_dtype=kv,
                    vocab=V) as ctx:
        ctx.upload_all(w)
        ctx.set_weight_storage(mb.MB_W_BF16)
        h = ctx.prefill(ids, n)
        h_or = st.prefill(ids, n)
        assert np.abs(h - h_or).max() < TOL[kv]
        pos = n.copy()
        for f in range(frames):
            codes, cont = ctx.local_frame(h)
            g_text, g_logits = ctx.local_logits(h, codes)
            for b in range(B):
                o_text, o_logits = m.local_logits(h_or[b], codes[b])
                chk.frame(b, f"frame {f} voice {b}", codes[b], cont[b], o_text, o_logits, TOL[kv],
                          g_text[b], g_logits[b])
            rows = np.stack([synth.frame_row(codes[b]) for b in range(B)])
            h = ctx.decode_step(rows, pos)
            h_or = st.decode_step(rows, pos)
            assert np.abs(h - h_or).max() < TOL[kv], f
            pos = pos + 1
        if C == 256:
            assert pos.max() > C  # the ring wrapped
    chk.summary(f"bf16 weights few voices kv={kv} C={C}")
    assert chk.codes_equal + chk.codes_tied == 16 * frames * B


@pytest.mark.parametrize("B", [64, 256])
def test_bf16_weights_many_voices(B):
    """bf16 K/V and bf16 weights at the benchmark's voice counts, where the
    decode projections run the row-tiled two-product split-bf16 kernel with
    bf16 weights (several row tiles, the LayerNorm scale applied to the rows,
    fc_out split over k) and the local head's projections the same at B rows.
    The GPU runs every voice; the oracle, on the rounded weights, follows
    six voices spread over the row tiles, teacher-forced by the GPU's codes:
    prefill hidden states, every frame's logits and codes, and the hidden
    state after each of 5 decode steps within the bf16 bar."""
    say(f"bf16 weights: kv=bf16 voices={B}")
    L, V, C = 2, 64, 128
    w = synth.model_weights(n_layers=L, vocab=V, seed=23, bias_std=0.02, ln_std=0.1)
    w["model.text_lm_head.weight"][:, 9] = w["model.text_lm_head.weight"][:, 7]  # never stops
    m = oracle.Model(rounded_weights(w), n_layers=L, vocab=V)
    g = np.random.default_rng(B)
    lens = g.integers(8, 60, size=B)
    prompts = [synth.prompt(300 + b, n_frames=int(lens[b]) // 2,
                            n_text=int(lens[b]) - 3 - int(lens[b]) // 2, vocab=V) for b in range(B)]
    n = np.array([p.shape[0] for p in prompts], np.int32)
    ids = np.full((B, n.max(), 17), 1024, np.int32)
    for b, p in enumerate(prompts):
        ids[b, :n[b]] = p
    watch = sorted({0, 17, B // 2 - 1, B // 2 + 5, B - 16, B - 1})
    st = oracle.ModelState(m, len(watch), C, kv_bf16=True)
    h_or = st.prefill(np.ascontiguousarray(ids[watch]), n[watch])
    tol = TOL[mb.MB_KV_BF16]
    chk = FrameCheck(len(watch))
    with mb.Context(n_layers=L, capacity=C, max_seqs=B, max_rows=int(n.max()),
                    kv_dtype=mb.MB_KV_BF16, vocab=V) as ctx:
        ctx.upload_all(w)
        ctx.set_weight_storage(mb.MB_W_BF16)
        h = ctx.prefill(ids, n)
        assert np.isfinite(h).all()
        assert np.abs(h[watch] - h_or).max() < tol
        pos = n.copy()
        for f in range(5):
            codes, cont = ctx.local_frame(h)
            assert cont.all()
            g_text, g_logits = ctx.local_logits(h, codes)
            for i, b in enumerate(watch):
                o_text, o_logits = m.local_logits(h_or[i], codes[b])
                chk.frame(i, f"frame {f} voice {b}", codes[b], cont[b], o_text, o_logits, tol,
                          g_text[b], g_logits[b])
            rows = np.stack([synth.frame_row(codes[b]) for b in range(B)])
            h = ctx.decode_step(rows, pos)
            h_or = st.decode_step(rows[watch], pos[watch])
            assert np.abs(h[watch] - h_or).max() < tol, f
            pos = pos + 1
    chk.summary(f"bf16 weights kv=bf16 voices={B}")
    assert chk.codes_equal + chk.codes_tied == len(watch) * 5 * 16


def test_weight_storage_switches_back():
    """MB_W_BF16, then MB_W_F32 again on the same context: the copies are
    derived again, the fp32 model's results come back and the bf16 period's
    rounded copies are freed (the context's device bytes return to the fp32
    figure)."""
    say("bf16 weights: switch back to fp32")
    L, V, B, C = 1, 32, 2, 64
    w = synth.model_weights(n_layers=L, vocab=V, seed=5, bias_std=0.02, ln_std=0.1)
    ids, n = _prompts(B, V)
    want32 = oracle.ModelState(oracle.Model(w, n_layers=L, vocab=V), B, C).prefill(ids, n)
    want16 = oracle.ModelState(oracle.Model(rounded_weights(w), n_layers=L, vocab=V), B,
                               C).prefill(ids, n)
    with mb.Context(n_layers=L, capacity=C, max_seqs=B, max_rows=64, vocab=V) as ctx:
        ctx.upload_all(w)
        assert np.abs(ctx.prefill(ids, n) - want32).max() < 1e-4
        bytes32 = ctx.device_bytes()
        ctx.set_weight_storage(mb.MB_W_BF16)
        ctx.ring_reset()
        assert np.abs(ctx.prefill(ids, n) - want16).max() < 1e-4
        assert ctx.device_bytes() != bytes32
        ctx.set_weight_storage(mb.MB_W_F32)
        ctx.ring_reset()
        assert np.abs(ctx.prefill(ids, n) - want32).max() < 1e-4
        # the rounded copies are freed again: the fp32 footprint comes back
        assert ctx.device_bytes() == bytes32
        with pytest.raises(mb.MbError) as e:
            ctx.set_weight_storage(7)
        assert e.value.code == mb.MB_ERR_ARG


def test_bf16_weights_c0_single_voice_60_frames():
    """The benchmark's one-voice frame with bf16 storage at full size: 12
    layers, vocab 32000, the 281-row voice-clone prompt, ring 1024 (fp32
    K/V), 60 greedy frames per call.  Each frame runs the global layers'
    attention as per-wave partials merged by the O projection and makes the
    code choices of channels 0-14 inside the next local step's QKV
    projection; every code, logit and hidden state is compared with the
    oracle on the rounded weights."""
    say("bf16 weights, C0 size: prefill 281 rows + 60 frames, B=1")
    w = synth.model_weights(n_layers=12, vocab=32000, seed=0)
    w["model.text_lm_head.weight"][:, 9] = w["model.text_lm_head.weight"][:, 7]  # never ends
    m = oracle.Model(rounded_weights(w), n_layers=12, vocab=32000)
    rows = synth.prompt(0, n_frames=150, n_text=128, vocab=32000)
    st = oracle.ModelState(m, 1, 1024)
    h_or = st.prefill_all(0, rows)[-1][None]
    chk = FrameCheck(1)
    tol = TOL[mb.MB_KV_F32]
    with mb.Context(n_layers=12, capacity=1024, max_seqs=1, max_rows=512, vocab=32000) as ctx:
        ctx.upload_all(w)
        ctx.set_weight_storage(mb.MB_W_BF16)
        h = ctx.prefill(rows[None], [rows.shape[0]])
        max_h = float(np.abs(h - h_or).max())
        assert max_h < tol
        pos = rows.shape[0]
        for f in range(60):
            codes, cont = ctx.local_frame(h)
            g_text, g_logits = ctx.local_logits(h, codes)
            o_text, o_logits = m.local_logits(h_or[0], codes[0])
            chk.frame(0, f"frame {f}", codes[0], cont[0], o_text, o_logits, tol, g_text[0],
                      g_logits[0])
            assert cont[0]
            row = synth.frame_row(codes[0])[None]
            h = ctx.decode_step(row, [pos])
            h_or = st.decode_step(row, [pos])
            d = float(np.abs(h - h_or).max())
            max_h = max(max_h, d)
            assert d < tol, f
            pos += 1
    chk.summary("bf16 weights C0")
    say(f"  bf16 weights C0: max |hidden diff| {max_h:.2e}")
    assert chk.codes_equal + chk.codes_tied == 960
