"""GPU parity of the decoder (fp32 MFMA projections, LN, GELU, embeddings,
greedy local head) through the C ABI, against the oracle.

Bars: hidden states and logits within 1e-4 of the oracle with fp32 K/V and
2e-2 with bf16 K/V (the oracle rounds its stored K/V to bf16 the same way),
ring slot positions exact.

Greedy codes are checked frame by frame against the oracle teacher-forced by
the GPU's own codes (tests/frame_check.py): every code of every frame is
compared, the GPU's code must be exactly the penalised argmax of its own
logits (read back through mb_local_logits), and a code may differ from the
oracle's choice only at a near tie that the logits difference explains.
"""
import numpy as np
import pytest

import mockbird_amd as mb
from mockbird_amd import synth
from oracle import oracle
from conftest import say
from frame_check import FrameCheck

pytestmark = pytest.mark.gpu

TOL = {mb.MB_KV_F32: 1e-4, mb.MB_KV_BF16: 2e-2}


def _ctx(weights, n_layers, vocab, B, C, kv=mb.MB_KV_F32, max_rows=512):
    ctx = mb.Context(n_layers=n_layers, capacity=C, max_seqs=B, max_rows=max_rows, kv_dtype=kv,
                     vocab=vocab)
    ctx.upload_all(weights)
    return ctx


@pytest.mark.parametrize("kv", [mb.MB_KV_F32, mb.MB_KV_BF16])
def test_small_model_prefill_decode_frames(kv):
    """2 layers with non-zero biases and LayerNorm parameters, 3 voices of
    different prompt lengths, prefill + 6 frames, every frame's logits and
    codes compared."""
    say(f"small model kv={kv}")
    L, V, B, C = 2, 64, 3, 96
    w = synth.model_weights(n_layers=L, vocab=V, seed=7, bias_std=0.02, ln_std=0.1)
    m = oracle.Model(w, n_layers=L, vocab=V)
    prompts = [synth.prompt(10 + b, n_frames=3 + 7 * b, n_text=5 + b, vocab=V) for b in range(B)]
    n = np.array([p.shape[0] for p in prompts], np.int32)
    ids = np.full((B, n.max(), 17), 1024, np.int32)
    ids[:, :, 0] = 0
    for b, p in enumerate(prompts):
        ids[b, :n[b]] = p
    st = oracle.ModelState(m, B, C, kv_bf16=(kv == mb.MB_KV_BF16))
    chk = FrameCheck(B)
    with _ctx(w, L, V, B, C, kv) as ctx:
        h = ctx.prefill(ids, n)
        h_or = st.prefill(ids, n)
        assert np.abs(h - h_or).max() < TOL[kv]
        for l in range(L):
            for b in range(B):
                k, v, sp = ctx.read_ring(l, b)
                assert np.array_equal(sp, st.slot_pos[b, l])
                live = sp >= 0
                assert np.abs(k[live] - st.K[b, l][live]).max() < TOL[kv]
        pos = n.copy()
        for f in range(6):
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
    chk.summary(f"small model kv={kv}")
    assert chk.codes_equal + chk.codes_tied >= 16 * 6  # at least one voice went on every frame


def test_model_errors():
    say("model errors")
    L, V = 1, 16
    w = synth.model_weights(n_layers=L, vocab=V, seed=1)
    with mb.Context(n_layers=L, capacity=8, max_seqs=1, max_rows=8, vocab=V, wrap=False) as ctx:
        with pytest.raises(mb.MbError) as e:  # nothing uploaded yet
            ctx.prefill(np.zeros((1, 2, 17), np.int32), [2])
        assert e.value.code == mb.MB_ERR_STATE and "weight not uploaded" in str(e.value)
        ctx.upload_all(w)
        bad = np.full((1, 2, 17), 1024, np.int32)
        bad[0, :, 0] = V  # text id out of range
        with pytest.raises(mb.MbError) as e:
            ctx.prefill(bad, [2])
        assert e.value.code == mb.MB_ERR_ARG
        ok = np.full((1, 2, 17), 1024, np.int32)
        ok[0, :, 0] = 6
        h = ctx.prefill(ok, [2])
        assert np.isfinite(h).all() and np.abs(h).max() > 0
        with pytest.raises(mb.MbError) as e:  # the non-wrapping ring is full at position 8
            ctx.decode_step(synth.frame_row([0] * 16)[None], [8])
        assert e.value.code == mb.MB_ERR_RANGE
        ctx.cancel(True)
        with pytest.raises(mb.MbError) as e:
            ctx.decode_step(synth.frame_row([0] * 16)[None], [2])
        assert e.value.code == mb.MB_ERR_CANCELLED
        ctx.cancel(False)
        ctx.decode_step(synth.frame_row([0] * 16)[None], [2])


def _c0_weights(n_layers=12, vocab=32000, seed=0):
    w = synth.model_weights(n_layers=n_layers, vocab=vocab, seed=seed)
    # the benchmark model never ends its utterance: the assistant column equals
    # the audio_end column, so "continue iff assistant >= end" always holds
    w["model.text_lm_head.weight"][:, 9] = w["model.text_lm_head.weight"][:, 7]
    return w


def _c0_setup():
    w = _c0_weights()
    m = oracle.Model(w, n_layers=12, vocab=32000)
    rows = synth.prompt(0, n_frames=150, n_text=128, vocab=32000)
    st = oracle.ModelState(m, 1, 1024)
    h_or = st.prefill_all(0, rows)[-1][None]
    return w, m, rows, st, h_or


def test_c0_single_voice_60_frames():
    """The single-stream configuration: 12 layers, d=768, vocab 32000,
    281-row voice-clone prompt (150 code frames + 128 text ids), ring 1024,
    60 greedy frames driven call by call (nextFrame, then decodeStep of the
    frame row); every code, logit and hidden state compared with the
    oracle."""
    say("C0: prefill 281 rows + 60 frames, B=1, per call")
    w, m, rows, st, h_or = _c0_setup()
    chk = FrameCheck(1)
    max_h = 0.0
    with _ctx(w, 12, 32000, 1, 1024) as ctx:
        h = ctx.prefill(rows[None], [rows.shape[0]])
        max_h = float(np.abs(h - h_or).max())
        assert max_h < 1e-4
        pos = rows.shape[0]
        gpu_codes = []
        for f in range(60):
            codes, cont = ctx.local_frame(h)
            g_text, g_logits = ctx.local_logits(h, codes)
            o_text, o_logits = m.local_logits(h_or[0], codes[0])
            chk.frame(0, f"frame {f}", codes[0], cont[0], o_text, o_logits, 1e-4, g_text[0],
                      g_logits[0])
            assert cont[0]
            gpu_codes.append(codes[0].copy())
            row = synth.frame_row(codes[0])[None]
            h = ctx.decode_step(row, [pos])
            h_or = st.decode_step(row, [pos])
            d = float(np.abs(h - h_or).max())
            max_h = max(max_h, d)
            assert d < 1e-4, f
            pos += 1
        for l in (0, 11):
            k, v, sp = ctx.read_ring(l, 0)
            assert np.array_equal(sp, st.slot_pos[0, l])
            live = sp >= 0
            assert np.abs(k[live] - st.K[0, l][live]).max() < 1e-4
            assert np.abs(v[live] - st.V[0, l][live]).max() < 1e-4
    chk.summary("C0 per call")
    say(f"  C0 per call: max |hidden diff| {max_h:.2e}")
    assert chk.codes_equal + chk.codes_tied == 960
    assert chk.codes_equal >= 950
    _C0_RUN["codes"] = np.stack(gpu_codes)


_C0_RUN = {}  # the per-call run's codes, for the frame-loop test that follows it


def test_c0_device_frame_loop_60_frames():
    """C0's 60 frames through mb_decode_frames (one eager frame, then 59
    replays of the captured frame graph), followed by the oracle teacher-
    forced with the GPU's codes: every code is the oracle's choice or a near
    tie within 2.4 x the logits bar, the final hidden state, position and
    ring contents match, and the codes equal the per-call run's bit for bit."""
    say("C0: prefill 281 rows + 60 frames, B=1, device frame loop (graph replay)")
    w, m, rows, st, h_or = _c0_setup()
    chk = FrameCheck(1)
    with _ctx(w, 12, 32000, 1, 1024) as ctx:
        h = ctx.prefill(rows[None], [rows.shape[0]])
        codes, cont, h_end, p_end = ctx.decode_frames(h, [rows.shape[0]], 60)
        assert cont.all() and p_end[0] == rows.shape[0] + 60
        pos = rows.shape[0]
        for f in range(60):
            o_text, o_logits = m.local_logits(h_or[0], codes[f, 0])
            chk.frame(0, f"frame {f}", codes[f, 0], cont[f, 0], o_text, o_logits, 1e-4,
                      bar=2.4e-4)
            h_or = st.decode_step(synth.frame_row(codes[f, 0])[None], [pos])
            pos += 1
        d = float(np.abs(h_end - h_or).max())
        assert d < 1e-4
        for l in (0, 5, 11):
            k, v, sp = ctx.read_ring(l, 0)
            assert np.array_equal(sp, st.slot_pos[0, l])
            live = sp >= 0
            assert np.abs(k[live] - st.K[0, l][live]).max() < 1e-4
            assert np.abs(v[live] - st.V[0, l][live]).max() < 1e-4
    chk.summary("C0 frame loop")
    say(f"  C0 frame loop: final |hidden diff| {d:.2e}")
    assert chk.codes_equal + chk.codes_tied == 960
    assert chk.codes_equal >= 950
    if "codes" in _C0_RUN:
        assert np.array_equal(_C0_RUN["codes"], codes[:, 0]), "graph loop differs from per-call frames"


def _c3_prompts(B):
    g = np.random.default_rng(33)
    lens = g.integers(64, 400, size=B)
    prompts = [synth.prompt(1000 + b, n_frames=int(lens[b]) // 2,
                            n_text=int(lens[b]) - 3 - int(lens[b]) // 2, vocab=32000)
               for b in range(B)]
    n = np.array([p.shape[0] for p in prompts], np.int32)
    ids = np.full((B, n.max(), 17), 1024, np.int32)
    for b, p in enumerate(prompts):
        ids[b, :n[b]] = p
    return prompts, n, ids


def test_c3_many_voices():
    """256 voices with prompt lengths U[64, 400), bf16 KV, ring 1024, the
    configuration's 300 frames.  The GPU runs every voice; the oracle follows
    8 of them (shortest, longest and six others), teacher-forced: 40 frames
    driven call by call with every watched voice's logits, codes and hidden
    states compared, then 260 through mb_decode_frames (graph replay) with
    the codes compared -- all 8 voices for the first 20 of them (hidden
    states checked there), the shortest and the longest voice through all
    260, so the longest reaches position 698 -- and the hidden state checked
    at the end."""
    say("C3: B=256 prefill + 40 per-call frames + 260 graph frames, 8 voices checked")
    B, C = 256, 1024
    w = _c0_weights()
    prompts, n, ids = _c3_prompts(B)
    watch = sorted({int(np.argmin(n)), int(np.argmax(n)), 0, 37, 101, 160, 200, 222})
    assert len(watch) == 8
    m = oracle.Model(w, n_layers=12, vocab=32000)
    tol = TOL[mb.MB_KV_BF16]
    sub_n = n[watch]
    sub_ids = np.full((len(watch), sub_n.max(), 17), 1024, np.int32)
    for i, b in enumerate(watch):
        sub_ids[i, :n[b]] = prompts[b]
    st = oracle.ModelState(m, len(watch), C, kv_bf16=True)
    h_or = st.prefill(sub_ids, sub_n)
    chk = FrameCheck(len(watch))
    max_h = 0.0
    with _ctx(w, 12, 32000, B, C, kv=mb.MB_KV_BF16, max_rows=int(n.max())) as ctx:
        h = ctx.prefill(ids, n)
        assert np.isfinite(h).all()
        max_h = float(np.abs(h[watch] - h_or).max())
        assert max_h < tol
        pos = n.copy()
        for f in range(40):
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
            d = float(np.abs(h[watch] - h_or).max())
            max_h = max(max_h, d)
            assert d < tol, f
            pos = pos + 1
        G = 260
        codes, cont, h_end, p_end = ctx.decode_frames(h, pos, G)
        assert cont.all() and (p_end == pos + G).all()
        assert int(p_end.max()) == int(n.max()) + 300 <= C
        for f in range(20):
            for i, b in enumerate(watch):
                o_text, o_logits = m.local_logits(h_or[i], codes[f, b])
                chk.frame(i, f"graph frame {f} voice {b}", codes[f, b], cont[f, b], o_text,
                          o_logits, tol, bar=2.4 * tol)
            h_or = st.decode_step(np.stack([synth.frame_row(codes[f, b]) for b in watch]),
                                  pos[watch] + f)
        # the shortest and the longest voice on to the 300th frame
        ends = [watch.index(int(np.argmin(n))), watch.index(int(np.argmax(n)))]
        st2 = st.select(ends)
        h2 = h_or[ends]
        far = [watch[i] for i in ends]
        for f in range(20, G):
            for j, b in enumerate(far):
                o_text, o_logits = m.local_logits(h2[j], codes[f, b])
                chk.frame(ends[j], f"graph frame {f} voice {b}", codes[f, b], cont[f, b], o_text,
                          o_logits, tol, bar=2.4 * tol)
            h2 = st2.decode_step(np.stack([synth.frame_row(codes[f, b]) for b in far]),
                                 pos[far] + f)
        d = float(np.abs(h_end[far] - h2).max())
        assert d < tol
        for l in (0, 11):
            for j, b in enumerate(far):
                k, v, sp = ctx.read_ring(l, b)
                assert np.array_equal(sp, st2.slot_pos[j, l]), (l, b)
    chk.summary("C3")
    say(f"  C3: max |hidden diff| {max(max_h, d):.2e}")
    total = 8 * 60 * 16 + 2 * (G - 20) * 16
    assert chk.codes_equal + chk.codes_tied == total
    assert chk.codes_equal >= 0.99 * total


def _crafted_head_weights(hi=3, lo=5):
    """A 2-layer model whose local ln_f has scale 0 and shift e_0, so every
    local step's output is exactly e_0: each audio head's logits are then its
    row 0 exactly (also through the LayerNorm-folded head), and the text
    decision is text_head[0][9] = 1 against text_head[0][7] = 0 (always go
    on).  Row 0 of every head holds 1.0 at id `hi`, fp32(0.8333333) at id
    `lo`, 0.81 at id 11 and -1 elsewhere."""
    row = np.full(1024, -1.0, np.float32)
    row[hi], row[lo], row[11] = 1.0, np.float32(0.8333333), 0.81
    return _row_head_weights(row), row


def _row_head_weights(row):
    """_crafted_head_weights' model with `row` as every audio head's logits."""
    w = synth.model_weights(n_layers=2, vocab=64, seed=5)
    w["model.local_transformer.ln_f.weight"] = np.zeros(768, np.float32)
    e0 = np.zeros(768, np.float32)
    e0[0] = 1.0
    w["model.local_transformer.ln_f.bias"] = e0
    th = w["model.text_lm_head.weight"]
    th[0, 7], th[0, 9] = 0.0, 1.0
    for k in range(16):
        w[f"model.audio_lm_heads.{k}.weight"][0] = row
    return w


def _expected_codes(row, n_frames, penalty, seen, f32=False):
    out = []
    for _ in range(n_frames):
        tok = oracle.argmax_penalty(row, sorted(seen), penalty, f32=f32)[0]
        out.append(tok)
        seen.add(tok)
    return out


@pytest.mark.parametrize("B", [1, 2])
def test_penalty_is_the_double_and_settings_reach_the_frame_graph(B):
    """The repetition penalty is applied as the double 1.2: after id 3 (logit
    1.0) is drawn, 1.0 / 1.2 = 0.83333333 still beats id 5's fp32(0.8333333)
    = 0.83333331, which 1.0 / 1.2f = 0.83333330 would not.  Then the penalty
    changes to 1.25 between two mb_decode_frames calls on the same buffers:
    the second call's replayed frames must use 1.25 (id 11 wins its second
    frame; a stale 1.2 would give id 3).  Every channel of both voices
    follows the oracle's penalised argmax, and the per-call path agrees."""
    say("crafted penalty: double 1.2, then 1.25 through the frame graph")
    w, row = _crafted_head_weights()
    assert _expected_codes(row, 2, float(np.float32(1.2)), set()) == [3, 5]  # the case discriminates
    seen = set()
    want1 = _expected_codes(row, 3, 1.2, seen)
    assert want1 == [3, 3, 3]
    want2 = _expected_codes(row, 3, 1.25, seen)
    assert want2 == [5, 11, 3]
    stale = _expected_codes(row, 2, 1.2, {3, 5})
    assert stale[0] == 3  # what a replay with the old penalty would pick
    ids, n = _prompt_batch(B, 64, 90)
    with _ctx(w, 2, 64, B, 64) as ctx:
        h = ctx.prefill(ids, n)
        c1, f1, h1, p1 = ctx.decode_frames(h, n, 3)
        ctx.set_local_head(7, 9, 1.25)
        c2, f2, _, _ = ctx.decode_frames(h1, p1, 3)
    assert f1.all() and f2.all()
    for f in range(3):
        assert (c1[f] == want1[f]).all(), (f, c1[f])
        assert (c2[f] == want2[f]).all(), (f, c2[f])
    with _ctx(w, 2, 64, B, 64) as ref:  # the same frames call by call
        h = ref.prefill(ids, n)
        pos = n.copy()
        for f in range(6):
            if f == 3:
                ref.set_local_head(7, 9, 1.25)
            codes, cont = ref.local_frame(h)
            assert (codes == (want1 + want2)[f]).all(), (f, codes)
            h = ref.decode_step(np.stack([synth.frame_row(c) for c in codes]), pos)
            pos = pos + 1


@pytest.mark.parametrize("B", [1, 2])
def test_penalty_precision_f32_is_the_wgsl_arithmetic(B):
    """MB_PENALTY_F32, the WGSL engine's arithmetic (kernels-decode.ts:454-461):
    id 5 holds 1.0 and id 3 fp32(0.8333333).  Once 5 has been drawn, its f32
    penalised score 1.0 / 1.2f rounds to exactly fp32(0.8333333), a tie that
    the lower id 3 wins, while the double 1.0 / 1.2 = 0.83333333 keeps 5.
    Per call and through the frame graph (the precision switched between two
    mb_decode_frames calls on the same buffers, so the graph must be taken
    again), every channel of both voices follows the oracle's f32 or double
    choice, and the oracle's f32 path (plain fp32 division) agrees with the
    kernel's (a double quotient rounded once to f32)."""
    say("penalty precision: f32 (WGSL engine) against f64 (CPU path)")
    w, row = _crafted_head_weights(hi=5, lo=3)
    want64 = _expected_codes(row, 3, 1.2, set())
    want32 = _expected_codes(row, 3, 1.2, set(), f32=True)
    assert want64[:2] == [5, 5] and want32[:2] == [5, 3]  # the case discriminates
    ids, n = _prompt_batch(B, 64, 90)
    with _ctx(w, 2, 64, B, 64) as ctx:
        h = ctx.prefill(ids, n)
        c1, f1, h1, p1 = ctx.decode_frames(h, n, 3)
        ctx.clear_seen()
        ctx.set_penalty_precision(mb.MB_PENALTY_F32)
        c2, f2, _, _ = ctx.decode_frames(h1, p1, 3)
        with pytest.raises(mb.MbError) as e:
            ctx.set_penalty_precision(2)
        assert e.value.code == mb.MB_ERR_ARG
    assert f1.all() and f2.all()
    for f in range(3):
        assert (c1[f] == want64[f]).all(), (f, c1[f])
        assert (c2[f] == want32[f]).all(), (f, c2[f])
    with _ctx(w, 2, 64, B, 64) as ref:  # the f32 frames call by call
        ref.set_penalty_precision(mb.MB_PENALTY_F32)
        h = ref.prefill(ids, n)
        pos = n.copy()
        for f in range(3):
            codes, cont = ref.local_frame(h)
            assert (codes == want32[f]).all(), (f, codes)
            h = ref.decode_step(np.stack([synth.frame_row(c) for c in codes]), pos)
            pos = pos + 1


@pytest.mark.parametrize("B,f32", [(1, False), (1, True), (2, False)])
def test_code_choice_ties_nan_and_penalised_candidates(B, f32):
    """The greedy choice on a crafted row (every channel's logits): 2.0 at ids
    40 and 41 (one lane's ids) and 700 (another lane's), 1.7 at 300, NaN at
    ids 5 and 1000, -3e38 elsewhere.  Frame by frame the lowest id of the
    highest score wins, a NaN never does, the seen ids' penalised scores
    (2.0 / 1.2) tie each other across lanes and lose to 1.7 until it is seen
    too: codes 40, 41, 700, 300, then 40 again.  One voice makes each choice
    but the last inside the next step's projection, two voices in the argmax
    launch; both follow the oracle's penalised argmax."""
    say(f"code choice: ties, NaN, penalised candidates (B={B}, f32={f32})")
    row = np.full(1024, -3e38, np.float32)
    row[[40, 41, 700]] = 2.0
    row[300] = 1.7
    row[[5, 1000]] = np.nan
    w = _row_head_weights(row)
    frames = 6
    want = _expected_codes(row, frames, 1.2, set(), f32=f32)
    assert want == [40, 41, 700, 300, 40, 40], want  # the row discriminates
    ids, n = _prompt_batch(B, 64, 90)
    with _ctx(w, 2, 64, B, 64) as ctx:
        if f32:
            ctx.set_penalty_precision(mb.MB_PENALTY_F32)
        h = ctx.prefill(ids, n)
        pos = n.copy()
        for f in range(frames):
            codes, cont = ctx.local_frame(h)
            assert cont.all() and (codes == want[f]).all(), (f, codes)
            h = ctx.decode_step(np.stack([synth.frame_row(c) for c in codes]), pos)
            pos = pos + 1


def test_prefill_rows_and_local_steps():
    """PrefillRunner.run's whole hidden block (prefill.ts:325-603), also cut
    to one layer by its layerCount argument, and the nextFrameSteps probe (decode.ts:970-1030) against the oracle: every row of
    a ragged 3-voice prefill, then local steps 0, 1, 2, 9 and 16 fed with the
    codes of the frame just chosen."""
    say("prefill_rows + local_steps, 2 layers, 3 voices")
    L, V, B, C = 2, 64, 3, 96
    w = _c0_weights(n_layers=L, vocab=V, seed=11)
    m = oracle.Model(w, n_layers=L, vocab=V)
    prompts = [synth.prompt(40 + b, n_frames=4 + 5 * b, n_text=3 + 2 * b, vocab=V) for b in range(B)]
    n = np.array([p.shape[0] for p in prompts], np.int32)
    ids = np.full((B, n.max(), 17), 1024, np.int32)
    for b, p in enumerate(prompts):
        ids[b, :n[b]] = p
    m1 = oracle.Model(w, n_layers=1, vocab=V)
    with _ctx(w, L, V, B, C) as ctx:
        hid1 = ctx.prefill_rows(ids, n, layer_count=1)
        for b in range(B):
            ref = oracle.ModelState(m1, 1, C).prefill_all(0, prompts[b])
            assert np.abs(hid1[b, :n[b]] - ref).max() < 1e-4, b
        assert (ctx.read_ring(1, 0)[2] == -1).all()
        hid = ctx.prefill_rows(ids, n)
        for b in range(B):
            ref = oracle.ModelState(m, 1, C).prefill_all(0, prompts[b])
            assert np.abs(hid[b, :n[b]] - ref).max() < 1e-4, b
            assert not hid[b, n[b]:].any()
        h = np.stack([hid[b, n[b] - 1] for b in range(B)])
        codes, cont = ctx.local_frame(h)
        assert cont.all()
        for s in (0, 1, 2, 9, 16):
            out = ctx.local_steps(h, s)
            for b in range(B):
                ref = m.local_steps(h[b], s, codes[b])
                assert np.abs(out[b] - ref).max() < 1e-4, (s, b)
        with pytest.raises(mb.MbError):
            ctx.local_steps(h, 17)


def _per_call_frames(ctx, h, pos, max_pos, F, latch):
    """The frame loop driven call by call on device buffers: local frame, then
    the decode step of its row; positions advance for voices that continued
    (with `latch`, a voice that stopped stays stopped)."""
    import torch

    B = pos.shape[0]
    dev = h.device
    codes = torch.zeros((B, 16), dtype=torch.int32, device=dev)
    cont = torch.zeros(B, dtype=torch.int32, device=dev)
    rows = torch.zeros((B, 17), dtype=torch.int32, device=dev)
    alive = torch.ones(B, dtype=torch.int32, device=dev)
    out_codes, out_cont = [], []
    for f in range(F):
        ctx.local_frame_dev(B, h.data_ptr(), codes.data_ptr(), cont.data_ptr(), rows.data_ptr())
        ctx.decode_step_dev(B, rows.data_ptr(), pos.data_ptr(), max_pos, h.data_ptr())
        eff = cont * alive if latch else cont
        if latch:
            alive = eff.clone()
        pos += eff
        torch.cuda.synchronize()
        out_codes.append(codes.cpu().numpy().copy())
        out_cont.append(eff.cpu().numpy().copy())
    return np.stack(out_codes), np.stack(out_cont)


def _prompt_batch(B, V, seed):
    prompts = [synth.prompt(seed + b, n_frames=3 + 4 * b, n_text=4 + b, vocab=V) for b in range(B)]
    n = np.array([p.shape[0] for p in prompts], np.int32)
    ids = np.full((B, n.max(), 17), 1024, np.int32)
    for b, p in enumerate(prompts):
        ids[b, :n[b]] = p
    return ids, n


def test_device_frame_loop_matches_per_call_frames():
    """mb_decode_frames_dev (frame 0 as plain launches, later frames replayed
    from a captured HIP graph) against the same frames driven call by call:
    codes, flags, positions and hidden states agree bit for bit over three
    calls -- a capture, a recapture for new output buffers, and a replay of
    the cached graph."""
    torch = pytest.importorskip("torch")
    say("device frame loop vs per-call frames (capture, recapture, replay)")
    L, V, B, C, F = 2, 64, 4, 128, 12
    w = _c0_weights(n_layers=L, vocab=V, seed=21)
    ids, n = _prompt_batch(B, V, 60)
    max_pos = int(n.max()) + F
    dev = torch.device("cuda")
    with _ctx(w, L, V, B, C) as ref:
        ref.set_stream(torch.cuda.current_stream().cuda_stream)
        h = torch.from_numpy(ref.prefill(ids, n)).to(dev)
        pos = torch.from_numpy(n.copy()).to(dev)
        want_codes, want_cont = _per_call_frames(ref, h, pos, max_pos, F, latch=False)
        want_h, want_pos = h.cpu().numpy(), pos.cpu().numpy()
    assert want_cont.all()
    with _ctx(w, L, V, B, C) as ctx:
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        h = torch.from_numpy(ctx.prefill(ids, n)).to(dev)
        pos = torch.from_numpy(n.copy()).to(dev)
        bufs = [(torch.full((4, B, 16), -1, dtype=torch.int32, device=dev),
                 torch.full((4, B), -1, dtype=torch.int32, device=dev)) for _ in range(2)]
        got = []
        for cb, fb in [bufs[0], bufs[1], bufs[1]]:
            ctx.decode_frames_dev(B, 4, h.data_ptr(), pos.data_ptr(), max_pos, cb.data_ptr(),
                                  fb.data_ptr())
            torch.cuda.synchronize()
            got.append((cb.cpu().numpy().copy(), fb.cpu().numpy().copy()))
        assert np.array_equal(np.concatenate([g[1] for g in got]), want_cont)
        assert np.array_equal(np.concatenate([g[0] for g in got]), want_codes)
        assert np.array_equal(pos.cpu().numpy(), want_pos)
        assert np.array_equal(h.cpu().numpy(), want_h)


def test_device_frame_loop_stops_voices():
    """An untied model whose voices stop at different frames: within one call a
    stopped voice stays stopped and keeps its position; the voices still
    going match the call-by-call loop bit for bit."""
    torch = pytest.importorskip("torch")
    say("device frame loop with stopping voices")
    L, V, B, C, F = 2, 64, 6, 128, 10
    w = synth.model_weights(n_layers=L, vocab=V, seed=21, bias_std=0.02, ln_std=0.1)
    ids, n = _prompt_batch(B, V, 80)
    max_pos = int(n.max()) + F
    dev = torch.device("cuda")
    with _ctx(w, L, V, B, C) as ref:
        ref.set_stream(torch.cuda.current_stream().cuda_stream)
        h = torch.from_numpy(ref.prefill(ids, n)).to(dev)
        pos = torch.from_numpy(n.copy()).to(dev)
        want_codes, want_cont = _per_call_frames(ref, h, pos, max_pos, F, latch=True)
        want_h, want_pos = h.cpu().numpy(), pos.cpu().numpy()
    with _ctx(w, L, V, B, C) as ctx:
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        h = torch.from_numpy(ctx.prefill(ids, n)).to(dev)
        pos = torch.from_numpy(n.copy()).to(dev)
        cb = torch.full((F, B, 16), -1, dtype=torch.int32, device=dev)
        fb = torch.full((F, B), -1, dtype=torch.int32, device=dev)
        ctx.decode_frames_dev(B, F, h.data_ptr(), pos.data_ptr(), max_pos, cb.data_ptr(),
                              fb.data_ptr())
        torch.cuda.synchronize()
        got_codes, got_cont = cb.cpu().numpy(), fb.cpu().numpy()
    say(f"  frames continued per voice: {want_cont.sum(0).tolist()}")
    assert want_cont[0].any() and not want_cont[-1].all(), "expected a mix of going and stopped voices"
    assert np.array_equal(got_cont, want_cont)
    live = want_cont.astype(bool)
    assert np.array_equal(got_codes[live], want_codes[live])
    assert np.array_equal(pos.cpu().numpy(), want_pos)
    going = want_cont[-1].astype(bool)
    assert np.array_equal(h.cpu().numpy()[going], want_h[going])
    # the latch: once 0, a voice's flag stays 0
    assert (np.diff(got_cont, axis=0) <= 0).all()
