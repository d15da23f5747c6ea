"""The oracle's decoder pieces against properties the reference fixes.

- a decode step at position S-1 reproduces the last row of an S-row prefill
  bit for bit (decode.ts appends into the ring the prefill filled, so the two
  paths must agree exactly);
- the causal-prefix property: the first n rows of a prefill do not depend on
  later rows (the reference's 8-row and 195-row captures satisfy it exactly);
- the prompt layout of buildVoiceCloneRows (policy.ts:49-80) in two
  independent implementations;
- hand-made greedy cases for the repetition penalty and the stop rule
  (policy.ts:273-302).
"""
import numpy as np
import pytest

from mockbird_amd import synth
from oracle import oracle


@pytest.fixture(scope="module")
def tiny():
    w = synth.model_weights(n_layers=2, vocab=64, seed=3, bias_std=0.02, ln_std=0.1)
    return oracle.Model(w, n_layers=2, vocab=64), w


def _rows(seed, n_frames, n_text, vocab=64):
    return synth.prompt(seed, n_frames=n_frames, n_text=n_text, vocab=vocab)


def test_decode_step_reproduces_prefill_last_row(tiny):
    m, _ = tiny
    rows = _rows(1, 5, 6)
    S = rows.shape[0]
    full = oracle.ModelState(m, 1, 64)
    h_all = full.prefill_all(0, rows)
    part = oracle.ModelState(m, 1, 64)
    part.prefill_all(0, rows[:-1])
    h = part.decode_step(rows[-1][None], [S - 1])
    assert np.array_equal(h[0], h_all[-1])
    assert np.array_equal(part.K, full.K) and np.array_equal(part.V, full.V)


def test_causal_prefix(tiny):
    m, _ = tiny
    rows = _rows(2, 6, 9)
    a = oracle.ModelState(m, 1, 64).prefill_all(0, rows)
    b = oracle.ModelState(m, 1, 64).prefill_all(0, rows[:7])
    assert np.array_equal(a[:7], b)


def test_prompt_layout_c0():
    rows = synth.prompt(0, n_frames=150, n_text=128, vocab=32000)
    assert rows.shape == (281, 17)
    g = np.random.default_rng([0, 0x5EED])
    codes = g.integers(0, 1024, size=(150, 16), dtype=np.int32)
    text = g.integers(0, 32000, size=128, dtype=np.int32)
    assert np.array_equal(rows, oracle.build_rows(codes, text))
    assert rows[0, 0] == 6 and (rows[0, 1:] == 1024).all()
    assert (rows[1:151, 0] == 8).all() and np.array_equal(rows[1:151, 1:], codes)
    assert rows[151, 0] == 7 and np.array_equal(rows[152:280, 0], text)
    assert rows[280, 0] == 6 and (rows[151:, 1:] == 1024).all()
    fr = synth.frame_row(list(range(16)))
    assert fr[0] == 9 and np.array_equal(fr[1:], np.arange(16))


def test_repetition_penalty_cases():
    ap = oracle.argmax_penalty
    # positive seen logit divided: 1.1 / 1.2 < 1.0
    assert ap(np.array([1.0, 1.1, 0.5], np.float32), [1])[0] == 0
    # negative seen logit multiplied: -1.0 * 1.2 < -1.1
    assert ap(np.array([-1.0, -1.1], np.float32), [0])[0] == 1
    # nothing seen: plain argmax; penalty 1: plain argmax
    assert ap(np.array([1.0, 1.1], np.float32), [])[0] == 1
    assert ap(np.array([1.0, 1.1], np.float32), [1], penalty=1.0)[0] == 1
    # exact tie keeps the lowest id
    assert ap(np.array([0.5, 0.5, 0.2], np.float32), [])[0] == 0
    # the penalty is the JS double 1.2 (mossTtsRuntime.js:506-521): the fp32
    # logit 1.2f divided by it is 1.00000004 > 1.0, not a tie
    assert ap(np.array([1.0, 1.2, 0.0], np.float32), [1])[0] == 1
    assert ap(np.array([1.0, 1.2, 0.0], np.float32), [1], penalty=float(np.float32(1.2)))[0] == 0
    # a winner that s / 1.2 and s / 1.2f decide differently:
    # 1 / 1.2 = 0.83333333 > fp32(0.8333333) = 0.83333331 > 1 / 1.2f = 0.83333330
    crafted = np.array([1.0, 0.8333333], np.float32)
    assert ap(crafted, [0])[0] == 0
    assert ap(crafted, [0], penalty=float(np.float32(1.2)))[0] == 1
    # negative seen logits are multiplied: -1.0 * 1.2 = -1.2 > fp32(-1.2) = -1.20000005
    assert ap(np.array([-1.0, -1.2], np.float32), [0])[0] == 0
    assert ap(np.array([-1.0, -1.2], np.float32), [0], penalty=float(np.float32(1.2)))[0] == 0
    # zero counts as non-negative (divided), NaN never wins
    assert ap(np.array([0.0, -0.1], np.float32), [0])[0] == 0
    assert ap(np.array([np.nan, -5.0], np.float32), [])[0] == 1


def test_repetition_penalty_f32_mode():
    """The WGSL engine's f32 arithmetic (kernels-decode.ts:454-461), pinned
    against numpy's float32 arithmetic on random logits and seen sets, with
    the case where the two precisions pick differently: 1.0 / 1.2f rounds to
    exactly fp32(0.8333333), a tie the lower id wins."""
    ap = oracle.argmax_penalty
    crafted = np.array([0.8333333, 1.0], np.float32)
    assert ap(crafted, [1])[0] == 1
    assert ap(crafted, [1], f32=True)[0] == 0
    assert np.float32(1.0) / np.float32(1.2) == np.float32(0.8333333)
    g = np.random.default_rng(12)
    p32 = np.float32(1.2)
    for _ in range(200):
        logits = g.standard_normal(1024).astype(np.float32)
        seen = sorted(set(g.integers(0, 1024, size=int(g.integers(0, 40))).tolist()))
        s = logits.copy()
        for i in seen:
            s[i] = s[i] * p32 if s[i] < 0 else s[i] / p32
        want = int(np.argmax(s)) if seen else int(np.argmax(logits))
        assert ap(logits, seen, f32=True)[0] == want


def test_stop_rule(tiny):
    m, w = tiny
    h = np.random.default_rng(4).standard_normal(768).astype(np.float32)
    cont, e, a = m.text_decide(h)
    col = w["model.text_lm_head.weight"]
    assert np.isclose(e, float(h.astype(np.float64) @ col[:, 7]), rtol=1e-12)
    assert np.isclose(a, float(h.astype(np.float64) @ col[:, 9]), rtol=1e-12)
    assert cont == (a >= e)


def test_local_frame_updates_history_only_when_continuing(tiny):
    m, w = tiny
    st = oracle.ModelState(m, 2, 64)
    g = np.random.default_rng(5)
    hidden = g.standard_normal((2, 768)).astype(np.float32)
    codes, cont, margins = st.local_frame(hidden)
    for b in range(2):
        bits = np.unpackbits(st.seen[b].view(np.uint8), bitorder="little").reshape(16, 1024)
        if cont[b]:
            assert all(bits[c, codes[b, c]] for c in range(16)) and bits.sum() == 16
            assert (margins[b, 1:] >= 0).all()
        else:
            assert bits.sum() == 0


def test_local_steps_rederive_the_frame(tiny):
    """nextFrameSteps (decode.ts:970-1030) run to step s, then the step's own
    head, reproduces what the greedy frame chose at that step: the text
    decision from step 0 and code s-1 (with its margin) from step s >= 1.  A
    wrong embedding at any step (assistant slot, channel or code index)
    changes later codes."""
    m, w = tiny
    g = np.random.default_rng(6)
    col = w["model.text_lm_head.weight"]
    heads = [w[f"model.audio_lm_heads.{k}.weight"] for k in range(16)]
    n_cont = 0
    for trial in range(4):
        hidden = g.standard_normal(768).astype(np.float32)
        st = oracle.ModelState(m, 1, 64)
        codes, cont, margins = st.local_frame(hidden[None])
        h0 = m.local_steps(hidden, 0, codes[0])
        c, e, a = m.text_decide(h0)
        assert c == cont[0] and np.isclose(a - e, margins[0, 0], rtol=1e-12)
        if not cont[0]:
            continue
        n_cont += 1
        seen = [[] for _ in range(16)]
        for s in range(1, 17):
            h = m.local_steps(hidden, s, codes[0])
            logits = oracle.gemm(h[None], heads[s - 1])[0]
            tok, bv, sv = oracle.argmax_penalty(logits, seen[s - 1])
            assert tok == codes[0, s - 1], (trial, s)
            assert np.isclose(bv - sv, margins[0, s], rtol=1e-9, atol=1e-12)
    assert n_cont >= 1
