"""The oracle's model composition against an independent float64 restatement
of the reference's CPU decoder.

`RefDecoder` below is written from tools/onnx-probe/ref-decode.mjs alone, in
numpy float64, sharing no code with oracle/mb_oracle.c:

- embedRow ........ ref-decode.mjs:163-174 (wte[id0] + audio_k[id_{k+1}], pads skipped)
- layerNorm, gemv,
  geluTanh, RoPE .. :85-124 (RoPE angle in double, as the JS computes it)
- attend .......... :138-161 (scale 0.125, softmax over the whole cache)
- prefill ......... :175-204 (per layer: every row's attention, then every row's MLP)
- decodeStep ...... :207-234 (each layer's MLP right after its own attention)
- localStep ....... :238-272 (step 0 takes the global hidden, step 1 wte[text],
                    step s >= 2 audio_{s-2}[previous code]; position = step)
- argmaxPenalty ... :273-286 (strict >, HF penalty with the double 1.2)
- the frame loop .. :378-421 (text decision, 16 channels, the frame row
                    [assistant, codes] decoded at the next position)

The C oracle and the restatement run the same tiny 2-layer model, with
non-zero biases and LayerNorm scales and shifts so that a parameter read from
the wrong place shows.  Every prefill row's ln_f output, every ring row (K
roped at its position, V), every decode step's hidden state, every local step's
ln_f output, the text-decision dot products and all 16 channels' logits must
agree within 1e-4, the bar north_star sets for fp32 (the two differ only by
the oracle's fp32 storage of each op's output and its fp32 RoPE angle:
measured about 1e-6).  Greedy codes and continue flags must be equal wherever
the restatement's margin exceeds that bar.

Each mutant plants one plausible misreading of ref-decode.mjs in the
restatement (LN1's parameters used for the MLP, audio channel k embedded from
table k+1, local step 1 fed wte[audio_end], the attention residual dropped,
the frame row decoded one position past the prompt's end, each decode
layer's MLP run on the pre-attention state).  Every mutant must miss the C
oracle by far more than the bar, so the comparison would catch the same
misreading in the oracle.  (Shifting every local-head position by the same
amount is not among them: RoPE scores depend only on position differences,
so that shift changes nothing but rounding.)
"""
import numpy as np
import pytest

from mockbird_amd import synth
from oracle import oracle

D, H, HD, F, NVQ, PAD, EPS = 768, 12, 64, 3072, 16, 1024, 1e-5
TOL = 1e-4
AUDIO_END, ASSISTANT = 7, 9
PENALTY = 1.2

MUTANTS = ("ln1_for_mlp", "embed_channel_shift", "step1_audio_end", "no_attn_residual",
           "decode_pos_plus_one", "mlp_before_attention")


class RefDecoder:
    """float64 restatement of ref-decode.mjs for a weight dict with the
    exported graph's tensor names (ref-decode.mjs:40-80)."""

    def __init__(self, w, n_layers, mut=()):
        self.mut = set(mut)
        g = lambda n: np.asarray(w[n], np.float64)
        self.layers = []
        for i in range(n_layers):
            p = f"core.model.transformer.h.{i}."
            self.layers.append(self._layer(g, p))
        self.loc = self._layer(g, "model.local_transformer.h.0.")
        self.lnf = (g("core.model.transformer.ln_f.weight"), g("core.model.transformer.ln_f.bias"))
        self.loc_lnf = (g("model.local_transformer.ln_f.weight"),
                        g("model.local_transformer.ln_f.bias"))
        self.wte = g("core.model.transformer.wte.weight")
        self.aud = [g(f"core.model.audio_embeddings.{k}.weight") for k in range(NVQ)]
        self.text_head = g("model.text_lm_head.weight")
        self.heads = [g(f"model.audio_lm_heads.{k}.weight") for k in range(NVQ)]
        self.inv_freq = np.array([10000.0 ** (-(2 * i) / HD) for i in range(HD // 2)])

    @staticmethod
    def _layer(g, p):
        return {k: g(p + n) for k, n in (
            ("ln1w", "ln_1.weight"), ("ln1b", "ln_1.bias"), ("ln2w", "ln_2.weight"),
            ("ln2b", "ln_2.bias"), ("attn", "attn.c_attn.weight"), ("attnb", "attn.c_attn.bias"),
            ("proj", "attn.c_proj.weight"), ("projb", "attn.c_proj.bias"),
            ("fcin", "mlp.fc_in.weight"), ("fcinb", "mlp.fc_in.bias"),
            ("fcout", "mlp.fc_out.weight"), ("fcoutb", "mlp.fc_out.bias"))}

    # ---- kernels (ref-decode.mjs:85-161)
    @staticmethod
    def layer_norm(x, w, b):
        m = x.sum() / D
        v = ((x - m) ** 2).sum() / D
        return (x - m) / np.sqrt(v + EPS) * w + b

    @staticmethod
    def gelu(v):
        return 0.5 * v * (1 + np.tanh(0.7978845608028654 * (v + 0.044715 * v * v * v)))

    def rope(self, v, pos):
        v = v.reshape(H, HD)
        ang = pos * self.inv_freq
        c, s = np.repeat(np.cos(ang), 2), np.repeat(np.sin(ang), 2)
        partner = np.empty_like(v)
        partner[:, 0::2] = -v[:, 1::2]
        partner[:, 1::2] = v[:, 0::2]
        return (v * c + partner * s).reshape(D)

    @staticmethod
    def attend(q, ks, vs):
        K, V = np.stack(ks).reshape(-1, H, HD), np.stack(vs).reshape(-1, H, HD)
        out = np.zeros((H, HD))
        for h in range(H):
            s = K[:, h] @ q.reshape(H, HD)[h] * 0.125
            p = np.exp(s - s.max())
            out[h] = (p / p.sum()) @ V[:, h]
        return out.reshape(D)

    def embed_row(self, row):
        x = self.wte[row[0]].copy()
        for k in range(NVQ):
            if row[k + 1] == PAD:
                continue
            table = self.aud[(k + 1) % NVQ] if "embed_channel_shift" in self.mut else self.aud[k]
            x += table[row[k + 1]]
        return x

    # ---- one layer's two halves
    def _attn(self, L, x, cache, pos):
        qkv = self.layer_norm(x, L["ln1w"], L["ln1b"]) @ L["attn"] + L["attnb"]
        q, k, v = qkv[:D], qkv[D:2 * D], qkv[2 * D:]
        cache[0].append(self.rope(k, pos))
        cache[1].append(v)
        proj = self.attend(self.rope(q, pos), cache[0], cache[1]) @ L["proj"] + L["projb"]
        return proj if "no_attn_residual" in self.mut else x + proj

    def _mlp(self, L, x):
        w, b = (L["ln1w"], L["ln1b"]) if "ln1_for_mlp" in self.mut else (L["ln2w"], L["ln2b"])
        a = self.gelu(self.layer_norm(x, w, b) @ L["fcin"] + L["fcinb"])
        return x + a @ L["fcout"] + L["fcoutb"]

    def _layer_step(self, L, x, cache, pos):
        if "mlp_before_attention" in self.mut:
            return self._attn(L, self._mlp(L, x), cache, pos)
        return self._mlp(L, self._attn(L, x, cache, pos))

    # ---- the model (ref-decode.mjs:175-272)
    def prefill(self, rows):
        hs = [self.embed_row(r) for r in rows]
        kv = []
        for L in self.layers:
            cache = ([], [])
            if "mlp_before_attention" in self.mut:
                hs = [self._mlp(L, h) for h in hs]
            for i in range(len(hs)):
                hs[i] = self._attn(L, hs[i], cache, i)
            if "mlp_before_attention" not in self.mut:
                hs = [self._mlp(L, h) for h in hs]
            kv.append(cache)
        return [self.layer_norm(h, *self.lnf) for h in hs], kv

    def decode_step(self, x, kv, pos):
        if "decode_pos_plus_one" in self.mut:
            pos += 1
        for L, cache in zip(self.layers, kv):
            x = self._layer_step(L, x, cache, pos)
        return self.layer_norm(x, *self.lnf)

    def local_step(self, e, cache, step):
        return self.layer_norm(self._layer_step(self.loc, e, cache, step), *self.loc_lnf)

    def step1_input(self):
        return self.wte[AUDIO_END if "step1_audio_end" in self.mut else ASSISTANT]

    @staticmethod
    def argmax_penalty(vals, seen):
        best, best_val, second = 0, -np.inf, -np.inf
        for i, s in enumerate(vals):
            if seen and i in seen:
                s = s * PENALTY if s < 0 else s / PENALTY
            if s > best_val:
                best, best_val, second = i, s, best_val
            elif s > second:
                second = s
        return best, best_val - second


def _tiny(seed=3):
    w = synth.model_weights(n_layers=2, vocab=64, seed=seed, bias_std=0.05, ln_std=0.2)
    return w


def _run_both(w, ref, n_frames=3, rows=None, cap=64):
    """Run the C oracle and `ref` side by side through prefill and the frame
    loop (each frame teacher-forced with the C oracle's codes).  Returns
    (max abs difference over every compared value, list of code/flag
    disagreements whose restatement margin exceeds TOL, frames continued)."""
    m = oracle.Model(w, n_layers=2, vocab=64)
    if rows is None:
        rows = synth.prompt(5, n_frames=5, n_text=6, vocab=64)
    S = rows.shape[0]
    st = oracle.ModelState(m, 1, cap)
    h_or = st.prefill_all(0, rows)
    h_ref, kv = ref.prefill(rows)
    diff = float(np.abs(h_or - np.stack(h_ref)).max())
    for l in range(2):
        diff = max(diff, float(np.abs(st.K[0, l, :S] - np.stack(kv[l][0])).max()),
                   float(np.abs(st.V[0, l, :S] - np.stack(kv[l][1])).max()))
    bad, n_cont = [], 0
    hidden_or, hidden_ref = h_or[-1], h_ref[-1]
    seen = [set() for _ in range(NVQ)]
    pos = S
    for f in range(n_frames):
        codes, cont, _ = st.local_frame(hidden_or[None])
        cache = ([], [])
        h0 = ref.local_step(hidden_ref, cache, 0)
        t_end, t_asst = h0 @ ref.text_head[:, AUDIO_END], h0 @ ref.text_head[:, ASSISTANT]
        text2, logits = m.local_logits(hidden_or, codes[0])
        diff = max(diff, abs(text2[0] - t_end), abs(text2[1] - t_asst))
        diff = max(diff, float(np.abs(m.local_steps(hidden_or, 0, codes[0]) - h0).max()))
        if (t_asst >= t_end) != bool(cont[0]) and abs(t_asst - t_end) > TOL:
            bad.append((f, "continue"))
        if not cont[0]:
            break
        n_cont += 1
        for ch in range(NVQ):
            e = ref.step1_input() if ch == 0 else ref.aud[ch - 1][codes[0, ch - 1]]
            h = ref.local_step(e, cache, ch + 1)
            diff = max(diff, float(np.abs(m.local_steps(hidden_or, ch + 1, codes[0]) - h).max()))
            lg = h @ ref.heads[ch]
            diff = max(diff, float(np.abs(logits[ch] - lg).max()))
            tok, margin = ref.argmax_penalty(lg, seen[ch])
            if tok != codes[0, ch] and margin > TOL:
                bad.append((f, ch, tok, int(codes[0, ch]), margin))
            seen[ch].add(int(codes[0, ch]))
        row = synth.frame_row(codes[0])
        hidden_or = st.decode_step(row[None], [pos])[0]
        hidden_ref = ref.decode_step(ref.embed_row(row), kv, pos)
        diff = max(diff, float(np.abs(hidden_or - hidden_ref).max()))
        pos += 1
    return diff, bad, n_cont


@pytest.fixture(scope="module")
def tiny_run():
    w = _tiny()
    return w, _run_both(w, RefDecoder(w, 2))


def test_oracle_matches_float64_restatement(tiny_run):
    w, (diff, bad, n_cont) = tiny_run
    print(f"max |oracle - float64 restatement| = {diff:.2e}; frames continued {n_cont}")
    assert n_cont >= 2, "the model must decode codes for the comparison to cover the local head"
    assert diff < TOL
    assert not bad, bad


def test_stop_decision_matches(tiny_run):
    """A frame whose text decision stops (untied head) compares the same way:
    the restatement's loop breaks at the same frame."""
    w, _ = tiny_run
    w2 = dict(w)
    head = w["model.text_lm_head.weight"].copy()
    head[:, ASSISTANT] = head[:, AUDIO_END] - np.float32(0.05)  # assistant < end for typical h
    w2["model.text_lm_head.weight"] = head
    m = oracle.Model(w2, n_layers=2, vocab=64)
    ref = RefDecoder(w2, 2)
    g = np.random.default_rng(9)
    stops = 0
    for _ in range(6):
        hid = g.standard_normal(D).astype(np.float32)
        st = oracle.ModelState(m, 1, 64)
        _, cont, margins = st.local_frame(hid[None])
        h0 = ref.local_step(hid.astype(np.float64), ([], []), 0)
        a_minus_e = h0 @ head[:, ASSISTANT].astype(np.float64) - h0 @ head[:, AUDIO_END].astype(np.float64)
        assert abs(margins[0, 0] - a_minus_e) < TOL
        assert bool(cont[0]) == (a_minus_e >= 0)
        stops += not cont[0]
    assert stops >= 1


@pytest.mark.parametrize("mut", MUTANTS)
def test_mutant_misses_the_oracle(tiny_run, mut):
    w, (diff_ok, _, _) = tiny_run
    diff, bad, _ = _run_both(w, RefDecoder(w, 2, mut=(mut,)))
    print(f"{mut}: max diff {diff:.2e}, code disagreements {len(bad)}")
    assert diff > 100 * TOL or bad, f"mutant {mut} is not caught"
    assert diff > 1000 * diff_ok or bad


def test_embed_row_structured_tables():
    """or_embed_row on tables built so that each (table, row) leaves its own
    mark: wte[t] has t+1 in dimension 0; audio table k row i has (i+1) in
    dimension 1+k and 1 in dimension 17+k.  The embedding of a row then
    reads back which table and which id fed each channel, and which channels
    were skipped as pads, with no arithmetic to retype."""
    V = 40
    w = synth.model_weights(n_layers=1, vocab=V, seed=2)
    wte = np.zeros((V, D), np.float32)
    wte[:, 0] = np.arange(1, V + 1)
    w["core.model.transformer.wte.weight"] = wte
    for k in range(NVQ):
        t = np.zeros((1024, D), np.float32)
        t[:, 1 + k] = np.arange(1, 1025)
        t[:, 17 + k] = 1
        w[f"core.model.audio_embeddings.{k}.weight"] = t
    m = oracle.Model(w, n_layers=1, vocab=V)
    g = np.random.default_rng(12)
    for trial in range(20):
        row = np.full(17, PAD, np.int32)
        row[0] = g.integers(0, V)
        live = g.random(NVQ) < 0.6
        ids = g.integers(0, 1024, NVQ)
        row[1:][live] = ids[live]
        if trial == 0:
            row[1:] = PAD  # a text row: every channel padded
        if trial == 1:
            row[1:] = 1023  # every channel at the last id
            live[:] = True
            ids[:] = 1023
        if trial == 0:
            live[:] = False
        x = m.embed_row(row)
        assert x[0] == row[0] + 1
        for k in range(NVQ):
            assert x[1 + k] == (ids[k] + 1 if live[k] else 0), (trial, k)
            assert x[17 + k] == (1 if live[k] else 0), (trial, k)
        assert not x[33:].any()


def test_embed_row_accumulates_in_fp32_channel_order():
    """ref-decode.mjs:163-174 adds into a Float32Array, channel by channel:
    values chosen so that fp32 order matters (1 + 2^-24 + 2^-24 rounds back to
    1 when added one at a time, but 2^-23 added at once survives)."""
    V = 16
    w = synth.model_weights(n_layers=1, vocab=V, seed=2)
    wte = np.zeros((V, D), np.float32)
    wte[:, 0] = 1.0
    w["core.model.transformer.wte.weight"] = wte
    for k in range(NVQ):
        t = np.zeros((1024, D), np.float32)
        t[:, 0] = np.float32(2.0 ** -24)
        w[f"core.model.audio_embeddings.{k}.weight"] = t
    m = oracle.Model(w, n_layers=1, vocab=V)
    row = np.zeros(17, np.int32)
    assert m.embed_row(row)[0] == np.float32(1.0)


def test_attend_prefill_wrapped_ring_brute_force():
    """Ring.attend_prefill over a ring that has wrapped several times, against
    float64 attention over the visible set computed from the write history
    alone: a slot holds the latest position written to it (pos mod C), and a
    query at position cur sees the stored positions p with p <= cur and
    cur - p < C."""
    C, B = 8, 2
    g = np.random.default_rng(21)
    ring = oracle.Ring(B, C)
    hist = [dict() for _ in range(B)]  # position -> (roped k, v)
    pos0 = np.array([0, 3], np.int32)
    n_empty = [0]
    for chunk in range(3):
        n = np.array([7, 9], np.int32) if chunk < 2 else np.array([5, 4], np.int32)
        qkv = g.standard_normal((B, 9, 2304), dtype=np.float32)
        q = ring.write(qkv, pos0, n)
        for b in range(B):
            for r in range(n[b]):
                p = int(pos0[b]) + r
                hist[b][p] = (oracle.rope(qkv[b, r, 768:1536], p), qkv[b, r, 1536:])
        out = ring.attend_prefill(q, pos0, n)
        for b in range(B):
            stored = {}
            for p in sorted(hist[b]):
                stored[p % C] = p
            for r in range(n[b]):
                cur = int(pos0[b]) + r
                vis = sorted(p for p in stored.values() if p <= cur and cur - p < C)
                if not vis:  # its own row was overwritten later in the chunk: no live slot
                    assert not out[b, r].any(), (chunk, b, r)
                    n_empty[0] += 1
                    continue
                K = np.stack([hist[b][p][0] for p in vis]).astype(np.float64).reshape(-1, H, HD)
                V = np.stack([hist[b][p][1] for p in vis]).astype(np.float64).reshape(-1, H, HD)
                qq = q[b, r].astype(np.float64).reshape(H, HD)
                want = np.zeros((H, HD))
                for h in range(H):
                    s = K[:, h] @ qq[h] * 0.125
                    p_ = np.exp(s - s.max())
                    want[h] = (p_ / p_.sum()) @ V[:, h]
                assert np.abs(out[b, r] - want.reshape(D)).max() < 1e-5, (chunk, b, r)
        pos0 = pos0 + n
    assert n_empty[0] >= 1  # the 9-row chunks overwrite their own first row
