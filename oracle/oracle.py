"""ctypes wrapper over the C oracle (liboracle.so) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py may
import this module; it checks results and is never the thing measured or shipped.
Every function here is a thin call into oracle/mb_oracle.c, whose header lists
the reference file:line each piece restates.

Ring arrays here use the reference's layout (prefill.ts:55-56): per sequence
(and per layer where stated) K and V are [slot][768] with head-major columns
head*64 + dim, and slot_pos[slot] holds the absolute position in that slot.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
#: MB_ORACLE_LIB names another build of the same source (the sanitized one,
#: oracle/_asan/liboracle.so, for tests/test_oracle_sanitized.py)
_LIB = os.environ.get("MB_ORACLE_LIB") or os.path.join(_HERE, "liboracle.so")
#: the fp32-accumulating build of mb_oracle.c: the CPU throughput baseline
#: only (bench.py's cpu_baseline leg), never a checker
_LIB_FP32 = os.path.join(_HERE, "liboracle_fp32.so")
_lib = None
_libs = {}

D, H, HD, QKV, FFN, NVQ, ROW, PAD, CODES = 768, 12, 64, 2304, 3072, 16, 17, 1024, 1024

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")


def build() -> str:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB


def lib():
    global _lib
    if _lib is None:
        _lib = _load(_LIB)
    return _lib


def lib_fp32():
    """The fp32 baseline build (same functions, fp32 accumulators)."""
    return _load(_LIB_FP32, codec=False)


def _load(path, codec=True):
    if path in _libs:
        return _libs[path]
    if not os.path.exists(path):
        build()
    L = C.CDLL(path)
    L.or_inv_freq.argtypes = [_f32p]
    L.or_bf16_round.argtypes = [C.c_float]
    L.or_bf16_round.restype = C.c_float
    L.or_bf16_round_array.argtypes = [_f32p, C.c_int64, _f32p]
    L.or_rope.argtypes = [_f32p, C.c_int, C.c_int64, _f32p]
    L.or_slot_of.argtypes = [C.c_int64, C.c_int, C.c_int]
    L.or_slot_live.argtypes = [C.c_int64, C.c_int64, C.c_int]
    L.or_ring_write.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _f32p, C.c_int64,
                                _i32p, _i32p, C.c_void_p, _f32p, _f32p, _i32p]
    L.or_decode_attention.argtypes = [C.c_int, C.c_int, _f32p, _i32p, _f32p, _f32p, _i32p, _f32p]
    L.or_prefill_attention.argtypes = [C.c_int, C.c_int, C.c_int, _f32p, _i32p, _i32p, _f32p,
                                       _f32p, _i32p, _f32p]
    L.or_layernorm.argtypes = [_f32p, C.c_void_p, C.c_void_p, C.c_int, _f32p]
    L.or_gemm.argtypes = [C.c_int, C.c_int, C.c_int, _f32p, _f32p, C.c_void_p, _f32p]
    L.or_gelu_tanh.argtypes = [C.c_float]
    L.or_gelu_tanh.restype = C.c_float
    L.or_argmax_penalty.argtypes = [_f32p, C.c_int, _u32p, C.c_double, C.c_void_p, C.c_void_p]
    L.or_argmax_penalty_prec.argtypes = [_f32p, C.c_int, _u32p, C.c_double, C.c_int, C.c_void_p,
                                         C.c_void_p]
    L.or_build_rows.argtypes = [C.c_int, _i32p, C.c_int, _i32p, _i32p]
    L.or_embed_row.argtypes = [C.c_void_p, _i32p, _f32p]
    L.or_text_decide.argtypes = [C.c_void_p, _f32p, C.c_void_p, C.c_void_p]
    L.or_model_prefill.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, _i32p, _f32p,
                                   _f32p, _i32p, _f32p]
    L.or_model_decode_step.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, _i32p, C.c_int,
                                       _f32p, _f32p, _i32p, _f32p]
    L.or_local_frame.argtypes = [C.c_void_p, _f32p, _u32p, _i32p, C.c_void_p]
    L.or_local_steps.argtypes = [C.c_void_p, _f32p, C.c_int, _i32p, _f32p]
    L.or_local_logits.argtypes = [C.c_void_p, _f32p, _i32p, _f64p, _f32p]
    L.or_model_prefill_batch.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                         _i32p, _i32p, _f32p, _f32p, _i32p, _f32p]
    L.or_model_decode_step_batch.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int,
                                             _i32p, _i32p, _f32p, _f32p, _i32p, _f32p]
    L.or_local_frame_batch.argtypes = [C.c_void_p, C.c_int, _f32p, _u32p, _i32p, _i32p,
                                       C.c_void_p]
    if codec:
        L.or_erf_as.argtypes = [C.c_double]
        L.or_erf_as.restype = C.c_double
        L.or_gelu_erf.argtypes = [C.c_float]
        L.or_gelu_erf.restype = C.c_float
        L.or_codec_slots.argtypes = [C.c_void_p]
        L.or_codec_slots.restype = C.c_int64
        L.or_codec_rvq.argtypes = [C.c_void_p, _i32p, _f32p]
        L.or_codec_decode_batch.argtypes = [C.c_void_p, C.c_int, _f32p, _f32p, _i32p, _i32p,
                                            C.c_int, _i32p, _f32p]
        L.or_codec_decode_batch.restype = C.c_int
    _libs[path] = L
    return L


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def inv_freq() -> np.ndarray:
    out = np.zeros(32, np.float32)
    lib().or_inv_freq(out)
    return out


def bf16_round(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty_like(x)
    lib().or_bf16_round_array(x, x.size, out)
    return out


def rope(x: np.ndarray, pos: int) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty_like(x)
    lib().or_rope(x, x.size // 64, int(pos), out)
    return out


def slot_of(pos: int, cap: int, wrap: bool = True) -> int:
    return lib().or_slot_of(int(pos), int(cap), int(wrap))


def slot_live(stored: int, cur: int, cap: int) -> bool:
    return bool(lib().or_slot_live(int(stored), int(cur), int(cap)))


class Ring:
    """Per-sequence rings for one layer: K, V [B][C][768] fp32 and slot_pos [B][C]."""

    def __init__(self, B: int, cap: int, kv_bf16: bool = False, wrap: bool = True):
        self.B, self.C, self.kv_bf16, self.wrap = B, cap, kv_bf16, wrap
        self.K = np.zeros((B, cap, D), np.float32)
        self.V = np.zeros((B, cap, D), np.float32)
        self.slot_pos = np.full((B, cap), -1, np.int32)

    def write(self, qkv: np.ndarray, pos0, n) -> np.ndarray:
        """qkv [B][rows_max][2304]; returns roped q [B][rows_max][768]."""
        qkv = _c(qkv, np.float32)
        B, rows_max = qkv.shape[0], qkv.shape[1]
        q = np.zeros((B, rows_max, D), np.float32)
        rc = lib().or_ring_write(B, self.C, int(self.wrap), int(self.kv_bf16), rows_max, qkv, QKV,
                                 _c(pos0, np.int32), _c(n, np.int32), q.ctypes.data, self.K,
                                 self.V, self.slot_pos)
        if rc != 0:
            raise ValueError("position does not fit the ring")
        return q

    def append(self, qkv: np.ndarray, pos) -> np.ndarray:
        """One row per sequence: qkv [B][2304] at positions pos[B]; returns q [B][768]."""
        B = qkv.shape[0]
        return self.write(qkv.reshape(B, 1, QKV), pos, np.ones(B, np.int32))[:, 0]

    def attend(self, q: np.ndarray, pos) -> np.ndarray:
        q = _c(q, np.float32)
        out = np.zeros((q.shape[0], D), np.float32)
        lib().or_decode_attention(q.shape[0], self.C, q, _c(pos, np.int32), self.K, self.V,
                                  self.slot_pos, out)
        return out

    def attend_prefill(self, q: np.ndarray, pos0, n) -> np.ndarray:
        q = _c(q, np.float32)
        B, rows_max = q.shape[0], q.shape[1]
        out = np.zeros((B, rows_max, D), np.float32)
        lib().or_prefill_attention(B, self.C, rows_max, q, _c(pos0, np.int32), _c(n, np.int32),
                                   self.K, self.V, self.slot_pos, out)
        return out


def layernorm(x, w=None, b=None) -> np.ndarray:
    x = _c(x, np.float32)
    n = x.shape[-1]
    flat = x.reshape(-1, n)
    out = np.empty_like(flat)
    wp = _c(w, np.float32) if w is not None else None
    bp = _c(b, np.float32) if b is not None else None
    row = np.empty(n, np.float32)
    for r in range(flat.shape[0]):
        lib().or_layernorm(np.ascontiguousarray(flat[r]), wp.ctypes.data if wp is not None else None,
                           bp.ctypes.data if bp is not None else None, n, row)
        out[r] = row
    return out.reshape(x.shape)


def gemm(x, W, bias=None) -> np.ndarray:
    x = _c(x, np.float32)
    W = _c(W, np.float32)
    M, K = x.shape
    N = W.shape[1]
    y = np.zeros((M, N), np.float32)
    bp = _c(bias, np.float32) if bias is not None else None
    lib().or_gemm(M, K, N, x, W, bp.ctypes.data if bp is not None else None, y)
    return y


def gelu(x) -> np.ndarray:
    f = np.vectorize(lambda v: lib().or_gelu_tanh(float(v)), otypes=[np.float32])
    return f(np.asarray(x, np.float32))


def argmax_penalty(logits, seen_ids=(), penalty: float = 1.2, f32: bool = False):
    """Penalised argmax; f32 selects the WGSL engine's f32 penalty arithmetic."""
    logits = _c(logits, np.float32)
    seen = np.zeros((logits.size + 31) // 32, np.uint32)
    for i in seen_ids:
        seen[i >> 5] |= np.uint32(1 << (i & 31))
    bv, sv = C.c_double(), C.c_double()
    tok = lib().or_argmax_penalty_prec(logits, logits.size, seen, C.c_double(penalty), int(f32),
                                       C.byref(bv), C.byref(sv))
    return tok, bv.value, sv.value


def build_rows(codes: np.ndarray, text: np.ndarray) -> np.ndarray:
    codes = _c(codes, np.int32).reshape(-1, NVQ)
    text = _c(text, np.int32)
    rows = np.zeros((codes.shape[0] + text.size + 3, ROW), np.int32)
    n = lib().or_build_rows(codes.shape[0], codes.reshape(-1), text.size, text, rows.reshape(-1))
    assert n == rows.shape[0]
    return rows


# ------------------------------------------------------------------- model

class _Layer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "ln1_w", "ln1_b", "attn_w", "attn_b", "proj_w", "proj_b",
        "ln2_w", "ln2_b", "fc_in_w", "fc_in_b", "fc_out_w", "fc_out_b")]


class _Model(C.Structure):
    _fields_ = [
        ("n_layers", C.c_int), ("vocab", C.c_int),
        ("layers", C.c_void_p),
        ("lnf_w", C.c_void_p), ("lnf_b", C.c_void_p),
        ("wte", C.c_void_p),
        ("audio_emb", C.c_void_p * NVQ),
        ("local", _Layer),
        ("local_lnf_w", C.c_void_p), ("local_lnf_b", C.c_void_p),
        ("text_head", C.c_void_p),
        ("audio_heads", C.c_void_p * NVQ),
        ("audio_end_id", C.c_int), ("assistant_id", C.c_int),
        ("penalty", C.c_double),
        ("penalty_f32", C.c_int),
    ]


_LAYER_KEYS = ("ln_1.weight", "ln_1.bias", "attn.c_attn.weight", "attn.c_attn.bias",
               "attn.c_proj.weight", "attn.c_proj.bias", "ln_2.weight", "ln_2.bias",
               "mlp.fc_in.weight", "mlp.fc_in.bias", "mlp.fc_out.weight", "mlp.fc_out.bias")


class Model:
    """Oracle view of a weight dict named as in mockbird_amd.synth (the
    reference's ONNX tensor names, ref-decode.mjs:40-80)."""

    def __init__(self, weights: dict, n_layers: int, vocab: int, penalty: float = 1.2,
                 audio_end_id: int = 7, assistant_id: int = 9, fp32: bool = False,
                 penalty_f32: bool = False):
        # fp32 selects the fp32-accumulating baseline build (timing only)
        self._lib = lib_fp32() if fp32 else lib()
        self._keep = {k: _c(v, np.float32) for k, v in weights.items()}
        w = self._keep
        self._layers = (_Layer * n_layers)()
        for i in range(n_layers):
            p = f"core.model.transformer.h.{i}."
            self._layers[i] = _Layer(*[w[p + k].ctypes.data for k in _LAYER_KEYS])
        m = _Model()
        m.n_layers, m.vocab = n_layers, vocab
        m.layers = C.cast(self._layers, C.c_void_p)
        m.lnf_w = w["core.model.transformer.ln_f.weight"].ctypes.data
        m.lnf_b = w["core.model.transformer.ln_f.bias"].ctypes.data
        m.wte = w["core.model.transformer.wte.weight"].ctypes.data
        for k in range(NVQ):
            m.audio_emb[k] = w[f"core.model.audio_embeddings.{k}.weight"].ctypes.data
            m.audio_heads[k] = w[f"model.audio_lm_heads.{k}.weight"].ctypes.data
        lp = "model.local_transformer.h.0."
        m.local = _Layer(*[w[lp + k].ctypes.data for k in _LAYER_KEYS])
        m.local_lnf_w = w["model.local_transformer.ln_f.weight"].ctypes.data
        m.local_lnf_b = w["model.local_transformer.ln_f.bias"].ctypes.data
        m.text_head = w["model.text_lm_head.weight"].ctypes.data
        m.audio_end_id, m.assistant_id, m.penalty = audio_end_id, assistant_id, penalty
        m.penalty_f32 = int(penalty_f32)
        self._m = m
        self.n_layers, self.vocab = n_layers, vocab

    @property
    def ptr(self):
        return C.addressof(self._m)

    def embed_row(self, row17) -> np.ndarray:
        x = np.zeros(D, np.float32)
        self._lib.or_embed_row(self.ptr, _c(row17, np.int32), x)
        return x

    def local_steps(self, hidden, max_step: int, codes) -> np.ndarray:
        """ln_f output of local-head step `max_step` with the codes fed in."""
        out = np.zeros(D, np.float32)
        self._lib.or_local_steps(self.ptr, _c(hidden, np.float32), int(max_step), _c(codes, np.int32),
                             out)
        return out

    def local_logits(self, hidden, codes):
        """The frame head teacher-forced with `codes` [16]: returns
        (text2 = (audio_end, assistant) dot products of step 0 [2] float64,
        audio-head logits of every channel [16][1024] before the penalty)."""
        text2 = np.zeros(2, np.float64)
        logits = np.zeros((NVQ, CODES), np.float32)
        self._lib.or_local_logits(self.ptr, _c(hidden, np.float32), _c(codes, np.int32), text2,
                                  logits)
        return text2, logits

    def text_decide(self, h):
        e, a = C.c_double(), C.c_double()
        c = self._lib.or_text_decide(self.ptr, _c(h, np.float32), C.byref(e), C.byref(a))
        return bool(c), e.value, a.value


class ModelState:
    """Per-voice global rings for every layer: K/V [B][L][C][768], slot_pos
    [B][L][C], and per-voice repetition history seen [B][16][32]."""

    def __init__(self, model: Model, B: int, cap: int, kv_bf16: bool = False, wrap: bool = True):
        self.m, self.B, self.C, self.kv_bf16, self.wrap = model, B, cap, kv_bf16, wrap
        L = model.n_layers
        self.K = np.zeros((B, L, cap, D), np.float32)
        self.V = np.zeros((B, L, cap, D), np.float32)
        self.slot_pos = np.full((B, L, cap), -1, np.int32)
        self.seen = np.zeros((B, NVQ, 32), np.uint32)

    def prefill(self, ids: np.ndarray, n_rows) -> np.ndarray:
        """ids [B][rows_max][17] -> last-row hidden [B][768]."""
        ids = _c(ids, np.int32)
        out = np.zeros((self.B, D), np.float32)
        rc = self.m._lib.or_model_prefill_batch(self.m.ptr, self.B, self.C, int(self.wrap),
                                          int(self.kv_bf16), ids.shape[1], _c(n_rows, np.int32),
                                          ids, self.K, self.V, self.slot_pos, out)
        if rc != 0:
            raise ValueError("prompt does not fit the ring")
        return out

    def prefill_all(self, b: int, ids: np.ndarray) -> np.ndarray:
        """Single voice b, every row's hidden state [S][768]."""
        ids = _c(ids, np.int32)
        S = ids.shape[0]
        out = np.zeros((S, D), np.float32)
        K, V, sp = self.K[b], self.V[b], self.slot_pos[b]
        rc = self.m._lib.or_model_prefill(self.m.ptr, self.C, int(self.wrap), int(self.kv_bf16), S, ids, K,
                                    V, sp, out)
        if rc != 0:
            raise ValueError("prompt does not fit the ring")
        return out

    def decode_step(self, rows17: np.ndarray, pos) -> np.ndarray:
        out = np.zeros((self.B, D), np.float32)
        rc = self.m._lib.or_model_decode_step_batch(self.m.ptr, self.B, self.C, int(self.wrap),
                                              int(self.kv_bf16), _c(rows17, np.int32),
                                              _c(pos, np.int32), self.K, self.V, self.slot_pos, out)
        if rc != 0:
            raise ValueError("decode position exceeds the KV ring")
        return out

    def select(self, voices) -> "ModelState":
        """A new state holding copies of the given voices' rings and
        repetition history, in that order."""
        idx = list(voices)
        out = ModelState(self.m, len(idx), self.C, kv_bf16=self.kv_bf16, wrap=self.wrap)
        out.K[:] = self.K[idx]
        out.V[:] = self.V[idx]
        out.slot_pos[:] = self.slot_pos[idx]
        out.seen[:] = self.seen[idx]
        return out

    def local_frame(self, hidden: np.ndarray):
        """-> codes [B][16], cont [B], margins [B][17]."""
        codes = np.zeros((self.B, NVQ), np.int32)
        cont = np.zeros(self.B, np.int32)
        margins = np.zeros((self.B, 17), np.float64)
        self.m._lib.or_local_frame_batch(self.m.ptr, self.B, _c(hidden, np.float32), self.seen, codes,
                                   cont, margins.ctypes.data)
        return codes, cont.astype(bool), margins


# ------------------------------------------------------------------ the codec
class _CodecLayer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in
                ("qkv", "o", "f1", "f2", "ln1_w", "ln1_b", "ln2_w", "ln2_b", "s1", "s2")]


class _Codec(C.Structure):
    _fields_ = [("rvq_w", C.c_void_p * 16), ("rvq_b", C.c_void_p * 16),
                ("rvq_book", C.c_void_p * 16), ("rvq_out", C.c_void_p), ("rvq_out_b", C.c_void_p),
                ("layers", C.c_int * 4), ("context", C.c_int * 4), ("in_proj", C.c_void_p * 4),
                ("out_proj", C.c_void_p * 4), ("layer", C.POINTER(_CodecLayer)),
                ("kv_bf16", C.c_int)]


def erf_as(x: float) -> float:
    """erf by Abramowitz & Stegun 7.1.26 (the reference's GELU_ERF form)."""
    return lib().or_erf_as(float(x))


def gelu_erf(x: float) -> float:
    return lib().or_gelu_erf(float(x))


class CodecOracle:
    """The codec decoder (codec_oracle.c) for B voices with their own rings:
    the reference's per-position order, rings of exactly `context` slots."""

    def __init__(self, weights: dict, B: int, layers=(4, 2, 2, 4),
                 context=(500, 1696, 2480, 3248), kv_bf16: bool = False):
        self.B, self.layers, self.context = B, tuple(layers), tuple(context)
        self._keep = {k: _c(v, np.float32) for k, v in weights.items()}
        w = self._keep
        st = _Codec()
        for k in range(16):
            p = f"model.quantizer.quantizers.{k}."
            st.rvq_w[k] = w[p + "out_proj.weight"].ctypes.data
            st.rvq_b[k] = w[p + "out_proj.bias"].ctypes.data
            st.rvq_book[k] = w[p + "codebook.weight"].ctypes.data
        st.rvq_out = w["model.quantizer.output_proj.weight"].ctypes.data
        st.rvq_out_b = w["model.quantizer.output_proj.bias"].ctypes.data
        layer_structs = []
        for s in range(4):
            p = f"model.decoder.{(1, 3, 5, 7)[s]}."
            st.layers[s] = self.layers[s]
            st.context[s] = self.context[s]
            st.in_proj[s] = w[p + "input_proj.weight"].ctypes.data
            st.out_proj[s] = w[p + "output_proj.weight"].ctypes.data
            for i in range(self.layers[s]):
                q = p + f"transformer.layers.{i}."
                layer_structs.append(_CodecLayer(
                    w[q + "self_attn.in_proj.weight"].ctypes.data,
                    w[q + "self_attn.out_proj.weight"].ctypes.data,
                    w[q + "ffn.0.weight"].ctypes.data, w[q + "ffn.2.weight"].ctypes.data,
                    w[q + "norm1.weight"].ctypes.data, w[q + "norm1.bias"].ctypes.data,
                    w[q + "norm2.weight"].ctypes.data, w[q + "norm2.bias"].ctypes.data,
                    w[q + "layer_scale_1.scale"].ctypes.data,
                    w[q + "layer_scale_2.scale"].ctypes.data))
        self._layers = (_CodecLayer * len(layer_structs))(*layer_structs)
        st.layer = C.cast(self._layers, C.POINTER(_CodecLayer))
        st.kv_bf16 = int(kv_bf16)
        self._st = st
        self.slots = int(lib().or_codec_slots(C.byref(st)))
        self.K = np.zeros((B, self.slots, 256), np.float32)
        self.V = np.zeros((B, self.slots, 256), np.float32)
        self.slot_pos = np.full((B, self.slots), -1, np.int32)
        self.pos = np.zeros((B, 4), np.int32)

    def reset(self, voices=None):
        for b in (range(self.B) if voices is None else voices):
            self.slot_pos[b] = -1
            self.pos[b] = 0

    def rvq(self, codes) -> np.ndarray:
        """One frame's RVQ front for one voice: codes[16] -> [4][192]."""
        out = np.zeros((4, 192), np.float32)
        lib().or_codec_rvq(C.byref(self._st), _c(codes, np.int32), out)
        return out

    def decode(self, codes: np.ndarray) -> np.ndarray:
        """codes [n][B][16] -> pcm [B][2][n * 3840], continuing every voice."""
        codes = _c(codes, np.int32)
        n = codes.shape[0]
        pcm = np.zeros((self.B, 2, n * 3840), np.float32)
        rc = lib().or_codec_decode_batch(C.byref(self._st), self.B, self.K, self.V, self.slot_pos,
                                         self.pos, n, codes, pcm)
        if rc != 0:
            raise MemoryError("codec oracle allocation failed")
        return pcm

    def layer_ring(self, layer: int, voice: int):
        """(K [context][256], V, slot_pos [context]) of one layer's ring."""
        start, s_of = 0, []
        for s in range(4):
            for _ in range(self.layers[s]):
                s_of.append((start, self.context[s]))
                start += self.context[s]
        a, c = s_of[layer]
        return (self.K[voice, a:a + c], self.V[voice, a:a + c], self.slot_pos[voice, a:a + c])
