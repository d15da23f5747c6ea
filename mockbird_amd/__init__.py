"""mockbird_amd -- MI355X (gfx950) decoder hot path for MOSS-TTS-Nano.

The product is the C-ABI library ``libmockbird_hip.so`` (include/mockbird_hip.h)
built from ``csrc/``.  This module is the Python view of that ABI used by the
tests and the benchmark: it loads the in-tree library with ctypes and fails
loudly when it is missing -- there is no CPU fallback.  The JavaScript host
(``engine/``) binds the same ABI through the N-API addon.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
# MB_HIP_LIB names another build of the same library (the host-sanitized one
# of mockbird_amd.build.build_sanitized); there is no other implementation
LIB_PATH = os.environ.get("MB_HIP_LIB") or os.path.join(PKG, "libmockbird_hip.so")

MB_OK, MB_ERR_ARG, MB_ERR_RANGE, MB_ERR_HIP, MB_ERR_STATE, MB_ERR_CANCELLED, MB_ERR_NOMEM = range(7)
MB_KV_F32, MB_KV_BF16 = 0, 1
MB_DT_F32, MB_DT_BF16 = 0, 1
MB_W_F32, MB_W_BF16 = 0, 1
MB_PENALTY_F64, MB_PENALTY_F32 = 0, 1
MB_EPI_STORE, MB_EPI_GELU, MB_EPI_ADD, MB_EPI_SCALE_ADD, MB_EPI_GELU_ERF = 0, 1, 2, 3, 4
#: the codec decoder's shape (codec.ts:1-30)
CODEC_LAYERS, CODEC_CONTEXT, CODEC_SAMPLES = (4, 2, 2, 4), (500, 1696, 2480, 3248), 3840
D, H, HD, QKV, FFN, NVQ, ROW, PAD, CODES = 768, 12, 64, 2304, 3072, 16, 17, 1024, 1024

#: every symbol include/mockbird_hip.h declares (checked by the CPU tests)
EXPORTS = (
    "mb_abi_version", "mb_create", "mb_destroy", "mb_last_error", "mb_set_stream",
    "mb_get_stream", "mb_synchronize", "mb_device_bytes", "mb_upload_tensor", "mb_cancel",
    "mb_ring_reset", "mb_ring_poison", "mb_read_ring", "mb_write_ring", "mb_ring_append", "mb_ring_write_rows",
    "mb_decode_attention", "mb_prefill_attention", "mb_ring_append_dev",
    "mb_ring_write_rows_dev", "mb_decode_attention_dev", "mb_prefill_attention_dev",
    "mb_set_local_head", "mb_set_penalty_precision", "mb_set_weight_storage", "mb_prefill", "mb_prefill_rows", "mb_decode_step", "mb_local_frame",
    "mb_local_steps", "mb_local_logits", "mb_clear_seen", "mb_decode_step_dev", "mb_local_frame_dev",
    "mb_linear_dev", "mb_split_weights_dev", "mb_linear_split_dev", "mb_linear_noalloc_dev", "mb_decode_frames_dev", "mb_decode_frames", "mb_append_attend",
    "mb_append_attend_dev", "mb_codec_init", "mb_codec_reset", "mb_codec_decode",
    "mb_codec_decode_dev", "mb_codec_read_ring",
)


class MbError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[mb error {code}] {msg}")
        self.code = code


class Config(C.Structure):
    _fields_ = [
        ("n_layers", C.c_int32), ("vocab", C.c_int32), ("capacity", C.c_int32),
        ("max_seqs", C.c_int32), ("max_rows", C.c_int32), ("kv_dtype", C.c_int32),
        ("wrap", C.c_int32), ("device", C.c_int32),
    ]


class CodecConfig(C.Structure):
    _fields_ = [("max_voices", C.c_int32), ("kv_dtype", C.c_int32),
                ("layers", C.c_int32 * 4), ("context", C.c_int32 * 4)]


_lib = None
_vp, _i32, _i64, _f32 = C.c_void_p, C.c_int32, C.c_int64, C.c_float


def load():
    """Load libmockbird_hip.so (built by mockbird_amd.build); raise if absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m mockbird_amd.build` "
            "(the HIP library is the only implementation; there is no fallback)")
    # One HIP runtime per process: when PyTorch is present it carries its own
    # libamdhip64.so.7, and a second copy loaded from /opt/rocm would own the
    # device first and leave torch with "no ROCm-capable device".  Importing
    # torch first makes the dynamic loader bind this library to torch's copy
    # (same soname), so device pointers and streams are shared.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    L = C.CDLL(LIB_PATH)
    sig = {
        "mb_abi_version": ([], C.c_int),
        "mb_create": ([C.POINTER(Config), C.POINTER(_vp)], C.c_int),
        "mb_destroy": ([_vp], None),
        "mb_last_error": ([_vp], C.c_char_p),
        "mb_set_stream": ([_vp, _vp], C.c_int),
        "mb_get_stream": ([_vp], _vp),
        "mb_synchronize": ([_vp], C.c_int),
        "mb_device_bytes": ([_vp], _i64),
        "mb_upload_tensor": ([_vp, C.c_char_p, _vp, _vp, C.c_int], C.c_int),
        "mb_cancel": ([_vp, C.c_int], C.c_int),
        "mb_ring_reset": ([_vp, C.c_int, _vp], C.c_int),
        "mb_ring_poison": ([_vp, C.c_int, C.c_int, C.c_int, _f32], C.c_int),
        "mb_read_ring": ([_vp, C.c_int, C.c_int, C.c_int, C.c_int, _vp, _vp, _vp], C.c_int),
        "mb_write_ring": ([_vp, C.c_int, C.c_int, C.c_int, C.c_int, _vp, _vp, _vp], C.c_int),
        "mb_ring_append": ([_vp, C.c_int, C.c_int, _vp, _vp, _vp], C.c_int),
        "mb_ring_write_rows": ([_vp, C.c_int, C.c_int, C.c_int, _vp, _vp, _vp, _vp], C.c_int),
        "mb_decode_attention": ([_vp, C.c_int, C.c_int, _vp, _vp, _vp], C.c_int),
        "mb_prefill_attention": ([_vp, C.c_int, C.c_int, C.c_int, _vp, _vp, _vp, _vp], C.c_int),
        "mb_ring_append_dev": ([_vp, C.c_int, C.c_int, _vp, C.c_int, _i64, _vp, _vp, _i64], C.c_int),
        "mb_ring_write_rows_dev": ([_vp, C.c_int, C.c_int, C.c_int, _vp, C.c_int, _vp, _vp, _vp,
                                    C.c_int], C.c_int),
        "mb_decode_attention_dev": ([_vp, C.c_int, C.c_int, _vp, _i64, _vp, _i32, _vp, _i64],
                                    C.c_int),
        "mb_prefill_attention_dev": ([_vp, C.c_int, C.c_int, C.c_int, _vp, C.c_int, _vp, _vp, _vp],
                                     C.c_int),
        "mb_set_local_head": ([_vp, _i32, _i32, C.c_double], C.c_int),
        "mb_set_weight_storage": ([_vp, _i32], C.c_int),
        "mb_set_penalty_precision": ([_vp, _i32], C.c_int),
        "mb_prefill": ([_vp, C.c_int, C.c_int, _vp, _vp, _vp], C.c_int),
        "mb_prefill_rows": ([_vp, C.c_int, C.c_int, _vp, _vp, C.c_int, _vp], C.c_int),
        "mb_local_steps": ([_vp, C.c_int, _vp, C.c_int, _vp], C.c_int),
        "mb_local_logits": ([_vp, C.c_int, _vp, _vp, _vp, _vp], C.c_int),
        "mb_decode_step": ([_vp, C.c_int, _vp, _vp, _vp], C.c_int),
        "mb_local_frame": ([_vp, C.c_int, _vp, _vp, _vp], C.c_int),
        "mb_clear_seen": ([_vp, C.c_int, _vp], C.c_int),
        "mb_decode_step_dev": ([_vp, C.c_int, _vp, _vp, _i32, _vp], C.c_int),
        "mb_local_frame_dev": ([_vp, C.c_int, _vp, _vp, _vp, _vp], C.c_int),
        "mb_linear_dev": ([_vp, C.c_int, C.c_int, C.c_int, _vp, C.c_int64, _vp, _vp, _vp,
                           C.c_int64, C.c_int], C.c_int),
        "mb_linear_noalloc_dev": ([_vp, C.c_int, C.c_int, C.c_int, _vp, C.c_int64, _vp, _vp, _vp,
                                   C.c_int64, C.c_int], C.c_int),
        "mb_split_weights_dev": ([_vp, _vp, C.c_int, C.c_int, _vp], C.c_int),
        "mb_linear_split_dev": ([_vp, C.c_int, C.c_int, C.c_int, _vp, C.c_int64, _vp, _vp, _vp,
                                 C.c_int64, C.c_int], C.c_int),
        "mb_decode_frames_dev": ([_vp, C.c_int, C.c_int, _vp, _vp, _i32, _vp, _vp], C.c_int),
        "mb_decode_frames": ([_vp, C.c_int, C.c_int, _vp, _vp, _vp, _vp], C.c_int),
        "mb_append_attend": ([_vp, C.c_int, C.c_int, _vp, _vp, _vp, _vp], C.c_int),
        "mb_append_attend_dev": ([_vp, C.c_int, C.c_int, _vp, C.c_int, _i64, _vp, _i32, _vp, _i64,
                                  _vp, _i64], C.c_int),
        "mb_codec_init": ([_vp, C.POINTER(CodecConfig)], C.c_int),
        "mb_codec_reset": ([_vp, C.c_int, _vp], C.c_int),
        "mb_codec_decode": ([_vp, C.c_int, C.c_int, _vp, _vp], C.c_int),
        "mb_codec_decode_dev": ([_vp, C.c_int, C.c_int, _vp, _vp], C.c_int),
        "mb_codec_read_ring": ([_vp, C.c_int, C.c_int, _vp, _vp, _vp, _vp], C.c_int),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _lib = L
    return L


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


def _f32c(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _i32c(a):
    return np.ascontiguousarray(a, dtype=np.int32)


class Context:
    """One mb_ctx: rings for `max_seqs` sequences on one GPU."""

    def __init__(self, n_layers: int = 12, capacity: int = 1024, max_seqs: int = 1,
                 max_rows: int = 512, kv_dtype: int = MB_KV_F32, wrap: bool = True,
                 vocab: int = 32000, device: int = 0):
        self.lib = load()
        self.cfg = Config(n_layers, vocab, capacity, max_seqs, max_rows, kv_dtype, int(wrap), device)
        h = _vp()
        rc = self.lib.mb_create(C.byref(self.cfg), C.byref(h))
        if rc != MB_OK:
            raise MbError(rc, "mb_create failed (see stderr)")
        self.h = h

    # -- plumbing
    def close(self):
        if getattr(self, "h", None):
            self.lib.mb_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def check(self, rc: int):
        if rc != MB_OK:
            raise MbError(rc, self.lib.mb_last_error(self.h).decode())

    @property
    def capacity(self):
        return self.cfg.capacity

    def set_stream(self, stream_handle: int | None):
        self.check(self.lib.mb_set_stream(self.h, stream_handle))

    def synchronize(self):
        self.check(self.lib.mb_synchronize(self.h))

    def device_bytes(self) -> int:
        return self.lib.mb_device_bytes(self.h)

    def upload(self, name: str, arr: np.ndarray):
        a = _f32c(arr)
        dims = (C.c_int64 * a.ndim)(*a.shape)
        self.check(self.lib.mb_upload_tensor(self.h, name.encode(), a.ctypes.data, dims, a.ndim))

    def upload_all(self, weights: dict):
        for k, v in weights.items():
            self.upload(k, v)

    def cancel(self, on: bool = True):
        self.check(self.lib.mb_cancel(self.h, int(on)))

    # -- ring
    def ring_reset(self, seq_ids=None):
        if seq_ids is None:
            self.check(self.lib.mb_ring_reset(self.h, -1, None))
        else:
            s = _i32c(seq_ids)
            self.check(self.lib.mb_ring_reset(self.h, s.size, s.ctypes.data))

    def ring_poison(self, layer: int, seq: int, n_slots: int, sentinel: float = -12345.5):
        self.check(self.lib.mb_ring_poison(self.h, layer, seq, n_slots, sentinel))

    def read_ring(self, layer: int, seq: int, slot0: int = 0, n: int | None = None):
        n = self.capacity - slot0 if n is None else n
        k = np.zeros((n, D), np.float32)
        v = np.zeros((n, D), np.float32)
        sp = np.zeros(n, np.int32)
        self.check(self.lib.mb_read_ring(self.h, layer, seq, slot0, n, k.ctypes.data, v.ctypes.data,
                                         sp.ctypes.data))
        return k, v, sp

    def write_ring(self, layer: int, seq: int, slot0: int = 0, k=None, v=None, slot_pos=None):
        """Store k, v [n][768] and slot_pos [n] (any may be None) into slots
        [slot0, slot0 + n): the inverse of read_ring."""
        parts = [x for x in (k, v, slot_pos) if x is not None]
        if not parts:
            return
        n = len(parts[0])
        k = None if k is None else _f32c(k).reshape(n, D)
        v = None if v is None else _f32c(v).reshape(n, D)
        sp = None if slot_pos is None else _i32c(slot_pos).reshape(n)
        if any(len(x) != n for x in (k, v, sp) if x is not None):
            raise ValueError("k, v and slot_pos cover different numbers of slots")
        self.check(self.lib.mb_write_ring(self.h, layer, seq, slot0, n,
                                          None if k is None else k.ctypes.data,
                                          None if v is None else v.ctypes.data,
                                          None if sp is None else sp.ctypes.data))

    def ring_append(self, layer: int, qkv: np.ndarray, pos) -> np.ndarray:
        qkv, pos = _f32c(qkv), _i32c(pos)
        B = qkv.shape[0]
        q = np.zeros((B, D), np.float32)
        self.check(self.lib.mb_ring_append(self.h, layer, B, qkv.ctypes.data, pos.ctypes.data,
                                           q.ctypes.data))
        return q

    def ring_write_rows(self, layer: int, qkv: np.ndarray, pos0, n_rows) -> np.ndarray:
        qkv, pos0, n_rows = _f32c(qkv), _i32c(pos0), _i32c(n_rows)
        B, R = qkv.shape[0], qkv.shape[1]
        q = np.zeros((B, R, D), np.float32)
        self.check(self.lib.mb_ring_write_rows(self.h, layer, B, R, qkv.ctypes.data,
                                               pos0.ctypes.data, n_rows.ctypes.data, q.ctypes.data))
        return q

    def decode_attention(self, layer: int, q: np.ndarray, pos) -> np.ndarray:
        q, pos = _f32c(q), _i32c(pos)
        out = np.zeros((q.shape[0], D), np.float32)
        self.check(self.lib.mb_decode_attention(self.h, layer, q.shape[0], q.ctypes.data,
                                                pos.ctypes.data, out.ctypes.data))
        return out

    def append_attend(self, layer: int, qkv: np.ndarray, pos, want_q: bool = True):
        """Fused append + decode attention: returns (roped q or None, out)."""
        qkv, pos = _f32c(qkv), _i32c(pos)
        B = qkv.shape[0]
        q = np.zeros((B, D), np.float32) if want_q else None
        out = np.zeros((B, D), np.float32)
        self.check(self.lib.mb_append_attend(self.h, layer, B, qkv.ctypes.data, pos.ctypes.data,
                                             _ptr(q), out.ctypes.data))
        return q, out

    def prefill_attention(self, layer: int, q: np.ndarray, pos0, n_rows) -> np.ndarray:
        q, pos0, n_rows = _f32c(q), _i32c(pos0), _i32c(n_rows)
        B, R = q.shape[0], q.shape[1]
        out = np.zeros((B, R, D), np.float32)
        self.check(self.lib.mb_prefill_attention(self.h, layer, B, R, q.ctypes.data,
                                                 pos0.ctypes.data, n_rows.ctypes.data,
                                                 out.ctypes.data))
        return out

    # -- device-pointer forms (integer device addresses, e.g. torch tensor.data_ptr())
    def ring_append_dev(self, layer, B, qkv_ptr, pos_ptr, q_ptr, qkv_dtype=MB_DT_F32,
                        qkv_stride=QKV, q_stride=D):
        self.check(self.lib.mb_ring_append_dev(self.h, layer, B, qkv_ptr, qkv_dtype, qkv_stride,
                                               pos_ptr, q_ptr, q_stride))

    def ring_write_rows_dev(self, layer, B, rows_max, qkv_ptr, pos0_ptr, n_ptr, q_ptr,
                            qkv_dtype=MB_DT_F32, q_dtype=MB_DT_F32):
        self.check(self.lib.mb_ring_write_rows_dev(self.h, layer, B, rows_max, qkv_ptr, qkv_dtype,
                                                   pos0_ptr, n_ptr, q_ptr, q_dtype))

    def decode_attention_dev(self, layer, B, q_ptr, pos_ptr, max_pos, out_ptr, q_stride=D,
                             out_stride=D):
        self.check(self.lib.mb_decode_attention_dev(self.h, layer, B, q_ptr, q_stride, pos_ptr,
                                                    max_pos, out_ptr, out_stride))

    def append_attend_dev(self, layer, B, qkv_ptr, pos_ptr, max_pos, out_ptr, q_ptr=None,
                          qkv_dtype=MB_DT_F32, qkv_stride=QKV, q_stride=D, out_stride=D):
        self.check(self.lib.mb_append_attend_dev(self.h, layer, B, qkv_ptr, qkv_dtype, qkv_stride,
                                                 pos_ptr, max_pos, q_ptr, q_stride, out_ptr,
                                                 out_stride))

    def prefill_attention_dev(self, layer, B, rows_max, q_ptr, pos0_ptr, n_ptr, out_ptr,
                              q_dtype=MB_DT_F32):
        self.check(self.lib.mb_prefill_attention_dev(self.h, layer, B, rows_max, q_ptr, q_dtype,
                                                     pos0_ptr, n_ptr, out_ptr))

    # -- the codec decoder
    def codec_init(self, max_voices: int, layers=CODEC_LAYERS, context=CODEC_CONTEXT,
                   kv_dtype: int = MB_KV_F32):
        cfg = CodecConfig(max_voices, kv_dtype, (C.c_int32 * 4)(*layers),
                          (C.c_int32 * 4)(*context))
        self.check(self.lib.mb_codec_init(self.h, C.byref(cfg)))
        self.codec_layers, self.codec_context = tuple(layers), tuple(context)

    def codec_reset(self, voices=None):
        if voices is None:
            self.check(self.lib.mb_codec_reset(self.h, -1, None))
        else:
            v = _i32c(voices)
            self.check(self.lib.mb_codec_reset(self.h, v.size, _ptr(v)))

    def codec_decode(self, codes: np.ndarray) -> np.ndarray:
        """codes [n_frames][B][16] -> pcm [B][2][n_frames * 3840]."""
        codes = _i32c(codes)
        n, B = codes.shape[0], codes.shape[1]
        pcm = np.zeros((B, 2, n * CODEC_SAMPLES), np.float32)
        self.check(self.lib.mb_codec_decode(self.h, B, n, _ptr(codes), _ptr(pcm)))
        return pcm

    def codec_decode_dev(self, B, n_frames, codes_ptr, pcm_ptr):
        self.check(self.lib.mb_codec_decode_dev(self.h, B, n_frames, codes_ptr, pcm_ptr))

    def codec_read_ring(self, layer: int, voice: int):
        """(k [slots][256], v [slots][256], slot_pos [slots]) of one codec layer and voice."""
        n = C.c_int32(0)
        self.check(self.lib.mb_codec_read_ring(self.h, layer, voice, None, None, None, C.byref(n)))
        k = np.zeros((n.value, 256), np.float32)
        v = np.zeros((n.value, 256), np.float32)
        sp = np.zeros(n.value, np.int32)
        self.check(self.lib.mb_codec_read_ring(self.h, layer, voice, _ptr(k), _ptr(v), _ptr(sp),
                                               None))
        return k, v, sp

    def decode_frames_dev(self, B, n_frames, hidden_ptr, pos_ptr, max_pos, codes_ptr, cont_ptr):
        self.check(self.lib.mb_decode_frames_dev(self.h, B, n_frames, hidden_ptr, pos_ptr, max_pos,
                                                 codes_ptr, cont_ptr))

    def decode_frames(self, hidden: np.ndarray, pos, n_frames: int):
        """Host form of the frame loop: returns (codes [n][B][16], cont [n][B],
        hidden after the last frame [B][768], positions after it [B])."""
        h, p = _f32c(hidden).copy(), _i32c(pos).copy()
        B = h.shape[0]
        codes = np.zeros((n_frames, B, NVQ), np.int32)
        cont = np.zeros((n_frames, B), np.int32)
        self.check(self.lib.mb_decode_frames(self.h, B, n_frames, h.ctypes.data, p.ctypes.data,
                                             codes.ctypes.data, cont.ctypes.data))
        return codes, cont.astype(bool), h, p

    def linear_dev(self, M, N, K, a_ptr, lda, w_ptr, bias_ptr, c_ptr, ldc, epi=0):
        self.check(self.lib.mb_linear_dev(self.h, M, N, K, a_ptr, lda, w_ptr, bias_ptr, c_ptr, ldc,
                                          epi))

    def split_weights_dev(self, w_ptr, K, N, wx_ptr):
        self.check(self.lib.mb_split_weights_dev(self.h, w_ptr, K, N, wx_ptr))

    def linear_split_dev(self, M, N, K, a_ptr, lda, wx_ptr, bias_ptr, c_ptr, ldc, epi=0):
        self.check(self.lib.mb_linear_split_dev(self.h, M, N, K, a_ptr, lda, wx_ptr, bias_ptr,
                                                c_ptr, ldc, epi))

    def linear_noalloc_dev(self, M, N, K, a_ptr, lda, w_ptr, bias_ptr, c_ptr, ldc, epi=0):
        self.check(self.lib.mb_linear_noalloc_dev(self.h, M, N, K, a_ptr, lda, w_ptr, bias_ptr,
                                                  c_ptr, ldc, epi))

    # -- model
    def set_local_head(self, audio_end_id: int = 7, assistant_id: int = 9, penalty: float = 1.2):
        self.check(self.lib.mb_set_local_head(self.h, audio_end_id, assistant_id, penalty))

    def set_penalty_precision(self, precision: int = MB_PENALTY_F64):
        """MB_PENALTY_F64 (default: the reference CPU path's JS doubles) or
        MB_PENALTY_F32 (the WGSL engine's f32 penalty arithmetic)."""
        self.check(self.lib.mb_set_penalty_precision(self.h, precision))

    def set_weight_storage(self, storage: int = MB_W_F32):
        """MB_W_F32 (default) or MB_W_BF16: the decoder's projection weights
        rounded to bf16 once and read as bf16 (mb_set_weight_storage)."""
        self.check(self.lib.mb_set_weight_storage(self.h, storage))

    def prefill(self, ids: np.ndarray, n_rows) -> np.ndarray:
        """ids [B][rows_max][17] -> last-row hidden [B][768]."""
        ids, n_rows = _i32c(ids), _i32c(n_rows)
        B, R = ids.shape[0], ids.shape[1]
        out = np.zeros((B, D), np.float32)
        self.check(self.lib.mb_prefill(self.h, B, R, ids.ctypes.data, n_rows.ctypes.data,
                                       out.ctypes.data))
        return out

    def prefill_rows(self, ids: np.ndarray, n_rows, layer_count: int = 0) -> np.ndarray:
        """ids [B][rows_max][17] -> hidden of every row [B][rows_max][768]
        after the first `layer_count` layers (0: all) and ln_f."""
        ids, n_rows = _i32c(ids), _i32c(n_rows)
        B, R = ids.shape[0], ids.shape[1]
        out = np.zeros((B, R, D), np.float32)
        self.check(self.lib.mb_prefill_rows(self.h, B, R, ids.ctypes.data, n_rows.ctypes.data,
                                            int(layer_count), out.ctypes.data))
        return out

    def local_steps(self, hidden: np.ndarray, max_step: int) -> np.ndarray:
        """ln_f output of local-head step `max_step` (no greedy choices)."""
        hidden = _f32c(hidden)
        out = np.zeros_like(hidden)
        self.check(self.lib.mb_local_steps(self.h, hidden.shape[0], hidden.ctypes.data, max_step,
                                           out.ctypes.data))
        return out

    def local_logits(self, hidden: np.ndarray, codes: np.ndarray):
        """The frame head teacher-forced with codes [B][16]: returns (text2
        [B][2] float64 = (audio_end, assistant) dot products of step 0,
        logits [B][16][1024] before the repetition penalty)."""
        hidden, codes = _f32c(hidden), _i32c(codes)
        B = hidden.shape[0]
        text2 = np.zeros((B, 2), np.float64)
        logits = np.zeros((B, NVQ, CODES), np.float32)
        self.check(self.lib.mb_local_logits(self.h, B, hidden.ctypes.data, codes.ctypes.data,
                                            text2.ctypes.data, logits.ctypes.data))
        return text2, logits

    def decode_step(self, rows17: np.ndarray, pos) -> np.ndarray:
        rows17, pos = _i32c(rows17), _i32c(pos)
        out = np.zeros((rows17.shape[0], D), np.float32)
        self.check(self.lib.mb_decode_step(self.h, rows17.shape[0], rows17.ctypes.data,
                                           pos.ctypes.data, out.ctypes.data))
        return out

    def local_frame(self, hidden: np.ndarray):
        hidden = _f32c(hidden)
        B = hidden.shape[0]
        codes = np.zeros((B, NVQ), np.int32)
        cont = np.zeros(B, np.int32)
        self.check(self.lib.mb_local_frame(self.h, B, hidden.ctypes.data, codes.ctypes.data,
                                           cont.ctypes.data))
        return codes, cont.astype(bool)

    def clear_seen(self, seq_ids=None):
        if seq_ids is None:
            self.check(self.lib.mb_clear_seen(self.h, -1, None))
        else:
            s = _i32c(seq_ids)
            self.check(self.lib.mb_clear_seen(self.h, s.size, s.ctypes.data))

    def decode_step_dev(self, B, rows_ptr, pos_ptr, max_pos, hidden_ptr):
        self.check(self.lib.mb_decode_step_dev(self.h, B, rows_ptr, pos_ptr, max_pos, hidden_ptr))

    def local_frame_dev(self, B, hidden_ptr, codes_ptr, cont_ptr, rows_out_ptr):
        self.check(self.lib.mb_local_frame_dev(self.h, B, hidden_ptr, codes_ptr, cont_ptr,
                                               rows_out_ptr))
