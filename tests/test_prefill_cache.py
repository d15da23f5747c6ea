"""The prefill-cache file (mockbird_amd.prefill_cache) against the reference
oracle's reader, tools/onnx-probe/ref-decode.mjs:327-372: an int32 row count
S, then S hidden rows, then per layer S K rows followed by S V rows, all
768-float little-endian.  The context here is a host stand-in with the ring
calls' semantics (no GPU); the GPU test of the same module drives a real
context (test_gpu_ring_snapshot.py)."""
import struct

import numpy as np
import pytest

from mockbird_amd import prefill_cache as pc

D = 768


class HostRings:
    """read_ring / write_ring / ring_reset over numpy arrays, wrapping ring."""

    class _Cfg:
        pass

    def __init__(self, n_layers, capacity, seqs):
        self.cfg = self._Cfg()
        self.cfg.n_layers = n_layers
        self.capacity = capacity
        self.k = np.full((n_layers, seqs, capacity, D), np.nan, np.float32)
        self.v = np.full((n_layers, seqs, capacity, D), np.nan, np.float32)
        self.sp = np.full((n_layers, seqs, capacity), -1, np.int32)

    def read_ring(self, layer, seq, slot0=0, n=None):
        n = self.capacity - slot0 if n is None else n
        s = slice(slot0, slot0 + n)
        return self.k[layer, seq, s].copy(), self.v[layer, seq, s].copy(), self.sp[layer, seq, s].copy()

    def write_ring(self, layer, seq, slot0=0, k=None, v=None, slot_pos=None):
        n = len(slot_pos)
        s = slice(slot0, slot0 + n)
        assert np.all((slot_pos == -1) | (slot_pos % self.capacity == np.arange(slot0, slot0 + n)))
        self.k[layer, seq, s], self.v[layer, seq, s], self.sp[layer, seq, s] = k, v, slot_pos

    def ring_reset(self, seqs):
        for q in seqs:
            self.sp[:, q] = -1


def reference_reader(buf: bytes, layers: int):
    """The reference reader's walk over the buffer (ref-decode.mjs:331-356):
    offsets advance row by row, hidden rows first, then per layer the K rows
    and then the V rows."""
    S = struct.unpack_from("<i", buf, 0)[0]
    off = 4
    hidden = []
    for _ in range(S):
        hidden.append(np.frombuffer(buf, "<f4", D, off))
        off += D * 4
    kv = []
    for _ in range(layers):
        nk, nv = [], []
        for _ in range(S):
            nk.append(np.frombuffer(buf, "<f4", D, off))
            off += D * 4
        for _ in range(S):
            nv.append(np.frombuffer(buf, "<f4", D, off))
            off += D * 4
        kv.append((np.stack(nk), np.stack(nv)))
    assert off == 4 + S * 4 * D + layers * 2 * S * 4 * D == len(buf)
    return np.stack(hidden), kv


def _filled(L=3, C=20, seqs=2, S=7, seed=1):
    g = np.random.default_rng(seed)
    ctx = HostRings(L, C, seqs)
    for layer in range(L):
        for q in range(seqs):
            ctx.write_ring(layer, q, 0, g.standard_normal((S, D), np.float32),
                           g.standard_normal((S, D), np.float32), np.arange(S, dtype=np.int32))
    return ctx, g


def test_save_matches_reference_reader(tmp_path):
    ctx, g = _filled()
    S = 7
    hidden = g.standard_normal((S, D), np.float32)
    path = tmp_path / "ref-prefill.bin"
    assert pc.save(str(path), ctx, 1, hidden) == S
    buf = path.read_bytes()
    assert len(buf) == pc.file_bytes(S, 3)
    h, kv = reference_reader(buf, 3)
    assert np.array_equal(h, hidden)
    for layer, (k, v) in enumerate(kv):
        assert np.array_equal(k, ctx.k[layer, 1, :S])
        assert np.array_equal(v, ctx.v[layer, 1, :S])
        assert not np.array_equal(k, ctx.k[layer, 0, :S])  # voice 1, not voice 0


def test_load_of_a_reference_written_file(tmp_path):
    """A file laid out as the reference's writer lays it out
    (ref-decode.mjs:362-369: row count, hidden rows, then each layer's K rows
    and V rows) loads into positions 0 .. S-1 and clears the rest."""
    L, S = 2, 5
    g = np.random.default_rng(4)
    hidden = g.standard_normal((S, D), np.float32)
    ks = [g.standard_normal((S, D), np.float32) for _ in range(L)]
    vs = [g.standard_normal((S, D), np.float32) for _ in range(L)]
    parts = [struct.pack("<i", S)] + [r.tobytes() for r in hidden]
    for layer in range(L):
        parts += [r.tobytes() for r in ks[layer]] + [r.tobytes() for r in vs[layer]]
    path = tmp_path / "ref-prefill.bin"
    path.write_bytes(b"".join(parts))
    ctx = HostRings(L, 16, 2)
    ctx.sp[:, 0, 9] = 9  # a stale position from an earlier utterance
    h = pc.load(str(path), ctx, 0)
    assert np.array_equal(h, hidden)
    for layer in range(L):
        k, v, sp = ctx.read_ring(layer, 0)
        assert np.array_equal(sp[:S], np.arange(S)) and (sp[S:] == -1).all()
        assert np.array_equal(k[:S], ks[layer]) and np.array_equal(v[:S], vs[layer])
        assert (ctx.sp[layer, 1] == -1).all()  # the other voice untouched


def test_save_last_row_and_round_trip(tmp_path):
    ctx, g = _filled(S=6)
    last = g.standard_normal(D, np.float32)
    p1 = tmp_path / "a.bin"
    pc.save_last_row(str(p1), ctx, 0, 6, last)
    h, _, _ = pc.read(str(p1), 3)
    assert np.array_equal(h[-1], last) and not h[:-1].any()
    other = HostRings(3, 20, 1)
    pc.load(str(p1), other, 0)
    p2 = tmp_path / "b.bin"
    pc.save(str(p2), other, 0, h)
    assert p1.read_bytes() == p2.read_bytes()


def test_rejects(tmp_path):
    ctx, g = _filled(S=7)
    # slot 3 holds a position other than 3: not expressible in the file
    ctx.sp[1, 0, 3] = 23
    with pytest.raises(ValueError, match="slot 3"):
        pc.save(str(tmp_path / "x.bin"), ctx, 0, np.zeros((7, D), np.float32))
    with pytest.raises(ValueError, match="last row"):
        pc.save(str(tmp_path / "x.bin"), ctx, 1, np.zeros(D, np.float32))
    with pytest.raises(ValueError, match="do not fit"):
        pc.save(str(tmp_path / "x.bin"), ctx, 1, np.zeros((21, D), np.float32))
    good = tmp_path / "g.bin"
    pc.save(str(good), ctx, 1, np.zeros((7, D), np.float32))
    with pytest.raises(ValueError, match="expected"):
        pc.read(str(good), 2)  # written for 3 layers
    (tmp_path / "t.bin").write_bytes(good.read_bytes()[:-4])
    with pytest.raises(ValueError, match="expected"):
        pc.read(str(tmp_path / "t.bin"), 3)
    with pytest.raises(ValueError, match="do not fit"):
        pc.load(str(good), HostRings(3, 6, 1), 0)
