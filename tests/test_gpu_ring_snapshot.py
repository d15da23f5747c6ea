"""mb_write_ring (the inverse of mb_read_ring) and the prefill-cache file
through a real context: stores land where read-back finds them (fp32 exact,
bf16 rounded to nearest even as the oracle rounds), positions the ring could
not hold are refused with nothing written, and a voice restored from a
prefill-cache file decodes bit for bit as the voice that wrote it
(tools/onnx-probe/ref-decode.mjs:327-372 is the reference's use: reload a
prefill instead of recomputing it)."""
import numpy as np
import pytest

import mockbird_amd as mb
from mockbird_amd import prefill_cache, synth
from oracle import oracle
from conftest import say

pytestmark = pytest.mark.gpu

D = 768


def _rows(g, n):
    x = g.standard_normal((n, D), np.float32)
    x[0, :4] = [1.00390625, 1.01171875, -3.0e38, 1e-40]  # bf16 ties (to even), a huge and a tiny value
    return x


@pytest.mark.parametrize("kv", [mb.MB_KV_F32, mb.MB_KV_BF16])
def test_write_read_round_trip(kv):
    say(f"mb_write_ring round trip kv={kv}")
    g = np.random.default_rng(11)
    L, C, S = 2, 40, 3
    with mb.Context(n_layers=L, capacity=C, max_seqs=S, max_rows=8, kv_dtype=kv) as ctx:
        ctx.ring_reset()
        k, v = _rows(g, 17), _rows(g, 17)
        slots = np.arange(5, 22)
        sp = np.where(slots % 3 == 0, -1, slots + C * (slots % 4)).astype(np.int32)
        ctx.write_ring(1, 2, 5, k, v, sp)
        rk, rv, rsp = ctx.read_ring(1, 2, 5, 17)
        want = (lambda x: x) if kv == mb.MB_KV_F32 else oracle.bf16_round
        assert np.array_equal(rsp, sp)
        assert np.array_equal(rk, want(k)) and np.array_equal(rv, want(v))
        if kv == mb.MB_KV_BF16:
            assert rk[0, 0] == 1.0 and rk[0, 1] == 1.015625  # ties to even
        # the neighbouring slots, layer and voices are untouched
        assert (ctx.read_ring(1, 2, 0, 5)[2] == -1).all() and (ctx.read_ring(1, 2, 22)[2] == -1).all()
        assert (ctx.read_ring(0, 2)[2] == -1).all() and (ctx.read_ring(1, 1)[2] == -1).all()
        # a NULL part leaves that part as it was
        ctx.write_ring(1, 2, 5, slot_pos=np.full(17, -1, np.int32))
        rk2, rv2, rsp2 = ctx.read_ring(1, 2, 5, 17)
        assert (rsp2 == -1).all() and np.array_equal(rk2, rk) and np.array_equal(rv2, rv)
        v2 = g.standard_normal((3, D), np.float32)
        ctx.write_ring(1, 2, 6, v=v2)
        assert np.array_equal(ctx.read_ring(1, 2, 6, 3)[1], want(v2))
        assert np.array_equal(ctx.read_ring(1, 2, 6, 3)[0], rk[1:4])


def test_write_ring_refuses_positions_the_ring_cannot_hold():
    say("mb_write_ring refusals")
    g = np.random.default_rng(12)
    for wrap in (True, False):
        with mb.Context(n_layers=1, capacity=16, max_seqs=1, max_rows=8, wrap=wrap) as ctx:
            ctx.ring_reset()
            k = g.standard_normal((4, D), np.float32)
            for bad in ([3, 4, 5, 7], [3, 4, -2, 6], [3, 4, 5, 5]):
                with pytest.raises(mb.MbError):
                    ctx.write_ring(0, 0, 3, k, k, np.array(bad, np.int32))
                assert (ctx.read_ring(0, 0)[2] == -1).all()  # nothing written
            if not wrap:  # pos mod C is not enough on a non-wrapping ring
                with pytest.raises(mb.MbError):
                    ctx.write_ring(0, 0, 3, k, k, np.array([3, 4, 5, 22], np.int32))
            else:
                ctx.write_ring(0, 0, 3, k, k, np.array([3, 20, 5, 38], np.int32))
                assert list(ctx.read_ring(0, 0, 3, 4)[2]) == [3, 20, 5, 38]
            for slot0, n in ((-1, 2), (15, 2), (0, 17)):
                with pytest.raises(mb.MbError):
                    ctx.write_ring(0, 0, slot0, np.zeros((n, D), np.float32))
            with pytest.raises(mb.MbError):
                ctx.write_ring(1, 0, 0, k)  # layer out of range
            with pytest.raises(mb.MbError):
                ctx.write_ring(0, 1, 0, k)  # voice out of range


@pytest.mark.parametrize("kv", [mb.MB_KV_F32, mb.MB_KV_BF16])
def test_prefill_cache_restore_decodes_identically(kv, tmp_path):
    """Voice A prefills and its rings and hidden rows go to a prefill-cache
    file; a fresh context loads the file; both then decode the same 4 frames
    and agree bit for bit, and the restored rings write the same file back."""
    say(f"prefill cache restore kv={kv}")
    L, V, C = 2, 64, 96
    w = synth.model_weights(n_layers=L, vocab=V, seed=9, bias_std=0.02, ln_std=0.1)
    rows = synth.prompt(3, n_frames=9, n_text=6, vocab=V)
    S = rows.shape[0]
    path = str(tmp_path / "ref-prefill.bin")
    with mb.Context(n_layers=L, capacity=C, max_seqs=1, max_rows=64, kv_dtype=kv, vocab=V) as a, \
            mb.Context(n_layers=L, capacity=C, max_seqs=1, max_rows=64, kv_dtype=kv, vocab=V) as b:
        a.upload_all(w)
        b.upload_all(w)
        hid = a.prefill_rows(rows[None], [S])[0]
        assert prefill_cache.save(path, a, 0, hid) == S
        # b holds another utterance first: the load must clear it
        other = synth.prompt(4, n_frames=20, n_text=9, vocab=V)
        b.prefill(other[None], [other.shape[0]])
        hb = prefill_cache.load(path, b, 0)
        assert np.array_equal(hb, hid)
        for layer in range(L):
            ka, va, spa = a.read_ring(layer, 0)
            kb, vb, spb = b.read_ring(layer, 0)
            assert np.array_equal(spa, spb)
            live = spa >= 0
            assert np.array_equal(ka[live], kb[live]) and np.array_equal(va[live], vb[live])
        ha, hb = hid[-1][None], hb[-1][None]
        for f in range(4):
            ca, conta = a.local_frame(ha)
            cb, contb = b.local_frame(hb)
            assert np.array_equal(ca, cb) and np.array_equal(conta, contb), f
            ha = a.decode_step(synth.frame_row(ca[0])[None], [S + f])
            hb = b.decode_step(synth.frame_row(cb[0])[None], [S + f])
            assert np.array_equal(ha, hb), f
        b2 = str(tmp_path / "again.bin")
        b.ring_reset()
        prefill_cache.load(path, b, 0)
        prefill_cache.save(b2, b, 0, hid)
        assert open(b2, "rb").read() == open(path, "rb").read()
