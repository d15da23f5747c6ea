"""GPU parity of the ring append (RoPE on K, slot = pos mod C) and of the
split-softmax decode attention, through the C ABI, against the oracle.

Bars: slot positions, K and V ring contents and the roped q are bit-exact
(fp32 and bf16 storage); attention outputs within 1e-4 of the oracle on the
same stored values, and within 2e-2 of the fp32 oracle when K/V are stored
in bf16.
"""
import numpy as np
import pytest

import mockbird_amd as mb
from mockbird_amd import synth
from oracle import oracle
from conftest import say

pytestmark = pytest.mark.gpu

KV = [("f32", mb.MB_KV_F32), ("bf16", mb.MB_KV_BF16)]


def _oracle_ring(B, C, kv, wrap=True):
    return oracle.Ring(B, C, kv_bf16=(kv == mb.MB_KV_BF16), wrap=wrap)


def _check_ring(ctx, ring, layer, seqs):
    for b in seqs:
        k, v, sp = ctx.read_ring(layer, b)
        assert np.array_equal(sp, ring.slot_pos[b]), f"slot positions differ, seq {b}"
        live = sp >= 0
        assert np.array_equal(k[live], ring.K[b][live]), f"K differs, seq {b}"
        assert np.array_equal(v[live], ring.V[b][live]), f"V differs, seq {b}"


@pytest.mark.parametrize("name,kv", KV)
def test_append_and_attention_small(name, kv):
    say(f"small ring parity kv={name}")
    B, C, L = 5, 64, 2
    rng = np.random.default_rng(11)
    with mb.Context(n_layers=L, capacity=C, max_seqs=B, max_rows=200, kv_dtype=kv) as ctx:
        ring = _oracle_ring(B, C, kv)
        ring32 = _oracle_ring(B, C, mb.MB_KV_F32)
        # prefill-style rows: ragged counts, some starting late enough to wrap inside the call
        n = np.array([1, 17, 64, 50, 64], np.int32)
        pos0 = np.array([0, 3, 0, 40, 100], np.int32)
        qkv = synth.qkv_rows(1, (B, 64))
        q_gpu = ctx.ring_write_rows(1, qkv, pos0, n)
        q_or = ring.write(qkv, pos0, n)
        ring32.write(qkv, pos0, n)
        for b in range(B):
            assert np.array_equal(q_gpu[b, :n[b]], q_or[b, :n[b]])
        _check_ring(ctx, ring, 1, range(B))
        pos = pos0 + n
        for step in range(70):  # appends that wrap every ring at least once
            qkv1 = rng.standard_normal((B, 2304), dtype=np.float32)
            q1 = ctx.ring_append(1, qkv1, pos)
            assert np.array_equal(q1, ring.append(qkv1, pos))
            ring32.append(qkv1, pos)
            out = ctx.decode_attention(1, q1, pos)
            want = ring.attend(q1, pos)
            assert np.abs(out - want).max() < 1e-4, step
            if kv == mb.MB_KV_BF16:
                assert np.abs(out - ring32.attend(q1, pos)).max() < 2e-2
            pos = pos + 1
        _check_ring(ctx, ring, 1, range(B))
        # layer 0 was never written: every slot still empty
        assert (ctx.read_ring(0, 2)[2] == -1).all()


@pytest.mark.parametrize("name,kv", KV)
@pytest.mark.parametrize("C", [1, 2, 3])
def test_tiny_rings(name, kv, C):
    """Rings of 1-3 slots, where every append past the first C evicts: the
    fused launch and the two-launch form against the oracle, ring contents
    bit-exact.  With one slot the window is the new row alone, so the output
    is that row's stored V exactly (the softmax of one score is 1)."""
    say(f"tiny ring C={C} kv={name}")
    B = 4
    rng = np.random.default_rng(40 + C)
    pos = np.array([0, 1, 7, 70_001], np.int32)
    with mb.Context(n_layers=1, capacity=C, max_seqs=B, max_rows=C, kv_dtype=kv) as fused, \
            mb.Context(n_layers=1, capacity=C, max_seqs=B, max_rows=C, kv_dtype=kv) as twin:
        ring = _oracle_ring(B, C, kv)
        for step in range(2 * C + 3):
            qkv = rng.standard_normal((B, 2304), dtype=np.float32)
            q_f, out_f = fused.append_attend(0, qkv, pos)
            q_t = twin.ring_append(0, qkv, pos)
            out_t = twin.decode_attention(0, q_t, pos)
            q_or = ring.append(qkv, pos)
            assert np.array_equal(q_f, q_or) and np.array_equal(q_t, q_or), step
            assert np.array_equal(out_f, out_t), step
            assert np.abs(out_f - ring.attend(q_or, pos)).max() < 1e-4, step
            if C == 1:
                for b in range(B):
                    assert np.array_equal(out_f[b], ring.V[b][0]), (step, b)
            pos = pos + 1
        _check_ring(fused, ring, 0, range(B))
        _check_ring(twin, ring, 0, range(B))


def test_empty_batches_are_no_ops():
    """B = 0 through every host-pointer ring and attention entry point: no
    error, empty outputs, and the rings stay empty."""
    say("empty batches")
    with mb.Context(n_layers=1, capacity=8, max_seqs=2, max_rows=8) as ctx:
        none = np.zeros(0, np.int32)
        assert ctx.ring_append(0, np.zeros((0, 2304), np.float32), none).shape == (0, 768)
        q, out = ctx.append_attend(0, np.zeros((0, 2304), np.float32), none)
        assert q.shape == (0, 768) and out.shape == (0, 768)
        assert ctx.decode_attention(0, np.zeros((0, 768), np.float32), none).shape == (0, 768)
        rows = ctx.ring_write_rows(0, np.zeros((0, 4, 2304), np.float32), none, none)
        assert rows.shape == (0, 4, 768)
        out = ctx.prefill_attention(0, np.zeros((0, 4, 768), np.float32), none, none)
        assert out.shape == (0, 4, 768)
        for b in range(2):
            assert (ctx.read_ring(0, b)[2] == -1).all()


def test_rope_positions_beyond_the_table():
    """Positions below 65536 take cos/sin from the context's table, later ones
    are evaluated in-kernel; both must reproduce the oracle bit for bit."""
    say("rope table boundary")
    pos = np.array([0, 1, 65534, 65535, 65536, 65537, 1_000_003, 2**24 + 1], np.int32)
    B = pos.size
    with mb.Context(n_layers=1, capacity=7, max_seqs=B, max_rows=1) as ctx:
        ring = oracle.Ring(B, 7)
        qkv = synth.qkv_rows(3, (B,))
        q = ctx.ring_append(0, qkv, pos)
        assert np.array_equal(q, ring.append(qkv, pos))
        _check_ring(ctx, ring, 0, range(B))


def test_non_wrapping_ring_reports_range_error():
    say("non-wrapping ring overflow")
    with mb.Context(n_layers=1, capacity=8, max_seqs=1, max_rows=8, wrap=False) as ctx:
        qkv = np.zeros((1, 2304), np.float32)
        ctx.ring_append(0, qkv, [7])
        with pytest.raises(mb.MbError) as e:
            ctx.ring_append(0, qkv, [8])
        assert e.value.code == mb.MB_ERR_RANGE and "exceeds the KV ring" in str(e.value)
        # more rows than slots in one call is refused before any launch
        with pytest.raises(mb.MbError) as e:
            ctx.ring_write_rows(0, np.zeros((1, 9, 2304), np.float32), [0], [9])
        assert e.value.code == mb.MB_ERR_ARG


def test_poison_reset_and_empty_attention():
    say("poison / reset")
    with mb.Context(n_layers=1, capacity=16, max_seqs=2, max_rows=16) as ctx:
        ctx.ring_poison(0, 1, 3, -12345.5)
        k, v, sp = ctx.read_ring(0, 1, 0, 4)
        assert (k[:3] == -12345.5).all() and (v[:3] == -12345.5).all() and (k[3] == 0).all()
        assert (sp == -1).all()  # poison does not make a slot live
        rng = np.random.default_rng(5)
        for p in range(20):
            q = ctx.ring_append(0, rng.standard_normal((2, 2304), dtype=np.float32), [p, p])
        ctx.ring_reset([1])
        assert (ctx.read_ring(0, 1)[2] == -1).all()
        assert (ctx.read_ring(0, 0)[2] >= 0).all()
        qkv = rng.standard_normal((2, 2304), dtype=np.float32)
        q = ctx.ring_append(0, qkv, [0, 20])
        out = ctx.decode_attention(0, q, [0, 20])
        # sequence 1 sees only the row it just appended: its V, exactly weighted 1
        assert np.abs(out[1] - qkv[1, 1536:]).max() < 1e-6
        # a query with nothing live returns zeros
        ctx.ring_reset([1])
        assert np.abs(ctx.decode_attention(0, q, [0, 20])[1]).max() == 0.0


@pytest.mark.parametrize("name,kv", KV)
def test_c1_full_size(name, kv):
    """B=64 sequences, C=2048, positions U[1, 6144) (about two thirds wrapped),
    rings filled through the row writer on the device, one append + attention
    step; every sequence checked against the oracle slot for slot and by the
    closed-form window."""
    torch = pytest.importorskip("torch")
    say(f"C1 full size kv={name}")
    B, C = 64, 2048
    g = np.random.default_rng(20260101)
    pos = g.integers(1, 6144, size=B).astype(np.int32)
    start = np.maximum(0, pos - (C - 1)).astype(np.int32)
    nfill = (pos - start).astype(np.int32)
    sample = range(B)
    dev = torch.device("cuda")
    tg = torch.Generator(device=dev)
    tg.manual_seed(7)
    host_rows = {b: [] for b in sample}
    with mb.Context(n_layers=1, capacity=C, max_seqs=B, max_rows=256, kv_dtype=kv) as ctx:
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        chunk = 256
        for c0 in range(0, int(nfill.max()), chunk):
            qkv = torch.randn((B, chunk, 2304), generator=tg, device=dev, dtype=torch.float32)
            n = torch.from_numpy(np.clip(nfill - c0, 0, chunk).astype(np.int32)).to(dev)
            p0 = torch.from_numpy((start + c0).astype(np.int32)).to(dev)
            ctx.ring_write_rows_dev(0, B, chunk, qkv.data_ptr(), p0.data_ptr(), n.data_ptr(), 0)
            host = qkv.cpu().numpy()
            for b in sample:
                host_rows[b].append(host[b, :max(0, min(chunk, nfill[b] - c0))])
        step = torch.randn((B, 2304), generator=tg, device=dev, dtype=torch.float32)
        q = torch.empty((B, 768), device=dev)
        out = torch.empty((B, 768), device=dev)
        pos_d = torch.from_numpy(pos).to(dev)
        ctx.ring_append_dev(0, B, step.data_ptr(), pos_d.data_ptr(), q.data_ptr())
        ctx.decode_attention_dev(0, B, q.data_ptr(), pos_d.data_ptr(), int(pos.max()), out.data_ptr())
        torch.cuda.synchronize()
        q_h, out_h, step_h = q.cpu().numpy(), out.cpu().numpy(), step.cpu().numpy()
        assert np.isfinite(out_h).all()
        for b in range(B):  # closed-form window for every sequence
            sp = ctx.read_ring(0, b)[2]
            lo = max(0, pos[b] - C + 1)
            want = np.full(C, -1, np.int32)
            for p in range(lo, pos[b] + 1):
                want[p % C] = p
            assert np.array_equal(sp, want), b
        for b in sample:
            ring = _oracle_ring(1, C, kv)
            rows = np.concatenate(host_rows[b] + [step_h[b][None]])[None]
            qo = ring.write(rows, [start[b]], [nfill[b] + 1])[0, -1]
            assert np.array_equal(qo, q_h[b])
            k, v, sp = ctx.read_ring(0, b)
            assert np.array_equal(sp, ring.slot_pos[0])
            assert np.array_equal(k, ring.K[0]) and np.array_equal(v, ring.V[0])
            want = ring.attend(q_h[b][None], [pos[b]])[0]
            assert np.abs(out_h[b] - want).max() < 1e-4, b


def test_c4_eviction_stress():
    """B=32, C=4096, positions 0..5000 (every ring wraps and evicts); at
    4095, 4096, 4097 and 5000: slot positions of every sequence exact, two
    sequences' rings bit-exact and attention within 1e-4 of the oracle."""
    say("C4 eviction stress")
    B, C = 32, 4096
    watch = [0, 17]
    rings = {b: _oracle_ring(1, C, mb.MB_KV_F32) for b in watch}
    checks = (4095, 4096, 4097, 5000)
    with mb.Context(n_layers=1, capacity=C, max_seqs=B, max_rows=1) as ctx:
        for p in range(5001):
            qkv = np.random.default_rng([44, p]).standard_normal((B, 2304), dtype=np.float32)
            posv = np.full(B, p, np.int32)
            q = ctx.ring_append(0, qkv, posv)
            for b in watch:
                assert np.array_equal(q[b], rings[b].append(qkv[b][None], [p])[0])
            if p in checks:
                say(f"  checkpoint {p}")
                out = ctx.decode_attention(0, q, posv)
                lo = max(0, p - C + 1)
                want_sp = np.full(C, -1, np.int32)
                for pp in range(lo, p + 1):
                    want_sp[pp % C] = pp
                for b in range(B):
                    assert np.array_equal(ctx.read_ring(0, b)[2], want_sp), (p, b)
                for b in watch:
                    k, v, sp = ctx.read_ring(0, b)
                    assert np.array_equal(k, rings[b].K[0]) and np.array_equal(v, rings[b].V[0])
                    want = rings[b].attend(q[b][None], [p])[0]
                    assert np.abs(out[b] - want).max() < 1e-4, (p, b)


def test_c4_bf16_wrapped_full_size():
    """B=32, C=4096, bf16 KV, as the wrapped decode workload runs it: rows
    written through the row writer and fused append + attention steps at the
    checkpoints 4095 (the ring just full, nothing evicted), 4096 (slot 0 now
    holds 4096, position 0 evicted), 4097 and 5000 (window 905..5000; rows
    4098..4999 written by the row writer in between).  At every checkpoint
    every sequence's slot positions follow the closed-form window, and 8
    sequences' rings are bit-exact and their attention within 1e-4 of the
    oracle's on the same stored values."""
    torch = pytest.importorskip("torch")
    say("C4 bf16 wrapped full size")
    B, C, P = 32, 4096, 5000
    steps = (4095, 4096, 4097, P)
    watch = [0, 5, 11, 16, 21, 26, 30, 31]
    dev = torch.device("cuda")
    chunk = 256
    rings = {b: _oracle_ring(1, C, mb.MB_KV_BF16) for b in watch}
    with mb.Context(n_layers=1, capacity=C, max_seqs=B, max_rows=chunk, kv_dtype=mb.MB_KV_BF16) as ctx:
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)

        def write_rows(lo, hi):
            for c0 in range(lo, hi, chunk):
                nrow = min(chunk, hi - c0)
                rows = np.random.default_rng([45, c0]).standard_normal((B, chunk, 2304),
                                                                        dtype=np.float32)
                qkv = torch.from_numpy(rows).to(dev)
                n = torch.full((B,), nrow, dtype=torch.int32, device=dev)
                p0 = torch.full((B,), c0, dtype=torch.int32, device=dev)
                ctx.ring_write_rows_dev(0, B, chunk, qkv.data_ptr(), p0.data_ptr(), n.data_ptr(), 0)
                for b in watch:
                    rings[b].write(rows[b:b + 1, :nrow], [c0], [nrow])

        written = 0
        for p in steps:
            write_rows(written, p)
            say(f"  checkpoint {p}")
            step = np.random.default_rng([46, p]).standard_normal((B, 2304), dtype=np.float32)
            step_d = torch.from_numpy(step).to(dev)
            pos_d = torch.full((B,), p, dtype=torch.int32, device=dev)
            out = torch.empty((B, 768), device=dev)
            ctx.append_attend_dev(0, B, step_d.data_ptr(), pos_d.data_ptr(), p, out.data_ptr())
            torch.cuda.synchronize()
            written = p + 1
            out_h = out.cpu().numpy()
            assert np.isfinite(out_h).all()
            want_sp = np.full(C, -1, np.int32)
            for pp in range(max(0, p - C + 1), p + 1):
                want_sp[pp % C] = pp
            for b in range(B):
                assert np.array_equal(ctx.read_ring(0, b)[2], want_sp), (p, b)
            for b in watch:
                qo = rings[b].append(step[b][None], [p])[0]
                k, v, sp = ctx.read_ring(0, b)
                assert np.array_equal(sp, rings[b].slot_pos[0])
                assert np.array_equal(k, rings[b].K[0]) and np.array_equal(v, rings[b].V[0]), (p, b)
                want = rings[b].attend(qo[None], [p])[0]
                assert np.abs(out_h[b] - want).max() < 1e-4, (p, b)


@pytest.mark.parametrize("name,kv", KV)
def test_append_attend_equals_append_then_attention(name, kv):
    """The fused append + attention launch against the two calls in sequence
    on a twin context (bit-exact: same stored rows, same fold order) and
    against the oracle; rings that wrap, a ring holding only the new row, and
    positions beyond the RoPE table."""
    say(f"fused append+attention kv={name}")
    B, C = 6, 96
    rng = np.random.default_rng(21)
    pos = np.array([0, 5, 95, 96, 300, 70_000], np.int32)
    with mb.Context(n_layers=2, capacity=C, max_seqs=B, max_rows=C, kv_dtype=kv) as fused, \
            mb.Context(n_layers=2, capacity=C, max_seqs=B, max_rows=C, kv_dtype=kv) as twin:
        ring = _oracle_ring(B, C, kv)
        start = np.maximum(0, pos - C + 1).astype(np.int32)
        n = (pos - start).astype(np.int32)
        fill = rng.standard_normal((B, C, 2304), dtype=np.float32)
        for ctx in (fused, twin):
            ctx.ring_write_rows(1, fill, start, n)
        ring.write(fill, start, n)
        for step in range(5):
            qkv = rng.standard_normal((B, 2304), dtype=np.float32)
            q_f, out_f = fused.append_attend(1, qkv, pos)
            q_t = twin.ring_append(1, qkv, pos)
            out_t = twin.decode_attention(1, q_t, pos)
            assert np.array_equal(q_f, q_t), step
            assert np.array_equal(out_f, out_t), step
            q_or = ring.append(qkv, pos)
            assert np.array_equal(q_f, q_or), step
            assert np.abs(out_f - ring.attend(q_or, pos)).max() < 1e-4, step
            pos = pos + 1
        _check_ring(fused, ring, 1, range(B))
        # without q_out the output is the same
        qkv = rng.standard_normal((B, 2304), dtype=np.float32)
        _, out_a = fused.append_attend(0, qkv, pos, want_q=False)
        q_t = twin.ring_append(0, qkv, pos)
        assert np.array_equal(out_a, twin.decode_attention(0, q_t, pos))


@pytest.mark.parametrize("name,kv", KV)
def test_few_units_long_windows(name, kv):
    """Launches of few (query, head) units take more waves per block (enough
    to read the window in one batch each, up to the cap): 2 sequences (24
    units) with windows of 700 to 2048 slots, one of them wrapped, through
    the fused append + attention and the two-launch path, against the oracle
    at every step and bit-exact between the two paths."""
    say(f"long windows (few units) kv={name}")
    B, C = 2, 2048
    rng = np.random.default_rng(33)
    pos = np.array([700, 2300], np.int32)
    with mb.Context(n_layers=1, capacity=C, max_seqs=B, max_rows=128, kv_dtype=kv) as fused, \
            mb.Context(n_layers=1, capacity=C, max_seqs=B, max_rows=128, kv_dtype=kv) as twin:
        ring = _oracle_ring(B, C, kv)
        start = np.maximum(0, pos - C + 1).astype(np.int32)
        n = (pos - start).astype(np.int32)
        for c0 in range(0, int(n.max()), 128):
            fill = rng.standard_normal((B, 128, 2304), dtype=np.float32)
            nn = np.clip(n - c0, 0, 128).astype(np.int32)
            for ctx in (fused, twin):
                ctx.ring_write_rows(0, fill, (start + c0).astype(np.int32), nn)
            ring.write(fill, (start + c0).astype(np.int32), nn)
        for step in range(4):
            qkv = rng.standard_normal((B, 2304), dtype=np.float32)
            q_f, out_f = fused.append_attend(0, qkv, pos)
            q_t = twin.ring_append(0, qkv, pos)
            out_t = twin.decode_attention(0, q_t, pos)
            assert np.array_equal(q_f, q_t), step
            assert np.array_equal(out_f, out_t), step
            q_or = ring.append(qkv, pos)
            err = np.abs(out_f - ring.attend(q_or, pos)).max()
            assert err < 1e-4, (step, err)
            pos = pos + 1
        _check_ring(fused, ring, 0, range(B))


def test_append_attend_range_error_on_a_non_wrapping_ring():
    say("fused append+attention range error")
    import torch

    with mb.Context(n_layers=1, capacity=8, max_seqs=2, max_rows=8, wrap=False) as ctx:
        qkv = np.zeros((2, 2304), np.float32)
        with pytest.raises(mb.MbError) as e:
            ctx.append_attend(0, qkv, [3, 8])
        assert e.value.code == mb.MB_ERR_RANGE
        d = torch.zeros((2, 2304), device="cuda")
        p = torch.tensor([3, 7], dtype=torch.int32, device="cuda")
        out = torch.empty((2, 768), device="cuda")
        with pytest.raises(mb.MbError) as e:
            ctx.append_attend_dev(0, 2, d.data_ptr(), p.data_ptr(), 8, out.data_ptr())
        assert e.value.code == mb.MB_ERR_RANGE and "exceeds the KV ring" in str(e.value)
        ctx.append_attend_dev(0, 2, d.data_ptr(), p.data_ptr(), 7, out.data_ptr())
        ctx.synchronize()
        assert torch.isfinite(out).all()


@pytest.mark.parametrize("name,kv", KV)
def test_c1_full_size_fused_matches_two_launches(name, kv):
    """B=64, C=2048, positions U[1, 6144): two layers filled with the same
    rows; layer 0 steps with append then attention, layer 1 with the fused
    launch.  Outputs and ring contents must be identical, and the outputs
    agree with the unfused path for three consecutive steps."""
    torch = pytest.importorskip("torch")
    say(f"C1 full size fused kv={name}")
    B, C = 64, 2048
    g = np.random.default_rng(20260101)
    pos = g.integers(1, 6144, size=B).astype(np.int32)
    start = np.maximum(0, pos - (C - 1)).astype(np.int32)
    nfill = (pos - start).astype(np.int32)
    dev = torch.device("cuda")
    tg = torch.Generator(device=dev)
    tg.manual_seed(9)
    with mb.Context(n_layers=2, capacity=C, max_seqs=B, max_rows=256, kv_dtype=kv) as ctx:
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        chunk = 256
        for c0 in range(0, int(nfill.max()), chunk):
            qkv = torch.randn((B, chunk, 2304), generator=tg, device=dev, dtype=torch.float32)
            n = torch.from_numpy(np.clip(nfill - c0, 0, chunk).astype(np.int32)).to(dev)
            p0 = torch.from_numpy((start + c0).astype(np.int32)).to(dev)
            for layer in (0, 1):
                ctx.ring_write_rows_dev(layer, B, chunk, qkv.data_ptr(), p0.data_ptr(), n.data_ptr(), 0)
        q0 = torch.empty((B, 768), device=dev)
        q1 = torch.empty((B, 768), device=dev)
        out0 = torch.empty((B, 768), device=dev)
        out1 = torch.empty((B, 768), device=dev)
        for s in range(3):
            step = torch.randn((B, 2304), generator=tg, device=dev, dtype=torch.float32)
            pos_d = torch.from_numpy(pos + s).to(dev)
            mp = int(pos.max()) + s
            ctx.ring_append_dev(0, B, step.data_ptr(), pos_d.data_ptr(), q0.data_ptr())
            ctx.decode_attention_dev(0, B, q0.data_ptr(), pos_d.data_ptr(), mp, out0.data_ptr())
            ctx.append_attend_dev(1, B, step.data_ptr(), pos_d.data_ptr(), mp, out1.data_ptr(),
                                  q_ptr=q1.data_ptr())
            torch.cuda.synchronize()
            assert torch.equal(q0, q1), s
            assert torch.equal(out0, out1), s
        for b in range(0, B, 7):
            k0, v0, sp0 = ctx.read_ring(0, b)
            k1, v1, sp1 = ctx.read_ring(1, b)
            assert np.array_equal(sp0, sp1) and np.array_equal(k0, k1) and np.array_equal(v0, v1), b
