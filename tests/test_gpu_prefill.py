"""GPU parity of the causal prefill attention (MFMA flash kernels) through the
C ABI, against the oracle.

fp32 queries (the model path, fp32 MFMA) must match the oracle within 1e-4 on
fp32 and on bf16 rings; bf16 queries (the bf16 MFMA path of the isolated
prefill workload) within 2e-2, with the roped bf16 queries and the ring
contents bit-exact.
"""
import numpy as np
import pytest

import mockbird_amd as mb
from mockbird_amd import synth
from oracle import oracle
from conftest import say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kv", [mb.MB_KV_F32, mb.MB_KV_BF16])
def test_prefill_fp32_ragged(kv):
    say(f"prefill fp32 ragged kv={kv}")
    B, R, C = 4, 150, 256
    n = np.array([150, 1, 64, 97], np.int32)
    pos0 = np.zeros(B, np.int32)
    qkv = synth.qkv_rows(21, (B, R))
    with mb.Context(n_layers=1, capacity=C, max_seqs=B, max_rows=R, kv_dtype=kv) as ctx:
        ring = oracle.Ring(B, C, kv_bf16=(kv == mb.MB_KV_BF16))
        q = ctx.ring_write_rows(0, qkv, pos0, n)
        qo = ring.write(qkv, pos0, n)
        for b in range(B):
            assert np.array_equal(q[b, :n[b]], qo[b, :n[b]])
        out = ctx.prefill_attention(0, q, pos0, n)
        want = ring.attend_prefill(qo, pos0, n)
        for b in range(B):
            err = np.abs(out[b, :n[b]] - want[b, :n[b]]).max()
            assert err < 1e-4, (b, err)


def test_prefill_continuation_over_a_wrapped_ring():
    """Rows appended after earlier context, wrapping the ring inside the call:
    each row sees exactly the window (cur - C, cur] of stored positions."""
    say("prefill continuation, wrapped ring")
    B, C = 2, 128
    with mb.Context(n_layers=1, capacity=C, max_seqs=B, max_rows=128) as ctx:
        ring = oracle.Ring(B, C)
        first = synth.qkv_rows(31, (B, 100))
        ctx.ring_write_rows(0, first, [0, 0], [100, 37])
        ring.write(first, [0, 0], [100, 37])
        more = synth.qkv_rows(32, (B, 96))
        pos0 = np.array([100, 37], np.int32)
        n = np.array([96, 96], np.int32)
        q = ctx.ring_write_rows(0, more, pos0, n)
        qo = ring.write(more, pos0, n)
        assert np.array_equal(q, qo)
        out = ctx.prefill_attention(0, q, pos0, n)
        want = ring.attend_prefill(qo, pos0, n)
        assert np.abs(out - want).max() < 1e-4


def test_prefill_rows_are_independent():
    """A sequence cut to its first 300 rows gets bit-identical outputs for
    those rows (the causal-prefix property of the reference captures)."""
    torch = pytest.importorskip("torch")
    say("prefill causal prefix")
    B, R, C = 2, 512, 1024
    dev = torch.device("cuda")
    with mb.Context(n_layers=1, capacity=C, max_seqs=B, max_rows=R) as ctx:
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        one = torch.from_numpy(synth.qkv_rows(41, (1, R))).to(dev)
        qkv = torch.cat([one, one])
        p0 = torch.zeros(B, dtype=torch.int32, device=dev)
        n = torch.tensor([R, 300], dtype=torch.int32, device=dev)
        q = torch.empty((B, R, 768), device=dev)
        out = torch.zeros((B, R, 768), device=dev)
        ctx.ring_write_rows_dev(0, B, R, qkv.data_ptr(), p0.data_ptr(), n.data_ptr(), q.data_ptr())
        ctx.prefill_attention_dev(0, B, R, q.data_ptr(), p0.data_ptr(), n.data_ptr(), out.data_ptr())
        torch.cuda.synchronize()
        o = out.cpu().numpy()
        assert np.array_equal(o[0, :300], o[1, :300])
        assert np.isfinite(o[0]).all()


def test_c2_bf16_prefill_full_size():
    """B=16, S=512 (128 text + 384 code rows), bf16 q/k/v ~ N(0,1), RoPE at
    pos = row, ring C=1024 written from slot 0, bf16 MFMA causal attention;
    all 16 sequences' roped q and rings bit-exact, attention within 2e-2."""
    torch = pytest.importorskip("torch")
    say("C2 bf16 prefill full size")
    B, S, C = 16, 512, 1024
    dev = torch.device("cuda")
    tg = torch.Generator(device=dev)
    tg.manual_seed(2)
    with mb.Context(n_layers=1, capacity=C, max_seqs=B, max_rows=S, kv_dtype=mb.MB_KV_BF16) as ctx:
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        qkv = torch.randn((B, S, 2304), generator=tg, device=dev).to(torch.bfloat16)
        p0 = torch.zeros(B, dtype=torch.int32, device=dev)
        n = torch.full((B,), S, dtype=torch.int32, device=dev)
        q = torch.empty((B, S, 768), dtype=torch.bfloat16, device=dev)
        out = torch.empty((B, S, 768), device=dev)
        ctx.ring_write_rows_dev(0, B, S, qkv.data_ptr(), p0.data_ptr(), n.data_ptr(), q.data_ptr(),
                                qkv_dtype=mb.MB_DT_BF16, q_dtype=mb.MB_DT_BF16)
        ctx.prefill_attention_dev(0, B, S, q.data_ptr(), p0.data_ptr(), n.data_ptr(), out.data_ptr(),
                                  q_dtype=mb.MB_DT_BF16)
        torch.cuda.synchronize()
        out_h = out.cpu().numpy()
        assert np.isfinite(out_h).all()
        for b in range(B):  # every sequence against the oracle
            x = qkv[b:b + 1].float().cpu().numpy()
            ring = oracle.Ring(1, C, kv_bf16=True)
            qo = ring.write(x, [0], [S])
            qo_bf = oracle.bf16_round(qo)
            q_gpu = q[b].float().cpu().numpy()
            assert np.array_equal(q_gpu, qo_bf[0])
            k, v, sp = ctx.read_ring(0, b)
            assert np.array_equal(sp, ring.slot_pos[0])
            assert np.array_equal(k, ring.K[0]) and np.array_equal(v, ring.V[0])
            want = ring.attend_prefill(qo_bf, [0], [S])[0]
            err = np.abs(out_h[b] - want).max()
            assert err < 2e-2, (b, err)


def _bf16_prefill(ctx, torch, x, pos0, n):
    """Rows of bf16 q | k | v through the bf16 ring write and the bf16 MFMA
    attention (device forms); returns (roped q, output) as float32 arrays."""
    dev = torch.device("cuda")
    B, R = x.shape[0], x.shape[1]
    qkv = torch.from_numpy(x).to(dev).to(torch.bfloat16)
    p0 = torch.from_numpy(np.asarray(pos0, np.int32)).to(dev)
    nt = torch.from_numpy(np.asarray(n, np.int32)).to(dev)
    q = torch.zeros((B, R, 768), dtype=torch.bfloat16, device=dev)
    out = torch.zeros((B, R, 768), device=dev)
    ctx.ring_write_rows_dev(0, B, R, qkv.data_ptr(), p0.data_ptr(), nt.data_ptr(), q.data_ptr(),
                            qkv_dtype=mb.MB_DT_BF16, q_dtype=mb.MB_DT_BF16)
    ctx.prefill_attention_dev(0, B, R, q.data_ptr(), p0.data_ptr(), nt.data_ptr(), out.data_ptr(),
                              q_dtype=mb.MB_DT_BF16)
    torch.cuda.synchronize()
    return q.float().cpu().numpy(), out.cpu().numpy()


@pytest.mark.parametrize("C", [256, 1024])
def test_prefill_bf16_ragged_and_wrapped(C):
    """bf16 MFMA attention on ragged row counts (1, 77, 300 rows, several
    128-row query tiles), on a continuation after earlier context, and on
    rings that wrap inside the call: every row sees the window (cur - C, cur]
    of stored positions; q and the ring bit-exact, outputs within 2e-2."""
    torch = pytest.importorskip("torch")
    say(f"bf16 prefill ragged / wrapped C={C}")
    B, R = 4, 300
    first_n = np.array([0, 0, 180, 0], np.int32)
    pos0 = np.array([0, 0, 180, 0], np.int32)
    n = np.array([300, 1, 150, 77], np.int32)
    with mb.Context(n_layers=1, capacity=C, max_seqs=B, max_rows=R, kv_dtype=mb.MB_KV_BF16) as ctx:
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        ring = oracle.Ring(B, C, kv_bf16=True)
        first = synth.qkv_rows(51, (B, 180))
        ctx.ring_write_rows(0, first, np.zeros(B, np.int32), first_n)
        ring.write(first, np.zeros(B, np.int32), first_n)
        x = oracle.bf16_round(synth.qkv_rows(52, (B, R)))
        q_gpu, out = _bf16_prefill(ctx, torch, x, pos0, n)
        qo = oracle.bf16_round(ring.write(x, pos0, n))
        want = ring.attend_prefill(qo, pos0, n)
        for b in range(B):
            assert np.array_equal(q_gpu[b, :n[b]], qo[b, :n[b]]), b
            k, v, sp = ctx.read_ring(0, b)
            assert np.array_equal(sp, ring.slot_pos[b]), b
            assert np.array_equal(k, ring.K[b]) and np.array_equal(v, ring.V[b]), b
            err = np.abs(out[b, :n[b]] - want[b, :n[b]]).max()
            assert err < 2e-2, (b, err)
            assert not out[b, n[b]:].any(), b  # rows past n are not written


def test_prefill_bf16_rows_are_independent():
    """bf16 MFMA path: a sequence cut to its first 300 of 512 rows gets
    bit-identical outputs for those rows (tiles the shorter sequence skips or
    masks contribute nothing)."""
    torch = pytest.importorskip("torch")
    say("bf16 prefill causal prefix")
    B, R, C = 2, 512, 1024
    with mb.Context(n_layers=1, capacity=C, max_seqs=B, max_rows=R, kv_dtype=mb.MB_KV_BF16) as ctx:
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        one = synth.qkv_rows(61, (1, R))
        _, out = _bf16_prefill(ctx, torch, np.concatenate([one, one]), [0, 0], [R, 300])
        assert np.array_equal(out[0, :300], out[1, :300])
        assert np.isfinite(out[0]).all()
