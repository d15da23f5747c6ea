"""The reference's kernel-conformance cases (tests/gpu/kernels.test.mjs, the
WGSL kernels against CPU restatements) run through this library's C ABI on
the GPU, with the reference's inputs (its xorshift PRNG, seed 0x2f6e2b1,
kernels.test.mjs:22-30) and expected values from independent float64
computations:

- GEMV 768 -> 2304 with bias (kernels.test.mjs GEMV case): mb_linear_dev at
  M = 1, bar 1e-4 (the reference's is 5e-3);
- RoPE of one head at pos = 137: mb_ring_append's roped q and the stored K
  against the complex rotation, bar 1e-5 (the reference's);
- single-query attention over N = 512 ring slots x 12 heads at position 511:
  mb_decode_attention against float64 attention over the stored K / V, bar
  1e-5 on fp32 rings and 1e-4 on bf16 rings (bf16 values, fp32 arithmetic),
  and the bf16 result within 2e-2 of the fp32 one.
"""
import numpy as np
import pytest

import mockbird_amd as mb
from conftest import say
from kernel_cases import ATTN_SLOTS, D, H, HD, ROPE_POS, make_cases, rope_f64
from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def cases():
    return make_cases()


def test_gemv_reference_case(cases):
    torch = pytest.importorskip("torch")
    say("reference GEMV 768 -> 2304, M=1")
    x, W, bias = cases["gemv"]
    K, N = W.shape
    want = x.astype(np.float64) @ W.astype(np.float64) + bias.astype(np.float64)
    dev = torch.device("cuda")
    with mb.Context(n_layers=1, capacity=16, max_seqs=1, max_rows=16) as ctx:
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        tA = torch.from_numpy(x[None].copy()).to(dev)
        tW, tb = torch.from_numpy(W).to(dev), torch.from_numpy(bias).to(dev)
        tC = torch.zeros((1, N), device=dev)
        ctx.linear_dev(1, N, K, tA.data_ptr(), K, tW.data_ptr(), tb.data_ptr(), tC.data_ptr(), N,
                       mb.MB_EPI_STORE)
        torch.cuda.synchronize()
        got = tC.cpu().numpy()[0]
    assert np.abs(got - want).max() < 1e-4


@pytest.mark.parametrize("kv_name,kv", [("f32", mb.MB_KV_F32), ("bf16", mb.MB_KV_BF16)])
def test_rope_reference_case(cases, kv_name, kv):
    say(f"reference RoPE pos={ROPE_POS} kv={kv_name}")
    v = cases["rope"]
    want = rope_f64(v, ROPE_POS, oracle.inv_freq())
    qkv = np.zeros((1, 3 * D), np.float32)
    for h in range(H):  # the same head vector in every q and k head; v = the plain vector
        qkv[0, h * HD:(h + 1) * HD] = v
        qkv[0, D + h * HD:D + (h + 1) * HD] = v
        qkv[0, 2 * D + h * HD:2 * D + (h + 1) * HD] = v
    C = 256
    with mb.Context(n_layers=1, capacity=C, max_seqs=1, max_rows=16, kv_dtype=kv) as ctx:
        q = ctx.ring_append(0, qkv, [ROPE_POS])
        k, vv, sp = ctx.read_ring(0, 0, ROPE_POS % C, 1)
    assert sp[0] == ROPE_POS
    for h in range(H):
        assert np.abs(q[0, h * HD:(h + 1) * HD] - want).max() < 1e-5
    if kv == mb.MB_KV_F32:
        for h in range(H):
            assert np.abs(k[0, h * HD:(h + 1) * HD] - want).max() < 1e-5
        assert np.array_equal(vv[0], qkv[0, 2 * D:])
    else:  # stored K and V are the bf16 roundings of the fp32 values
        kf = np.tile(q[0, :HD], H)
        assert np.array_equal(k[0], oracle.bf16_round(kf))
        assert np.array_equal(vv[0], oracle.bf16_round(qkv[0, 2 * D:]))


def _attend_f64(q, K, V):
    """Single-query softmax attention per head, scale 1/sqrt(64), float64."""
    out = np.empty(D)
    for h in range(H):
        s = slice(h * HD, (h + 1) * HD)
        sc = K[:, s].astype(np.float64) @ q[s].astype(np.float64) * 0.125
        w = np.exp(sc - sc.max())
        out[s] = (w / w.sum()) @ V[:, s].astype(np.float64)
    return out


def test_attention_reference_case(cases):
    say(f"reference attention N={ATTN_SLOTS} x {H} heads, fp32 and bf16 rings")
    q, K, V = cases["attn"]
    n = ATTN_SLOTS
    qkv = np.zeros((1, n, 3 * D), np.float32)
    qkv[0, :, D:2 * D] = K
    qkv[0, :, 2 * D:] = V
    outs = {}
    for kv_name, kv in (("f32", mb.MB_KV_F32), ("bf16", mb.MB_KV_BF16)):
        with mb.Context(n_layers=1, capacity=n, max_seqs=1, max_rows=n, kv_dtype=kv) as ctx:
            ctx.ring_write_rows(0, qkv, [0], [n])
            ks, vs, sp = ctx.read_ring(0, 0)
            got = ctx.decode_attention(0, q[None], [n - 1])[0]
        assert np.array_equal(sp, np.arange(n, dtype=np.int32))
        want = _attend_f64(q, ks, vs)
        bar = 1e-5 if kv == mb.MB_KV_F32 else 1e-4
        assert np.abs(got - want).max() < bar, kv_name
        outs[kv_name] = got
    assert np.abs(outs["bf16"] - outs["f32"]).max() < 2e-2
