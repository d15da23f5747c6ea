"""GPU parity of the projections (row a7) through mb_linear_dev, against the
oracle's GEMM (double accumulation, fp32 output; pinned by a float64 closed
form in test_oracle_kernels.py).

The shapes cover both kernels the library picks from -- the streaming
split-K kernel for decode-sized M (16/32/64 rows per wave, one split or
many) and the LDS-tiled kernel for prefill-sized M -- at the model's
projection shapes (768 -> 2304, 768 -> 768, 768 -> 3072, 3072 -> 768, the
1024-code audio heads) plus ragged M and a narrow N.  Bar: max-abs 1e-4
(fp32 products and accumulation; outputs are O(1)).
"""
import numpy as np
import pytest

import mockbird_amd as mb
from oracle import oracle
from conftest import say

pytestmark = pytest.mark.gpu

SHAPES = [  # (M, N, K)
    (1, 2304, 768), (1, 768, 768), (1, 3072, 768), (1, 768, 3072), (1, 1024, 768),
    (2, 2304, 768), (3, 64, 768), (4, 768, 3072), (5, 1024, 768), (16, 2304, 768), (17, 768, 3072), (32, 1024, 768), (33, 3072, 768),
    (64, 2304, 768), (100, 768, 3072), (256, 2304, 768), (256, 768, 3072), (256, 1024, 768),
    (1000, 768, 768), (1024, 2304, 768), (1500, 768, 3072), (4096, 3072, 768),
]


@pytest.fixture(scope="module")
def ctx():
    with mb.Context(n_layers=1, capacity=16, max_seqs=1, max_rows=16) as c:
        yield c


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_linear_matches_oracle(ctx, M, N, K):
    torch = pytest.importorskip("torch")
    say(f"linear M={M} N={N} K={K}")
    g = np.random.default_rng([M, N, K])
    A = g.standard_normal((M, K), dtype=np.float32)
    W = (g.standard_normal((K, N), dtype=np.float32) * np.float32(0.02))
    bias = (g.standard_normal(N, dtype=np.float32) * np.float32(0.1))
    C0 = g.standard_normal((M, N), dtype=np.float32)
    dev = torch.device("cuda")
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    tA, tW, tb = (torch.from_numpy(x).to(dev) for x in (A, W, bias))
    want_lin = oracle.gemm(A, W, bias)
    for epi in (mb.MB_EPI_STORE, mb.MB_EPI_GELU, mb.MB_EPI_ADD):
        tC = torch.from_numpy(C0).to(dev)
        ctx.linear_dev(M, N, K, tA.data_ptr(), K, tW.data_ptr(), tb.data_ptr(), tC.data_ptr(), N, epi)
        torch.cuda.synchronize()
        got = tC.cpu().numpy()
        if epi == mb.MB_EPI_STORE:
            want = want_lin
        elif epi == mb.MB_EPI_GELU:
            want = oracle.gelu(want_lin) if M * N <= 300000 else None
        else:
            want = C0 + want_lin
        if want is None:  # large GELU case: compare the pre-activation through STORE above
            continue
        err = float(np.abs(got - want).max())
        assert err < 1e-4, (epi, err)


def test_linear_is_deterministic_and_strided(ctx):
    """Split-K partials are summed in split order by whichever block finishes
    last, so repeated calls are bit-identical; A and C may be row-strided."""
    torch = pytest.importorskip("torch")
    say("linear determinism + strides")
    for M in (1, 5):
        N, K = 768, 3072
        g = np.random.default_rng(9)
        A = g.standard_normal((M, K + 32), dtype=np.float32)
        W = g.standard_normal((K, N), dtype=np.float32) * np.float32(0.02)
        dev = torch.device("cuda")
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        tA, tW = torch.from_numpy(A).to(dev), torch.from_numpy(W).to(dev)
        outs = []
        for _ in range(5):
            tC = torch.zeros((M, N + 64), device=dev)
            ctx.linear_dev(M, N, K, tA.data_ptr(), K + 32, tW.data_ptr(), None, tC.data_ptr(), N + 64)
            torch.cuda.synchronize()
            outs.append(tC.cpu().numpy())
        for o in outs[1:]:
            assert np.array_equal(o, outs[0])
        assert not outs[0][:, N:].any()
        assert np.abs(outs[0][:, :N] - oracle.gemm(A[:, :K], W)).max() < 1e-4


def test_linear_rejects_bad_shapes(ctx):
    with pytest.raises(mb.MbError) as e:
        ctx.linear_dev(4, 100, 768, 16, 768, 16, None, 16, 100)  # N % 64 != 0
    assert e.value.code == mb.MB_ERR_ARG
    with pytest.raises(mb.MbError):
        ctx.linear_dev(4, 64, 768, 16, 700, 16, None, 16, 64)  # lda < K


CODEC_SHAPES = [  # (M, N, K): the codec's projections at 1-256 voices
    (4, 256, 192), (16, 768, 256), (64, 256, 256), (128, 1024, 256), (256, 256, 1024),
    (512, 768, 384), (1024, 256, 1024), (2048, 1024, 256), (8192, 256, 256),
    # streaming kernel at 384 tiles (two rounds); LDS-tiled 64 x 64 tiles at K = 256
    (2048, 768, 256), (4096, 768, 256),
]


@pytest.mark.parametrize("M,N,K", CODEC_SHAPES)
def test_linear_codec_epilogues(ctx, M, N, K):
    """MB_EPI_SCALE_ADD (C + s * A W, the codec's layer scale, LAYER_SCALE_ADD
    kernels-decode.ts:360-371) and MB_EPI_GELU_ERF (the exact GELU after the
    bias, GELU_ERF :392-415) on both GEMM kernels.  Expected: the oracle's
    GEMM, then the epilogue in float64 with scipy's erf (A&S 7.1.26, which
    the kernels use, is within 1.5e-7 of it).  Bar 1e-4 (outputs are O(1))."""
    torch = pytest.importorskip("torch")
    from scipy.special import erf
    say(f"linear codec epilogues M={M} N={N} K={K}")
    g = np.random.default_rng([M, N, K, 7])
    A = g.standard_normal((M, K), dtype=np.float32)
    W = g.standard_normal((K, N), dtype=np.float32) * np.float32(K ** -0.5)
    vec = g.standard_normal(N, dtype=np.float32) * np.float32(0.3)
    C0 = g.standard_normal((M, N), dtype=np.float32)
    dev = torch.device("cuda")
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    tA, tW, tv = (torch.from_numpy(x).to(dev) for x in (A, W, vec))
    lin = oracle.gemm(A, W).astype(np.float64)
    cases = {
        mb.MB_EPI_SCALE_ADD: C0.astype(np.float64) + vec.astype(np.float64) * lin,
        mb.MB_EPI_GELU_ERF: (lambda u: 0.5 * u * (1.0 + erf(u / np.sqrt(2.0))))(lin + vec),
    }
    for epi, want in cases.items():
        tC = torch.from_numpy(C0).to(dev)
        ctx.linear_dev(M, N, K, tA.data_ptr(), K, tW.data_ptr(), tv.data_ptr(), tC.data_ptr(), N, epi)
        torch.cuda.synchronize()
        err = float(np.abs(tC.cpu().numpy() - want).max())
        assert err < 1e-4, (epi, err)


def test_linear_scale_add_needs_the_scale(ctx):
    with pytest.raises(mb.MbError) as e:
        ctx.linear_dev(4, 256, 256, 16, 256, 16, None, 16, 256, mb.MB_EPI_SCALE_ADD)
    assert e.value.code == mb.MB_ERR_ARG


def test_gemv_rows_1_to_8(ctx):
    """Up to 8 rows take the GEMV kernel: 16-column strips over all of k, the
    four strips of a 64-column block numbered 8 apart, a last group of fewer
    than 32 strips in order.  Every row count 1..8 at shapes from one
    64-column block (N = 64) to 144 strips (2304) and 3072-deep k, each call
    made twice: both within 1e-4 of the oracle and bit-identical."""
    torch = pytest.importorskip("torch")
    dev = torch.device("cuda")
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    for N, K in ((64, 64), (128, 768), (2304, 768), (768, 3072), (1024, 192)):
        say(f"gemv N={N} K={K} M=1..8")
        g = np.random.default_rng([N, K, 11])
        W = g.standard_normal((K, N), dtype=np.float32) * np.float32(0.05)
        bias = g.standard_normal(N, dtype=np.float32) * np.float32(0.1)
        tW, tb = torch.from_numpy(W).to(dev), torch.from_numpy(bias).to(dev)
        for M in range(1, 9):
            A = g.standard_normal((M, K), dtype=np.float32)
            tA = torch.from_numpy(A).to(dev)
            want = oracle.gemm(A, W, bias)
            outs = []
            for _ in range(2):
                tC = torch.full((M, N), 7.0, device=dev)
                ctx.linear_dev(M, N, K, tA.data_ptr(), K, tW.data_ptr(), tb.data_ptr(), tC.data_ptr(), N)
                torch.cuda.synchronize()
                outs.append(tC.cpu().numpy())
            assert np.array_equal(outs[0], outs[1]), (M, N, K)
            err = float(np.abs(outs[0] - want).max())
            assert err < 1e-4, (M, N, K, err)


SPLIT_SHAPES = [  # (M, N, K): 16 / 32 / 48 / 64-row tiles, k split in two, ragged M
    (9, 2304, 768), (64, 768, 768), (100, 768, 3072), (256, 2304, 768), (256, 3072, 768),
    (256, 768, 3072), (256, 1024, 768), (300, 768, 768), (1000, 768, 768),
    # prefill sizes, the tiled kernel: 128-, 64- and 32-row workgroup tiles,
    # ragged M, K = 3072, the codec's N = 256 / 1024 at K = 256 / 1024
    (8192, 2304, 768), (8192, 768, 3072), (2000, 768, 768), (4100, 256, 1024),
    (8192, 1024, 256), (1030, 3072, 768),
]


def _bf16(x):
    """float32 -> bf16 (round to nearest even), returned as float32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return u.astype(np.uint32).view(np.float32)


@pytest.mark.parametrize("M,N,K", SPLIT_SHAPES)
def test_linear_split_bf16(ctx, M, N, K):
    """mb_linear_split_dev on weights from mb_split_weights_dev.  Each product
    a w is ah wh + ah wl + al wh (ah = bf16(a), al = bf16(a - ah), likewise
    w); with bf16's 8-bit significand the terms left out are each within
    2^-18 |a w|, so every output is within 2^-16 sum_k |a_k w_k| (+ fp32
    accumulation) of the exact product -- checked elementwise against the
    oracle's GEMM.  Plain bf16 products (ah wh alone) miss by ~2^-9 |a w|:
    the split must land at least 30x closer, which a dropped term fails.
    Two calls are bit-identical."""
    torch = pytest.importorskip("torch")
    say(f"linear split-bf16 M={M} N={N} K={K}")
    g = np.random.default_rng([M, N, K, 3])
    A = g.standard_normal((M, K), dtype=np.float32)
    W = g.standard_normal((K, N), dtype=np.float32) * np.float32(0.02)
    bias = g.standard_normal(N, dtype=np.float32) * np.float32(0.1)
    C0 = g.standard_normal((M, N), dtype=np.float32)
    dev = torch.device("cuda")
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    tA, tW, tb = (torch.from_numpy(x).to(dev) for x in (A, W, bias))
    tWx = torch.empty(2 * K * N, dtype=torch.bfloat16, device=dev)
    ctx.split_weights_dev(tW.data_ptr(), K, N, tWx.data_ptr())
    lin = oracle.gemm(A, W, bias).astype(np.float64)
    absprod = np.abs(A.astype(np.float64)) @ np.abs(W.astype(np.float64))
    bound = 2.0 ** -16 * absprod + 2e-6 * (1.0 + np.abs(lin))
    plain = (_bf16(A).astype(np.float64) @ _bf16(W).astype(np.float64)) + bias
    plain_err = float(np.abs(plain - lin).max())
    for epi in (mb.MB_EPI_STORE, mb.MB_EPI_GELU, mb.MB_EPI_ADD):
        outs = []
        for _ in range(2):
            tC = torch.from_numpy(C0).to(dev)
            ctx.linear_split_dev(M, N, K, tA.data_ptr(), K, tWx.data_ptr(), tb.data_ptr(),
                                 tC.data_ptr(), N, epi)
            torch.cuda.synchronize()
            outs.append(tC.cpu().numpy())
        assert np.array_equal(outs[0], outs[1]), epi
        got = outs[0].astype(np.float64)
        if epi == mb.MB_EPI_STORE:
            err = np.abs(got - lin)
            assert (err <= bound).all(), float((err / bound).max())
            assert float(err.max()) * 30 < plain_err, (float(err.max()), plain_err)
        elif epi == mb.MB_EPI_GELU:  # |gelu'| <= 1.13
            want = oracle.gelu(lin.astype(np.float32)).astype(np.float64)
            assert (np.abs(got - want) <= 1.2 * bound + 1e-6).all()
        else:
            want = C0.astype(np.float64) + lin
            assert (np.abs(got - want) <= bound + 2.0 ** -23 * np.abs(want)).all()


def test_linear_split_rejects_bad_shapes(ctx):
    """GEMV-sized M, K not a multiple of 128 (decode sizes), N not a
    multiple of 128 (prefill sizes) and misaligned weights are refused before
    any launch."""
    with pytest.raises(mb.MbError) as e:
        ctx.linear_split_dev(8, 768, 768, 16, 768, 16, None, 16, 768)  # M <= 8: the GEMV's
    assert e.value.code == mb.MB_ERR_STATE
    with pytest.raises(mb.MbError) as e:
        ctx.linear_split_dev(64, 768, 704, 16, 704, 16, None, 16, 768)  # K % 128 != 0
    assert e.value.code == mb.MB_ERR_ARG
    with pytest.raises(mb.MbError) as e:
        ctx.linear_split_dev(8192, 704, 768, 16, 768, 16, None, 16, 704)  # N % 128 != 0
    assert e.value.code == mb.MB_ERR_ARG
    with pytest.raises(mb.MbError) as e:
        ctx.split_weights_dev(16, 768, 768, 24)  # Wx not 16-byte aligned
    assert e.value.code == mb.MB_ERR_ARG


def test_linear_split_counters_reset_between_calls(ctx):
    """K = 3072 split-bf16 projections finish their k-split tiles in the
    kernel: the last split of a tile to count in on the tile's counter adds
    the partials and sets the counter back to zero.  Ten calls in a row over
    changing row counts (so the tiles and counters differ from call to call),
    each checked against the oracle: a counter left non-zero would make a
    later call skip or double a tile."""
    torch = pytest.importorskip("torch")
    dev = torch.device("cuda")
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    N, K = 768, 3072
    g = np.random.default_rng(77)
    W = g.standard_normal((K, N), dtype=np.float32) * np.float32(0.02)
    tW = torch.from_numpy(W).to(dev)
    tWx = torch.empty(2 * K * N, dtype=torch.bfloat16, device=dev)
    ctx.split_weights_dev(tW.data_ptr(), K, N, tWx.data_ptr())
    absW = np.abs(W.astype(np.float64))
    for M in (256, 100, 256, 64, 9, 300, 256, 128, 17, 256):
        say(f"split-bf16 K=3072 M={M}")
        A = g.standard_normal((M, K), dtype=np.float32)
        tA = torch.from_numpy(A).to(dev)
        tC = torch.full((M, N), 5.0, device=dev)
        ctx.linear_split_dev(M, N, K, tA.data_ptr(), K, tWx.data_ptr(), None, tC.data_ptr(), N)
        torch.cuda.synchronize()
        want = oracle.gemm(A, W).astype(np.float64)
        bound = 2.0 ** -16 * (np.abs(A.astype(np.float64)) @ absW) + 2e-6 * (1.0 + np.abs(want))
        err = np.abs(tC.cpu().numpy().astype(np.float64) - want)
        assert (err <= bound).all(), (M, float((err / bound).max()))
