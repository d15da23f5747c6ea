"""mb_linear_noalloc_dev, the projection entry point that allocates nothing,
against mb_linear_dev (the entry point it varies) through the C ABI.

Two calls in a row on one context, the second smaller, each with split-K
partials in the static scratch (K = 3072 at decode-sized M: 256 rows split
two ways on 32-row tiles, 64 rows four ways on 16-row tiles), so the second call reuses the
array the first one left its partials in: outputs equal
mb_linear_dev's bit for bit (same kernels, same summation order) and are
within 1e-4 of float64 (the fp32 bar).  The context's device memory does not
grow across the calls, while mb_linear_dev on the same shapes grows its
context's scratch.
"""
import numpy as np
import pytest

import mockbird_amd as mb
from conftest import say

pytestmark = pytest.mark.gpu

CASES = [  # (M, N, K, epi): the second call is smaller
    (256, 768, 3072, mb.MB_EPI_ADD),
    (64, 768, 3072, mb.MB_EPI_STORE),
]


def test_noalloc_linear_matches_linear_dev():
    torch = pytest.importorskip("torch")
    dev = torch.device("cuda")
    g = torch.Generator(device="cpu").manual_seed(77)
    inputs = []
    for M, N, K, epi in CASES:
        a = torch.randn(M, K, generator=g)
        w = torch.randn(K, N, generator=g) * 0.02
        b = torch.randn(N, generator=g) * 0.1
        c0 = torch.randn(M, N, generator=g)
        inputs.append((a.to(dev), w.to(dev), b.to(dev), c0.to(dev)))
    with mb.Context(n_layers=1, capacity=8, max_seqs=1, max_rows=8, vocab=16) as ctx, \
            mb.Context(n_layers=1, capacity=8, max_seqs=1, max_rows=8, vocab=16) as ref:
        s = torch.cuda.current_stream().cuda_stream
        ctx.set_stream(s)
        ref.set_stream(s)
        before = ctx.device_bytes()
        outs = []
        for (M, N, K, epi), (a, w, b, c0) in zip(CASES, inputs):
            say(f"no-alloc linear M={M} N={N} K={K} epi={epi}")
            c = c0.clone()
            ctx.linear_noalloc_dev(M, N, K, a.data_ptr(), K, w.data_ptr(), b.data_ptr(),
                                   c.data_ptr(), N, epi)
            want = c0.clone()
            ref.linear_dev(M, N, K, a.data_ptr(), K, w.data_ptr(), b.data_ptr(), want.data_ptr(),
                           N, epi)
            torch.cuda.synchronize()
            outs.append((c.cpu().numpy(), want.cpu().numpy()))
        assert ctx.device_bytes() == before, "the no-alloc entry point grew the context"
        assert ref.device_bytes() > before, "the reference path was expected to allocate partials"
    for (M, N, K, epi), (a, w, b, c0), (got, want) in zip(CASES, inputs, outs):
        assert np.array_equal(got, want), (M, N, K)
        x = a.cpu().double().numpy() @ w.cpu().double().numpy() + b.cpu().double().numpy()
        if epi == mb.MB_EPI_ADD:
            x = x + c0.cpu().double().numpy()
        err = float(np.abs(got - x).max() / max(1.0, float(np.abs(x).max())))
        say(f"  M={M}: bit-exact with mb_linear_dev; rel error vs float64 {err:.2e}")
        assert err < 1e-4


def test_noalloc_linear_rejects_bad_arguments():
    with mb.Context(n_layers=1, capacity=8, max_seqs=1, max_rows=8, vocab=16) as ctx:
        with pytest.raises(mb.MbError) as e:
            ctx.linear_noalloc_dev(4, 768, 3072, 0, 3072, 0, 0, 0, 768)
        assert e.value.code == mb.MB_ERR_ARG
        with pytest.raises(mb.MbError) as e:
            ctx.linear_noalloc_dev(4, 768, 3072, 16, 3072, 16, 0, 16, 768, epi=9)
        assert e.value.code == mb.MB_ERR_ARG
