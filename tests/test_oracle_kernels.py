"""Known-answer checks of the oracle's layer pieces.

The inputs are the reference's own kernel-conformance cases
(tests/gpu/kernels.test.mjs): its xorshift PRNG with seed 0x2f6e2b1
(kernels.test.mjs:22-30), drawn in the same order, on the same shapes
(LayerNorm d=768, GEMV 768x2304, RoPE pos=137, attention over N=512 ring
slots x 12 heads, argmax over 1024).  Each expected value comes from an
independent implementation -- numpy/torch in float64, complex rotation -- not
from the oracle's formulas, and the tolerances are at least as tight as the
reference's (2e-5, 5e-3, 1e-5, 1e-5, exact).
"""
import numpy as np
import pytest

from kernel_cases import XorShift, make_cases, rope_f64
from oracle import oracle


@pytest.fixture(scope="module")
def cases():
    return make_cases()


def test_xorshift_matches_js_semantics():
    """The Python port of the PRNG agrees with a JS engine running the same
    statements (kernels.test.mjs:22-30), so the cases below are the reference's."""
    import shutil
    import subprocess
    node = shutil.which("node")
    if node is None:
        pytest.skip("node is not installed")
    js = ("let seed=0x2f6e2b1;const rnd=()=>{seed^=seed<<13;seed>>>=0;seed^=seed>>17;"
          "seed^=seed<<5;seed>>>=0;return (seed/0xffffffff)*2-1;};"
          "const o=[];for(let i=0;i<2000;i++)o.push(rnd());console.log(JSON.stringify(o));")
    import json
    want = json.loads(subprocess.run([node, "-e", js], capture_output=True, text=True,
                                     check=True).stdout)
    r = XorShift()
    got = [r() for _ in range(2000)]
    assert got == want


def test_layernorm_vs_torch(cases):
    torch = pytest.importorskip("torch")
    x, g, b = cases["ln"]
    ref = torch.nn.functional.layer_norm(torch.from_numpy(x).double(), (768,),
                                         torch.from_numpy(g).double(), torch.from_numpy(b).double(),
                                         eps=1e-5).numpy()
    got = oracle.layernorm(x, g, b)
    assert np.abs(got - ref).max() < 2e-6  # reference tolerance 2e-5


def test_gemv_vs_float64(cases):
    x, W, bias = cases["gemv"]
    ref = x.astype(np.float64) @ W.astype(np.float64) + bias
    got = oracle.gemm(x[None], W, bias)[0]
    assert np.abs(got - ref).max() < 1e-6  # reference tolerance 5e-3


def test_rope_pos137_as_complex_rotation(cases):
    v = cases["rope"]
    ref = rope_f64(v, 137, oracle.inv_freq())
    got = oracle.rope(v, 137)
    assert np.abs(got - ref).max() < 1e-6  # reference tolerance 1e-5
    # the reference test's inline formula has the opposite sign (kernels.test.mjs:240);
    # it rotates the other way and disagrees with the engine convention the fixture pins
    z = v[0::2].astype(np.float64) + 1j * v[1::2].astype(np.float64)
    ang = np.float32(137) * oracle.inv_freq()
    zl = z * np.exp(-1j * ang.astype(np.float64))
    assert np.abs(got[1::2] - zl.imag).max() > 0.1


def test_attention_n512_vs_torch(cases):
    torch = pytest.importorskip("torch")
    q, K, V = cases["attn"]
    ring = oracle.Ring(1, 512)
    ring.K[0], ring.V[0] = K, V
    ring.slot_pos[0] = np.arange(512)
    got = ring.attend(q[None], [511])[0]
    qt = torch.from_numpy(q).double().view(12, 1, 64)
    kt = torch.from_numpy(K).double().view(512, 12, 64).transpose(0, 1)
    vt = torch.from_numpy(V).double().view(512, 12, 64).transpose(0, 1)
    ref = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt).reshape(768).numpy()
    assert np.abs(got - ref).max() < 1e-6  # reference tolerance 1e-5


def test_argmax_lowest_index_on_tie(cases):
    logits = cases["argmax"].copy()
    best = int(np.argmax(logits))  # numpy returns the first maximum
    assert oracle.argmax_penalty(logits)[0] == best
    logits[best + 7] = logits[best]
    logits[3] = logits[best]
    assert oracle.argmax_penalty(logits)[0] == min(3, best)


def test_gelu_tanh_vs_torch():
    torch = pytest.importorskip("torch")
    x = np.linspace(-8, 8, 2001, dtype=np.float32)
    ref = torch.nn.functional.gelu(torch.from_numpy(x).double(), approximate="tanh").numpy()
    assert np.abs(oracle.gelu(x) - ref).max() < 1e-6
    assert oracle.gelu(np.float32(0.0)) == 0.0


def test_bf16_rounding_matches_torch():
    """Round-to-nearest-even to bf16, checked against torch's own conversion,
    including exact ties, the largest finite values and infinities."""
    torch = pytest.importorskip("torch")
    g = np.random.default_rng(9)
    x = np.concatenate([
        g.standard_normal(100000).astype(np.float32) * 10,
        np.array([1 + 2**-8, 1 + 3 * 2**-8, -(1 + 2**-8), 3.4e38, -3.4e38, 1e-40, 0.0, -0.0,
                  np.inf, -np.inf], np.float32),
    ])
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    got = oracle.bf16_round(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
