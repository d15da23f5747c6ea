"""The reference's kernel-conformance inputs (tests/gpu/kernels.test.mjs):
its xorshift PRNG with seed 0x2f6e2b1 (kernels.test.mjs:22-30), drawn in the
same order, on the same shapes -- LayerNorm d=768, GEMV 768x2304, RoPE of one
64-dim head at pos=137, attention over N=512 ring slots x 12 heads, argmax
over 1024.  Shared by the oracle's known-answer tests and the GPU tests that
run the same cases through the C ABI."""
import numpy as np

D, H, HD = 768, 12, 64
ROPE_POS = 137
ATTN_SLOTS = 512


class XorShift:
    """kernels.test.mjs:22-30, with JS's int32/uint32 conversions."""

    def __init__(self, seed=0x2F6E2B1):
        self.s = seed

    @staticmethod
    def _i32(x):
        x &= 0xFFFFFFFF
        return x - (1 << 32) if x & 0x80000000 else x

    def __call__(self):
        i32 = self._i32
        s = i32(i32(self.s) ^ i32(self.s << 13)) & 0xFFFFFFFF
        s = i32(i32(s) ^ (i32(s) >> 17))
        s = i32(s ^ i32(s << 5)) & 0xFFFFFFFF
        self.s = s
        return (s / 0xFFFFFFFF) * 2 - 1


def make_cases() -> dict:
    """{"ln": (x, gamma, beta), "gemv": (x, W[768][2304], bias), "rope": v[64],
    "attn": (q[768], K[512][768], V[512][768]), "argmax": logits[1024]}, float32."""
    r = XorShift()
    c = {}
    x = np.zeros(D)
    b = np.zeros(D)
    for i in range(D):
        x[i] = r() * 4
        b[i] = r() * 0.1
    c["ln"] = (x.astype(np.float32), np.ones(D, np.float32), b.astype(np.float32))
    K, N = D, 3 * D
    xg = np.array([r() for _ in range(K)], np.float32)
    W = np.array([r() * 0.05 for _ in range(K * N)], np.float32).reshape(K, N)
    bias = np.array([r() * 0.02 for _ in range(N)], np.float32)
    c["gemv"] = (xg, W, bias)
    c["rope"] = np.array([r() for _ in range(HD)], np.float32)
    n = ATTN_SLOTS
    k = np.zeros(n * H * HD, np.float32)
    v = np.zeros(n * H * HD, np.float32)
    for i in range(k.size):
        k[i] = r()
        v[i] = r()
    q = np.array([r() for _ in range(H * HD)], np.float32)
    c["attn"] = (q, k.reshape(n, D), v.reshape(n, D))
    c["argmax"] = np.array([r() for _ in range(1024)], np.float32)
    return c


def rope_f64(v: np.ndarray, pos: int, inv_freq: np.ndarray) -> np.ndarray:
    """RoPE of one 64-dim head as a complex rotation in float64: pairs
    (2i, 2i+1) turn by pos * inv_freq[i] (angles formed in float32, as the
    engine forms them)."""
    z = v[0::2].astype(np.float64) + 1j * v[1::2].astype(np.float64)
    ang = (np.float32(pos) * inv_freq.astype(np.float32)).astype(np.float64)
    zr = z * np.exp(1j * ang)
    out = np.empty(v.shape[-1])
    out[0::2], out[1::2] = zr.real, zr.imag
    return out
