"""Pin the oracle's ring (slot = pos mod C, slot positions, live mask) against
the graph's own formulation of the same cache.

The codec graph spells the ring as a shift-append (docs/moss-tts-runtime-
analysis.md:663-682): concatenate the cached entries with the new one, keep
the last C, and mask an entry unless 0 <= cur - stored < C.  ShiftCache below
is that formulation, written as a Python list; the oracle's ring must expose
exactly the same visible (position -> K, V) set after every append, for tiny
capacities and arbitrary position streams (jumps, resets), and its attention
must equal textbook softmax attention over that set.
"""
import numpy as np
import pytest

from oracle import oracle

D = 768


class ShiftCache:
    def __init__(self, cap):
        self.C = cap
        self.entries = []  # (pos, k_roped, v)

    def append(self, pos, k_roped, v):
        self.entries = (self.entries + [(pos, k_roped, v)])[-self.C:]

    def visible(self, cur):
        return {p: (k, v) for p, k, v in self.entries if 0 <= cur - p < self.C}


def _attend_f64(q, vis):
    """Textbook softmax attention, scale 0.125, per 64-wide head, float64."""
    if not vis:
        return np.zeros(D)
    K = np.stack([k for k, _ in vis.values()]).astype(np.float64).reshape(-1, 12, 64)
    V = np.stack([v for _, v in vis.values()]).astype(np.float64).reshape(-1, 12, 64)
    qh = q.astype(np.float64).reshape(12, 64)
    s = np.einsum("hd,nhd->hn", qh, K) * 0.125
    p = np.exp(s - s.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    return np.einsum("hn,nhd->hd", p, V).reshape(D)


def _streams(rng, n_steps, cap):
    """Consecutive runs with occasional jumps (forward, past the window)."""
    pos, out = int(rng.integers(0, 3 * cap)), []
    for _ in range(n_steps):
        out.append(pos)
        pos += 1 if rng.random() > 0.1 else int(rng.integers(2, 3 * cap))
    return out


@pytest.mark.parametrize("cap", [1, 2, 3, 5, 8])
@pytest.mark.parametrize("kv_bf16", [False, True])
def test_ring_matches_shift_append(cap, kv_bf16):
    rng = np.random.default_rng(cap * 7 + kv_bf16)
    ring = oracle.Ring(1, cap, kv_bf16=kv_bf16)
    shift = ShiftCache(cap)
    for step, pos in enumerate(_streams(rng, 6 * cap + 10, cap)):
        qkv = rng.standard_normal((1, 2304), dtype=np.float32)
        q = ring.append(qkv, [pos])[0]
        k_roped = oracle.rope(qkv[0, 768:1536], pos)
        v = qkv[0, 1536:].copy()
        if kv_bf16:
            k_roped, v = oracle.bf16_round(k_roped), oracle.bf16_round(v)
        shift.append(pos, k_roped, v)
        vis = shift.visible(pos)
        # the same visible set, slot for slot
        live = {int(p): s for s, p in enumerate(ring.slot_pos[0])
                if oracle.slot_live(int(p), pos, cap)}
        assert set(live) == set(vis), (step, pos)
        for p, s in live.items():
            assert s == p % cap
            assert np.array_equal(ring.K[0, s], vis[p][0])
            assert np.array_equal(ring.V[0, s], vis[p][1])
        got = ring.attend(q[None], [pos])[0]
        assert np.abs(got - _attend_f64(q, vis)).max() < 1e-6


def test_reset_forgets_everything():
    ring = oracle.Ring(1, 4)
    rng = np.random.default_rng(1)
    for p in range(6):
        ring.append(rng.standard_normal((1, 2304), dtype=np.float32), [p])
    ring.slot_pos[:] = -1  # engine.reset (gpu.ts:237-242): every slot forgets its position
    q = ring.append(rng.standard_normal((1, 2304), dtype=np.float32), [0])
    assert sorted(ring.slot_pos[0].tolist()) == [-1, -1, -1, 0]
    # only the new row is visible: attention returns its V exactly
    assert np.abs(ring.attend(q, [0])[0] - ring.V[0, 0]).max() < 1e-7


def test_non_wrapping_ring_rejects_overflow():
    ring = oracle.Ring(1, 8, wrap=False)
    rng = np.random.default_rng(2)
    ring.append(rng.standard_normal((1, 2304), dtype=np.float32), [7])
    with pytest.raises(ValueError):
        ring.append(rng.standard_normal((1, 2304), dtype=np.float32), [8])


def test_eviction_boundaries_capacity_4096():
    """Step index = absolute position; after appending pos the window is
    (pos - C, pos].  Checked at 4095 (full, nothing evicted), 4096 (slot 0
    holds 4096, 0 evicted), 4097 and 5000 (window 905..5000)."""
    C = 4096
    ring = oracle.Ring(1, C)
    rng = np.random.default_rng(3)
    checks = {4095: (0, 4095), 4096: (1, 4096), 4097: (2, 4097), 5000: (905, 5000)}
    for p in range(5001):
        ring.append(rng.standard_normal((1, 2304), dtype=np.float32), [p])
        if p in checks:
            lo, hi = checks[p]
            sp = ring.slot_pos[0]
            live = sorted(int(x) for x in sp if oracle.slot_live(int(x), p, C))
            assert live == list(range(lo, hi + 1))
            assert sp[p % C] == p
            if p >= C:
                assert sp[(p + 1) % C] == p + 1 - C  # next to be evicted is the oldest


def test_attention_invariants():
    rng = np.random.default_rng(4)
    ring = oracle.Ring(1, 16)
    ring.slot_pos[0, :10] = np.arange(10)
    ring.K[0, :10] = rng.standard_normal(D, dtype=np.float32)  # identical keys: uniform weights
    ring.V[0, :10] = rng.standard_normal((10, D), dtype=np.float32)
    q = rng.standard_normal((1, D), dtype=np.float32)
    got = ring.attend(q, [9])[0]
    assert np.abs(got - ring.V[0, :10].astype(np.float64).mean(0)).max() < 1e-6
    # a permutation of the slots changes nothing
    perm = rng.permutation(16)
    r2 = oracle.Ring(1, 16)
    r2.K[0], r2.V[0], r2.slot_pos[0] = ring.K[0, perm], ring.V[0, perm], ring.slot_pos[0, perm]
    assert np.abs(r2.attend(q, [9])[0] - got).max() < 1e-6
