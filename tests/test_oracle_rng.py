"""Pins the oracle's RNG restatement (rng.rs) bit for bit against an
independent Python big-int xoshiro256++ / splitmix64, and re-runs the
reference's own rng unit tests (rng.rs:74-118) on it."""
import math

import numpy as np

M64 = (1 << 64) - 1


def py_xoshiro(seed):
    """rng.rs:8-36 written independently with Python integers."""
    z = (seed + 0x9E3779B97F4A7C15) & M64
    s = []
    for _ in range(4):
        z = (z + 0x9E3779B97F4A7C15) & M64
        x = z
        x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & M64
        x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & M64
        s.append(x ^ (x >> 31))

    def rotl(x, k):
        return ((x << k) | (x >> (64 - k))) & M64

    while True:
        r = (rotl((s[0] + s[3]) & M64, 23) + s[0]) & M64
        t = (s[1] << 17) & M64
        s[2] ^= s[0]
        s[3] ^= s[1]
        s[1] ^= s[2]
        s[0] ^= s[3]
        s[2] ^= t
        s[3] = rotl(s[3], 45)
        yield r


def test_u64_stream_matches_independent_restatement(orc):
    for seed in (0, 1, 7, 1234, 1234 ^ 0x1234, 0xFFFFFFFFFFFFFFFF):
        r = orc.Rng(seed)
        g = py_xoshiro(seed)
        for _ in range(2000):
            assert r.next_u64() == next(g)


def test_uniform_is_top_24_bits(orc):
    r, g = orc.Rng(7), py_xoshiro(7)
    for _ in range(2000):
        assert r.uniform() == (next(g) >> 40) * 2.0 ** -24


def test_normal_is_box_muller(orc):
    """normal = sqrt(-2 ln u1) cos(tau u2), u1 clamped to 1e-7 (rng.rs:54-59);
    f32 logf/cosf are within a few ulp of the f64 formula."""
    r, g = orc.Rng(99), py_xoshiro(99)
    for _ in range(2000):
        u1 = max((next(g) >> 40) * 2.0 ** -24, float(np.float32(1e-7)))
        u2 = (next(g) >> 40) * 2.0 ** -24
        want = math.sqrt(-2.0 * math.log(u1)) * math.cos(2 * math.pi * u2)
        assert abs(r.normal() - want) <= 2e-6 * max(1.0, abs(want))


def test_rand_vec_matches_normal_sequence(orc):
    a = orc.Rng(5).rand_vec(100)
    r = orc.Rng(5)
    assert np.array_equal(a, np.array([r.normal() for _ in range(100)], np.float32))
    big = orc.Rng(7).rand_vec(200000)
    assert abs(float(big.mean())) < 0.01 and abs(float(big.std()) - 1.0) < 0.01


# --- the reference's unit tests (rng.rs:74-118) on the restatement
def test_same_seed_same_sequence(orc):
    a, b = orc.Rng(1234), orc.Rng(1234)
    for _ in range(1000):
        assert a.next_u64() == b.next_u64()
    assert orc.Rng(1).next_u64() != orc.Rng(2).next_u64()


def test_uniform_in_range(orc):
    r = orc.Rng(7)
    for _ in range(10000):
        x = r.uniform()
        assert 0.0 <= x < 1.0


def test_below_in_range(orc):
    r = orc.Rng(9)
    for n in (1, 2, 7, 100):
        for _ in range(1000):
            assert r.below(n) < n
