/*
 * orc_rng.c -- restatement of the reference RNG (rng.rs).  Test
 * infrastructure: generates the seeded synthetic inputs shared by the oracle,
 * the parity tests and bench.py.  Parity: the reference's own unit-test
 * properties (rng.rs:74-118) and an independent Python big-int restatement
 * (tests/test_oracle_rng.py) pin it bit for bit.
 *
 * Rust's f32::ln / f32::cos / f32::sqrt lower to the C library's logf / cosf /
 * sqrtf on linux-gnu, which is what is called here.
 */
#include <math.h>

#include "orc.h"

static inline uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

/* Rng::new (rng.rs:8-22): splitmix64 seeded from seed + golden gamma. */
void orc_rng_new(orc_rng *r, uint64_t seed) {
    uint64_t z = seed + 0x9E3779B97F4A7C15ull;
    for (int i = 0; i < 4; i++) {
        z += 0x9E3779B97F4A7C15ull;
        uint64_t x = z;
        x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
        x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
        r->s[i] = x ^ (x >> 31);
    }
}

/* Rng::next_u64 (rng.rs:24-36): xoshiro256++. */
uint64_t orc_rng_next_u64(orc_rng *r) {
    uint64_t *s = r->s;
    uint64_t res = rotl64(s[0] + s[3], 23) + s[0];
    uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl64(s[3], 45);
    return res;
}

/* rng.rs:38-41 */
uint32_t orc_rng_next_u32(orc_rng *r) { return (uint32_t)(orc_rng_next_u64(r) >> 32); }

/* rng.rs:43-47 */
size_t orc_rng_below(orc_rng *r, size_t n) { return (size_t)(orc_rng_next_u64(r) % (uint64_t)n); }

/* rng.rs:49-52: 24-bit uniform in [0, 1). */
float orc_rng_uniform(orc_rng *r) {
    return (float)(orc_rng_next_u64(r) >> 40) * (1.0f / (float)(1ull << 24));
}

/* rng.rs:54-59: Box-Muller, u1 clamped to >= 1e-7. */
float orc_rng_normal(orc_rng *r) {
    float u1 = orc_rng_uniform(r);
    if (!(u1 > 1e-7f)) u1 = 1e-7f; /* f32::max(u1, 1e-7) */
    float u2 = orc_rng_uniform(r);
    const float tau = 6.28318530717958647692f; /* std::f32::consts::TAU */
    return sqrtf(-2.0f * logf(u1)) * cosf(tau * u2);
}

/* rand_vec (rng.rs:68-72). */
void orc_rand_vec(orc_rng *r, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = orc_rng_normal(r);
}

void orc_rand_uniform_vec(orc_rng *r, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = orc_rng_uniform(r);
}

/* Param::trunc_normal (nn.rs:77-89): a normal, redrawn at most 8 times while
 * |z| > 2, clamped to [-2, 2] (f32::clamp), times std. */
void orc_trunc_normal(orc_rng *r, float *out, size_t n, float std_) {
    for (size_t i = 0; i < n; i++) {
        float z = orc_rng_normal(r);
        int tries = 0;
        while (fabsf(z) > 2.0f && tries < 8) {
            z = orc_rng_normal(r);
            tries++;
        }
        if (z < -2.0f) z = -2.0f;
        if (z > 2.0f) z = 2.0f;
        out[i] = z * std_;
    }
}

/* Rng::shuffle (rng.rs:61-65): Fisher-Yates from the top. */
void orc_rng_shuffle(orc_rng *r, size_t *v, size_t n) {
    for (size_t i = n; i-- > 1;) {
        size_t j = orc_rng_below(r, i + 1);
        size_t t = v[i];
        v[i] = v[j];
        v[j] = t;
    }
}
