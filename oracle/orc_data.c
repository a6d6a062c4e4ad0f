/*
 * orc_data.c -- CPU oracle: data.rs batch assembly (crop, flip, normalise,
 * random erasing), the evaluation batch and mix_batch.  TEST INFRASTRUCTURE
 * ONLY (see orc.h).  Loops and draws in the reference's order.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "orc.h"

#define IMG 32
#define CH 3
#define PIX (CH * IMG * IMG)

static const float MEAN_[3] = {0.5071f, 0.4865f, 0.4409f};
static const float STD_[3] = {0.2673f, 0.2564f, 0.2762f};

/* norm (data.rs:96-98). */
static float norm_(uint8_t v, int c) { return ((float)v / 255.0f - MEAN_[c]) / STD_[c]; }

/* crop_flip_normalize (data.rs:331-362). */
void orc_crop_flip_normalize(const uint8_t *src, float *dst, long dy, long dx, int flip) {
    for (int c = 0; c < CH; c++) {
        const float border = -MEAN_[c] / STD_[c];
        for (int y = 0; y < IMG; y++) {
            const long sy = y + dy;
            float *row = dst + c * IMG * IMG + y * IMG;
            for (int x = 0; x < IMG; x++) {
                const long sx = (flip ? IMG - 1 - x : x) + dx;
                row[x] = (sy >= 0 && sy < IMG && sx >= 0 && sx < IMG)
                             ? norm_(src[c * IMG * IMG + sy * IMG + sx], c)
                             : border;
            }
        }
    }
}

/* ---- RandAugment (data.rs:102-314) on one u8 image [3][32][32] */
static uint8_t px_(const uint8_t *im, int c, long y, long x) {
    if (y < 0 || x < 0 || y >= IMG || x >= IMG) return 128;
    return im[c * IMG * IMG + y * IMG + x];
}

static uint8_t sat_u8(float v) {  /* v.clamp(0, 255) as u8 */
    if (!(v > 0.0f)) return 0;  /* NaN saturates to 0 in Rust's cast */
    if (v > 255.0f) v = 255.0f;
    return (uint8_t)v;
}

static void affine_(uint8_t *im, float a, float b, float tx, float c_, float d, float ty) {
    uint8_t src[PIX];
    memcpy(src, im, PIX);
    const float cy = (float)IMG / 2.0f - 0.5f, cx = (float)IMG / 2.0f - 0.5f;
    for (int ch = 0; ch < CH; ch++)
        for (int y = 0; y < IMG; y++)
            for (int x = 0; x < IMG; x++) {
                const float fy = (float)y - cy, fx = (float)x - cx;
                const float sx = a * fx + b * fy + tx + cx;
                const float sy = c_ * fx + d * fy + ty + cy;
                const float x0f = floorf(sx), y0f = floorf(sy);
                const float wx = sx - x0f, wy = sy - y0f;
                const long x0 = (long)x0f, y0 = (long)y0f;
                const float v = (float)px_(src, ch, y0, x0) * (1.0f - wx) * (1.0f - wy) +
                                (float)px_(src, ch, y0, x0 + 1) * wx * (1.0f - wy) +
                                (float)px_(src, ch, y0 + 1, x0) * (1.0f - wx) * wy +
                                (float)px_(src, ch, y0 + 1, x0 + 1) * wx * wy;
                im[ch * IMG * IMG + y * IMG + x] = sat_u8(v);
            }
}

static void blend_(uint8_t *im, const uint8_t *other, float f) {
    for (int i = 0; i < PIX; i++)
        im[i] = sat_u8((float)other[i] + f * ((float)im[i] - (float)other[i]));
}

static void grayscale_(const uint8_t *im, uint8_t *g) {
    for (int p = 0; p < IMG * IMG; p++) {
        const float v = 0.299f * (float)im[p] + 0.587f * (float)im[IMG * IMG + p] +
                        0.114f * (float)im[2 * IMG * IMG + p];
        const uint8_t u = sat_u8(v);
        for (int c = 0; c < CH; c++) g[c * IMG * IMG + p] = u;
    }
}

/* apply_op (data.rs:255-278) after its sign draw: operation op with
 * magnitude v in [0, 1] and sign +-1. */
void orc_ra_op(uint8_t *im, size_t op, float v, float sign) {
    const float f = 1.0f + sign * 0.9f * v;
    uint8_t tmp[PIX];
    switch (op) {
        case 0: affine_(im, 1.0f, sign * 0.3f * v, 0.0f, 0.0f, 1.0f, 0.0f); break;
        case 1: affine_(im, 1.0f, 0.0f, 0.0f, sign * 0.3f * v, 1.0f, 0.0f); break;
        case 2: affine_(im, 1.0f, 0.0f, sign * 10.0f * v, 0.0f, 1.0f, 0.0f); break;
        case 3: affine_(im, 1.0f, 0.0f, 0.0f, 0.0f, 1.0f, sign * 10.0f * v); break;
        case 4: {
            const float t = sign * 30.0f * v * 3.14159265358979323846f / 180.0f;
            affine_(im, cosf(t), -sinf(t), 0.0f, sinf(t), cosf(t), 0.0f);
            break;
        }
        case 5: {
            const unsigned bits = 8u - (unsigned)(4.0f * v);
            const uint8_t mask = (uint8_t)~((1u << (8 - bits)) - 1u);
            for (int i = 0; i < PIX; i++) im[i] &= mask;
            break;
        }
        case 6: {
            const uint8_t th = sat_u8(255.0f * (1.0f - v));
            for (int i = 0; i < PIX; i++)
                if (im[i] >= th) im[i] = (uint8_t)(255 - im[i]);
            break;
        }
        case 7:
            for (int c = 0; c < CH; c++) {
                uint8_t *s = im + c * IMG * IMG, lo = 255, hi = 0;
                for (int i = 0; i < IMG * IMG; i++) {
                    lo = s[i] < lo ? s[i] : lo;
                    hi = s[i] > hi ? s[i] : hi;
                }
                if (hi > lo) {
                    const float k = 255.0f / (float)(hi - lo);
                    for (int i = 0; i < IMG * IMG; i++) s[i] = sat_u8((float)(s[i] - lo) * k);
                }
            }
            break;
        case 8:
            for (int c = 0; c < CH; c++) {
                uint8_t *s = im + c * IMG * IMG;
                uint32_t hist[256] = {0}, cdf[256], acc = 0, lo = 0;
                for (int i = 0; i < IMG * IMG; i++) hist[s[i]]++;
                for (int i = 0; i < 256; i++) cdf[i] = acc += hist[i];
                for (int i = 0; i < 256; i++)
                    if (cdf[i] > 0) {
                        lo = cdf[i];
                        break;
                    }
                uint32_t den = IMG * IMG > lo ? IMG * IMG - lo : 0;
                if (den < 1) den = 1;
                for (int i = 0; i < IMG * IMG; i++) s[i] = (uint8_t)(((cdf[s[i]] - lo) * 255u) / den);
            }
            break;
        case 9:
            memset(tmp, 0, PIX);
            blend_(im, tmp, f);
            break;
        case 10:
            grayscale_(im, tmp);
            blend_(im, tmp, f);
            break;
        case 11: {
            grayscale_(im, tmp);
            uint32_t sum = 0;
            for (int i = 0; i < IMG * IMG; i++) sum += tmp[i];
            memset(tmp, (int)(uint8_t)(sum / (IMG * IMG)), PIX);
            blend_(im, tmp, f);
            break;
        }
        default: {
            uint8_t src[PIX];
            memcpy(src, im, PIX);
            memcpy(tmp, im, PIX);
            for (int c = 0; c < CH; c++)
                for (int y = 1; y < IMG - 1; y++)
                    for (int x = 1; x < IMG - 1; x++) {
                        float sm = 0.0f;
                        for (int dy = 0; dy < 3; dy++)
                            for (int dx = 0; dx < 3; dx++) {
                                const float w = (dy == 1 && dx == 1) ? 5.0f : 1.0f / 8.0f * 3.0f;
                                sm += w * (float)px_(src, c, y + dy - 1, x + dx - 1);
                            }
                        tmp[c * IMG * IMG + y * IMG + x] = sat_u8(sm / 8.0f);
                    }
            blend_(im, tmp, f);
        }
    }
}

/* randaugment (data.rs:303-314). */
static void apply_op_(uint8_t *im, size_t op, float v, orc_rng *r) {
    /* the sign is drawn for every operation, used or not */
    const float sign = (orc_rng_next_u32(r) & 1u) == 1u ? 1.0f : -1.0f;
    orc_ra_op(im, op, v, sign);
}

void orc_randaugment(uint8_t *im, float ra_mag, size_t ra_n, orc_rng *r) {
    if (ra_mag <= 0.0f) return;
    for (size_t k = 0; k < ra_n; k++) {
        const size_t op = orc_rng_below(r, 13);
        float v = ra_mag * (1.0f + 0.5f * orc_rng_normal(r));
        v = v < 0.0f ? 0.0f : (v > 1.0f ? 1.0f : v);
        apply_op_(im, op, v, r);
    }
}

/* make_batch_train (data.rs:384-416). */
void orc_cifar_batch_train(const uint8_t *images, const uint8_t *fine, const uint8_t *coarse,
                           const uint32_t *idx, size_t bs, size_t pad, float ra_mag, size_t ra_n,
                           float erase, size_t erase_side, uint64_t seed, float *out,
                           uint32_t *labels, uint32_t *coarse_out) {
    for (size_t b = 0; b < bs; b++) {
        const uint32_t i = idx[b];
        labels[b] = fine[i];
        coarse_out[b] = coarse[i];
        orc_rng r;
        orc_rng_new(&r, seed ^ ((uint64_t)b * 0x9E3779B97F4A7C15ull));
        uint8_t work[PIX];
        memcpy(work, images + (size_t)i * PIX, PIX);
        orc_randaugment(work, ra_mag, ra_n, &r);
        long dy = 0, dx = 0;
        if (pad > 0) {
            dy = (long)orc_rng_below(&r, 2 * pad + 1) - (long)pad;
            dx = (long)orc_rng_below(&r, 2 * pad + 1) - (long)pad;
        }
        const int flip = (orc_rng_next_u32(&r) & 1u) == 1u;
        float *dst = out + b * PIX;
        orc_crop_flip_normalize(work, dst, dy, dx, flip);
        if (erase <= 0.0f || orc_rng_uniform(&r) >= erase) continue;
        const long cy = (long)orc_rng_below(&r, IMG), cx = (long)orc_rng_below(&r, IMG);
        const long h = (long)erase_side / 2;
        for (int c = 0; c < CH; c++)
            for (long y = cy - h < 0 ? 0 : cy - h; y < (cy + h < IMG ? cy + h : IMG); y++)
                for (long x = cx - h < 0 ? 0 : cx - h; x < (cx + h < IMG ? cx + h : IMG); x++)
                    dst[c * IMG * IMG + y * IMG + x] = orc_rng_normal(&r);
    }
}

/* beta_like (data.rs:418-429). */
static float beta_like_(float a, orc_rng *r) {
    const float u = orc_rng_uniform(r);
    if (a >= 1.0f) return u;
    if (u < 0.5f) return powf(2.0f * u, 1.0f / a) * 0.5f;
    return 1.0f - powf(2.0f * (1.0f - u), 1.0f / a) * 0.5f;
}

/* mix_batch (data.rs:469-492) in place on x [bs][PIX]; perm, lam out. */
void orc_mix_batch(float *x, size_t bs, float alpha_mix, float alpha_cut, float sw, orc_rng *r,
                   uint32_t *perm, float *lam) {
    size_t *p = malloc((bs ? bs : 1) * sizeof(size_t));
    for (size_t i = 0; i < bs; i++) p[i] = i;
    for (size_t i = bs; i-- > 1;) {
        const size_t j = orc_rng_below(r, i + 1);
        const size_t t = p[i];
        p[i] = p[j];
        p[j] = t;
    }
    for (size_t i = 0; i < bs; i++) {
        perm[i] = (uint32_t)p[i];
        lam[i] = 1.0f;
    }
    if (!(alpha_mix <= 0.0f && alpha_cut <= 0.0f)) {
        const int cut = alpha_cut > 0.0f && (alpha_mix <= 0.0f || orc_rng_uniform(r) < sw);
        const float l = beta_like_(cut ? alpha_cut : alpha_mix, r);
        float *src = malloc(bs * PIX * sizeof(float));
        memcpy(src, x, bs * PIX * sizeof(float));
        if (cut) {
            const float rr = sqrtf(1.0f - l);
            size_t side = (size_t)((float)IMG * rr);
            if (side > IMG) side = IMG;
            const size_t cy = orc_rng_below(r, IMG), cx = orc_rng_below(r, IMG);
            const size_t y0 = cy >= side / 2 ? cy - side / 2 : 0;
            const size_t y1 = cy + side / 2 < IMG ? cy + side / 2 : IMG;
            const size_t x0 = cx >= side / 2 ? cx - side / 2 : 0;
            const size_t x1 = cx + side / 2 < IMG ? cx + side / 2 : IMG;
            const float area = (float)((y1 - y0) * (x1 - x0)) / (float)(IMG * IMG);
            for (size_t b = 0; b < bs; b++) {
                for (int c = 0; c < CH; c++)
                    for (size_t y = y0; y < y1; y++)
                        for (size_t xx = x0; xx < x1; xx++) {
                            const size_t o = c * IMG * IMG + y * IMG + xx;
                            x[b * PIX + o] = src[p[b] * PIX + o];
                        }
                lam[b] = 1.0f - area;
            }
        } else {
            for (size_t b = 0; b < bs; b++) {
                for (size_t i = 0; i < PIX; i++)
                    x[b * PIX + i] = l * src[b * PIX + i] + (1.0f - l) * src[p[b] * PIX + i];
                lam[b] = l;
            }
        }
        free(src);
    }
    free(p);
}

/* ---------------------------------------------------------------- train.rs
 * FNV-1a 64 of Trainer::fingerprint (train.rs:474-484): offset basis
 * 0xcbf29ce484222325, prime 0x100000001b3; per byte h = (h ^ b) * prime
 * (mod 2^64).  fnv_f32 folds a float as the 4 little-endian bytes of its bit
 * pattern. */
uint64_t orc_fnv1a_bytes(uint64_t h, const uint8_t *p, size_t n) {
    for (size_t i = 0; i < n; i++) {
        h ^= (uint64_t)p[i];
        h *= 0x00000100000001b3ull;
    }
    return h;
}

uint64_t orc_fnv1a_f32(uint64_t h, const float *v, size_t n) {
    for (size_t i = 0; i < n; i++) {
        uint32_t bits;
        memcpy(&bits, &v[i], 4);
        for (int k = 0; k < 4; k++) {
            h ^= (uint64_t)((bits >> (8 * k)) & 0xffu);
            h *= 0x00000100000001b3ull;
        }
    }
    return h;
}
