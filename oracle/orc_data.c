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

/* make_batch_train (data.rs:384-416) without RandAugment. */
void orc_cifar_batch_train(const uint8_t *images, const uint8_t *fine, const uint8_t *coarse,
                           const uint32_t *idx, size_t bs, size_t pad, float erase,
                           size_t erase_side, uint64_t seed, float *out, uint32_t *labels,
                           uint32_t *coarse_out) {
    for (size_t b = 0; b < bs; b++) {
        const uint32_t i = idx[b];
        labels[b] = fine[i];
        coarse_out[b] = coarse[i];
        orc_rng r;
        orc_rng_new(&r, seed ^ ((uint64_t)b * 0x9E3779B97F4A7C15ull));
        long dy = 0, dx = 0;
        if (pad > 0) {
            dy = (long)orc_rng_below(&r, 2 * pad + 1) - (long)pad;
            dx = (long)orc_rng_below(&r, 2 * pad + 1) - (long)pad;
        }
        const int flip = (orc_rng_next_u32(&r) & 1u) == 1u;
        float *dst = out + b * PIX;
        orc_crop_flip_normalize(images + (size_t)i * PIX, dst, dy, dx, flip);
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
