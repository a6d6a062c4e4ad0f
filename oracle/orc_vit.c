/*
 * orc_vit.c -- CPU oracle: vit.rs's DropPath, token merge and TaxoHead
 * combine, tok.rs's layout changes.  TEST INFRASTRUCTURE ONLY (see orc.h).
 */
#include <stdint.h>
#include <string.h>

#include "orc.h"

/* DropPath::forward (vit.rs:39-59) in place; mask [n] receives the factors. */
void orc_drop_path(size_t n, size_t per, float *x, float p, uint64_t seed, float *mask) {
    orc_rng r;
    orc_rng_new(&r, seed);
    const float keep = 1.0f - p;
    for (size_t i = 0; i < n; i++) mask[i] = orc_rng_uniform(&r) < keep ? 1.0f / keep : 0.0f;
    for (size_t i = 0; i < n; i++)
        if (mask[i] != 1.0f)
            for (size_t j = 0; j < per; j++) x[i * per + j] *= mask[i];
}

/* token_merge (vit.rs:612-630). */
void orc_token_merge(size_t n, size_t th, size_t c, const float *z, float *y) {
    const size_t t2 = th / 2;
    static const int off[4][2] = {{0, 0}, {0, 1}, {1, 0}, {1, 1}};
    for (size_t i = 0; i < n; i++)
        for (size_t oy = 0; oy < t2; oy++)
            for (size_t ox = 0; ox < t2; ox++) {
                const size_t o = ((i * t2 + oy) * t2 + ox) * 4 * c;
                for (int q = 0; q < 4; q++) {
                    const size_t s =
                        ((i * th + 2 * oy + (size_t)off[q][0]) * th + 2 * ox + (size_t)off[q][1]) * c;
                    memcpy(y + o + (size_t)q * c, z + s, c * sizeof(float));
                }
            }
}

/* TaxoHead::forward's combine (vit.rs:287-292) and the backward's coarse
 * gradient (vit.rs:296-306). */
void orc_taxo_combine(size_t n, size_t nf, size_t nc, const uint32_t *parent, float *zf,
                      const float *zc) {
    for (size_t i = 0; i < n; i++)
        for (size_t j = 0; j < nf; j++) zf[i * nf + j] += zc[i * nc + parent[j]];
}

void orc_taxo_combine_backward(size_t n, size_t nf, size_t nc, const uint32_t *parent,
                               const float *dzf, const float *dzc, float *dc) {
    for (size_t i = 0; i < n; i++) {
        memcpy(dc + i * nc, dzc + i * nc, nc * sizeof(float));
        for (size_t j = 0; j < nf; j++) dc[i * nc + parent[j]] += dzf[i * nf + j];
    }
}
