/*
 * orc_loss.c -- CPU oracle: loss.rs (soft targets, ce_soft, kl_distill,
 * hint_mse) and the batch targets of train.rs.  TEST INFRASTRUCTURE ONLY
 * (see orc.h).  Loops in the reference's order, f32, no contraction; the
 * row losses are added in row order (hint_mse's rayon sum has no fixed order
 * -- "parity unpinned" for that total's last bits).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

#include "orc.h"

/* taxo_target (loss.rs:11-28); groups[parent[y]] is every class with that
 * parent (data.rs:72-93). */
void orc_taxo_target(size_t y, const uint32_t *parent, size_t nf, float eps, float sib,
                     float *out) {
    size_t k = 0;
    for (size_t c = 0; c < nf; c++) k += parent[c] == parent[y];
    const float off_far = nf > k ? eps * (1.0f - sib) / (float)(nf - k) : 0.0f;
    for (size_t j = 0; j < nf; j++) out[j] = off_far;
    if (k > 1) {
        const float off_sib = eps * sib / (float)(k - 1);
        for (size_t c = 0; c < nf; c++)
            if (parent[c] == parent[y]) out[c] = off_sib;
    }
    out[y] = 1.0f - eps;
}

/* uniform_target (loss.rs:30-34). */
void orc_uniform_target(size_t y, size_t k, float eps, float *out) {
    for (size_t j = 0; j < k; j++) out[j] = eps / (float)k;
    out[y] += 1.0f - eps;
}

/* targets (train.rs:121-155); perm / lam may be NULL (identity, 1). */
void orc_soft_targets(size_t n, size_t nf, size_t nc, const uint32_t *labels,
                      const uint32_t *coarse, const uint32_t *perm, const float *lam,
                      const uint32_t *parent, int taxo, float eps, float sib, float *tf,
                      float *tc) {
    float *a = malloc(nf * sizeof(float)), *b = malloc(nf * sizeof(float));
    float *ca = malloc((nc ? nc : 1) * sizeof(float)), *cb = malloc((nc ? nc : 1) * sizeof(float));
    for (size_t i = 0; i < n; i++) {
        const size_t pi = perm ? perm[i] : i;
        const size_t ya = labels[i], yb = labels[pi];
        if (taxo) {
            orc_taxo_target(ya, parent, nf, eps, sib, a);
            orc_taxo_target(yb, parent, nf, eps, sib, b);
        } else {
            orc_uniform_target(ya, nf, eps, a);
            orc_uniform_target(yb, nf, eps, b);
        }
        const float l = lam ? lam[i] : 1.0f;
        for (size_t j = 0; j < nf; j++) tf[i * nf + j] = l * a[j] + (1.0f - l) * b[j];
        if (tc) {
            orc_uniform_target(coarse[i], nc, eps, ca);
            orc_uniform_target(coarse[pi], nc, eps, cb);
            for (size_t j = 0; j < nc; j++) tc[i * nc + j] = l * ca[j] + (1.0f - l) * cb[j];
        }
    }
    free(a);
    free(b);
    free(ca);
    free(cb);
}

/* ce_soft (loss.rs:39-83): returns the mean loss, *correct the hits. */
float orc_ce_soft(size_t n, size_t nc, const float *logits, const float *target,
                  const uint32_t *hard, float scale, float *dz, size_t *correct) {
    const float inv = 1.0f / (float)n;
    float loss = 0.0f;
    size_t hits = 0;
    for (size_t i = 0; i < n; i++) {
        const float *z = logits + i * nc, *t = target + i * nc;
        float *d = dz + i * nc;
        float mx = -INFINITY;
        size_t arg = 0;
        for (size_t j = 0; j < nc; j++)
            if (z[j] > mx) {
                mx = z[j];
                arg = j;
            }
        float sum = 0.0f;
        for (size_t j = 0; j < nc; j++) {
            const float e = expf(z[j] - mx);
            d[j] = e;
            sum += e;
        }
        const float lse = mx + logf(sum);
        float l = 0.0f;
        for (size_t j = 0; j < nc; j++) {
            l += t[j] * (lse - z[j]);
            d[j] = (d[j] / sum - t[j]) * inv * scale;
        }
        loss += l;
        hits += arg == hard[i];
    }
    if (correct) *correct = hits;
    return loss * inv;
}

static void soft_(const float *z, size_t nc, float it, float *o) {
    float mx = -INFINITY;
    for (size_t j = 0; j < nc; j++) mx = fmaxf(mx, z[j]);
    float s = 0.0f;
    for (size_t j = 0; j < nc; j++) {
        const float e = expf((z[j] - mx) * it);
        o[j] = e;
        s += e;
    }
    const float is = 1.0f / s;
    for (size_t j = 0; j < nc; j++) o[j] *= is;
}

/* kl_distill (loss.rs:87-130): dz += ...; returns the loss. */
float orc_kl_distill(size_t n, size_t nc, const float *student, const float *teacher, float temp,
                     float scale, float *dz) {
    const float inv = 1.0f / (float)n, it = 1.0f / temp;
    float *ps = malloc(nc * sizeof(float)), *pt = malloc(nc * sizeof(float));
    float total = 0.0f;
    for (size_t i = 0; i < n; i++) {
        soft_(student + i * nc, nc, it, ps);
        soft_(teacher + i * nc, nc, it, pt);
        float l = 0.0f;
        float *d = dz + i * nc;
        for (size_t j = 0; j < nc; j++) {
            if (pt[j] > 1e-9f) l += pt[j] * (logf(fmaxf(pt[j], 1e-9f)) - logf(fmaxf(ps[j], 1e-9f)));
            d[j] += temp * (ps[j] - pt[j]) * inv * scale;
        }
        total += l * temp * temp;
    }
    free(ps);
    free(pt);
    return total * inv;
}

/* hint_mse (loss.rs:133-151): dz += ...; returns the loss. */
float orc_hint_mse(size_t n, size_t c, const float *pred, const float *target, float scale,
                   float *dz) {
    const float inv = 1.0f / (float)(n * c);
    float total = 0.0f;
    for (size_t i = 0; i < n; i++) {
        float s = 0.0f;
        for (size_t j = 0; j < c; j++) {
            const float e = pred[i * c + j] - target[i * c + j];
            s += e * e;
            dz[i * c + j] += 2.0f * e * inv * scale;
        }
        total += s;
    }
    return total * inv * scale;
}
