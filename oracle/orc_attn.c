/*
 * orc_attn.c -- restatement of the reference attention core (attn.rs:21-343):
 * rel_index, Core::forward and Core::backward.  Test infrastructure only (see
 * orc.h).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "orc.h"

/* RelGeom::new + rel_index (attn.rs:21-72). */
size_t orc_rel_index(size_t th, size_t tw, size_t mh, size_t mw, uint32_t *idx) {
    long sy, sx, scale, oy, ox;
    if (mh == th) {
        sy = 2 * (long)th - 1;
        sx = 2 * (long)tw - 1;
        scale = 1;
        oy = (long)th - 1;
        ox = (long)tw - 1;
    } else {
        sy = 2 * ((long)th - 1) + (long)mh;
        sx = 2 * ((long)tw - 1) + (long)mw;
        scale = 2;
        oy = (long)mh - 1;
        ox = (long)mw - 1;
    }
    size_t z = 0;
    for (long qy = 0; qy < (long)th; qy++)
        for (long qx = 0; qx < (long)tw; qx++)
            for (long my = 0; my < (long)mh; my++)
                for (long mx = 0; mx < (long)mw; mx++) {
                    long dy = scale * qy - my + oy;
                    long dx = scale * qx - mx + ox;
                    idx[z++] = (uint32_t)(dy * sx + dx);
                }
    return (size_t)(sy * sx);
}

/* gather (attn.rs:116-123). */
static void gather(const float *src, size_t base, size_t stride, size_t off, size_t rows, size_t dh,
                   float *dst) {
    for (size_t r = 0; r < rows; r++) memcpy(dst + r * dh, src + base + r * stride + off, dh * sizeof(float));
}

/* scatter_add (attn.rs:125-141). */
static void scatter_add(float *dst, size_t base, size_t stride, size_t off, size_t rows, size_t dh,
                        const float *src) {
    for (size_t r = 0; r < rows; r++) {
        float *d = dst + base + r * stride + off;
        for (size_t z = 0; z < dh; z++) d[z] += src[r * dh + z];
    }
}

/* Core::forward (attn.rs:148-223), one image. */
static void forward_image(const orc_attn_desc *d, size_t i, const float *q, const float *kv,
                          const float *tau, const float *rel, float *p, float *o, float *wq,
                          float *wk, float *wv, float *ws, float *wo) {
    size_t h = d->h, dh = d->dh, tq = d->tq, tk = d->tk, c = h * dh;
    float *oi = o + i * tq * c;
    float *pi = p + i * h * tq * tk;
    size_t qbase = i * tq * d->qstride, kbase = i * tk * d->kvstride;
    for (size_t hd = 0; hd < h; hd++) {
        size_t hq = d->qoff + hd * dh, hk = d->koff + hd * dh, hv = d->voff + hd * dh;
        gather(q, qbase, d->qstride, hq, tq, dh, wq);
        gather(kv, kbase, d->kvstride, hk, tk, dh, wk);
        gather(kv, kbase, d->kvstride, hv, tk, dh, wv);
        /* S = Q K^T */
        orc_gemm_small(tq, tk, dh, wq, 0, wk, 1, ws, 0);
        float t = tau[hd];
        const float *rb = rel + hd * d->nrel;
        float *pr = pi + hd * tq * tk;
        for (size_t qi = 0; qi < tq; qi++) {
            const float *sr = ws + qi * tk;
            float *dr = pr + qi * tk;
            const uint32_t *ridx = d->relidx + qi * tk;
            float mx = -INFINITY;
            for (size_t kj = 0; kj < tk; kj++) {
                float val = t * sr[kj] + rb[ridx[kj]];
                dr[kj] = (d->mask_diag && kj == qi) ? -INFINITY : val;
                if (dr[kj] > mx) mx = dr[kj];
            }
            float sum = 0.0f;
            for (size_t kj = 0; kj < tk; kj++) {
                float e = (dr[kj] == -INFINITY) ? 0.0f : expf(dr[kj] - mx);
                dr[kj] = e;
                sum += e;
            }
            float inv = 1.0f / sum;
            for (size_t kj = 0; kj < tk; kj++) dr[kj] *= inv;
        }
        /* O = P V */
        orc_gemm_small(tq, dh, tk, pr, 0, wv, 0, wo, 0);
        for (size_t qi = 0; qi < tq; qi++) memcpy(oi + qi * c + hd * dh, wo + qi * dh, dh * sizeof(float));
    }
}

void orc_attn_forward(const orc_attn_desc *d, size_t n, const float *q, const float *kv,
                      const float *tau, const float *rel, float *p, float *o) {
    size_t tq = d->tq, tk = d->tk, dh = d->dh;
    int nt = orc_get_threads();
#pragma omp parallel num_threads(nt) if (nt > 1)
    {
        float *wq = (float *)malloc(tq * dh * sizeof(float));
        float *wk = (float *)malloc(tk * dh * sizeof(float));
        float *wv = (float *)malloc(tk * dh * sizeof(float));
        float *ws = (float *)malloc(tq * tk * sizeof(float));
        float *wo = (float *)malloc(tq * dh * sizeof(float));
#pragma omp for schedule(dynamic, 1)
        for (size_t i = 0; i < n; i++) forward_image(d, i, q, kv, tau, rel, p, o, wq, wk, wv, ws, wo);
        free(wq);
        free(wk);
        free(wv);
        free(ws);
        free(wo);
    }
}

/* Core::backward fold body (attn.rs:255-329), one image; at/ar are the fold
 * accumulators for dtau [h] and drel [h*nrel]. */
static void backward_image(const orc_attn_desc *d, size_t i, const float *q, const float *kv,
                           const float *tau, const float *p, const float *dout, float *dq,
                           float *dkv, float *at, float *ar, float *wq, float *wk, float *wv,
                           float *ws, float *wo, float *wdq, float *wdk, float *wdv) {
    size_t h = d->h, dh = d->dh, tq = d->tq, tk = d->tk, c = h * dh, nrel = d->nrel;
    size_t qbase = i * tq * d->qstride, kbase = i * tk * d->kvstride;
    float *dqi = dq + i * tq * d->qstride;
    float *dkvi = dkv + i * tk * d->kvstride;
    const float *doi = dout + i * tq * c;
    const float *pi = p + i * h * tq * tk;
    for (size_t hd = 0; hd < h; hd++) {
        size_t hq = d->qoff + hd * dh, hk = d->koff + hd * dh, hv = d->voff + hd * dh;
        gather(q, qbase, d->qstride, hq, tq, dh, wq);
        gather(kv, kbase, d->kvstride, hk, tk, dh, wk);
        gather(kv, kbase, d->kvstride, hv, tk, dh, wv);
        for (size_t qi = 0; qi < tq; qi++) memcpy(wo + qi * dh, doi + qi * c + hd * dh, dh * sizeof(float));
        const float *pr = pi + hd * tq * tk;

        /* dV = P^T dO */
        orc_gemm_small(tk, dh, tq, pr, 1, wo, 0, wdv, 0);
        scatter_add(dkvi, 0, d->kvstride, hv, tk, dh, wdv);

        /* dP = dO V^T, then the row softmax backward gives dS */
        orc_gemm_small(tq, tk, dh, wo, 0, wv, 1, ws, 0);
        for (size_t qi = 0; qi < tq; qi++) {
            float *sr = ws + qi * tk;
            const float *prr = pr + qi * tk;
            float dot = 0.0f;
            for (size_t kj = 0; kj < tk; kj++) dot += sr[kj] * prr[kj];
            for (size_t kj = 0; kj < tk; kj++) sr[kj] = prr[kj] * (sr[kj] - dot);
        }

        /* dtau needs the raw <q,k>: recomputed (attn.rs:292-308) */
        float t = tau[hd];
        orc_gemm_small(tq, tk, dh, wq, 0, wk, 1, wdq, 0);
        float acc = 0.0f;
        for (size_t z = 0; z < tq * tk; z++) acc += ws[z] * wdq[z];
        at[hd] += acc;
        for (size_t qi = 0; qi < tq; qi++) {
            const float *sr = ws + qi * tk;
            const uint32_t *ridx = d->relidx + qi * tk;
            for (size_t kj = 0; kj < tk; kj++) ar[hd * nrel + ridx[kj]] += sr[kj];
        }
        for (size_t z = 0; z < tq * tk; z++) ws[z] *= t;

        /* dQ = dS K, dK = dS^T Q */
        orc_gemm_small(tq, dh, tk, ws, 0, wk, 0, wdq, 0);
        scatter_add(dqi, 0, d->qstride, hq, tq, dh, wdq);
        orc_gemm_small(tk, dh, tq, ws, 1, wq, 0, wdk, 0);
        scatter_add(dkvi, 0, d->kvstride, hk, tk, dh, wdk);
    }
}

/* Core::backward (attn.rs:226-343): fold per image, reduce the per-leaf
 * dtau/drel, then add into dtau/drel. */
void orc_attn_backward(const orc_attn_desc *d, size_t n, const float *q, const float *kv,
                       const float *tau, const float *p, const float *dout, float *dq, float *dkv,
                       float *dtau, float *drel) {
    size_t h = d->h, dh = d->dh, tq = d->tq, tk = d->tk, nrel = d->nrel;
    size_t lo[256], hi[256];
    int nt = orc_get_threads();
    size_t nl = orc_fold_leaves(n, nt, lo, hi, 256);
    size_t per = h + h * nrel;
    float *accs = (float *)calloc(nl * per + 1, sizeof(float));
#pragma omp parallel for num_threads(nt) schedule(static, 1) if (nt > 1)
    for (size_t l = 0; l < nl; l++) {
        float *at = accs + l * per, *ar = at + h;
        float *wq = (float *)malloc(tq * dh * sizeof(float));
        float *wk = (float *)malloc(tk * dh * sizeof(float));
        float *wv = (float *)malloc(tk * dh * sizeof(float));
        float *ws = (float *)malloc(tq * tk * sizeof(float));
        float *wo = (float *)malloc(tq * dh * sizeof(float));
        /* w.dq doubles as the recomputed-S buffer (attn.rs:296-307). */
        size_t dqn = tq * tk > tq * dh ? tq * tk : tq * dh;
        float *wdq = (float *)malloc(dqn * sizeof(float));
        float *wdk = (float *)malloc(tk * dh * sizeof(float));
        float *wdv = (float *)malloc(tk * dh * sizeof(float));
        for (size_t i = lo[l]; i < hi[l]; i++)
            backward_image(d, i, q, kv, tau, p, dout, dq, dkv, at, ar, wq, wk, wv, ws, wo, wdq, wdk,
                           wdv);
        free(wq);
        free(wk);
        free(wv);
        free(ws);
        free(wo);
        free(wdq);
        free(wdk);
        free(wdv);
    }
    float *red = (float *)calloc(per, sizeof(float));
    for (size_t l = 0; l < nl; l++)
        for (size_t e = 0; e < per; e++) red[e] += accs[l * per + e];
    for (size_t e = 0; e < h; e++) dtau[e] += red[e];
    for (size_t e = 0; e < h * nrel; e++) drel[e] += red[h + e];
    free(red);
    free(accs);
}
