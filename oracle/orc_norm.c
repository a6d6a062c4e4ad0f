/*
 * orc_norm.c -- CPU oracle: norm.rs (LayerNorm, LayerScale, the SwiGLU gate,
 * the depthwise 3x3 convolution, SeqPool) over token tensors [rows][c].
 * TEST INFRASTRUCTURE ONLY (see orc.h).
 *
 * Each function restates the reference's loops in its order: per-row and
 * per-element arithmetic is sequential as written there (f32, no
 * contraction; LayerNorm statistics in f64).  The reference's channel
 * reductions (dgamma / dbeta, dlambda, dW / db, dp) are rayon fold + reduce
 * over rows or images, whose split is unspecified; here they run in row
 * (image) order in one f32 accumulator -- "parity unpinned" for that order.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "orc.h"

/* LayerNorm::forward (norm.rs:38-85).  xhat / invstd may be NULL (eval). */
void orc_ln_forward(size_t rows, size_t c, const float *x, const float *g, const float *b,
                    float eps, float *y, float *xhat, float *invstd) {
    for (size_t r = 0; r < rows; r++) {
        const float *xr = x + r * c;
        double s = 0.0, s2 = 0.0;
        for (size_t j = 0; j < c; j++) {
            s += (double)xr[j];
            s2 += (double)xr[j] * (double)xr[j];
        }
        const double m = (double)c;
        const double mu = s / m;
        double v = s2 / m - mu * mu;
        const float var = (float)(v > 0.0 ? v : 0.0);
        const float i = 1.0f / sqrtf(var + eps);
        if (invstd) invstd[r] = i;
        for (size_t j = 0; j < c; j++) {
            const float h = (xr[j] - (float)mu) * i;
            if (xhat) xhat[r * c + j] = h;
            y[r * c + j] = g[j] * h + b[j];
        }
    }
}

/* LayerNorm::backward (norm.rs:87-137): dg += sum dy xhat, db += sum dy;
 * dx = invstd (d - m1/c - xhat m2/c) with d = dy g. */
void orc_ln_backward(size_t rows, size_t c, const float *dy, const float *xhat,
                     const float *invstd, const float *g, float *dx, float *dg, float *db) {
    float *ag = calloc(c ? c : 1, sizeof(float)), *ab = calloc(c ? c : 1, sizeof(float));
    for (size_t r = 0; r < rows; r++)
        for (size_t j = 0; j < c; j++) {
            ag[j] += dy[r * c + j] * xhat[r * c + j];
            ab[j] += dy[r * c + j];
        }
    for (size_t j = 0; j < c; j++) {
        dg[j] += ag[j];
        db[j] += ab[j];
    }
    free(ag);
    free(ab);
    for (size_t r = 0; r < rows; r++) {
        const float *dr = dy + r * c, *xh = xhat + r * c;
        float m1 = 0.0f, m2 = 0.0f;
        for (size_t j = 0; j < c; j++) {
            const float d = dr[j] * g[j];
            m1 += d;
            m2 += d * xh[j];
        }
        const float inv = 1.0f / (float)c;
        for (size_t j = 0; j < c; j++) {
            const float d = dr[j] * g[j];
            dx[r * c + j] = invstd[r] * (d - m1 * inv - xh[j] * m2 * inv);
        }
    }
}

/* LayerScale::forward / backward (norm.rs:166-212). */
void orc_layerscale_forward(size_t rows, size_t c, const float *x, const float *l, float *y) {
    for (size_t r = 0; r < rows; r++)
        for (size_t j = 0; j < c; j++) y[r * c + j] = x[r * c + j] * l[j];
}

void orc_layerscale_backward(size_t rows, size_t c, const float *dy, const float *x,
                             const float *l, float *dx, float *dl) {
    float *a = calloc(c ? c : 1, sizeof(float));
    for (size_t r = 0; r < rows; r++)
        for (size_t j = 0; j < c; j++) a[j] += dy[r * c + j] * x[r * c + j];
    for (size_t j = 0; j < c; j++) dl[j] += a[j];
    free(a);
    for (size_t r = 0; r < rows; r++)
        for (size_t j = 0; j < c; j++) dx[r * c + j] = dy[r * c + j] * l[j];
}

static float sigmoidf_(float z) { return 1.0f / (1.0f + expf(-z)); }

/* SwiGlu's gate (norm.rs:255-262, 276-287). */
void orc_swiglu_forward(size_t rows, size_t h, const float *ab, float *u) {
    for (size_t r = 0; r < rows; r++)
        for (size_t j = 0; j < h; j++) {
            const float a = ab[r * 2 * h + j];
            u[r * h + j] = a * sigmoidf_(a) * ab[r * 2 * h + h + j];
        }
}

void orc_swiglu_backward(size_t rows, size_t h, const float *du, const float *ab, float *dab) {
    for (size_t r = 0; r < rows; r++)
        for (size_t j = 0; j < h; j++) {
            const float a = ab[r * 2 * h + j], b = ab[r * 2 * h + h + j];
            const float s = sigmoidf_(a);
            const float sa = a * s;
            const float d = du[r * h + j];
            dab[r * 2 * h + j] = d * b * s * (1.0f + a * (1.0f - s));
            dab[r * 2 * h + h + j] = d * sa;
        }
}

/* DwConv3::forward (norm.rs:338-375): y = b, then y += w[tap] x[src] over
 * the in-bounds taps in (ky, kx) order. */
void orc_dwconv3_forward(size_t n, size_t th, size_t tw, size_t c, const float *x,
                         const float *w, const float *b, float *y) {
    const size_t img = th * tw * c;
    for (size_t i = 0; i < n; i++) {
        const float *xi = x + i * img;
        float *yi = y + i * img;
        for (size_t oy = 0; oy < th; oy++)
            for (size_t ox = 0; ox < tw; ox++) {
                float *dst = yi + (oy * tw + ox) * c;
                memcpy(dst, b, c * sizeof(float));
                for (int ky = 0; ky < 3; ky++) {
                    const long sy = (long)oy + ky - 1;
                    if (sy < 0 || sy >= (long)th) continue;
                    for (int kx = 0; kx < 3; kx++) {
                        const long sx = (long)ox + kx - 1;
                        if (sx < 0 || sx >= (long)tw) continue;
                        const float *wr = w + (size_t)(ky * 3 + kx) * c;
                        const float *src = xi + ((size_t)sy * tw + (size_t)sx) * c;
                        for (size_t j = 0; j < c; j++) dst[j] += wr[j] * src[j];
                    }
                }
            }
    }
}

/* DwConv3::backward (norm.rs:377-452): dw [9][c] += sum dy x[src] and
 * db += sum dy over images, positions and taps in that order; dx scattered
 * from each output position's taps in raster order (dx is overwritten). */
void orc_dwconv3_backward(size_t n, size_t th, size_t tw, size_t c, const float *dy,
                          const float *x, const float *w, float *dx, float *dw, float *db) {
    const size_t img = th * tw * c;
    float *aw = calloc(c ? 9 * c : 1, sizeof(float)), *ab = calloc(c ? c : 1, sizeof(float));
    memset(dx, 0, n * img * sizeof(float));
    for (size_t i = 0; i < n; i++) {
        const float *dyi = dy + i * img, *xi = x + i * img;
        float *dxi = dx + i * img;
        for (size_t oy = 0; oy < th; oy++)
            for (size_t ox = 0; ox < tw; ox++) {
                const float *d = dyi + (oy * tw + ox) * c;
                for (size_t j = 0; j < c; j++) ab[j] += d[j];
                for (int ky = 0; ky < 3; ky++) {
                    const long sy = (long)oy + ky - 1;
                    if (sy < 0 || sy >= (long)th) continue;
                    for (int kx = 0; kx < 3; kx++) {
                        const long sx = (long)ox + kx - 1;
                        if (sx < 0 || sx >= (long)tw) continue;
                        const size_t s = ((size_t)sy * tw + (size_t)sx) * c;
                        float *acc = aw + (size_t)(ky * 3 + kx) * c;
                        const float *wr = w + (size_t)(ky * 3 + kx) * c;
                        for (size_t j = 0; j < c; j++) {
                            acc[j] += d[j] * xi[s + j];
                            dxi[s + j] += wr[j] * d[j];
                        }
                    }
                }
            }
    }
    for (size_t j = 0; j < 9 * c; j++) dw[j] += aw[j];
    for (size_t j = 0; j < c; j++) db[j] += ab[j];
    free(aw);
    free(ab);
}

/* SeqPool::forward (norm.rs:487-528): z [n][c]; w [n][t] the softmax weights. */
void orc_seqpool_forward(size_t n, size_t t, size_t c, const float *x, const float *p, float *z,
                         float *w) {
    for (size_t i = 0; i < n; i++) {
        const float *xi = x + i * t * c;
        float *wi = w + i * t, *zi = z + i * c;
        float mx = -INFINITY;
        for (size_t j = 0; j < t; j++) {
            float s = 0.0f;
            for (size_t k = 0; k < c; k++) s += xi[j * c + k] * p[k];
            wi[j] = s;
            if (s > mx) mx = s;
        }
        float sum = 0.0f;
        for (size_t j = 0; j < t; j++) {
            wi[j] = expf(wi[j] - mx);
            sum += wi[j];
        }
        const float inv = 1.0f / sum;
        for (size_t k = 0; k < c; k++) zi[k] = 0.0f;
        for (size_t j = 0; j < t; j++) {
            wi[j] *= inv;
            for (size_t k = 0; k < c; k++) zi[k] += wi[j] * xi[j * c + k];
        }
    }
}

/* SeqPool::backward (norm.rs:530-580): dx overwritten, dp += sum over images. */
void orc_seqpool_backward(size_t n, size_t t, size_t c, const float *dz, const float *w,
                          const float *x, const float *p, float *dx, float *dp) {
    float *adp = calloc(c ? c : 1, sizeof(float)), *dw = malloc((t ? t : 1) * sizeof(float));
    memset(dx, 0, n * t * c * sizeof(float));
    for (size_t i = 0; i < n; i++) {
        const float *xi = x + i * t * c, *dzi = dz + i * c, *wi = w + i * t;
        float *dxi = dx + i * t * c;
        float dot = 0.0f;
        for (size_t j = 0; j < t; j++) {
            float s = 0.0f;
            for (size_t k = 0; k < c; k++) {
                s += dzi[k] * xi[j * c + k];
                dxi[j * c + k] += wi[j] * dzi[k];
            }
            dw[j] = s;
            dot += s * wi[j];
        }
        for (size_t j = 0; j < t; j++) {
            const float ds = wi[j] * (dw[j] - dot);
            for (size_t k = 0; k < c; k++) {
                adp[k] += ds * xi[j * c + k];
                dxi[j * c + k] += ds * p[k];
            }
        }
    }
    for (size_t k = 0; k < c; k++) dp[k] += adp[k];
    free(adp);
    free(dw);
}
