/*
 * orc_nn.c -- restatement of the reference's ResNet layers around the convs
 * (nn.rs:102-110, 253-637): BatchNorm2d train/eval forward and backward with
 * f64 batch statistics, ReLU / residual-add helpers, global average pooling,
 * the scalar nn.rs Linear used as the ResNet classifier, softmax
 * cross-entropy with label smoothing, and the Nesterov SGD step.
 * Test infrastructure only (see orc.h).
 *
 * Every output element is computed by one sequential loop in the reference's
 * order, so the OpenMP split over channels / rows / elements does not change
 * any result.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "orc.h"

/* BatchNorm2d::batch_stats + run_train (nn.rs:297-348).  y [n][c][hw] is
 * normalised in place; xhat and invstd are kept for the backward; rm / rv are
 * updated with the unbiased variance. */
void orc_bn_train_forward(size_t n, size_t c, size_t hw, float *y, const float *gamma,
                          const float *beta, float *rm, float *rv, float *xhat, float *mean_out,
                          float *invstd, float mom, float eps, int relu) {
    const float m = (float)(n * hw);
    float *mean = (float *)malloc((c ? c : 1) * sizeof(float));
    float *var = (float *)malloc((c ? c : 1) * sizeof(float));
#pragma omp parallel for num_threads(orc_get_threads()) schedule(static)
    for (size_t ci = 0; ci < c; ci++) {
        double s = 0.0, s2 = 0.0;
        for (size_t i = 0; i < n; i++) {
            const float *row = y + i * c * hw + ci * hw;
            for (size_t p = 0; p < hw; p++) {
                double v = (double)row[p];
                s += v;
                s2 += v * v;
            }
        }
        double mu = s / (double)m;
        mean[ci] = (float)mu;
        double va = s2 / (double)m - mu * mu;
        var[ci] = (float)(va > 0.0 ? va : 0.0);
    }
    for (size_t ci = 0; ci < c; ci++) {
        invstd[ci] = 1.0f / sqrtf(var[ci] + eps);
        rm[ci] = (1.0f - mom) * rm[ci] + mom * mean[ci];
        float den = m - 1.0f;
        if (den < 1.0f) den = 1.0f;
        float unb = var[ci] * m / den;
        rv[ci] = (1.0f - mom) * rv[ci] + mom * unb;
        if (mean_out) mean_out[ci] = mean[ci];
    }
#pragma omp parallel for num_threads(orc_get_threads()) schedule(static)
    for (size_t idx = 0; idx < n * c; idx++) {
        size_t ci = idx % c;
        float mu = mean[ci], is = invstd[ci], g = gamma[ci], b = beta[ci];
        float *yc = y + idx * hw;
        float *xh = xhat + idx * hw;
        for (size_t p = 0; p < hw; p++) {
            float h = (yc[p] - mu) * is;
            xh[p] = h;
            float v = g * h + b;
            yc[p] = relu ? (v > 0.0f ? v : 0.0f) : v;
        }
    }
    free(mean);
    free(var);
}

/* BatchNorm2d::run_eval (nn.rs:350-365): a per-channel scale and shift. */
void orc_bn_eval_forward(size_t n, size_t c, size_t hw, float *y, const float *gamma,
                         const float *beta, const float *rm, const float *rv, float eps,
                         int relu) {
#pragma omp parallel for num_threads(orc_get_threads()) schedule(static)
    for (size_t idx = 0; idx < n * c; idx++) {
        size_t ci = idx % c;
        float is = 1.0f / sqrtf(rv[ci] + eps);
        float sc = gamma[ci] * is, sh = beta[ci] - gamma[ci] * is * rm[ci];
        float *yc = y + idx * hw;
        for (size_t p = 0; p < hw; p++) {
            float v = sc * yc[p] + sh;
            yc[p] = relu ? (v > 0.0f ? v : 0.0f) : v;
        }
    }
}

/* BatchNorm2d::backward (nn.rs:379-425): dx overwritten, dgamma / dbeta
 * accumulate (g.g += , b.g +=). */
void orc_bn_backward(size_t n, size_t c, size_t hw, const float *dy, const float *xhat,
                     const float *gamma, const float *invstd, float *dx, float *dgamma,
                     float *dbeta) {
    const float m = (float)(n * hw);
    float *dg = (float *)malloc((c ? c : 1) * sizeof(float));
    float *db = (float *)malloc((c ? c : 1) * sizeof(float));
#pragma omp parallel for num_threads(orc_get_threads()) schedule(static)
    for (size_t ci = 0; ci < c; ci++) {
        float a = 0.0f, b = 0.0f;
        for (size_t i = 0; i < n; i++) {
            size_t base = i * c * hw + ci * hw;
            for (size_t p = 0; p < hw; p++) {
                a += dy[base + p] * xhat[base + p];
                b += dy[base + p];
            }
        }
        dg[ci] = a;
        db[ci] = b;
    }
#pragma omp parallel for num_threads(orc_get_threads()) schedule(static)
    for (size_t idx = 0; idx < n * c; idx++) {
        size_t ci = idx % c;
        float s = gamma[ci] * invstd[ci] / m;
        const float *dyc = dy + idx * hw, *xh = xhat + idx * hw;
        float *dxc = dx + idx * hw;
        for (size_t p = 0; p < hw; p++) dxc[p] = s * (m * dyc[p] - db[ci] - xh[p] * dg[ci]);
    }
    for (size_t ci = 0; ci < c; ci++) {
        dgamma[ci] += dg[ci];
        dbeta[ci] += db[ci];
    }
    free(dg);
    free(db);
}

/* relu_back_ (nn.rs:432-439): d = 0 where y <= 0. */
void orc_relu_back(size_t len, float *d, const float *y) {
#pragma omp parallel for num_threads(orc_get_threads()) schedule(static)
    for (size_t i = 0; i < len; i++)
        if (y[i] <= 0.0f) d[i] = 0.0f;
}

/* add_ (nn.rs:441-443). */
void orc_add(size_t len, float *a, const float *b) {
#pragma omp parallel for num_threads(orc_get_threads()) schedule(static)
    for (size_t i = 0; i < len; i++) a[i] += b[i];
}

/* add_relu_ (nn.rs:446-450). */
void orc_add_relu(size_t len, float *a, const float *b) {
#pragma omp parallel for num_threads(orc_get_threads()) schedule(static)
    for (size_t i = 0; i < len; i++) {
        float v = a[i] + b[i];
        a[i] = v > 0.0f ? v : 0.0f;
    }
}

/* gap_forward (nn.rs:455-463): sequential f32 sum of each plane / hw. */
void orc_gap_forward(size_t nc, size_t hw, const float *x, float *y) {
#pragma omp parallel for num_threads(orc_get_threads()) schedule(static)
    for (size_t i = 0; i < nc; i++) {
        float s = 0.0f;
        for (size_t p = 0; p < hw; p++) s += x[i * hw + p];
        y[i] = s / (float)hw;
    }
}

/* gap_backward (nn.rs:465-473). */
void orc_gap_backward(size_t nc, size_t hw, const float *dy, float *dx) {
#pragma omp parallel for num_threads(orc_get_threads()) schedule(static)
    for (size_t i = 0; i < nc; i++) {
        float v = dy[i] / (float)hw;
        for (size_t p = 0; p < hw; p++) dx[i * hw + p] = v;
    }
}

/* nn.rs Linear::forward (nn.rs:500-517): y[i][o] = b[o] + sum_j w[o][j] x[i][j]
 * as one unfused sequential chain starting from the bias. */
void orc_fc_forward(size_t rows, size_t fin, size_t fout, const float *x, const float *w,
                    const float *b, float *y) {
#pragma omp parallel for num_threads(orc_get_threads()) schedule(static)
    for (size_t i = 0; i < rows; i++)
        for (size_t o = 0; o < fout; o++) {
            const float *wr = w + o * fin, *xr = x + i * fin;
            float s = b[o];
            for (size_t j = 0; j < fin; j++) s += wr[j] * xr[j];
            y[i * fout + o] = s;
        }
}

/* nn.rs Linear::backward_w + backward_x (nn.rs:519-564).  dw, db accumulate
 * over rows in row order (zero gradients skipped, as the reference does);
 * dx [rows][fin] is overwritten. */
void orc_fc_backward(size_t rows, size_t fin, size_t fout, const float *dy, const float *x,
                     const float *w, float *dw, float *db, float *dx) {
#pragma omp parallel for num_threads(orc_get_threads()) schedule(static)
    for (size_t o = 0; o < fout; o++) {
        for (size_t i = 0; i < rows; i++) {
            float g = dy[i * fout + o];
            if (g == 0.0f) continue;
            db[o] += g;
            float *wg = dw + o * fin;
            const float *xr = x + i * fin;
            for (size_t j = 0; j < fin; j++) wg[j] += g * xr[j];
        }
    }
#pragma omp parallel for num_threads(orc_get_threads()) schedule(static)
    for (size_t i = 0; i < rows; i++) {
        float *dxr = dx + i * fin;
        for (size_t j = 0; j < fin; j++) dxr[j] = 0.0f;
        for (size_t o = 0; o < fout; o++) {
            float g = dy[i * fout + o];
            if (g == 0.0f) continue;
            const float *wr = w + o * fin;
            for (size_t j = 0; j < fin; j++) dxr[j] += g * wr[j];
        }
    }
}

/* softmax_ce (nn.rs:566-637): mean loss over rows, number of rows whose first
 * maximal logit is the label, and dlogits already divided by the batch. */
float orc_softmax_ce(size_t rows, size_t nclass, const float *logits, const uint32_t *labels,
                     float smooth, float *dlogits, size_t *correct) {
    const float inv = 1.0f / (float)rows;
    float loss = 0.0f;
    size_t ok = 0;
    for (size_t i = 0; i < rows; i++) {
        const float *z = logits + i * nclass;
        float *d = dlogits + i * nclass;
        size_t y = labels[i];
        float mx = -INFINITY;
        size_t arg = 0;
        for (size_t j = 0; j < nclass; j++)
            if (z[j] > mx) {
                mx = z[j];
                arg = j;
            }
        if (arg == y) ok++;
        float sum = 0.0f;
        for (size_t j = 0; j < nclass; j++) {
            float e = expf(z[j] - mx);
            d[j] = e;
            sum += e;
        }
        float lse = mx + logf(sum);
        float on = 1.0f - smooth, off = smooth / (float)nclass;
        float l = on * (lse - z[y]);
        if (smooth > 0.0f) {
            float s = 0.0f;
            for (size_t j = 0; j < nclass; j++) s += lse - z[j];
            l += off * s;
        }
        for (size_t j = 0; j < nclass; j++) {
            float t = j == y ? on + off : off;
            d[j] = (d[j] / sum - t) * inv;
        }
        loss += l;
    }
    if (correct) *correct = ok;
    return loss * inv;
}

/* Param::step (nn.rs:102-110): Nesterov SGD with weight decay added to the
 * gradient; the gradient is zeroed. */
void orc_sgd_step(size_t len, float *v, float *g, float *m, float lr, float mom, float wd) {
#pragma omp parallel for num_threads(orc_get_threads()) schedule(static)
    for (size_t i = 0; i < len; i++) {
        float gi = g[i] + wd * v[i];
        m[i] = mom * m[i] + gi;
        v[i] -= lr * (gi + mom * m[i]);
        g[i] = 0.0f;
    }
}
