/*
 * orc_optim.c -- CPU oracle: optim.rs (Muon with Newton-Schulz, AdamW,
 * global-norm clip, weight EMA).  TEST INFRASTRUCTURE ONLY (see orc.h).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "orc.h"

/* Quintic coefficients (optim.rs:22-26). */
#define NS_A 3.4445f
#define NS_B (-4.7750f)
#define NS_C 2.0315f

/* f32::powi with a run-time exponent: LLVM lowers it to compiler-rt's
 * __powisf2, square-and-multiply from the low bit (published algorithm). */
float orc_powi(float a, int b) {
    const int recip = b < 0;
    float r = 1.0f;
    for (;;) {
        if (b & 1) r *= a;
        b /= 2;
        if (b == 0) break;
        a *= a;
    }
    return recip ? 1.0f / r : r;
}

/* newton_schulz (optim.rs:124-145) with load_maybe_t / store_maybe_t
 * (optim.rs:41-65) and NsScratch::quintic_step (optim.rs:67-121): X = G (or
 * G^T when rows > cols) / (||G||_F + 1e-7), with the squared norm summed in
 * f32 in element order; then `steps` times A = X X^T, AA = A A,
 * B = b A + c AA, X = a X + B X, every product through gemm_small. */
void orc_newton_schulz(float *g, size_t rows, size_t cols, size_t steps) {
    const int tr = rows > cols;
    const size_t m = tr ? cols : rows, n = tr ? rows : cols;
    float *x = malloc(m * n * sizeof(float)), *a = malloc(m * m * sizeof(float));
    float *aa = malloc(m * m * sizeof(float)), *t = malloc(m * n * sizeof(float));
    if (!tr) {
        memcpy(x, g, m * n * sizeof(float));
    } else {
        for (size_t i = 0; i < rows; i++)
            for (size_t j = 0; j < cols; j++) x[j * rows + i] = g[i * cols + j];
    }
    float ss = 0.0f;
    for (size_t i = 0; i < m * n; i++) ss += x[i] * x[i];
    const float norm = sqrtf(ss) + 1e-7f;
    const float inv = 1.0f / norm;
    for (size_t i = 0; i < m * n; i++) x[i] *= inv;
    for (size_t s = 0; s < steps; s++) {
        orc_gemm_small(m, m, n, x, 0, x, 1, a, 0);
        orc_gemm_small(m, m, m, a, 0, a, 0, aa, 0);
        for (size_t i = 0; i < m * m; i++) a[i] = NS_B * a[i] + NS_C * aa[i];
        orc_gemm_small(m, n, m, a, 0, x, 0, t, 0);
        for (size_t i = 0; i < m * n; i++) x[i] = NS_A * x[i] + t[i];
    }
    if (!tr) {
        memcpy(g, x, m * n * sizeof(float));
    } else {
        for (size_t i = 0; i < rows; i++)
            for (size_t j = 0; j < cols; j++) g[i * cols + j] = x[j * rows + i];
    }
    free(x);
    free(a);
    free(aa);
    free(t);
}

/* The Muon branch of Optim::step_all for one [rows x cols] parameter
 * (optim.rs:182-195): Nesterov momentum into g, Newton-Schulz, then
 * v -= lr * (0.2 sqrt(max(rows, cols)) g + wd v) with wd only when the
 * parameter decays; g is zeroed. */
void orc_muon_step(float *v, float *g, float *m, size_t rows, size_t cols, int decay, float lr,
                   float wd, float mom, size_t ns_steps) {
    const size_t n = rows * cols;
    const float wdp = decay ? wd : 0.0f;
    for (size_t i = 0; i < n; i++) {
        m[i] = mom * m[i] + g[i];
        g[i] += mom * m[i];
    }
    orc_newton_schulz(g, rows, cols, ns_steps);
    const float scale = 0.2f * sqrtf((float)(rows > cols ? rows : cols));
    for (size_t i = 0; i < n; i++) {
        v[i] -= lr * (scale * g[i] + wdp * v[i]);
        g[i] = 0.0f;
    }
}

/* The Muon branch of Optim::step_all over a list of parameters, which the
 * reference runs as a rayon par_iter over the parameters (optim.rs:177-196):
 * one OpenMP loop over the matrices, each updated by orc_muon_step on one
 * thread (the GEMM regions inside are nested, so they run serially).  The
 * updates touch disjoint arrays, so the result equals orc_muon_step called
 * per matrix in any order.  Used to time the CPU baseline. */
void orc_muon_steps(size_t nmat, float *const *v, float *const *g, float *const *m,
                    const size_t *rows, const size_t *cols, const int *decay, float lr, float wd,
                    float mom, size_t ns_steps, int threads) {
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1) if (threads > 1)
    for (size_t i = 0; i < nmat; i++)
        orc_muon_step(v[i], g[i], m[i], rows[i], cols[i], decay[i], lr, wd, mom, ns_steps);
}

/* Optim::step_adam (optim.rs:207-235) at step count t (the step uses t + 1
 * for the bias corrections; the caller increments t after the whole step). */
void orc_adam_step(size_t n, float *v, float *g, float *m, float *v2, int decay, float lr,
                   float wd, float b1, float b2, float eps, size_t t) {
    const float wdd = decay ? wd : 0.0f;
    const float c1 = 1.0f - orc_powi(b1, (int)t + 1);
    const float c2 = 1.0f - orc_powi(b2, (int)t + 1);
    for (size_t i = 0; i < n; i++) {
        m[i] = b1 * m[i] + (1.0f - b1) * g[i];
        v2[i] = b2 * v2[i] + (1.0f - b2) * g[i] * g[i];
        v[i] -= lr * ((m[i] / c1) / (sqrtf(v2[i] / c2) + eps) + wdd * v[i]);
        g[i] = 0.0f;
    }
}

/* clip_ (optim.rs:237-251) over nseg gradient tensors laid end to end in g:
 * the f64 sum of squares per tensor, in element order, then over tensors in
 * order (the reference's rayon sums add the same terms in an unspecified
 * order); norm = sqrt as f32; above `max` every gradient is scaled by
 * max / norm.  Returns the norm. */
float orc_clip(float *g, const size_t *lens, size_t nseg, float max) {
    double sq = 0.0;
    size_t off = 0;
    for (size_t s = 0; s < nseg; s++) {
        double p = 0.0;
        for (size_t i = 0; i < lens[s]; i++) p += (double)g[off + i] * (double)g[off + i];
        sq += p;
        off += lens[s];
    }
    const float norm = (float)sqrt(sq);
    if (norm > max && norm > 0.0f) {
        const float sc = max / norm;
        for (size_t i = 0; i < off; i++) g[i] *= sc;
    }
    return norm;
}

/* Ema::update (optim.rs:270-288) after the first call: t is the update count
 * including this one; d = min(decay, (1 + t) / (10 + t)); w = d w + (1 - d) v. */
void orc_ema_update(size_t n, float *w, const float *v, float decay, size_t t) {
    const float ceil_d = (1.0f + (float)t) / (10.0f + (float)t);
    const float d = decay < ceil_d ? decay : ceil_d;
    for (size_t i = 0; i < n; i++) w[i] = d * w[i] + (1.0f - d) * v[i];
}

/* lr_at (train.rs:21-28): linear warm-up, then a cosine to lo; f32 with the
 * C library's cosf (Rust's f32::cos on linux-gnu). */
float orc_lr_at(float peak, float lo, size_t step, size_t total, size_t warm) {
    if (warm > 0 && step < warm) return lo + (peak - lo) * (float)(step + 1) / (float)warm;
    const size_t span = total > warm ? total - warm : 1;
    const float t = (float)(step - warm) / (float)span;
    return lo + 0.5f * (peak - lo) * (1.0f + cosf(3.14159265358979323846f * t));
}
