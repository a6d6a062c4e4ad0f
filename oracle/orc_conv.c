/*
 * orc_conv.c -- restatement of the reference implicit-GEMM convolution
 * (conv.rs) and of the Conv2d batch drivers (nn.rs:113-250).  Test
 * infrastructure only (see orc.h).
 */
#include <stdlib.h>
#include <string.h>

#include "orc.h"

#define MR ORC_MR
#define NR ORC_NR
#define KC ORC_KC

static inline size_t div_ceil(size_t a, size_t b) { return (a + b - 1) / b; }
static inline size_t min_sz(size_t a, size_t b) { return a < b ? a : b; }

/* Conv2d::out_dim / spec (nn.rs:147-164). */
void orc_conv_spec_init(orc_conv_spec *sp, uint32_t cin, uint32_t cout, uint32_t k,
                        uint32_t stride, uint32_t pad, uint32_t h, uint32_t w) {
    sp->cin = cin;
    sp->cout = cout;
    sp->k = k;
    sp->stride = stride;
    sp->pad = pad;
    sp->h = h;
    sp->w = w;
    sp->oh = (h + 2 * pad - k) / stride + 1;
    sp->ow = (w + 2 * pad - k) / stride + 1;
}

static inline size_t ckk_of(const orc_conv_spec *sp) { return (size_t)sp->cin * sp->k * sp->k; }
static inline size_t hw_of(const orc_conv_spec *sp) { return (size_t)sp->oh * sp->ow; }

/* RowMap::new (conv.rs:49-59): row r = ci*k*k + kh*k + kw. */
void orc_rowmap(const orc_conv_spec *sp, uint32_t *out) {
    size_t r = 0;
    for (uint32_t ci = 0; ci < sp->cin; ci++)
        for (uint32_t kh = 0; kh < sp->k; kh++)
            for (uint32_t kw = 0; kw < sp->k; kw++, r++) {
                out[3 * r + 0] = ci;
                out[3 * r + 1] = kh;
                out[3 * r + 2] = kw;
            }
}

static inline void rm_get(const orc_conv_spec *sp, size_t r, size_t *ci, size_t *kh, size_t *kw) {
    size_t kk = (size_t)sp->k * sp->k;
    *ci = r / kk;
    *kh = (r % kk) / sp->k;
    *kw = r % sp->k;
}

/* gather_span (conv.rs:68-120): dst[t] = X[ci, oy*s+kh-pad, ox*s+kw-pad] for
 * the n output pixels starting at (oy0, ox0), 0 outside the image. */
static void gather_span(const float *x, size_t ci, size_t kh, size_t kw, const orc_conv_spec *sp,
                        size_t oy0, size_t ox0, size_t n, float *dst) {
    size_t h = sp->h, w = sp->w, ow = sp->ow, stride = sp->stride, pad = sp->pad;
    size_t base = ci * h * w;
    size_t oy = oy0, ox = ox0, t = 0;
    while (t < n) {
        size_t len = min_sz(n - t, ow - ox);
        size_t iy = oy * stride + kh;
        if (iy < pad || iy >= h + pad) {
            for (size_t u = 0; u < len; u++) dst[t + u] = 0.0f;
        } else {
            size_t rb = base + (iy - pad) * w;
            if (stride == 1) {
                size_t a = kw + ox;
                size_t lo = pad > a ? pad - a : 0;
                if (lo > len) lo = len;
                size_t hi = (w + pad) > a ? (w + pad) - a : 0;
                if (hi > len) hi = len;
                for (size_t u = 0; u < lo; u++) dst[t + u] = 0.0f;
                if (hi > lo) {
                    size_t s = rb + ox + kw + lo - pad;
                    memcpy(dst + t + lo, x + s, (hi - lo) * sizeof(float));
                }
                for (size_t u = (hi > lo ? hi : lo); u < len; u++) dst[t + u] = 0.0f;
            } else {
                for (size_t u = 0; u < len; u++) {
                    size_t ix = (ox + u) * stride + kw;
                    dst[t + u] = (ix < pad || ix >= w + pad) ? 0.0f : x[rb + ix - pad];
                }
            }
        }
        t += len;
        oy += 1;
        ox = 0;
    }
}

/* scatter_span (conv.rs:122-166): col2im accumulate. */
static void scatter_span(float *dx, size_t ci, size_t kh, size_t kw, const orc_conv_spec *sp,
                         size_t oy0, size_t ox0, size_t n, const float *src) {
    size_t h = sp->h, w = sp->w, ow = sp->ow, stride = sp->stride, pad = sp->pad;
    size_t base = ci * h * w;
    size_t oy = oy0, ox = ox0, t = 0;
    while (t < n) {
        size_t len = min_sz(n - t, ow - ox);
        size_t iy = oy * stride + kh;
        if (iy >= pad && iy < h + pad) {
            size_t rb = base + (iy - pad) * w;
            if (stride == 1) {
                size_t a = kw + ox;
                size_t lo = pad > a ? pad - a : 0;
                if (lo > len) lo = len;
                size_t hi = (w + pad) > a ? (w + pad) - a : 0;
                if (hi > len) hi = len;
                if (hi > lo) {
                    size_t s0 = rb + ox + kw + lo - pad;
                    for (size_t u = 0; u < hi - lo; u++) dx[s0 + u] += src[t + lo + u];
                }
            } else {
                for (size_t u = 0; u < len; u++) {
                    size_t ix = (ox + u) * stride + kw;
                    if (ix >= pad && ix < w + pad) dx[rb + ix - pad] += src[t + u];
                }
            }
        }
        t += len;
        oy += 1;
        ox = 0;
    }
}

/* Debug: full im2col matrix [ckk x hw] of one image, row by row through
 * gather_span (the reference never materialises it; this is the bit-exact
 * definition the GPU staging loads are checked against). */
void orc_im2col(const orc_conv_spec *sp, const float *x, float *col) {
    size_t ckk = ckk_of(sp), hw = hw_of(sp);
    for (size_t r = 0; r < ckk; r++) {
        size_t ci, kh, kw;
        rm_get(sp, r, &ci, &kh, &kw);
        gather_span(x, ci, kh, kw, sp, 0, 0, hw, col + r * hw);
    }
}

/* forward_image (conv.rs:168-203) with W already packed (wpack = PackedA of
 * W [cout x ckk]).  bp is a KC*NR panel. */
static void forward_image_packed(const orc_conv_spec *sp, const float *wpack, const float *x,
                                 float *y, float *bp) {
    size_t ckk = ckk_of(sp), hw = hw_of(sp);
    size_t mpan = div_ceil(sp->cout, MR), mpad = mpan * MR;
    size_t q = 0;
    for (size_t pc = 0; pc < ckk; pc += KC, q++) {
        size_t kc = min_sz(KC, ckk - pc);
        for (size_t j = 0; j < hw; j += NR) {
            size_t nr = min_sz(NR, hw - j);
            size_t oy = j / sp->ow, ox = j % sp->ow;
            for (size_t p = 0; p < kc; p++) {
                size_t ci, kh, kw;
                rm_get(sp, pc + p, &ci, &kh, &kw);
                float *dst = bp + p * NR;
                for (size_t t = nr; t < NR; t++) dst[t] = 0.0f;
                gather_span(x, ci, kh, kw, sp, oy, ox, nr, dst);
            }
            for (size_t i = 0; i < mpan; i++) {
                size_t mr = min_sz(sp->cout - i * MR, MR);
                size_t off = i * MR * hw + j;
                orc_micro_kernel(kc, wpack + q * KC * mpad + i * kc * MR, bp, y + off, hw, mr, nr,
                                 q > 0);
            }
        }
    }
}

/* dx_image (conv.rs:205-246) with W^T packed (wtpack = PackedA::pack_t of W,
 * m = ckk, k = cout). */
static void dx_image_packed(const orc_conv_spec *sp, const float *wtpack, const float *dy,
                            float *dx, float *bp, float *tile) {
    size_t ckk = ckk_of(sp), hw = hw_of(sp);
    size_t mpan = div_ceil(ckk, MR), mpad = mpan * MR;
    memset(dx, 0, (size_t)sp->cin * sp->h * sp->w * sizeof(float));
    size_t q = 0;
    for (size_t pc = 0; pc < sp->cout; pc += KC, q++) {
        size_t kc = min_sz(KC, sp->cout - pc);
        for (size_t j = 0; j < hw; j += NR) {
            size_t nr = min_sz(NR, hw - j);
            size_t oy = j / sp->ow, ox = j % sp->ow;
            for (size_t p = 0; p < kc; p++) {
                const float *src = dy + (pc + p) * hw + j;
                float *dst = bp + p * NR;
                memcpy(dst, src, nr * sizeof(float));
                for (size_t t = nr; t < NR; t++) dst[t] = 0.0f;
            }
            for (size_t i = 0; i < mpan; i++) {
                size_t mr = min_sz(MR, ckk - i * MR);
                orc_micro_kernel(kc, wtpack + q * KC * mpad + i * kc * MR, bp, tile, NR, mr, nr, 0);
                for (size_t r = 0; r < mr; r++) {
                    size_t ci, kh, kw;
                    rm_get(sp, i * MR + r, &ci, &kh, &kw);
                    scatter_span(dx, ci, kh, kw, sp, oy, ox, nr, tile + r * NR);
                }
            }
        }
    }
}

/* pack_colt (conv.rs:248-275): tmp is NR*KC, bp is KC*NR. */
static void pack_colt(const orc_conv_spec *sp, const float *x, size_t pc, size_t kc, size_t j,
                      size_t nr, float *tmp, float *bp) {
    size_t oy = pc / sp->ow, ox = pc % sp->ow;
    for (size_t t = 0; t < nr; t++) {
        size_t ci, kh, kw;
        rm_get(sp, j + t, &ci, &kh, &kw);
        gather_span(x, ci, kh, kw, sp, oy, ox, kc, tmp + t * KC);
    }
    for (size_t t = nr; t < NR; t++) memset(tmp + t * KC, 0, kc * sizeof(float));
    orc_transpose_to_panel(tmp, KC, kc, bp);
}

/* dw_image (conv.rs:277-322): dW[cout x ckk] += dY im2col(X)^T.  dypack holds
 * orc_packed_a_len(cout, hw) floats. */
static void dw_image_ws(const orc_conv_spec *sp, float *dypack, const float *dy, const float *x,
                        float *dw, float *tmp, float *bp) {
    size_t ckk = ckk_of(sp), hw = hw_of(sp);
    size_t mpan = div_ceil(sp->cout, MR), mpad = mpan * MR;
    orc_pack_a(dy, sp->cout, hw, 0, dypack);
    size_t q = 0;
    for (size_t pc = 0; pc < hw; pc += KC, q++) {
        size_t kc = min_sz(KC, hw - pc);
        for (size_t j = 0; j < ckk; j += NR) {
            size_t nr = min_sz(NR, ckk - j);
            pack_colt(sp, x, pc, kc, j, nr, tmp, bp);
            for (size_t i = 0; i < mpan; i++) {
                size_t mr = min_sz(MR, sp->cout - i * MR);
                orc_micro_kernel(kc, dypack + q * KC * mpad + i * kc * MR, bp,
                                 dw + i * MR * ckk + j, ckk, mr, nr, 1);
            }
        }
    }
}

void orc_conv_forward_image(const orc_conv_spec *sp, const float *x, const float *w, float *y) {
    size_t ckk = ckk_of(sp);
    float *wpack = (float *)calloc(orc_packed_a_len(sp->cout, ckk), sizeof(float));
    float *bp = (float *)calloc(KC * NR, sizeof(float));
    orc_pack_a(w, sp->cout, ckk, 0, wpack);
    forward_image_packed(sp, wpack, x, y, bp);
    free(bp);
    free(wpack);
}

void orc_conv_dx_image(const orc_conv_spec *sp, const float *dy, const float *w, float *dx) {
    size_t ckk = ckk_of(sp);
    float *wtpack = (float *)calloc(orc_packed_a_len(ckk, sp->cout), sizeof(float));
    float *bp = (float *)calloc(KC * NR, sizeof(float));
    float tile[MR * NR];
    orc_pack_a(w, ckk, sp->cout, 1, wtpack);
    dx_image_packed(sp, wtpack, dy, dx, bp, tile);
    free(bp);
    free(wtpack);
}

void orc_conv_dw_image(const orc_conv_spec *sp, const float *dy, const float *x, float *dw) {
    float *dypack = (float *)calloc(orc_packed_a_len(sp->cout, hw_of(sp)), sizeof(float));
    float *scratch = (float *)calloc(2 * KC * NR, sizeof(float));
    dw_image_ws(sp, dypack, dy, x, dw, scratch, scratch + KC * NR);
    free(scratch);
    free(dypack);
}

/* Conv2d::forward (nn.rs:166-185): pack W once, y zero-filled, parallel per
 * image. */
void orc_conv2d_forward(const orc_conv_spec *sp, size_t n, const float *x, const float *w,
                        float *y) {
    size_t ckk = ckk_of(sp), hw = hw_of(sp);
    size_t xstride = (size_t)sp->cin * sp->h * sp->w, ystride = (size_t)sp->cout * hw;
    float *wpack = (float *)calloc(orc_packed_a_len(sp->cout, ckk), sizeof(float));
    orc_pack_a(w, sp->cout, ckk, 0, wpack);
    memset(y, 0, n * ystride * sizeof(float));
    int nt = orc_get_threads();
#pragma omp parallel num_threads(nt) if (nt > 1)
    {
        float *bp = (float *)calloc(KC * NR, sizeof(float));
#pragma omp for schedule(dynamic, 1)
        for (size_t i = 0; i < n; i++) forward_image_packed(sp, wpack, x + i * xstride, y + i * ystride, bp);
        free(bp);
    }
    free(wpack);
}

/* Conv2d::backward_w (nn.rs:193-227): per-image fold into private dW, reduce,
 * then w.g += dw. */
void orc_conv2d_backward_w(const orc_conv_spec *sp, size_t n, const float *dy, const float *x,
                           float *dw) {
    size_t ckk = ckk_of(sp), hw = hw_of(sp), cout = sp->cout;
    size_t xstride = (size_t)sp->cin * sp->h * sp->w, ystride = cout * hw;
    size_t lo[256], hi[256];
    int nt = orc_get_threads();
    size_t nl = orc_fold_leaves(n, nt, lo, hi, 256);
    float *accs = (float *)calloc(nl * cout * ckk + 1, sizeof(float));
#pragma omp parallel for num_threads(nt) schedule(static, 1) if (nt > 1)
    for (size_t l = 0; l < nl; l++) {
        float *acc = accs + l * cout * ckk;
        float *dypack = (float *)calloc(orc_packed_a_len(cout, hw), sizeof(float));
        float *scratch = (float *)calloc(2 * KC * NR, sizeof(float));
        for (size_t i = lo[l]; i < hi[l]; i++)
            dw_image_ws(sp, dypack, dy + i * ystride, x + i * xstride, acc, scratch,
                        scratch + KC * NR);
        free(scratch);
        free(dypack);
    }
    float *red = (float *)calloc(cout * ckk, sizeof(float));
    for (size_t l = 0; l < nl; l++)
        for (size_t e = 0; e < cout * ckk; e++) red[e] += accs[l * cout * ckk + e];
    for (size_t e = 0; e < cout * ckk; e++) dw[e] += red[e];
    free(red);
    free(accs);
}

/* The dX half of Conv2d::backward (nn.rs:233-249): pack W^T, dx zeroed,
 * parallel per image. */
void orc_conv2d_backward_x(const orc_conv_spec *sp, size_t n, const float *dy, const float *w,
                           float *dx) {
    size_t ckk = ckk_of(sp), hw = hw_of(sp);
    size_t xstride = (size_t)sp->cin * sp->h * sp->w, ystride = (size_t)sp->cout * hw;
    float *wtpack = (float *)calloc(orc_packed_a_len(ckk, sp->cout), sizeof(float));
    orc_pack_a(w, ckk, sp->cout, 1, wtpack);
    int nt = orc_get_threads();
#pragma omp parallel num_threads(nt) if (nt > 1)
    {
        float *bp = (float *)calloc(KC * NR, sizeof(float));
        float tile[MR * NR];
#pragma omp for schedule(dynamic, 1)
        for (size_t i = 0; i < n; i++)
            dx_image_packed(sp, wtpack, dy + i * ystride, dx + i * xstride, bp, tile);
        free(bp);
    }
    free(wtpack);
}
