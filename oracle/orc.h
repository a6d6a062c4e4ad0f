/*
 * orc.h -- CPU oracle for the rustnn GEMM core.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference's
 * CPU algorithm (lsiddd/rustnn, Rust; cannot be built in this image: no
 * cargo/rustc).  It exists to check the HIP product path and to time the
 * reference-style CPU path as a baseline.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it.  Nothing in rustnn_amd/ links,
 * loads or calls it.
 *
 * Every function cites the reference file:line it restates.  Build flags:
 * -O3 -mavx2 -mfma -ffp-contract=off (Rust never contracts a*b+c into an FMA
 * unless mul_add is written; the AVX2 micro-kernel uses explicit FMAs).
 *
 * Parity status (what pins each part; the pins live in tests/):
 *   rng            -- reference unit-test properties (rng.rs:74-118) plus a
 *                     bit-level restatement of xoshiro256++ / splitmix64
 *                     checked against an independent Python big-int version.
 *   pack_a/pack_b/transpose_to_panel/im2col/rel_index -- closed-form index
 *                     formulas and brute force on small inputs (bit-exact).
 *   micro_kernel/matmul/gemm_small/matmul_dw -- naive f64 GEMM, the
 *                     check.rs:101-161 gemmcheck shapes, integer-valued
 *                     inputs (exact, order-independent).
 *   conv forward/dx/dw -- f64 direct convolution, torch-CPU conv2d fixtures
 *                     committed under tests/golden, integer inputs (exact),
 *                     and the check.rs:503-546 dircheck at its shapes.
 *   attention fwd/bwd -- closed-form f64 softmax attention, finite
 *                     differences for dtau/drel, the check.rs:294-358 shapes.
 *   optim (Muon/NS, AdamW, clip, EMA) -- float64 numpy restatements of the
 *                     same iterations, torch's AdamW (decoupled decay, a
 *                     different but equivalent formula), the Newton-Schulz
 *                     spectrum property and transposition symmetry.
 *   The multi-thread reduction order of rayon (dW fold/reduce, attention
 *   dtau/drel, linear bias, clip_'s norm) is "parity unpinned": no reference
 *   test pins it.
 */
#ifndef ORC_H
#define ORC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* gemm.rs:11-13 */
#define ORC_MR 6
#define ORC_NR 16
#define ORC_KC 256

/* ------------------------------------------------------------------ rng.rs */
typedef struct {
    uint64_t s[4];
} orc_rng;

void orc_rng_new(orc_rng *r, uint64_t seed);
uint64_t orc_rng_next_u64(orc_rng *r);
uint32_t orc_rng_next_u32(orc_rng *r);
size_t orc_rng_below(orc_rng *r, size_t n);
float orc_rng_uniform(orc_rng *r);
float orc_rng_normal(orc_rng *r);
void orc_rand_vec(orc_rng *r, float *out, size_t n);
void orc_rand_uniform_vec(orc_rng *r, float *out, size_t n);
void orc_trunc_normal(orc_rng *r, float *out, size_t n, float std_);
void orc_rng_shuffle(orc_rng *r, size_t *v, size_t n);

/* ------------------------------------------------------------- threading */
/* Number of OpenMP workers used by the parallel drivers (1 = the reference's
 * --threads 1 order).  Returns the previous value. */
int orc_set_threads(int t);
int orc_get_threads(void);
/* 1 = AVX2/FMA micro-kernel (gemm.rs:122-179), 0 = scalar (gemm.rs:181-214).
 * Returns the previous value.  Ignored (scalar) when the CPU lacks AVX2. */
int orc_set_simd(int on);

/* ----------------------------------------------------------------- gemm.rs */
/* Size in floats of a packed operand buffer: nb*KC*pad (gemm.rs:36-45). */
size_t orc_packed_a_len(size_t m, size_t k);
size_t orc_packed_b_len(size_t n, size_t k);
/* PackedA::pack / pack_t (gemm.rs:54-113).  `out` holds orc_packed_a_len
 * floats; positions the reference never writes are left untouched. */
void orc_pack_a(const float *a, size_t m, size_t k, int transposed, float *out);
/* PackedB::pack / pack_t (gemm.rs:340-400). */
void orc_pack_b(const float *b, size_t n, size_t k, int transposed, float *out);
/* transpose_to_panel (gemm.rs:277-304): bp[p*NR+t] = src[t*lds+p]. */
void orc_transpose_to_panel(const float *src, size_t lds, size_t kc, float *bp);
/* micro_kernel (gemm.rs:218-236). */
void orc_micro_kernel(size_t kc, const float *ap, const float *bp, float *c, size_t ldc,
                      size_t mr, size_t nr, int accumulate);
/* matmul (gemm.rs:434-493): C[m x n] (+)= op(A) op(B). */
void orc_matmul(size_t m, size_t n, size_t k, const float *a, int at, const float *b, int bt,
                float *c, int acc);
/* gemm_small (gemm.rs:500-545): sequential; k == 0 leaves C untouched. */
void orc_gemm_small(size_t m, size_t n, size_t k, const float *a, int at, const float *b, int bt,
                    float *c, int acc);
/* matmul_dw (gemm.rs:555-598): C[m x n] += A^T B, A [k x m], B [k x n]. */
void orc_matmul_dw(size_t m, size_t n, size_t k, const float *a, const float *b, float *c);
/* Leaf ranges of a rayon fold/reduce over `len` items (see orc_gemm.c). */
size_t orc_fold_leaves(size_t len, int threads, size_t *lo, size_t *hi, size_t max_leaves);

/* ----------------------------------------------------------------- conv.rs */
/* ConvSpec (conv.rs:9-37) with oh/ow from Conv2d::out_dim (nn.rs:147-164). */
typedef struct {
    uint32_t cin, cout, k, stride, pad, h, w, oh, ow;
} orc_conv_spec;

void orc_conv_spec_init(orc_conv_spec *sp, uint32_t cin, uint32_t cout, uint32_t k,
                        uint32_t stride, uint32_t pad, uint32_t h, uint32_t w);
/* RowMap (conv.rs:39-66): out[3*r + {0,1,2}] = (ci, kh, kw). */
void orc_rowmap(const orc_conv_spec *sp, uint32_t *out);
/* Full im2col of one image via gather_span (conv.rs:68-120): col[ckk x hw]. */
void orc_im2col(const orc_conv_spec *sp, const float *x, float *col);
/* Per-image kernels (conv.rs:168-322). */
void orc_conv_forward_image(const orc_conv_spec *sp, const float *x, const float *w, float *y);
void orc_conv_dx_image(const orc_conv_spec *sp, const float *dy, const float *w, float *dx);
void orc_conv_dw_image(const orc_conv_spec *sp, const float *dy, const float *x, float *dw);
/* Conv2d batch drivers (nn.rs:166-250).  forward: y = conv(x).  backward_w:
 * dw += sum over images.  backward_x: dx = col2im(W^T dY) (overwritten). */
void orc_conv2d_forward(const orc_conv_spec *sp, size_t n, const float *x, const float *w,
                        float *y);
void orc_conv2d_backward_w(const orc_conv_spec *sp, size_t n, const float *dy, const float *x,
                           float *dw);
void orc_conv2d_backward_x(const orc_conv_spec *sp, size_t n, const float *dy, const float *w,
                           float *dx);

/* ----------------------------------------------------------------- attn.rs */
/* rel_index (attn.rs:21-72).  Writes th*tw*mh*mw entries; returns nrel. */
size_t orc_rel_index(size_t th, size_t tw, size_t mh, size_t mw, uint32_t *idx);

/* Core (attn.rs:74-84) plus the strides/offsets passed to forward/backward. */
typedef struct {
    size_t h, dh, tq, tk;
    size_t qstride, qoff, kvstride, koff, voff;
    size_t nrel;
    const uint32_t *relidx; /* [tq*tk] */
    int mask_diag;
} orc_attn_desc;

/* Core::forward (attn.rs:148-223): p [n,h,tq,tk], o [n,tq,h*dh]. */
void orc_attn_forward(const orc_attn_desc *d, size_t n, const float *q, const float *kv,
                      const float *tau, const float *rel, float *p, float *o);
/* Core::backward (attn.rs:226-343): dq, dkv, dtau, drel accumulate (+=). */
void orc_attn_backward(const orc_attn_desc *d, size_t n, const float *q, const float *kv,
                       const float *tau, const float *p, const float *dout, float *dq, float *dkv,
                       float *dtau, float *drel);

/* --------------------------------------------------------------- linear.rs */
/* Linear::forward (linear.rs:44-63): y[rows x fout] = x W^T + b (b may be NULL). */
void orc_linear_forward(size_t rows, size_t fin, size_t fout, const float *x, const float *w,
                        const float *b, float *y);
/* Linear::backward (linear.rs:66-96): dw += dy^T x, db += colsum(dy) (db may be
 * NULL), dx = dy W. */
void orc_linear_backward(size_t rows, size_t fin, size_t fout, const float *dy, const float *x,
                         const float *w, float *dw, float *db, float *dx);

/* ------------------------------------------------------------------- nn.rs */
/* BatchNorm2d train forward (nn.rs:297-348), in place on y [n][c][hw]; writes
 * xhat, mean_out (may be NULL) and invstd; updates rm / rv. */
void orc_bn_train_forward(size_t n, size_t c, size_t hw, float *y, const float *gamma,
                          const float *beta, float *rm, float *rv, float *xhat, float *mean_out,
                          float *invstd, float mom, float eps, int relu);
/* BatchNorm2d eval forward (nn.rs:350-365), in place. */
void orc_bn_eval_forward(size_t n, size_t c, size_t hw, float *y, const float *gamma,
                         const float *beta, const float *rm, const float *rv, float eps, int relu);
/* BatchNorm2d::backward (nn.rs:379-425): dx overwritten; dgamma, dbeta +=. */
void orc_bn_backward(size_t n, size_t c, size_t hw, const float *dy, const float *xhat,
                     const float *gamma, const float *invstd, float *dx, float *dgamma,
                     float *dbeta);
/* relu_back_, add_, add_relu_ (nn.rs:430-450). */
void orc_relu_back(size_t len, float *d, const float *y);
void orc_add(size_t len, float *a, const float *b);
void orc_add_relu(size_t len, float *a, const float *b);
/* gap_forward / gap_backward (nn.rs:452-473); nc = n*c planes of hw. */
void orc_gap_forward(size_t nc, size_t hw, const float *x, float *y);
void orc_gap_backward(size_t nc, size_t hw, const float *dy, float *dx);
/* nn.rs Linear (the ResNet classifier, nn.rs:475-564). */
void orc_fc_forward(size_t rows, size_t fin, size_t fout, const float *x, const float *w,
                    const float *b, float *y);
void orc_fc_backward(size_t rows, size_t fin, size_t fout, const float *dy, const float *x,
                     const float *w, float *dw, float *db, float *dx);
/* softmax_ce (nn.rs:566-637): returns the mean loss. */
float orc_softmax_ce(size_t rows, size_t nclass, const float *logits, const uint32_t *labels,
                     float smooth, float *dlogits, size_t *correct);
/* Param::step (nn.rs:102-110). */
void orc_sgd_step(size_t len, float *v, float *g, float *m, float lr, float mom, float wd);

/* --------------------------------------------------------------- optim.rs */
float orc_powi(float a, int b);
void orc_newton_schulz(float *g, size_t rows, size_t cols, size_t steps);
void orc_muon_step(float *v, float *g, float *m, size_t rows, size_t cols, int decay, float lr,
                   float wd, float mom, size_t ns_steps);
void orc_muon_steps(size_t nmat, float *const *v, float *const *g, float *const *m,
                    const size_t *rows, const size_t *cols, const int *decay, float lr, float wd,
                    float mom, size_t ns_steps, int threads);
void orc_adam_step(size_t n, float *v, float *g, float *m, float *v2, int decay, float lr,
                   float wd, float b1, float b2, float eps, size_t t);
float orc_clip(float *g, const size_t *lens, size_t nseg, float max);
void orc_ema_update(size_t n, float *w, const float *v, float decay, size_t t);
float orc_lr_at(float peak, float lo, size_t step, size_t total, size_t warm);

/* ---------------------------------------------------------------- norm.rs */
void orc_ln_forward(size_t rows, size_t c, const float *x, const float *g, const float *b,
                    float eps, float *y, float *xhat, float *invstd);
void orc_ln_backward(size_t rows, size_t c, const float *dy, const float *xhat,
                     const float *invstd, const float *g, float *dx, float *dg, float *db);
void orc_layerscale_forward(size_t rows, size_t c, const float *x, const float *l, float *y);
void orc_layerscale_backward(size_t rows, size_t c, const float *dy, const float *x,
                             const float *l, float *dx, float *dl);
void orc_swiglu_forward(size_t rows, size_t h, const float *ab, float *u);
void orc_swiglu_backward(size_t rows, size_t h, const float *du, const float *ab, float *dab);
void orc_dwconv3_forward(size_t n, size_t th, size_t tw, size_t c, const float *x,
                         const float *w, const float *b, float *y);
void orc_dwconv3_backward(size_t n, size_t th, size_t tw, size_t c, const float *dy,
                          const float *x, const float *w, float *dx, float *dw, float *db);
void orc_seqpool_forward(size_t n, size_t t, size_t c, const float *x, const float *p, float *z,
                         float *w);
void orc_seqpool_backward(size_t n, size_t t, size_t c, const float *dz, const float *w,
                          const float *x, const float *p, float *dx, float *dp);

/* ---------------------------------------------------------------- loss.rs */
void orc_taxo_target(size_t y, const uint32_t *parent, size_t nf, float eps, float sib,
                     float *out);
void orc_uniform_target(size_t y, size_t k, float eps, float *out);
void orc_soft_targets(size_t n, size_t nf, size_t nc, const uint32_t *labels,
                      const uint32_t *coarse, const uint32_t *perm, const float *lam,
                      const uint32_t *parent, int taxo, float eps, float sib, float *tf,
                      float *tc);
float orc_ce_soft(size_t n, size_t nc, const float *logits, const float *target,
                  const uint32_t *hard, float scale, float *dz, size_t *correct);
float orc_kl_distill(size_t n, size_t nc, const float *student, const float *teacher, float temp,
                     float scale, float *dz);
float orc_hint_mse(size_t n, size_t c, const float *pred, const float *target, float scale,
                   float *dz);

/* ---------------------------------------------------------------- vit.rs */
void orc_drop_path(size_t n, size_t per, float *x, float p, uint64_t seed, float *mask);
void orc_token_merge(size_t n, size_t th, size_t c, const float *z, float *y);
void orc_taxo_combine(size_t n, size_t nf, size_t nc, const uint32_t *parent, float *zf,
                      const float *zc);
void orc_taxo_combine_backward(size_t n, size_t nf, size_t nc, const uint32_t *parent,
                               const float *dzf, const float *dzc, float *dc);

/* ---------------------------------------------------------------- data.rs */
void orc_crop_flip_normalize(const uint8_t *src, float *dst, long dy, long dx, int flip);
void orc_ra_op(uint8_t *im, size_t op, float v, float sign);
void orc_randaugment(uint8_t *im, float ra_mag, size_t ra_n, orc_rng *r);
void orc_cifar_batch_train(const uint8_t *images, const uint8_t *fine, const uint8_t *coarse,
                           const uint32_t *idx, size_t bs, size_t pad, float ra_mag, size_t ra_n,
                           float erase, size_t erase_side, uint64_t seed, float *out,
                           uint32_t *labels, uint32_t *coarse_out);
void orc_mix_batch(float *x, size_t bs, float alpha_mix, float alpha_cut, float sw, orc_rng *r,
                   uint32_t *perm, float *lam);

/* ---------------------------------------------------------------- train.rs */
uint64_t orc_fnv1a_bytes(uint64_t h, const uint8_t *p, size_t n);
uint64_t orc_fnv1a_f32(uint64_t h, const float *v, size_t n);

#ifdef __cplusplus
}
#endif
#endif
