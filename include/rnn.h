/*
 * rnn.h -- C ABI of the MI355X (gfx950) GEMM core of rustnn.
 *
 * Drop-in boundary for the reference's L2 kernels (lsiddd/rustnn, Rust): each
 * entry point names the reference function it replaces (file:line).  A thin
 * Rust FFI crate (extern "C" + #[link(name = "rnn")]) keeps the reference call
 * sites in conv.rs / attn.rs / linear.rs / nn.rs unchanged (the crate rnn-sys,
 * generated from this header).
 *
 * Conventions
 *  - Every float pointer is a DEVICE pointer (hipMalloc / torch CUDA tensor)
 *    holding IEEE binary32, row-major, tightly packed unless a stride says
 *    otherwise.  Shapes are element counts.
 *  - Work is enqueued on the context's stream; calls return once the work is
 *    enqueued (use rnn_ctx_synchronize to wait).  The library keeps no pointer
 *    after a call returns.
 *  - Return value: RNN_OK (0) or a negative RNN_E_* code.  rnn_ctx_last_error
 *    gives the message.  The reference aborts on a bad shape (slice bounds
 *    panic, panic=abort); the Rust shim maps a non-zero status to panic!.
 *  - Results are deterministic: every reduction (split-K, dW over images,
 *    attention dtau/drel over images) runs in a fixed order.
 *  - One stream per context; a context may be used from several host threads
 *    (calls are serialised by a per-context lock).
 */
#ifndef RNN_H
#define RNN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    RNN_OK = 0,
    RNN_E_INVALID = -1,     /* bad shape / argument */
    RNN_E_NULL = -2,        /* required pointer is NULL */
    RNN_E_HIP = -3,         /* HIP runtime error (message has hipGetErrorString) */
    RNN_E_NOMEM = -4,       /* device workspace allocation failed */
    RNN_E_UNSUPPORTED = -5, /* shape outside what the kernels implement */
};

typedef struct rnn_ctx rnn_ctx;

/* ------------------------------------------------------------- context */
/* Replaces the process-wide rayon pool + thread-local scratch
 * (main.rs:41-48, gemm.rs:411-420): one device, one stream, one workspace. */
int rnn_ctx_create(int device, rnn_ctx **out);
/* Runs any reductions the deferral below still holds (rnn_ctx_flush), waits
 * for the stream, then frees the context; returns the flush's status. */
int rnn_ctx_destroy(rnn_ctx *ctx);
/* Use `stream` (a hipStream_t; NULL = the null stream) for later calls. */
int rnn_ctx_set_stream(rnn_ctx *ctx, void *stream);
/* Deferred parameter-gradient reductions (no counterpart in the reference:
 * a launch-count device).  While on, the backward entry points whose last
 * step only sums partial results into a parameter gradient leave that step
 * queued: rnn_linear_backward (dW when split over rows, and db),
 * rnn_ln_backward / rnn_ln_backward_add (dgamma, dbeta), the LayerScale
 * backwards (dl), rnn_dwconv3_backward (dw, db), the column sums and
 * rnn_attn_backward up to 64 tokens (dtau, drel).
 * rnn_ctx_flush runs every queued reduction in one launch, in call order,
 * with the same sums in the same order as the immediate path (results are
 * bit-identical); those gradients are complete only after it.  Turning
 * deferral off flushes first.  The partials stay in a context arena that
 * grows (hipMalloc) when a step needs more. */
int rnn_ctx_set_defer(rnn_ctx *ctx, int on);
int rnn_ctx_flush(rnn_ctx *ctx);
void *rnn_ctx_stream(rnn_ctx *ctx);
int rnn_ctx_synchronize(rnn_ctx *ctx);
const char *rnn_ctx_last_error(rnn_ctx *ctx);
const char *rnn_status_string(int status);
/* Bytes of device workspace currently held by the context. */
size_t rnn_ctx_workspace_bytes(rnn_ctx *ctx);

/* Device memory for callers that hold host slices (the Rust shim keeps the
 * reference's Vec<f32> tensors and mirrors them on the device).  No reference
 * counterpart: the reference computes on host memory only. */
int rnn_dev_alloc(rnn_ctx *ctx, size_t bytes, void **out);
int rnn_dev_free(rnn_ctx *ctx, void *p);
/* Host -> device, ordered on the context stream; returns after the copy. */
int rnn_copy_to_device(rnn_ctx *ctx, void *dst_dev, const void *src_host, size_t bytes);
/* Device -> host after all work queued on the context stream. */
int rnn_copy_to_host(rnn_ctx *ctx, void *dst_host, const void *src_dev, size_t bytes);

/* ------------------------------------------------------------ gemm.rs */
/* matmul (gemm.rs:434-493): C[m x n] = op(A) op(B) (+ C if acc).
 * at=0: A is [m x k]; at=1: A is [k x m].  bt=0: B is [k x n]; bt=1: B is
 * [n x k].  m == 0 or n == 0: no-op.  k == 0: C = 0 unless acc. */
int rnn_matmul(rnn_ctx *ctx, size_t m, size_t n, size_t k, const float *a, int at, const float *b,
               int bt, float *c, int acc);

/* gemm_small (gemm.rs:500-545), batched: `count` independent problems,
 * problem i uses a + i*stride_a, b + i*stride_b, c + i*stride_c.  Replaces the
 * per-(image, head) sequential calls made from rayon workers with one launch.
 * k == 0 leaves C untouched (gemm_small quirk). */
int rnn_gemm_small_batched(rnn_ctx *ctx, size_t count, size_t m, size_t n, size_t k,
                           const float *a, size_t stride_a, int at, const float *b,
                           size_t stride_b, int bt, float *c, size_t stride_c, int acc);

/* matmul_dw (gemm.rs:555-598): C[m x n] += A^T B with A [k x m], B [k x n]
 * (dense weight gradient, K = rows). */
int rnn_matmul_dw(rnn_ctx *ctx, size_t m, size_t n, size_t k, const float *a, const float *b,
                  float *c);

/* ------------------------------------------------------------ conv.rs */
/* ConvSpec (conv.rs:9-20); oh/ow follow Conv2d::out_dim (nn.rs:147-150):
 * oh = (h + 2*pad - k)/stride + 1.  W is [cout][cin][k][k] (RowMap order,
 * conv.rs:39-66); x, y, dx, dy are NCHW. */
typedef struct {
    uint32_t cin, cout, k, stride, pad, h, w, oh, ow;
} rnn_conv_spec;

/* Fills oh/ow.  Returns RNN_E_INVALID for k > h + 2*pad, stride 0, ... */
int rnn_conv_spec_init(rnn_conv_spec *sp, uint32_t cin, uint32_t cout, uint32_t k,
                       uint32_t stride, uint32_t pad, uint32_t h, uint32_t w);

/* Conv2d::forward (nn.rs:166-185) -> conv::forward_image (conv.rs:168-203):
 * y[n][cout][oh][ow] = conv(x) (overwritten). */
int rnn_conv2d_forward(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *x,
                       const float *w, float *y);
/* Conv2d::backward_w (nn.rs:193-227) -> conv::dw_image (conv.rs:277-322):
 * dw[cout][cin*k*k] += sum over images of dY im2col(X)^T. */
int rnn_conv2d_backward_w(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *dy,
                          const float *x, float *dw);
/* The per-worker half of Conv2d::backward_w (nn.rs:201-219): the batch's
 * dW as *nz partial slabs of cout*cin*k*k floats in `slabs` (slab z: the sum
 * over the pixel tiles workgroup z owns), without the final reduce
 * (nn.rs:220-225).  Adding the slabs in slab order gives what
 * rnn_conv2d_backward_w adds; a train step can fold that sum into its
 * gradient pass.  `slabs` holds rnn_conv2d_backward_w_slab_floats(...)
 * floats (0: no slab plan for the shape -- k not 1 or 3, stride not 1 or 2). */
size_t rnn_conv2d_backward_w_slab_floats(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n);
int rnn_conv2d_backward_w_slabs(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n,
                                const float *dy, const float *x, float *slabs, int *nz);
/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): rnn_conv2d_backward_w with its partial slabs in a fixed
 * device scratch array of 16 MiB (RNN_NOALLOC_SCRATCH_BYTES) that the library
 * holds on each device until the process ends, instead of the context's
 * growing workspace.  Same kernels, same summation order, same result.  It
 * calls no hipMalloc / hipFree.  A shape whose slabs need more than the
 * scratch (cout*cin*k*k*4 bytes times the slab count; 9.4 MB for the ResNet
 * convs at batch 128) returns RNN_E_UNSUPPORTED.  Every call on one device
 * shares that scratch.  Outside graph capture the library orders them: a
 * call on another stream than the device's previous call first waits for
 * that call's kernels (hipStreamWaitEvent; one event per device, created by
 * the first such call).  Under graph capture it does not: captured calls
 * that could run at the same time on one GPU race, and the caller orders
 * them (one stream, or graph edges between them).  The scratch address is
 * looked up by the first call on a device (hipGetSymbolAddress); a failed
 * lookup returns RNN_E_HIP from this call only. */
int rnn_conv2d_backward_w_noalloc(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n,
                                  const float *dy, const float *x, float *dw);
/* dX half of Conv2d::backward (nn.rs:230-250) -> conv::dx_image
 * (conv.rs:205-246): dx[n][cin][h][w] = col2im(W^T dY) (overwritten). */
int rnn_conv2d_backward_x(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *dy,
                          const float *w, float *dx);

/* Packed weights (no counterpart in the reference: for callers that run
 * several forward / dX convolutions between weight updates, such as a train
 * step).  rnn_conv_pack_weights rewrites W into the slab order the forward
 * (dx = 0) or dX (dx = 1) kernel stages through LDS, so that each stage's
 * weights arrive as one contiguous copy; *floats receives the packed size
 * (RNN_E_UNSUPPORTED: the shape has no packed form, use the calls above).
 * The _packed calls take W and its packed copy wp and give results identical
 * to rnn_conv2d_forward / rnn_conv2d_backward_x; wp must be re-packed after
 * W changes. */
int rnn_conv_packed_floats(const rnn_conv_spec *sp, int dx, size_t *floats);
int rnn_conv_pack_weights(rnn_ctx *ctx, const rnn_conv_spec *sp, int dx, const float *w,
                          float *wp);
int rnn_conv2d_forward_packed(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *x,
                              const float *w, const float *wp, float *y);
int rnn_conv2d_backward_x_packed(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *dy,
                                 const float *w, const float *wp, float *dx);
/* Packed copies of several convolutions' weights, refreshed together in one
 * launch (no counterpart in the reference: for a network whose convolutions
 * run on packed weights and are re-packed after each weight update, such as
 * the rustvit trunk).  Convolution i has spec specs[i] and weights w[i] (on
 * the device, [cout][cin][k][k]; w[i] must stay allocated, at the same
 * address, while the object lives).  create allocates the packed copies of
 * both directions of every convolution and packs them on the context stream;
 * update re-packs all of them from the current W; get returns convolution
 * i's copy for the forward (dx = 0) or dX (dx = 1) -- for the _packed calls
 * with the same spec -- or NULL when that shape has no packed form. */
typedef struct rnn_conv_packs rnn_conv_packs;
int rnn_conv_packs_create(rnn_ctx *ctx, size_t count, const rnn_conv_spec *specs, const float **w,
                          rnn_conv_packs **out);
int rnn_conv_packs_update(rnn_ctx *ctx, rnn_conv_packs *p);
const float *rnn_conv_packs_get(const rnn_conv_packs *p, size_t i, int dx);
void rnn_conv_packs_destroy(rnn_conv_packs *p);

/* ------------------------------------------------------------ attn.rs */
/* Core (attn.rs:74-84) plus the stride/offset arguments of Core::forward /
 * Core::backward (attn.rs:148-160, 226-242).  Rows of head hd are read at
 * base + r*qstride + qoff + hd*dh (queries) and base + r*kvstride + koff/voff
 * + hd*dh (keys / values).  relidx is a HOST pointer to tq*tk entries
 * (rnn_rel_index); the library uploads it. */
typedef struct {
    uint32_t h, dh, tq, tk;
    size_t qstride, qoff, kvstride, koff, voff;
    uint32_t nrel;
    const uint32_t *relidx;
    int mask_diag;
} rnn_attn_desc;

/* rel_index (attn.rs:53-72): host-side table of th*tw*mh*mw entries;
 * *nrel receives the bias-table length per head. */
int rnn_rel_index(uint32_t th, uint32_t tw, uint32_t mh, uint32_t mw, uint32_t *idx,
                  uint32_t *nrel);

/* Core::forward (attn.rs:148-223): p[n][h][tq][tk] = softmax(tau*QK^T + rel,
 * diagonal masked when mask_diag), o[n][tq][h*dh] = P V. */
int rnn_attn_forward(rnn_ctx *ctx, const rnn_attn_desc *d, size_t n, const float *q,
                     const float *kv, const float *tau, const float *rel, float *p, float *o);
/* Core::backward (attn.rs:226-343): dq, dkv, dtau, drel ACCUMULATE (+=).
 * dq and dkv may alias (disjoint columns, as in SelfAttn, attn.rs:418-438). */
int rnn_attn_backward(rnn_ctx *ctx, const rnn_attn_desc *d, size_t n, const float *q,
                      const float *kv, const float *tau, const float *p, const float *dout,
                      float *dq, float *dkv, float *dtau, float *drel);
/* Core::backward with dq and/or dkv OVERWRITTEN instead of accumulated
 * (flags: RNN_ATTN_SET_DQ, RNN_ATTN_SET_DKV; dtau and drel always
 * accumulate).  SelfAttn::backward (attn.rs:418-438) accumulates into freshly
 * zeroed dq and dkv buffers and CrossAttn::backward (attn.rs:533-551) into a
 * zeroed dq: the same values, without the clearing pass and the read of the
 * old contents.  flags 0 is rnn_attn_backward. */
#define RNN_ATTN_SET_DQ 1u
#define RNN_ATTN_SET_DKV 2u
int rnn_attn_backward_ex(rnn_ctx *ctx, const rnn_attn_desc *d, size_t n, const float *q,
                         const float *kv, const float *tau, const float *p, const float *dout,
                         float *dq, float *dkv, float *dtau, float *drel, uint32_t flags);

/* ---------------------------------------------------------- linear.rs */
/* Linear::forward (linear.rs:44-63): y[rows x fout] = x W^T + b (b may be NULL). */
int rnn_linear_forward(rnn_ctx *ctx, size_t rows, size_t fin, size_t fout, const float *x,
                       const float *w, const float *b, float *y);
/* Linear::forward feeding a residual branch (vit.rs:155-176): y = x W^T + b
 * as rnn_linear_forward, and out += (y l) m with m = mask[r / rpi] (mask may
 * be NULL: m = 1) -- rnn_residual_add_scaled(out, y, ...) -- in the GEMM's
 * epilogue (two passes when rpi is not a power of two).  out is neither x
 * nor y. */
int rnn_linear_forward_residual(rnn_ctx *ctx, size_t rows, size_t fin, size_t fout,
                                const float *x, const float *w, const float *b, float *y,
                                const float *l, const float *mask, size_t rpi, float *out);
/* Linear::backward (linear.rs:66-96): dw += dy^T x; db += colsum(dy) (db may
 * be NULL); dx = dy W (overwritten). */
int rnn_linear_backward(rnn_ctx *ctx, size_t rows, size_t fin, size_t fout, const float *dy,
                        const float *x, const float *w, float *dw, float *db, float *dx);
/* rnn_linear_backward with dx accumulated instead of overwritten when flags
 * has RNN_LINEAR_ACC_DX: dx += dy W, the old value first, as add_ (nn.rs:441-443)
 * of a separately computed dx.  Block::backward (vit.rs:175-232) sums its
 * branches' input gradients this way without a separate pass. */
#define RNN_LINEAR_ACC_DX 1u
int rnn_linear_backward_ex(rnn_ctx *ctx, size_t rows, size_t fin, size_t fout, const float *dy,
                           const float *x, const float *w, float *dw, float *db, float *dx,
                           uint32_t flags);

/* ------------------------------------------ host-slice forms (Rust shim) */
/* The same entry points over HOST memory, for the Rust shim, whose callers
 * keep the reference's Vec<f32> tensors (nn.rs Tensor, linear.rs, attn.rs
 * Tok): each call copies its operands into a device staging block the
 * context keeps (it only grows), runs the device entry point on the context
 * stream, runs any deferred reductions, copies the outputs back and returns
 * after the stream has finished.  Arguments, accumulation and the k = 0 /
 * empty cases are those of the device form; a host pointer passed for two
 * operands (a fused QKV buffer as q and kv; dq == dkv as SelfAttn::backward
 * passes them, attn.rs:418-438) is staged once.  Each replaces the same
 * reference function as its device form:
 *   rnn_matmul_host              matmul        (gemm.rs:434-493)
 *   rnn_gemm_small_batched_host  gemm_small    (gemm.rs:500-545), C read back whole
 *   rnn_matmul_dw_host           matmul_dw     (gemm.rs:555-598)
 *   rnn_conv2d_forward_host      Conv2d::forward    (nn.rs:166-185)
 *   rnn_conv2d_backward_w_host   Conv2d::backward_w (nn.rs:193-227)
 *   rnn_conv2d_backward_x_host   dX of Conv2d::backward (nn.rs:230-250)
 *   rnn_attn_forward_host        Core::forward (attn.rs:148-223)
 *   rnn_attn_backward_host       Core::backward (attn.rs:226-343)
 *   rnn_linear_forward_host      Linear::forward (linear.rs:44-64)
 *   rnn_linear_backward_host     Linear::backward (linear.rs:66-96) */
int rnn_matmul_host(rnn_ctx *ctx, size_t m, size_t n, size_t k, const float *a, int at,
                    const float *b, int bt, float *c, int acc);
int rnn_gemm_small_batched_host(rnn_ctx *ctx, size_t count, size_t m, size_t n, size_t k,
                                const float *a, size_t stride_a, int at, const float *b,
                                size_t stride_b, int bt, float *c, size_t stride_c, int acc);
int rnn_matmul_dw_host(rnn_ctx *ctx, size_t m, size_t n, size_t k, const float *a,
                       const float *b, float *c);
int rnn_conv2d_forward_host(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *x,
                            const float *w, float *y);
int rnn_conv2d_backward_w_host(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n,
                               const float *dy, const float *x, float *dw);
int rnn_conv2d_backward_x_host(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n,
                               const float *dy, const float *w, float *dx);
int rnn_attn_forward_host(rnn_ctx *ctx, const rnn_attn_desc *d, size_t n, const float *q,
                          const float *kv, const float *tau, const float *rel, float *p,
                          float *o);
int rnn_attn_backward_host(rnn_ctx *ctx, const rnn_attn_desc *d, size_t n, const float *q,
                           const float *kv, const float *tau, const float *p, const float *dout,
                           float *dq, float *dkv, float *dtau, float *drel);
int rnn_linear_forward_host(rnn_ctx *ctx, size_t rows, size_t fin, size_t fout, const float *x,
                            const float *w, const float *b, float *y);
int rnn_linear_backward_host(rnn_ctx *ctx, size_t rows, size_t fin, size_t fout,
                             const float *dy, const float *x, const float *w, float *dw,
                             float *db, float *dx);

/* -------------------------------------------------------------- nn.rs */
/* The ResNet layers around the convs.  Elementwise formulas round exactly as
 * the reference's (no FMA contraction); per-channel sums are f64 in a fixed
 * order.  x, y, dy, dx are NCHW [n][c][hw]; per-channel arrays hold c floats. */

/* BatchNorm2d::forward / forward_relu in train mode (nn.rs:253-348): batch
 * statistics (f64 sums), y = [relu](gamma*(x - mean)*invstd + beta), running
 * mean / unbiased running variance updated with `momentum` (0.1 in rustnn).
 * mean and invstd are written for rnn_bn_backward.  y may alias x; the
 * reference keeps xhat for the backward, this API keeps x instead (a caller
 * that normalises in place must keep a copy of x).  running_mean and
 * running_var may both be NULL (statistics only, no running update). */
int rnn_bn_forward_train(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *x, float *y,
                         const float *gamma, const float *beta, float *running_mean,
                         float *running_var, float *mean, float *invstd, float momentum, float eps,
                         int relu);
/* BatchNorm2d forward in eval mode (run_eval, nn.rs:350-365). */
int rnn_bn_forward_eval(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *x, float *y,
                        const float *gamma, const float *beta, const float *running_mean,
                        const float *running_var, float eps, int relu);
/* BatchNorm2d::backward (nn.rs:379-425): dx overwritten, dgamma / dbeta
 * ACCUMULATE.  x, mean, invstd as passed to / written by the train forward.
 * relu_out (may be NULL): apply relu_back_ (nn.rs:432-439) to dy first, i.e.
 * use 0 where relu_out <= 0 (dy itself is not modified). */
int rnn_bn_backward(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *dy,
                    const float *relu_out, const float *x, const float *mean, const float *invstd,
                    const float *gamma, float *dx, float *dgamma, float *dbeta);
/* relu_back_ (nn.rs:432-439): d = 0 where y <= 0. */
int rnn_relu_back(rnn_ctx *ctx, size_t len, float *d, const float *y);
/* add_ (nn.rs:441-443): a += b. */
int rnn_add(rnn_ctx *ctx, size_t len, float *a, const float *b);
/* add_ after relu_back_ (nn.rs:432-443) without changing b: a += b where
 * y > 0 (the value relu_back_(b, y) then add_(a, b) leave in a); a must
 * not be b. */
int rnn_add_relu_back(rnn_ctx *ctx, size_t len, float *a, const float *b, const float *y);
/* add_relu_ (nn.rs:446-450): a = max(a + b, 0). */
int rnn_add_relu(rnn_ctx *ctx, size_t len, float *a, const float *b);
/* gap_forward (nn.rs:455-463): y[n][c] = plane sum (pixel order) / hw. */
int rnn_gap_forward(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *x, float *y);
/* gap_backward (nn.rs:465-473): dx[n][c][p] = dy[n][c] / hw. */
int rnn_gap_backward(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *dy, float *dx);
/* nn.rs Linear (the ResNet classifier, nn.rs:475-564), bit-identical to the
 * reference's scalar loops.  forward: y[i][o] = b[o] + sum_j w[o][j] x[i][j].
 * backward: dw, db ACCUMULATE over rows in order; dx (may be NULL) is
 * overwritten. */
int rnn_fc_forward(rnn_ctx *ctx, size_t rows, size_t fin, size_t fout, const float *x,
                   const float *w, const float *b, float *y);
int rnn_fc_backward(rnn_ctx *ctx, size_t rows, size_t fin, size_t fout, const float *dy,
                    const float *x, const float *w, float *dw, float *db, float *dx);
/* softmax_ce (nn.rs:566-637): dlogits = (softmax - smoothed target) / rows;
 * *loss (device, may be NULL) = mean loss; *correct (device u32, may be NULL)
 * = rows whose first maximal logit is the label.  labels: device u32[rows].
 * rows <= 8192, nclass <= 1024.  A label >= nclass (a panic in the reference)
 * gives NaN for that row instead of an out-of-bounds read. */
int rnn_softmax_ce(rnn_ctx *ctx, size_t rows, size_t nclass, const float *logits,
                   const uint32_t *labels, float smooth, float *dlogits, float *loss,
                   uint32_t *correct);
/* Param::step (nn.rs:102-110): Nesterov SGD, g zeroed.  Pass wd = 0 for the
 * parameters the reference does not decay (BN gamma / beta, biases). */
int rnn_sgd_step(rnn_ctx *ctx, size_t len, float *v, float *g, float *m, float lr, float momentum,
                 float wd);

/* ----------------------------------------------------------- norm.rs */
/* Token tensors are [rows = n*t][c] row-major, channel fastest (tok.rs).
 * Parameter gradients (dg, db, dl, dw, dp) accumulate (+=), as Param::g does;
 * dx is overwritten. */
/* LayerNorm::forward (norm.rs:38-85): per row f64 sums, mu, var = max(s2/c -
 * mu^2, 0) as f32, invstd = 1/sqrt(var + eps); y = g (x - mu) invstd + b.
 * Training keeps xhat [rows][c] and invstd [rows]; pass both NULL for eval. */
int rnn_ln_forward(rnn_ctx *ctx, size_t rows, size_t c, const float *x, const float *g,
                   const float *b, float eps, float *y, float *xhat, float *invstd);
/* LayerNorm::backward (norm.rs:87-137). */
int rnn_ln_backward(rnn_ctx *ctx, size_t rows, size_t c, const float *dy, const float *xhat,
                    const float *invstd, const float *g, float *dx, float *dg, float *db);
/* rnn_ln_backward followed by add_ (Block::backward, vit.rs:175-232: the
 * norm's input gradient plus the residual's, dy = n2.backward(dh2) + dz and
 * dy += n1.backward(dh)): dx = the LayerNorm input gradient + add, in the
 * same pass for c <= 512.  add may be dx (in place). */
int rnn_ln_backward_add(rnn_ctx *ctx, size_t rows, size_t c, const float *dy, const float *xhat,
                        const float *invstd, const float *g, const float *add, float *dx,
                        float *dg, float *db);
/* rnn_ln_backward_add, then the DropPath + LayerScale backward that reads
 * its dx (the next block's first op in a backward over Blocks, vit.rs:175-
 * 232): lsdx = (dx m) l and dl += sum (dx m) lsx, m = mask[r / rpi] or 1
 * when NULL -- the values rnn_ln_backward_add then
 * rnn_drop_layerscale_backward(dx, lsx, l, mask, rpi, lsdx, dl) give, bit
 * for bit, in the same pass for c <= 512.  lsdx must not overlap dy, add,
 * dx or lsx. */
int rnn_ln_backward_add_ls(rnn_ctx *ctx, size_t rows, size_t c, const float *dy,
                           const float *xhat, const float *invstd, const float *g,
                           const float *add, float *dx, float *dg, float *db, const float *lsx,
                           const float *l, const float *mask, size_t rpi, float *lsdx,
                           float *dl);
/* LayerScale::forward / backward (norm.rs:166-212): y = x l per channel (y may
 * be x); dl += sum dy x, dx = dy l (dx may be dy). */
int rnn_layerscale_forward(rnn_ctx *ctx, size_t rows, size_t c, const float *x, const float *l,
                           float *y);
int rnn_layerscale_backward(rnn_ctx *ctx, size_t rows, size_t c, const float *dy, const float *x,
                            const float *l, float *dx, float *dl);
/* DropPath::backward then LayerScale::backward (vit.rs:61-73,
 * norm.rs:182-212) in one pass that reads dy without changing it:
 * g = dy * mask[r / rpi] (mask NULL: g = dy), dl += sum_r g x, dx = g l
 * (dx must not be dy).  Block::backward's branches (vit.rs:175-232) read the
 * same dy twice or three times, so no copy of it is needed. */
int rnn_drop_layerscale_backward(rnn_ctx *ctx, size_t rows, size_t c, const float *dy,
                                 const float *x, const float *l, const float *mask, size_t rpi,
                                 float *dx, float *dl);
/* The first residual's branch gradients in a Block backward (vit.rs:175-232)
 * in one pass over dy: da = (dy m1) l1 with dl1 += sum (dy m1) a (the
 * DropPath + LayerScale of the attention branch), ddw = da gamma with
 * dgamma += sum da dwo (the depthwise branch's gamma gate) and, for a reader
 * block (cm set), dc = (dy m2) lm with dlm += sum (dy m2) cm.  Each value
 * equals what rnn_drop_layerscale_backward (lsm, then ls1) and
 * rnn_layerscale_backward (gamma) called in turn write; m1 / m2 = mask[r /
 * rpi] or 1 when NULL.  dy, a, dwo and cm are not changed; the outputs must
 * not overlap them or each other. */
int rnn_block_branch_backward(rnn_ctx *ctx, size_t rows, size_t c, const float *dy,
                              const float *a, const float *l1, const float *m1, const float *dwo,
                              const float *gamma, const float *cm, const float *lm,
                              const float *m2, size_t rpi, float *da, float *dl1, float *ddw,
                              float *dgamma, float *dc, float *dlm);
/* y = x + (a l) m, m = mask[r / rpi] per image (mask may be NULL: m = 1): one
 * residual branch of Block::forward, x + DropPath(LayerScale(a))
 * (vit.rs:155-176: the LayerScale, the DropPath scaling and add_ in that
 * rounding order) in one pass.  y may be x (in place); a is left unchanged,
 * as the LayerScale backward (rnn_drop_layerscale_backward) reads it. */
int rnn_residual_add_scaled(rnn_ctx *ctx, size_t rows, size_t c, const float *x, const float *a,
                            const float *l, const float *mask, size_t rpi, float *y);
/* The SwiGLU gate between SwiGlu's two Linear calls (norm.rs:250-288): ab is
 * [rows][2h] (a | b), u = a sigmoid(a) b [rows][h]; the backward writes
 * dab [rows][2h] from du [rows][h]. */
int rnn_swiglu_forward(rnn_ctx *ctx, size_t rows, size_t h, const float *ab, float *u);
int rnn_swiglu_backward(rnn_ctx *ctx, size_t rows, size_t h, const float *du, const float *ab,
                        float *dab);
/* DwConv3 (norm.rs:296-457): depthwise 3x3, pad 1, over n images of th x tw
 * tokens, channel-last; w [9][c] (tap-major), b [c]. */
int rnn_dwconv3_forward(rnn_ctx *ctx, size_t n, size_t th, size_t tw, size_t c, const float *x,
                        const float *w, const float *b, float *y);
int rnn_dwconv3_backward(rnn_ctx *ctx, size_t n, size_t th, size_t tw, size_t c, const float *dy,
                         const float *x, const float *w, float *dx, float *dw, float *db);
/* rnn_dwconv3_backward with dx accumulated (dx += the input gradient, the old
 * value first) when flags has RNN_DW3_ACC_DX; dx must not be dy. */
#define RNN_DW3_ACC_DX 1u
int rnn_dwconv3_backward_ex(rnn_ctx *ctx, size_t n, size_t th, size_t tw, size_t c,
                            const float *dy, const float *x, const float *w, float *dx, float *dw,
                            float *db, uint32_t flags);
/* Block::forward's first branch (vit.rs:150-160) in one pass: d =
 * DwConv3(h) as rnn_dwconv3_forward computes it; a += gamma d (rnn_axpy_cols);
 * y = x + (a l) m, m = mask[image] (mask may be NULL; rnn_residual_add_scaled
 * with th * tw rows per image).  h, a, x, y, d are [n][th][tw][c]; gamma, l
 * [c]; a is updated in place and y may be x; d, a, h and y are distinct, and x
 * is not a. */
int rnn_dwconv3_branch_forward(rnn_ctx *ctx, size_t n, size_t th, size_t tw, size_t c,
                               const float *h, const float *w, const float *b, float *d, float *a,
                               const float *gamma, const float *x, const float *l,
                               const float *mask, float *y);
/* SeqPool (norm.rs:459-586): w = softmax_t(x p), z = sum_t w_t x_t; z [n][c];
 * the forward writes the softmax weights w [n][t] that the backward reads.
 * t <= 1024. */
int rnn_seqpool_forward(rnn_ctx *ctx, size_t n, size_t t, size_t c, const float *x,
                        const float *p, float *z, float *w);
int rnn_seqpool_backward(rnn_ctx *ctx, size_t n, size_t t, size_t c, const float *dz,
                         const float *w, const float *x, const float *p, float *dx, float *dp);

/* ----------------------------------------------------------- loss.rs */
/* Soft targets of a batch (targets, train.rs:121-155): tf [n][nf] = lam a +
 * (1 - lam) b with a / b the targets of labels[i] / labels[perm[i]] --
 * taxo_target (loss.rs:11-28, sibling share sib of eps, parent [nf] the
 * superclass of each fine class) when taxo, else uniform_target
 * (loss.rs:30-34); tc [n][nc] (may be NULL) the same over coarse labels with
 * uniform smoothing.  perm NULL = identity, lam NULL = all 1. */
int rnn_soft_targets(rnn_ctx *ctx, size_t n, size_t nf, size_t nc, const uint32_t *labels,
                     const uint32_t *coarse, const uint32_t *perm, const float *lam,
                     const uint32_t *parent, int taxo, float eps, float sib, float *tf,
                     float *tc);
/* The dominant label of each mixed image (Trainer::make_batch,
 * train.rs:313-320): dom[i] = labels[i] when lam[i] >= 0.5, else
 * labels[perm[i]] -- the hard label ce_soft counts hits against. */
int rnn_mix_dominant(rnn_ctx *ctx, size_t n, const uint32_t *labels, const uint32_t *perm,
                     const float *lam, uint32_t *dom);
/* ce_soft (loss.rs:39-83): dz [n][nclass] overwritten with scale (softmax -
 * target) / n; *loss (device, may be NULL) the mean loss; *correct (device,
 * may be NULL) the argmax hits against hard. */
int rnn_ce_soft(rnn_ctx *ctx, size_t n, size_t nclass, const float *logits, const float *target,
                const uint32_t *hard, float scale, float *dz, float *loss, uint32_t *correct);
/* kl_distill (loss.rs:87-130): teacher detached; dz += temp (ps - pt) / n *
 * scale; *loss = mean of temp^2 KL(pt || ps). */
int rnn_kl_distill(rnn_ctx *ctx, size_t n, size_t nclass, const float *student,
                   const float *teacher, float temp, float scale, float *dz, float *loss);
/* hint_mse (loss.rs:133-151): dz += 2 (pred - target) / (n c) * scale; *loss =
 * scale * mean squared error. */
int rnn_hint_mse(rnn_ctx *ctx, size_t n, size_t c, const float *pred, const float *target,
                 float scale, float *dz, float *loss);
/* build_loss (train.rs:70-118) in one call: the soft-target cross-entropy of
 * the logits (scale 1), of the coarse head when coarse_w > 0 and taxo (scale
 * coarse_w), and with the exits (io->e1 set): the exits' cross-entropies
 * (exit_w1, exit_w2), their distillation from the logits when alpha > 0
 * (loss::kl_distill, temp) and the hint MSEs of h1 / h2 against feat when
 * beta > 0.  Gradients are written (the reference's zeroed Grads receive
 * them): dlogits, dcoarse (zeros without the coarse term), de1 / de2 (their
 * cross-entropy, then the distillation added), dh1 / dh2 (zeros when beta
 * is 0).  *total = ce (+ coarse_w lc) (+ (w1 l1 + w2 l2)) (+ alpha (k1 + k2))
 * (+ (h1 + h2)) in f32, the reference's order and grouping; *ce the logits'
 * loss; *correct its argmax hits (device pointers, any may be NULL).  nc:
 * coarse classes (0: no coarse head); d4: the width of h1 / h2 / feat. */
typedef struct {
    float coarse_w, exit_w1, exit_w2, alpha, temp, beta;
    int taxo;
} rnn_loss_cfg;
typedef struct {
    const float *logits, *coarse, *e1, *e2, *h1, *h2, *feat;
    float *dlogits, *dcoarse, *de1, *de2, *dh1, *dh2;
} rnn_loss_io;
int rnn_build_loss(rnn_ctx *ctx, size_t n, size_t nf, size_t nc, size_t d4, const float *tf,
                   const float *tc, const uint32_t *hard, const uint32_t *hardc,
                   const rnn_loss_cfg *cfg, const rnn_loss_io *io, float *total, float *ce,
                   uint32_t *correct);

/* ----------------------------------------------------------- vit.rs */
/* DropPath (vit.rs:25-74) on n images of `per` floats, in place: image i is
 * kept with the i-th uniform of Rng::new(seed) (rng.rs) below 1 - p and
 * scaled by 1 / (1 - p), else zeroed; mask [n] (device) receives the factors
 * for the backward.  0 < p < 1 (the reference skips the layer otherwise). */
int rnn_drop_path_forward(rnn_ctx *ctx, size_t n, size_t per, float *x, float p, uint64_t seed,
                          float *mask);
int rnn_drop_path_backward(rnn_ctx *ctx, size_t n, size_t per, float *dy, const float *mask);
/* The masks alone of `count` DropPath layers over n images, in one launch:
 * masks[k] (device, [n]) receives rnn_drop_path_forward's factors for p[k]
 * and seeds[k] (p, seeds and masks are host arrays).  A layer whose mask is
 * drawn here is applied with rnn_drop_path_backward (the same per-image
 * scaling).  Batches DropPath::forward's draws (vit.rs:44-51) of a step. */
int rnn_drop_path_masks(rnn_ctx *ctx, size_t count, size_t n, const float *p,
                        const uint64_t *seeds, float *const *masks);
/* y[r][j] += l[j] x[r][j]: Block's depthwise gate a += gamma * dw(h)
 * (vit.rs:150-158).  Its backward is rnn_layerscale_backward. */
int rnn_axpy_cols(rnn_ctx *ctx, size_t rows, size_t c, float *y, const float *l, const float *x);
/* token_merge / token_merge_back (vit.rs:612-650): [n][th*th][c] <->
 * [n][(th/2)^2][4c], the 2x2 neighbours (0,0), (0,1), (1,0), (1,1)
 * concatenated; th even; the backward overwrites dz. */
int rnn_token_merge(rnn_ctx *ctx, size_t n, size_t th, size_t c, const float *z, float *y);
int rnn_token_merge_backward(rnn_ctx *ctx, size_t n, size_t th, size_t c, const float *dy,
                             float *dz);
/* TaxoHead (vit.rs:282-312): zf[i][j] += zc[i][parent[j]]; the backward's
 * coarse gradient dc = dzc + the fine gradients summed by parent (in class
 * order).  parent (device u32 [nf]). */
int rnn_taxo_head_combine(rnn_ctx *ctx, size_t n, size_t nf, size_t nc, const uint32_t *parent,
                          float *zf, const float *zc);
int rnn_taxo_head_combine_backward(rnn_ctx *ctx, size_t n, size_t nf, size_t nc,
                                   const uint32_t *parent, const float *dzf, const float *dzc,
                                   float *dc);
/* Tok::from_tensor / to_tensor (tok.rs): [n][c][hw] <-> [n][hw][c]. */
int rnn_nchw_to_tokens(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *x, float *t);
int rnn_tokens_to_nchw(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *t, float *x);

/* ----------------------------------------------------------- data.rs */
/* make_batch_train (data.rs:384-416): for batch slot b, image idx[b] of the
 * device-resident dataset (images [nimg][3][32][32] u8, fine / coarse labels
 * u8), with Rng::new(seed ^ b * 0x9E3779B97F4A7C15): ra_n RandAugment
 * operations of magnitude ra_mag (none when ra_mag <= 0; ra_n <= 16), crop
 * offsets in [-pad, pad], a horizontal flip,
 * normalisation (border = -mean/std), random erasing with probability erase
 * of an erase_side square of N(0,1) noise.  out [bs][3][32][32]; labels,
 * coarse_out [bs] u32.  An index past nimg gives a NaN image and label
 * 0xffffffff. */
int rnn_cifar_batch_train(rnn_ctx *ctx, const uint8_t *images, const uint8_t *fine,
                          const uint8_t *coarse, size_t nimg, const uint32_t *idx, size_t bs,
                          size_t pad, float ra_mag, size_t ra_n, float erase, size_t erase_side,
                          uint64_t seed, float *out, uint32_t *labels, uint32_t *coarse_out);
/* make_batch_eval (data.rs:494-512): images start .. start + bs normalised
 * (mirrored when flip); labels may be NULL. */
int rnn_cifar_batch_eval(rnn_ctx *ctx, const uint8_t *images, const uint8_t *fine, size_t nimg,
                         size_t start, size_t bs, int flip, float *out, uint32_t *labels);
/* FNV-1a 64 continued over host bytes, or over host floats' bit patterns as
 * 4 little-endian bytes each (fnv_f32, train.rs:478-484): the building blocks
 * of Trainer::fingerprint (train.rs:450-470).  Host only. */
uint64_t rnn_fnv1a_bytes(uint64_t hash, const uint8_t *bytes, size_t n);
uint64_t rnn_fnv1a_f32(uint64_t hash, const float *values, size_t n);
/* The host generator of the trainer (rng.rs): state = Rng::new(seed); next. */
int rnn_rng_seed(uint64_t seed, uint64_t *state);
uint64_t rnn_rng_next_u64(uint64_t *state);
/* Normal draws from the caller's generator state (4 u64, advanced), host
 * only: rand_vec (rng.rs:70-72) times scale -- Param::kaiming (nn.rs:95-100)
 * with scale = sqrt(2 / fan_in) as f32 -- and Param::trunc_normal
 * (nn.rs:77-89): up to 8 redraws while |z| > 2, clamped to [-2, 2], times
 * std.  The initial weights of the reference's models, bit for bit. */
int rnn_rng_normal_vec(uint64_t *state, size_t n, float scale, float *out);
int rnn_rng_trunc_normal(uint64_t *state, size_t n, float std_, float *out);
/* mix_batch's draws (data.rs:469-492) from the caller's generator state (4
 * u64, advanced): perm [bs] (shuffle), lam [bs], *cut (cutmix or mixup), *l
 * and, for cutmix, rect = y0, y1, x0, x1.  Host only. */
int rnn_mix_plan(uint64_t *rng_state, size_t bs, float alpha_mix, float alpha_cut, float sw,
                 uint32_t *perm, float *lam, int *cut, float *l, int *rect);
/* The blend of that plan on the device (cutmix / mixup, data.rs:434-467):
 * out [bs][3][32][32] from x (not aliased), perm on the device, rect on the
 * host. */
int rnn_mix_apply(rnn_ctx *ctx, const float *x, float *out, size_t bs, const uint32_t *perm,
                  int cut, float l, const int *rect);

/* ----------------------------------------------------------- optim.rs */
/* Newton-Schulz orthogonalisation (newton_schulz, optim.rs:124-145), in
 * place on `count` [rows x cols] matrices at g + i*stride: X = G (G^T when
 * rows > cols) / (||G||_F + 1e-7), then `steps` quintic steps
 * X = a X + (b A + c A A) X with A = X X^T (a, b, c = 3.4445, -4.7750,
 * 2.0315), each product a batched GEMM over the matrices. */
int rnn_newton_schulz(rnn_ctx *ctx, size_t count, size_t rows, size_t cols, size_t steps,
                      float *g, size_t stride);

/* One parameter of Optim::step_all (nn.rs Param, nn.rs:43-53): device
 * buffers; v2 (AdamW's second moment, zero-initialised) may be NULL for a
 * Muon matrix; rows = 0 marks a tensor that is not a matrix. */
typedef struct {
    float *v, *g, *m, *v2;
    size_t len, rows, cols;
    int decay;
} rnn_param;

/* Optim (optim.rs:147-235).  rnn_optim_create = Optim::new(muon, ns_steps)
 * with mom 0.95, b1 0.9, b2 0.999, eps 1e-8, t 0 (rnn_optim_set changes
 * them).  rnn_optim_step = Optim::step_all(params, lr, wd): matrices with
 * both sides > 1 take the Muon step when muon is set (Nesterov momentum,
 * Newton-Schulz, v -= lr (0.2 sqrt(max(rows, cols)) g + wd v)), the rest
 * AdamW with bias corrections at t + 1; every g is zeroed; t += 1.  Same-shape
 * matrices run Newton-Schulz together. */
typedef struct rnn_optim rnn_optim;
int rnn_optim_create(rnn_ctx *ctx, int muon, size_t ns_steps, rnn_optim **out);
int rnn_optim_destroy(rnn_optim *opt);
int rnn_optim_set(rnn_optim *opt, float mom, float b1, float b2, float eps, size_t t);
size_t rnn_optim_t(const rnn_optim *opt);
int rnn_optim_step(rnn_optim *opt, size_t nparam, const rnn_param *params, float lr, float wd);
/* clip_ (optim.rs:237-251) on a flat gradient: the f64 sum of squares in a
 * fixed order; norm = sqrt as f32; above `max` every element is scaled by
 * max / norm.  *norm (device, may be NULL) receives the norm. */
int rnn_clip_grad_norm(rnn_ctx *ctx, size_t len, float *g, float max, float *norm);
/* clip_ (optim.rs:237-251) over the gradients of a parameter list, as the
 * reference calls it (train.rs:372-375): one f64 sum of squares over every
 * gradient, norm = sqrt as f32 into *norm (device, may be NULL); above `max`
 * every gradient is scaled by max / norm.  The list's pointer table is kept on
 * the device and uploaded again only when the list changes. */
int rnn_clip_params(rnn_ctx *ctx, size_t nparam, const rnn_param *params, float max,
                    float *norm);
/* Ema::update (optim.rs:283-287): w = d w + (1 - d) v, with d computed by
 * the caller as min(decay, (1 + t) / (10 + t)). */
int rnn_ema_update(rnn_ctx *ctx, size_t len, float *w, const float *v, float d);
/* Ema::update over a whole parameter list (train.rs:377-379): w[i] = d w[i] +
 * (1 - d) params[i].v, one launch for the list (pointer table cached as in
 * rnn_clip_params). */
int rnn_ema_update_params(rnn_ctx *ctx, size_t nparam, float *const *w, const rnn_param *params,
                          float d);
/* f32::powi as the reference's bias corrections compute it. */
float rnn_powi_f32(float a, int b);
/* lr_at (train.rs:21-28), host only: linear warm-up over `warm` steps, then a
 * cosine from peak down to lo at step `total`, in f32. */
float rnn_lr_at(float peak, float lo, size_t step, size_t total, size_t warm);

/* ----------------------------------------------------------- model.rs */
/* Device-resident CIFAR ResNet (ResNet::new, model.rs:113-135): depth_n
 * blocks per stage (6n+2 layers), widths width/2w/4w, nclass outputs, Kaiming
 * initialisation from rng.rs seeded with `seed` (bit-identical to the
 * reference's).  Parameters, gradients, momenta, running statistics and the
 * activations of the last train forward live on the device. */
typedef struct rnn_resnet rnn_resnet;
int rnn_resnet_create(rnn_ctx *ctx, size_t depth_n, size_t width, size_t nclass, uint64_t seed,
                      rnn_resnet **out);
int rnn_resnet_destroy(rnn_resnet *net);
/* Total floats of all parameters / BN running buffers; number of parameter
 * tensors and the length (and weight-decay flag) of tensor i, in the
 * reference's for_each_param order (model.rs:164-175). */
size_t rnn_resnet_num_params(const rnn_resnet *net);
size_t rnn_resnet_num_buffers(const rnn_resnet *net);
size_t rnn_resnet_num_tensors(const rnn_resnet *net);
int rnn_resnet_tensor_len(const rnn_resnet *net, size_t i, size_t *len, int *decay);
/* Device copies of the state in for_each_param order (which 0 = values,
 * 1 = gradients, 2 = momenta) or for_each_buffer order (which 3 = BN running
 * mean / var): exactly one of dst (read out) and src (write in) is set. */
int rnn_resnet_copy(rnn_resnet *net, int which, float *dst, const float *src);
/* ResNet::forward (model.rs:138-150): x [n][3][h][w] -> logits [n][nclass].
 * train = 1 uses batch statistics, updates the running ones and keeps the
 * activations for rnn_resnet_backward. */
int rnn_resnet_forward(rnn_resnet *net, size_t n, size_t h, size_t w, const float *x, int train,
                       float *logits);
/* ResNet::backward (model.rs:152-162): gradients ACCUMULATE into the
 * parameters' g after the last train forward. */
int rnn_resnet_backward(rnn_resnet *net, const float *dlogits);
/* ResNet::step (model.rs:205-207): Param::step on every parameter. */
int rnn_resnet_step(rnn_resnet *net, float lr, float momentum, float wd);
/* One train step (train.rs:686-699): forward(train), softmax_ce with label
 * smoothing, backward, step.  labels: device u32[n].  loss / correct (device,
 * may be NULL) receive the mean loss and the hit count.  Replayed from a
 * hipGraph from the second call on for a given (n, h, w).  x and labels both
 * NULL: the batch is the one already in the network's input slots
 * (rnn_resnet_inputs), nothing is copied. */
int rnn_resnet_train_step(rnn_resnet *net, size_t n, size_t h, size_t w, const float *x,
                          const uint32_t *labels, float smooth, float lr, float momentum, float wd,
                          float *loss, uint32_t *correct);
/* The network's own input slots for batches of n x 3 x h x w (planning that
 * shape): device x[n][3][h][w] and labels u32[n] that a loader may fill in
 * place before rnn_resnet_train_step(x = labels = NULL) -- the batch
 * assembly of train.rs:670-684 writing straight to where the step reads.
 * Valid until the shape changes or the network is destroyed. */
int rnn_resnet_inputs(rnn_resnet *net, size_t n, size_t h, size_t w, float **x,
                      uint32_t **labels);
/* Logits of the last forward (device [n][nclass]). */
int rnn_resnet_logits(rnn_resnet *net, float *logits);
/* Train-step graph: enable / disable (drops a recorded graph); state 1 when a
 * graph is recorded, 0 otherwise, with *why the reason recording failed. */
int rnn_resnet_set_graph(rnn_resnet *net, int on);
int rnn_resnet_graph_state(const rnn_resnet *net, const char **why);
/* ResNet::flops (model.rs:179-198): forward FLOP per image at h x w. */
uint64_t rnn_resnet_flops(const rnn_resnet *net, size_t h, size_t w);

/* ------------------------------------------ debug exports (bit-exact tests) */
/* im2col of ONE image through the same staging index math the conv kernels
 * use: col[cin*k*k][oh*ow] (gather_span, conv.rs:68-120). */
/* The device buffers the train step keeps for block `block` of a ResNet
 * (test access, read-only): which = 0 y1 (c1 output), 1 h (b1 + ReLU), 2 y2
 * (c2 output), 3 ys (shortcut conv output), 4 out (block output), 5 / 6 / 7
 * the output gradients of c1 / c2 / the shortcut conv of the last backward,
 * 8 / 9 the batch mean then invstd of b1 / b2 ([2 cout]), 10 the block's
 * input (the previous block's output; for block 0 the stem's ReLU output).
 * *len: floats. */
int rnn_dbg_resnet_buffer(rnn_resnet *net, size_t block, int which, const float **ptr,
                          size_t *len);
/* The grouped weight-gradient launch(es) of the train step (every 3x3
 * stride-1 conv's dW in one persistent launch), enqueued once more on the
 * context's stream over the buffers the last backward left (its output
 * gradients and activations; the slabs are rewritten with the same values),
 * when `launch` is set.  *flops: the launch's algorithmic FLOP (0 when the
 * current plan has no grouped launch).  No counterpart in the reference: it
 * exists to time that kernel alone (benchmarks). */
int rnn_dbg_resnet_dw_group(rnn_resnet *net, int launch, double *flops);
int rnn_dbg_im2col(rnn_ctx *ctx, const rnn_conv_spec *sp, const float *x_img, float *col);
/* PackedA::pack / pack_t (gemm.rs:54-113) into out[nb*256*mpad] (positions the
 * reference never writes are left untouched). */
int rnn_dbg_pack_a(rnn_ctx *ctx, const float *a, size_t m, size_t k, int transposed, float *out);
/* PackedB::pack / pack_t (gemm.rs:340-400) into out[nb*256*npad]. */
int rnn_dbg_pack_b(rnn_ctx *ctx, const float *b, size_t n, size_t k, int transposed, float *out);
/* rel_index computed on the device into idx (device, th*tw*mh*mw u32). */
int rnn_dbg_rel_index(rnn_ctx *ctx, uint32_t th, uint32_t tw, uint32_t mh, uint32_t mw,
                      uint32_t *idx);

#ifdef __cplusplus
}
#endif
#endif
