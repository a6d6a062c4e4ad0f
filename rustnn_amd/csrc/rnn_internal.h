// Internal declarations shared by the HIP sources of librnn.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <mutex>
#include <vector>

#include "../../include/rnn.h"

struct rnn_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    bool own_stream = false;
    int num_cus = 256;
    // Growing device workspace (split-K partials, packed weights, attention
    // reductions).  Reallocated only when a call needs more; the stream is
    // synchronised first so no in-flight kernel still reads the old block.
    void *ws = nullptr;
    size_t ws_bytes = 0;
    // Attention relative-index tables (forward index + inverse CSR), uploaded
    // once per distinct table.
    std::vector<uint32_t> rel_host;  // last uploaded relidx (host copy)
    uint32_t *rel_dev = nullptr;     // [tq*tk] relidx, then CSR rowptr[nrel+1], then pos[tq*tk]
    size_t rel_cap = 0;              // u32 capacity of rel_dev
    uint32_t *rel_pinned = nullptr;  // staging for the async upload
    size_t rel_pinned_cap = 0;
    uint32_t rel_nrel = 0;
    std::recursive_mutex mu;
    char err[512] = {0};
};

// Records a message and returns `code`.
int rnn_fail(rnn_ctx *ctx, int code, const char *fmt, ...);

#define RNN_HIP(ctx, expr)                                                              \
    do {                                                                                \
        hipError_t e_ = (expr);                                                         \
        if (e_ != hipSuccess)                                                           \
            return rnn_fail((ctx), RNN_E_HIP, "%s failed: %s (%s:%d)", #expr,           \
                            hipGetErrorString(e_), __FILE__, __LINE__);                 \
    } while (0)

// Checks the launch status of the kernel just enqueued.
#define RNN_LAUNCHED(ctx)                                                               \
    do {                                                                                \
        hipError_t e_ = hipGetLastError();                                              \
        if (e_ != hipSuccess)                                                           \
            return rnn_fail((ctx), RNN_E_HIP, "kernel launch failed: %s (%s:%d)",       \
                            hipGetErrorString(e_), __FILE__, __LINE__);                 \
    } while (0)

// Returns a device workspace of at least `bytes` (256-byte aligned), or
// nullptr after recording RNN_E_NOMEM / RNN_E_HIP in ctx.
void *rnn_workspace(rnn_ctx *ctx, size_t bytes);

// Bump allocator over one workspace block.
struct WsCarve {
    size_t off = 0;
    size_t take(size_t bytes) {
        size_t o = off;
        off += (bytes + 255) & ~size_t(255);
        return o;
    }
};

static inline size_t rnn_div_up(size_t a, size_t b) { return (a + b - 1) / b; }
static inline size_t rnn_round_up(size_t a, size_t b) { return rnn_div_up(a, b) * b; }

// fp32 MFMA operand / accumulator vectors.
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Index of the calling wave in its workgroup, as a wave-uniform (scalar)
// value: loops and branches on it stay scalar instead of exec-masked.
__device__ __forceinline__ int wave_index() {
    return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

// Entry points implemented in the kernel sources, called from the C ABI.
int rnn_gemm_launch(rnn_ctx *ctx, size_t count, size_t m, size_t n, size_t k, const float *a,
                    size_t stride_a, int at, const float *b, size_t stride_b, int bt, float *c,
                    size_t stride_c, int acc, const float *bias);
int rnn_colsum_launch(rnn_ctx *ctx, size_t rows, size_t cols, const float *x, float *out);
// Specialised forward (dx = 0) / dX (dx = 1) convolution; RNN_E_UNSUPPORTED
// when (k, stride, pad) has no specialisation.
int rnn_conv_fast(rnn_ctx *ctx, int dx, const rnn_conv_spec *sp, size_t n, const float *src,
                  const float *w, float *dst);
// dW += over the batch (k = 1 or 3).
int rnn_conv_dw(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *dy, const float *x,
                float *dw);

// ResNet layer launchers (nn.hip).  Per-channel BN coefficients: train mode
// uses (mean, invstd, gamma, beta); eval mode (eval = true) uses the
// precomputed scale / shift in the mean / invstd slots.
struct RnnBnCoef {
    bool eval;
    const float *mean, *invstd, *gamma, *beta;
};
// f64 elements of BN partial-sum scratch for n images of c channels.
size_t rnn_bn_scratch_doubles(size_t n, size_t c);
// Batch statistics: mean / invstd, and running mean / var when rm is set.
int rnn_bn_stats_launch(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *x, double *part,
                        float *mean, float *invstd, float *rm, float *rv, float mom, float eps);
// out = [relu](bn(x) [+ skip | + sbn(skip)]); skip_mode 0 / 1 / 2 (2 and 1
// imply relu).
int rnn_bn_apply_launch(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *x,
                        const RnnBnCoef &bn, int relu, int skip_mode, const float *skip,
                        const RnnBnCoef &sbn, float *out);
int rnn_bn_eval_prep_launch(rnn_ctx *ctx, size_t c, const float *gamma, const float *beta,
                            const float *rm, const float *rv, float eps, float *sc, float *sh);
// BN backward with relu_back by `mask` folded in (mask may be null); dgamma /
// dbeta accumulate (may be null); dgdb[2c] is scratch.
int rnn_bn_backward_launch(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *dy,
                           const float *mask, const float *x, const float *mean,
                           const float *invstd, const float *gamma, float *dx, float *dgamma,
                           float *dbeta, double *part, float *dgdb);
// a += [mask] b.
int rnn_add_launch(rnn_ctx *ctx, size_t len, float *a, const float *b, const float *mask);
int rnn_gap_forward_launch(rnn_ctx *ctx, size_t nc, size_t hw, const float *x, float *y);
int rnn_gap_backward_launch(rnn_ctx *ctx, size_t nc, size_t hw, const float *dy, float *dx);
int rnn_fc_forward_launch(rnn_ctx *ctx, size_t rows, size_t fin, size_t fout, const float *x,
                          const float *w, const float *b, float *y);
int rnn_fc_backward_launch(rnn_ctx *ctx, size_t rows, size_t fin, size_t fout, const float *dy,
                           const float *x, const float *w, float *dw, float *db, float *dx);
// scal (device, may be null) overrides smooth with scal[3].
int rnn_softmax_ce_launch(rnn_ctx *ctx, size_t rows, size_t nclass, const float *logits,
                          const uint32_t *labels, float smooth, const float *scal, float *dl,
                          float *loss, uint32_t *correct);
// Nesterov SGD over [0, len), weight decay on [0, ndecay); scal (device, may
// be null) overrides (lr, mom, wd) with scal[0..3].
int rnn_sgd_launch(rnn_ctx *ctx, size_t len, size_t ndecay, float *v, float *g, float *m, float lr,
                   float mom, float wd, const float *scal);
int rnn_set_scalars_launch(rnn_ctx *ctx, float *scal, float a, float b, float c, float d);
