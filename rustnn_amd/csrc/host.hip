// Host-slice entry points for the Rust shim (rnn-sys): the reference's layer
// code keeps its tensors in host Vec<f32> (nn.rs Tensor, linear.rs, attn.rs
// Tok), so each *_host call copies its operands into a staging block on the
// device, runs the device entry point of the same name on the context's
// stream, copies the outputs back and waits for the stream.  Semantics --
// accumulation, the k = 0 cases, aliasing of dq / dkv -- are those of the
// device entry points, which the reference functions cited in include/rnn.h
// define.
#include "rnn_internal.h"

#include <algorithm>
#include <vector>

namespace {

enum StageMode { ST_IN = 1, ST_OUT = 2, ST_INOUT = 3 };

struct StageBuf {
    const void *host;
    size_t bytes;
    int mode;
    size_t off;
};

// One call's operands in the context's staging block.  A host pointer named
// twice (a fused QKV buffer read as queries and as keys / values, or dq and
// dkv aliasing in SelfAttn::backward) is staged once, so accumulation into
// aliased outputs stays in one device copy.
struct Stage {
    rnn_ctx *ctx;
    std::vector<StageBuf> bufs;
    char *base = nullptr;

    explicit Stage(rnn_ctx *c) : ctx(c) {}

    int add(const void *host, size_t bytes, int mode) {
        if (!host) return -1;
        for (size_t i = 0; i < bufs.size(); i++)
            if (bufs[i].host == host) {
                bufs[i].bytes = std::max(bufs[i].bytes, bytes);
                bufs[i].mode |= mode;
                return (int)i;
            }
        bufs.push_back({host, bytes, mode, 0});
        return (int)bufs.size() - 1;
    }

    // Sizes the staging block (it only grows; the stream is synchronised
    // before an old block is freed) and queues the host -> device copies.
    int commit() {
        size_t total = 0;
        for (auto &b : bufs) {
            b.off = total;
            total += rnn_round_up(std::max<size_t>(b.bytes, 1), 256);
        }
        if (total > ctx->hstage_bytes) {
            if (ctx->hstage) {
                RNN_HIP(ctx, hipStreamSynchronize(ctx->stream));
                (void)hipFree(ctx->hstage);
                ctx->hstage = nullptr;
                ctx->hstage_bytes = 0;
            }
            RNN_HIP(ctx, hipMalloc(&ctx->hstage, total));
            ctx->hstage_bytes = total;
        }
        base = (char *)ctx->hstage;
        for (auto &b : bufs)
            if ((b.mode & ST_IN) && b.bytes)
                RNN_HIP(ctx, hipMemcpyAsync(base + b.off, b.host, b.bytes, hipMemcpyHostToDevice,
                                            ctx->stream));
        return RNN_OK;
    }

    template <class T>
    T *dev(int i) const {
        return i < 0 ? nullptr : (T *)(base + bufs[i].off);
    }

    // Runs the reductions a deferral holds (the outputs must be complete),
    // queues the device -> host copies and waits for them.
    int finish() {
        int rc = rnn_ctx_flush(ctx);
        if (rc) return rc;
        for (auto &b : bufs)
            if ((b.mode & ST_OUT) && b.bytes)
                RNN_HIP(ctx, hipMemcpyAsync(const_cast<void *>(b.host), base + b.off, b.bytes,
                                            hipMemcpyDeviceToHost, ctx->stream));
        RNN_HIP(ctx, hipStreamSynchronize(ctx->stream));
        return RNN_OK;
    }
};

constexpr size_t F = sizeof(float);

// Floats a strided head buffer spans: rows r of n images at r*stride, the
// last row's heads ending at off + h*dh (attn.rs:74-141).
size_t rows_extent(size_t n, size_t t, size_t stride, size_t off, size_t hdh) {
    return n * t == 0 ? 0 : (n * t - 1) * stride + off + hdh;
}

}  // namespace

extern "C" {

int rnn_matmul_host(rnn_ctx *ctx, size_t m, size_t n, size_t k, const float *a, int at,
                    const float *b, int bt, float *c, int acc) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (m == 0 || n == 0) return RNN_OK;
    if (!c || (k && (!a || !b))) return rnn_fail(ctx, RNN_E_NULL, "matmul_host: null operand");
    Stage s(ctx);
    const int ia = s.add(a, m * k * F, ST_IN), ib = s.add(b, k * n * F, ST_IN);
    const int ic = s.add(c, m * n * F, acc ? ST_INOUT : ST_OUT);
    int rc = s.commit();
    if (rc) return rc;
    rc = rnn_matmul(ctx, m, n, k, s.dev<float>(ia), at, s.dev<float>(ib), bt, s.dev<float>(ic),
                    acc);
    return rc ? rc : s.finish();
}

int rnn_gemm_small_batched_host(rnn_ctx *ctx, size_t count, size_t m, size_t n, size_t k,
                                const float *a, size_t stride_a, int at, const float *b,
                                size_t stride_b, int bt, float *c, size_t stride_c, int acc) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (count == 0 || m == 0 || n == 0) return RNN_OK;
    if (!c || (k && (!a || !b)))
        return rnn_fail(ctx, RNN_E_NULL, "gemm_small_batched_host: null operand");
    Stage s(ctx);
    const int ia = s.add(a, ((count - 1) * stride_a + m * k) * F, ST_IN);
    const int ib = s.add(b, ((count - 1) * stride_b + k * n) * F, ST_IN);
    // C is read back whole: k = 0 leaves it untouched, and the gaps between
    // strided problems keep the caller's values
    const int ic = s.add(c, ((count - 1) * stride_c + m * n) * F, ST_INOUT);
    int rc = s.commit();
    if (rc) return rc;
    rc = rnn_gemm_small_batched(ctx, count, m, n, k, s.dev<float>(ia), stride_a, at,
                                s.dev<float>(ib), stride_b, bt, s.dev<float>(ic), stride_c, acc);
    return rc ? rc : s.finish();
}

int rnn_matmul_dw_host(rnn_ctx *ctx, size_t m, size_t n, size_t k, const float *a,
                       const float *b, float *c) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (m == 0 || n == 0 || k == 0) return RNN_OK;
    if (!a || !b || !c) return rnn_fail(ctx, RNN_E_NULL, "matmul_dw_host: null operand");
    Stage s(ctx);
    const int ia = s.add(a, k * m * F, ST_IN), ib = s.add(b, k * n * F, ST_IN);
    const int ic = s.add(c, m * n * F, ST_INOUT);
    int rc = s.commit();
    if (rc) return rc;
    rc = rnn_matmul_dw(ctx, m, n, k, s.dev<float>(ia), s.dev<float>(ib), s.dev<float>(ic));
    return rc ? rc : s.finish();
}

int rnn_conv2d_forward_host(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *x,
                            const float *w, float *y) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (!sp) return rnn_fail(ctx, RNN_E_NULL, "conv2d_forward_host: null spec");
    if (n == 0) return RNN_OK;
    Stage s(ctx);
    const int ix = s.add(x, n * sp->cin * sp->h * sp->w * F, ST_IN);
    const int iw = s.add(w, (size_t)sp->cout * sp->cin * sp->k * sp->k * F, ST_IN);
    const int iy = s.add(y, n * sp->cout * sp->oh * sp->ow * F, ST_OUT);
    int rc = s.commit();
    if (rc) return rc;
    rc = rnn_conv2d_forward(ctx, sp, n, s.dev<float>(ix), s.dev<float>(iw), s.dev<float>(iy));
    return rc ? rc : s.finish();
}

int rnn_conv2d_backward_w_host(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n,
                               const float *dy, const float *x, float *dw) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (!sp) return rnn_fail(ctx, RNN_E_NULL, "conv2d_backward_w_host: null spec");
    if (n == 0) return RNN_OK;
    Stage s(ctx);
    const int idy = s.add(dy, n * sp->cout * sp->oh * sp->ow * F, ST_IN);
    const int ix = s.add(x, n * sp->cin * sp->h * sp->w * F, ST_IN);
    const int iw = s.add(dw, (size_t)sp->cout * sp->cin * sp->k * sp->k * F, ST_INOUT);
    int rc = s.commit();
    if (rc) return rc;
    rc = rnn_conv2d_backward_w(ctx, sp, n, s.dev<float>(idy), s.dev<float>(ix), s.dev<float>(iw));
    return rc ? rc : s.finish();
}

int rnn_conv2d_backward_x_host(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n,
                               const float *dy, const float *w, float *dx) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (!sp) return rnn_fail(ctx, RNN_E_NULL, "conv2d_backward_x_host: null spec");
    if (n == 0) return RNN_OK;
    Stage s(ctx);
    const int idy = s.add(dy, n * sp->cout * sp->oh * sp->ow * F, ST_IN);
    const int iw = s.add(w, (size_t)sp->cout * sp->cin * sp->k * sp->k * F, ST_IN);
    const int ix = s.add(dx, n * sp->cin * sp->h * sp->w * F, ST_OUT);
    int rc = s.commit();
    if (rc) return rc;
    rc = rnn_conv2d_backward_x(ctx, sp, n, s.dev<float>(idy), s.dev<float>(iw), s.dev<float>(ix));
    return rc ? rc : s.finish();
}

int rnn_attn_forward_host(rnn_ctx *ctx, const rnn_attn_desc *d, size_t n, const float *q,
                          const float *kv, const float *tau, const float *rel, float *p,
                          float *o) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (!d) return rnn_fail(ctx, RNN_E_NULL, "attn_forward_host: null descriptor");
    if (n == 0) return RNN_OK;
    Stage s(ctx);
    const size_t hdh = (size_t)d->h * d->dh;
    const int iq = s.add(q, rows_extent(n, d->tq, d->qstride, d->qoff, hdh) * F, ST_IN);
    const int ikv = s.add(
        kv, rows_extent(n, d->tk, d->kvstride, std::max(d->koff, d->voff), hdh) * F, ST_IN);
    const int it = s.add(tau, (size_t)d->h * F, ST_IN);
    const int ir = s.add(rel, (size_t)d->h * d->nrel * F, ST_IN);
    const int ip = s.add(p, n * d->h * d->tq * d->tk * F, ST_OUT);
    const int io = s.add(o, n * d->tq * d->h * d->dh * F, ST_OUT);
    int rc = s.commit();
    if (rc) return rc;
    rc = rnn_attn_forward(ctx, d, n, s.dev<float>(iq), s.dev<float>(ikv), s.dev<float>(it),
                          s.dev<float>(ir), s.dev<float>(ip), s.dev<float>(io));
    return rc ? rc : s.finish();
}

int rnn_attn_backward_host(rnn_ctx *ctx, const rnn_attn_desc *d, size_t n, const float *q,
                           const float *kv, const float *tau, const float *p, const float *dout,
                           float *dq, float *dkv, float *dtau, float *drel) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (!d) return rnn_fail(ctx, RNN_E_NULL, "attn_backward_host: null descriptor");
    if (n == 0) return RNN_OK;
    Stage s(ctx);
    const size_t hdh = (size_t)d->h * d->dh;
    const size_t nq = rows_extent(n, d->tq, d->qstride, d->qoff, hdh);
    const size_t nkv = rows_extent(n, d->tk, d->kvstride, std::max(d->koff, d->voff), hdh);
    const int iq = s.add(q, nq * F, ST_IN);
    const int ikv = s.add(kv, nkv * F, ST_IN);
    const int it = s.add(tau, (size_t)d->h * F, ST_IN);
    const int ip = s.add(p, n * d->h * d->tq * d->tk * F, ST_IN);
    const int id = s.add(dout, n * d->tq * hdh * F, ST_IN);
    const int idq = s.add(dq, nq * F, ST_INOUT);
    const int idkv = s.add(dkv, nkv * F, ST_INOUT);
    const int idt = s.add(dtau, (size_t)d->h * F, ST_INOUT);
    const int idr = s.add(drel, (size_t)d->h * d->nrel * F, ST_INOUT);
    int rc = s.commit();
    if (rc) return rc;
    rc = rnn_attn_backward(ctx, d, n, s.dev<float>(iq), s.dev<float>(ikv), s.dev<float>(it),
                           s.dev<float>(ip), s.dev<float>(id), s.dev<float>(idq),
                           s.dev<float>(idkv), s.dev<float>(idt), s.dev<float>(idr));
    return rc ? rc : s.finish();
}

int rnn_linear_forward_host(rnn_ctx *ctx, size_t rows, size_t fin, size_t fout, const float *x,
                            const float *w, const float *b, float *y) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (rows == 0 || fout == 0) return RNN_OK;
    Stage s(ctx);
    const int ix = s.add(x, rows * fin * F, ST_IN), iw = s.add(w, fout * fin * F, ST_IN);
    const int ib = s.add(b, fout * F, ST_IN), iy = s.add(y, rows * fout * F, ST_OUT);
    int rc = s.commit();
    if (rc) return rc;
    rc = rnn_linear_forward(ctx, rows, fin, fout, s.dev<float>(ix), s.dev<float>(iw),
                            s.dev<float>(ib), s.dev<float>(iy));
    return rc ? rc : s.finish();
}

int rnn_linear_backward_host(rnn_ctx *ctx, size_t rows, size_t fin, size_t fout,
                             const float *dy, const float *x, const float *w, float *dw,
                             float *db, float *dx) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (rows == 0) return RNN_OK;
    Stage s(ctx);
    const int idy = s.add(dy, rows * fout * F, ST_IN), ix = s.add(x, rows * fin * F, ST_IN);
    const int iw = s.add(w, fout * fin * F, ST_IN), idw = s.add(dw, fout * fin * F, ST_INOUT);
    const int idb = s.add(db, fout * F, ST_INOUT), idx = s.add(dx, rows * fin * F, ST_OUT);
    int rc = s.commit();
    if (rc) return rc;
    rc = rnn_linear_backward(ctx, rows, fin, fout, s.dev<float>(idy), s.dev<float>(ix),
                             s.dev<float>(iw), s.dev<float>(idw), s.dev<float>(idb),
                             s.dev<float>(idx));
    return rc ? rc : s.finish();
}

}  // extern "C"
