// Context, stream, workspace and error reporting of librnn.so.
//
// Replaces the reference's process-wide rayon pool (main.rs:41-48) and the
// thread-local / per-task packing scratch (gemm.rs:411-420, nn.rs:178,
// attn.rs:170) with one device context: a stream and a device workspace that
// only grows, so steady-state calls never allocate.
#include "rnn_internal.h"

#include <algorithm>

#include <cstring>

// The fixed scratch of the no-allocation entry points: partial results that
// the other entry points keep in the context's growing workspace.  Every
// device the library runs on holds one copy until the process ends.  In host
// code the array's name is only a stand-in for the device symbol; the device
// address of each device's copy comes from hipGetSymbolAddress, looked up once
// per device (with that device current) and kept in g_scratch_addr.
static __device__ __align__(256) float scratch[RNN_NOALLOC_SCRATCH_BYTES / sizeof(float)];

static std::mutex g_scratch_mu;
static std::map<int, float *> g_scratch_addr;

// Device address of `device`'s scratch copy; device must be current.
static int scratch_address(int device, float **out) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    auto it = g_scratch_addr.find(device);
    if (it != g_scratch_addr.end()) {
        *out = it->second;
        return RNN_OK;
    }
    float *ptr = nullptr;
    hipError_t e = hipGetSymbolAddress((void **)&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) return RNN_E_HIP;
    g_scratch_addr[device] = ptr;
    *out = ptr;
    return RNN_OK;
}

// Per device: the lock the no-allocation calls hold while they enqueue, and
// the event recorded after the last call's kernels with the stream it was
// recorded on, so that a call on another stream waits for that one first.
struct NoallocOrder {
    std::mutex mu;
    hipEvent_t last = nullptr;
    hipStream_t last_stream = nullptr;
    bool pending = false;
};
static std::mutex g_order_mu;
static std::map<int, NoallocOrder> g_order;

static NoallocOrder &noalloc_order(int device) {
    std::lock_guard<std::mutex> lk(g_order_mu);
    return g_order[device];
}

int rnn_noalloc_scratch(rnn_ctx *ctx, float **out) {
    if (ctx->noalloc_scratch) {
        *out = ctx->noalloc_scratch;
        return RNN_OK;
    }
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return RNN_E_HIP;
    if (cur != ctx->device && hipSetDevice(ctx->device) != hipSuccess) return RNN_E_HIP;
    const int rc = scratch_address(ctx->device, &ctx->noalloc_scratch);
    if (cur != ctx->device) (void)hipSetDevice(cur);
    if (rc != RNN_OK) return rnn_fail(ctx, rc, "no-allocation scratch: hipGetSymbolAddress failed");
    *out = ctx->noalloc_scratch;
    return RNN_OK;
}

int rnn_noalloc_run(rnn_ctx *ctx, const std::function<int()> &enqueue) {
    NoallocOrder &o = noalloc_order(ctx->device);
    std::lock_guard<std::mutex> lk(o.mu);
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    RNN_HIP(ctx, hipStreamIsCapturing(ctx->stream, &cap));
    const bool eager = cap == hipStreamCaptureStatusNone;
    // the previous call on this device ran on another stream: this stream
    // waits for its kernels before reusing the scratch
    if (eager && o.pending && o.last_stream != ctx->stream)
        RNN_HIP(ctx, hipStreamWaitEvent(ctx->stream, o.last, 0));
    const int rc = enqueue();
    if (rc != RNN_OK || !eager) return rc;
    if (!o.last) RNN_HIP(ctx, hipEventCreateWithFlags(&o.last, hipEventDisableTiming));
    RNN_HIP(ctx, hipEventRecord(o.last, ctx->stream));
    o.last_stream = ctx->stream;
    o.pending = true;
    return RNN_OK;
}

int rnn_fail(rnn_ctx *ctx, int code, const char *fmt, ...) {
    if (ctx) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(ctx->err, sizeof(ctx->err), fmt, ap);
        va_end(ap);
    }
    return code;
}

void *rnn_workspace(rnn_ctx *ctx, size_t bytes) {
    bytes = rnn_round_up(bytes ? bytes : 256, 256);
    if (bytes <= ctx->ws_bytes) return ctx->ws;
    if (ctx->ws) {
        // Earlier kernels on this stream may still read the old block.
        hipError_t e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) {
            rnn_fail(ctx, RNN_E_HIP, "hipStreamSynchronize: %s", hipGetErrorString(e));
            return nullptr;
        }
        (void)hipFree(ctx->ws);
        ctx->ws = nullptr;
        ctx->ws_bytes = 0;
    }
    size_t want = bytes + bytes / 4;  // headroom against creeping regrowth
    hipError_t e = hipMalloc(&ctx->ws, want);
    if (e != hipSuccess) {
        ctx->ws = nullptr;
        rnn_fail(ctx, RNN_E_NOMEM, "workspace hipMalloc(%zu): %s", want, hipGetErrorString(e));
        return nullptr;
    }
    ctx->ws_bytes = want;
    return ctx->ws;
}

int rnn_dev_table(rnn_ctx *ctx, RnnDevTable &t, const void *src, size_t bytes, void **dev) {
    if (t.dev && bytes == t.host.size() &&
        (bytes == 0 || std::memcmp(t.host.data(), src, bytes) == 0)) {
        *dev = t.dev;
        return RNN_OK;
    }
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    RNN_HIP(ctx, hipStreamIsCapturing(ctx->stream, &cs));
    if (cs != hipStreamCaptureStatusNone)
        return rnn_fail(ctx, RNN_E_INVALID,
                        "tensor list changed during graph capture (call once before capturing)");
    RNN_HIP(ctx, hipStreamSynchronize(ctx->stream));
    const size_t want = rnn_round_up(bytes ? bytes : 256, 256);
    if (want > t.cap) {
        if (t.dev) (void)hipFree(t.dev);
        t.dev = nullptr;
        t.cap = 0;
        hipError_t e = hipMalloc(&t.dev, want);
        if (e != hipSuccess) {
            t.dev = nullptr;
            return rnn_fail(ctx, RNN_E_NOMEM, "table hipMalloc(%zu): %s", want,
                            hipGetErrorString(e));
        }
        t.cap = want;
    }
    if (bytes) RNN_HIP(ctx, hipMemcpy(t.dev, src, bytes, hipMemcpyHostToDevice));
    t.host.assign((const char *)src, (const char *)src + bytes);
    *dev = t.dev;
    return RNN_OK;
}

void rnn_dev_table_free(RnnDevTable &t) {
    if (t.dev) (void)hipFree(t.dev);
    t.dev = nullptr;
    t.cap = 0;
    t.host.clear();
}

// ------------------------------------------ deferred gradient reductions
void *rnn_defer_take(rnn_ctx *ctx, size_t bytes) {
    bytes = rnn_round_up(std::max<size_t>(bytes, 1), 256);
    while (ctx->dblk < ctx->darena.size()) {
        auto &b = ctx->darena[ctx->dblk];
        if (ctx->doff + bytes <= b.second) {
            void *p = b.first + ctx->doff;
            ctx->doff += bytes;
            return p;
        }
        ctx->dblk++;
        ctx->doff = 0;
    }
    // a new block (earlier blocks keep their pending partials)
    const size_t want = std::max<size_t>(bytes, (size_t)64 << 20);
    char *mem = nullptr;
    hipError_t e = hipMalloc((void **)&mem, want);
    if (e != hipSuccess) {
        rnn_fail(ctx, RNN_E_NOMEM, "deferred partials hipMalloc(%zu): %s", want,
                 hipGetErrorString(e));
        return nullptr;
    }
    ctx->darena.emplace_back(mem, want);
    ctx->dblk = ctx->darena.size() - 1;
    ctx->doff = bytes;
    return mem;
}

void rnn_defer_push(rnn_ctx *ctx, const RnnDeferSeg &s) { ctx->dsegs.push_back(s); }

namespace {

constexpr int DEFER_BATCH = 48;  // segments per launch (kernel arguments by value)

struct DeferBatch {
    RnnDeferSeg seg[DEFER_BATCH];
    unsigned blk0[DEFER_BATCH + 1];  // first block of each segment, then the total
    int nseg;
};

unsigned defer_blocks(const RnnDeferSeg &s) {
    const size_t per = s.kind == RNN_DEFER_COLS     ? 16
                       : s.kind == RNN_DEFER_ATTN    ? 32
                       : s.kind == RNN_DEFER_CHUNKS4 ? 1024
                                                     : 256;
    return (unsigned)rnn_div_up((size_t)s.len, per);
}

// Every queued reduction of a batch: block b serves the segment whose block
// range holds it, with the code of that segment's own reduction kernel.
__global__ __launch_bounds__(256) void deferred_reduce_kernel(DeferBatch b) {
    int lo = 0, hi = b.nseg - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (b.blk0[mid] <= blockIdx.x)
            lo = mid;
        else
            hi = mid - 1;
    }
    const RnnDeferSeg &s = b.seg[lo];
    const unsigned blk = blockIdx.x - b.blk0[lo];
    if (s.kind == RNN_DEFER_COLS) {
        rnn_colsum_red_block(s.nrow, (size_t)s.len, (size_t)s.split, (const double *)s.part,
                             s.out0, s.out1, blk);
        return;
    }
    if (s.kind == RNN_DEFER_ATTN) {
        const int h = (int)(s.len - s.split);
        rnn_attn_reduce_block((const double *)s.part, (const float *)s.part2, s.nrow, h,
                              (int)(s.split / h), s.out1, s.out0, blk);
        return;
    }
    const long long e = (long long)blk * 256 + threadIdx.x;
    if (s.kind == RNN_DEFER_CHUNKS4) {
        if (4 * e < s.len) rnn_chunk_sum4((const float *)s.part, s.nrow, s.len, s.out0, s.acc, 4 * e);
        return;
    }
    if (e >= s.len) return;
    if (s.kind == RNN_DEFER_CHUNKS)
        rnn_chunk_sum((const float *)s.part, s.nrow, s.len, s.out0, s.acc, e);
    else
        rnn_rows64_sum((const double *)s.part, s.nrow, s.len, s.out0, e);
}

int defer_flush(rnn_ctx *ctx) {
    for (size_t i0 = 0; i0 < ctx->dsegs.size(); i0 += DEFER_BATCH) {
        DeferBatch b{};
        b.nseg = (int)std::min<size_t>(DEFER_BATCH, ctx->dsegs.size() - i0);
        unsigned tot = 0;
        for (int k = 0; k < b.nseg; k++) {
            b.seg[k] = ctx->dsegs[i0 + k];
            b.blk0[k] = tot;
            tot += defer_blocks(b.seg[k]);
        }
        b.blk0[b.nseg] = tot;
        if (tot == 0) continue;
        hipLaunchKernelGGL(deferred_reduce_kernel, dim3(tot), dim3(256), 0, ctx->stream, b);
        RNN_LAUNCHED(ctx);
    }
    ctx->dsegs.clear();
    ctx->dblk = 0;
    ctx->doff = 0;
    return RNN_OK;
}

}  // namespace

extern "C" {

const char *rnn_status_string(int s) {
    switch (s) {
        case RNN_OK: return "ok";
        case RNN_E_INVALID: return "invalid argument";
        case RNN_E_NULL: return "null pointer";
        case RNN_E_HIP: return "HIP runtime error";
        case RNN_E_NOMEM: return "out of device memory";
        case RNN_E_UNSUPPORTED: return "unsupported shape";
        default: return "unknown status";
    }
}

int rnn_ctx_create(int device, rnn_ctx **out) {
    if (!out) return RNN_E_NULL;
    *out = nullptr;
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) return RNN_E_HIP;
    if (device < 0 || device >= ndev) return RNN_E_INVALID;
    if (hipSetDevice(device) != hipSuccess) return RNN_E_HIP;
    rnn_ctx *c = new rnn_ctx();
    c->device = device;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess) c->num_cus = prop.multiProcessorCount;
    // A stream of default priority (non-blocking w.r.t. the null stream).
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return RNN_E_HIP;
    }
    c->own_stream = true;
    *out = c;
    return RNN_OK;
}

int rnn_ctx_destroy(rnn_ctx *ctx) {
    if (!ctx) return RNN_E_NULL;
    (void)hipSetDevice(ctx->device);
    // gradient reductions still queued by the deferral run before the
    // arena that holds their partials is freed
    int rc = RNN_OK;
    if (!ctx->dsegs.empty()) rc = defer_flush(ctx);
    if (hipStreamSynchronize(ctx->stream) != hipSuccess && rc == RNN_OK) rc = RNN_E_HIP;
    if (ctx->ws) (void)hipFree(ctx->ws);
    if (ctx->hstage) (void)hipFree(ctx->hstage);
    for (auto &b : ctx->darena) (void)hipFree(b.first);
    for (auto &t : ctx->rel_tables) {
        if (t.dev) (void)hipFree(t.dev);
        if (t.pinned) (void)hipHostFree(t.pinned);
    }
    for (auto &kv : ctx->tables) rnn_dev_table_free(kv.second);
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return rc;
}

int rnn_ctx_set_stream(rnn_ctx *ctx, void *stream) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (ctx->stream == (hipStream_t)stream) return RNN_OK;
    // Work queued on the old stream may still use the workspace.
    RNN_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->stream);
    ctx->stream = (hipStream_t)stream;
    ctx->own_stream = false;
    return RNN_OK;
}

void *rnn_ctx_stream(rnn_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

int rnn_ctx_set_defer(rnn_ctx *ctx, int on) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (!on && !ctx->dsegs.empty()) {
        const int rc = defer_flush(ctx);
        if (rc) return rc;
    }
    ctx->defer = on != 0;
    return RNN_OK;
}

int rnn_ctx_flush(rnn_ctx *ctx) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    return defer_flush(ctx);
}

int rnn_ctx_synchronize(rnn_ctx *ctx) {
    if (!ctx) return RNN_E_NULL;
    RNN_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return RNN_OK;
}

const char *rnn_ctx_last_error(rnn_ctx *ctx) { return ctx ? ctx->err : "null context"; }

size_t rnn_ctx_workspace_bytes(rnn_ctx *ctx) { return ctx ? ctx->ws_bytes : 0; }

int rnn_dev_alloc(rnn_ctx *ctx, size_t bytes, void **out) {
    if (!ctx || !out) return RNN_E_NULL;
    *out = nullptr;
    if (bytes == 0) return RNN_OK;
    RNN_HIP(ctx, hipSetDevice(ctx->device));
    hipError_t e = hipMalloc(out, bytes);
    if (e != hipSuccess) {
        *out = nullptr;
        return rnn_fail(ctx, RNN_E_NOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    }
    return RNN_OK;
}

int rnn_dev_free(rnn_ctx *ctx, void *p) {
    if (!ctx) return RNN_E_NULL;
    if (!p) return RNN_OK;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    RNN_HIP(ctx, hipStreamSynchronize(ctx->stream));  // queued kernels may still use p
    RNN_HIP(ctx, hipFree(p));
    return RNN_OK;
}

int rnn_copy_to_device(rnn_ctx *ctx, void *dst_dev, const void *src_host, size_t bytes) {
    if (!ctx) return RNN_E_NULL;
    if (bytes == 0) return RNN_OK;
    if (!dst_dev || !src_host) return rnn_fail(ctx, RNN_E_NULL, "copy_to_device: null pointer");
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    RNN_HIP(ctx, hipMemcpyAsync(dst_dev, src_host, bytes, hipMemcpyHostToDevice, ctx->stream));
    RNN_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return RNN_OK;
}

int rnn_copy_to_host(rnn_ctx *ctx, void *dst_host, const void *src_dev, size_t bytes) {
    if (!ctx) return RNN_E_NULL;
    if (bytes == 0) return RNN_OK;
    if (!dst_host || !src_dev) return rnn_fail(ctx, RNN_E_NULL, "copy_to_host: null pointer");
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    RNN_HIP(ctx, hipMemcpyAsync(dst_host, src_dev, bytes, hipMemcpyDeviceToHost, ctx->stream));
    RNN_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return RNN_OK;
}

int rnn_conv_spec_init(rnn_conv_spec *sp, uint32_t cin, uint32_t cout, uint32_t k,
                       uint32_t stride, uint32_t pad, uint32_t h, uint32_t w) {
    if (!sp) return RNN_E_NULL;
    if (cin == 0 || cout == 0 || k == 0 || stride == 0 || h == 0 || w == 0) return RNN_E_INVALID;
    if (k > h + 2 * pad || k > w + 2 * pad) return RNN_E_INVALID;
    sp->cin = cin;
    sp->cout = cout;
    sp->k = k;
    sp->stride = stride;
    sp->pad = pad;
    sp->h = h;
    sp->w = w;
    sp->oh = (h + 2 * pad - k) / stride + 1;  // Conv2d::out_dim (nn.rs:147-150)
    sp->ow = (w + 2 * pad - k) / stride + 1;
    return RNN_OK;
}

// rel_index (attn.rs:53-72) with RelGeom (attn.rs:21-46): equal grids give
// offsets in [-(th-1), th-1]; a memory grid of twice the resolution measures
// the offset in half tokens, 2*q - m.
int rnn_rel_index(uint32_t th, uint32_t tw, uint32_t mh, uint32_t mw, uint32_t *idx,
                  uint32_t *nrel) {
    if (!idx || !nrel) return RNN_E_NULL;
    if (th == 0 || tw == 0 || mh == 0 || mw == 0) return RNN_E_INVALID;
    int64_t sy, sx, scale, oy, ox;
    if (mh == th) {
        sy = 2 * (int64_t)th - 1;
        sx = 2 * (int64_t)tw - 1;
        scale = 1;
        oy = (int64_t)th - 1;
        ox = (int64_t)tw - 1;
    } else {
        sy = 2 * ((int64_t)th - 1) + mh;
        sx = 2 * ((int64_t)tw - 1) + mw;
        scale = 2;
        oy = (int64_t)mh - 1;
        ox = (int64_t)mw - 1;
    }
    size_t z = 0;
    for (int64_t qy = 0; qy < th; qy++)
        for (int64_t qx = 0; qx < tw; qx++)
            for (int64_t my = 0; my < mh; my++)
                for (int64_t mx = 0; mx < mw; mx++) {
                    int64_t dy = scale * qy - my + oy, dx = scale * qx - mx + ox;
                    idx[z++] = (uint32_t)(dy * sx + dx);
                }
    *nrel = (uint32_t)(sy * sx);
    return RNN_OK;
}

}  // extern "C"
