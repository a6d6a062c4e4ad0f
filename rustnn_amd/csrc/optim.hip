// optim.rs on the device: Muon (Nesterov momentum + Newton-Schulz
// orthogonalisation over the batched GEMM core), AdamW, the global-norm clip
// and the weight EMA.
//
// Reference: newton_schulz (optim.rs:124-145) runs three quintic steps per
// matrix through gemm_small, one rayon task per parameter; step_all
// (optim.rs:177-205) splits the parameters into Muon matrices and AdamW
// tensors; step_adam (optim.rs:207-235); clip_ (optim.rs:237-251);
// Ema::update (optim.rs:270-288).
//
// Here the Muon matrices of one shape go through Newton-Schulz together: the
// 3 products of a quintic step are 3 batched GEMM launches over all matrices
// of that shape, and the elementwise parts are one launch each.  The squared
// Frobenius norm of each matrix is summed in f64 in a fixed order (the
// reference sums in f32 in element order).  Every elementwise formula keeps
// the reference's operation order (no contraction), so AdamW, the momentum,
// the Muon update and the EMA round as the reference does.
#include "rnn_internal.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <vector>

#pragma clang fp contract(off)

namespace {

constexpr float NS_A = 3.4445f;
constexpr float NS_B = -4.7750f;
constexpr float NS_C = 2.0315f;
constexpr int OPT_THREADS = 256;
constexpr int NS_CHUNK = 4096;  // elements of one matrix per block in the norm passes

// One Muon matrix of a same-shape group.
struct MuonMat {
    float *v, *g, *m;
};

// Block sums of g'^2 after the momentum update, in element order per thread
// then a fixed tree: matrix blockIdx.y, chunk blockIdx.x.
__global__ __launch_bounds__(OPT_THREADS) void muon_momentum_kernel(const MuonMat *__restrict__ mats,
                                                                    size_t len, float mom,
                                                                    int momentum, double *part) {
    __shared__ double red[OPT_THREADS / 64];
    const MuonMat mt = mats[blockIdx.y];
    const size_t e0 = (size_t)blockIdx.x * NS_CHUNK, e1 = min(len, e0 + NS_CHUNK);
    double s = 0.0;
    for (size_t e = e0 + threadIdx.x; e < e1; e += OPT_THREADS) {
        float gi = mt.g[e];
        if (momentum) {
            // Optim::step_all (optim.rs:186-189): m = mom m + g; g += mom m
            const float mi = mom * mt.m[e] + gi;
            mt.m[e] = mi;
            gi += mom * mi;
            mt.g[e] = gi;
        }
        s += (double)gi * (double)gi;
    }
    for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = red[0];
        for (int w = 1; w < OPT_THREADS / 64; w++) t += red[w];
        part[(size_t)blockIdx.y * gridDim.x + blockIdx.x] = t;
    }
}

// X[i] = G[i] / (||G[i]||_F + 1e-7), transposed when rows > cols
// (load_maybe_t, optim.rs:41-53, and the normalisation, optim.rs:133-136).
__global__ __launch_bounds__(OPT_THREADS) void ns_load_kernel(const MuonMat *__restrict__ mats,
                                                              const double *__restrict__ part,
                                                              int nchunk, int rows, int cols,
                                                              int tr, float *x) {
    const MuonMat mt = mats[blockIdx.y];
    double ss = 0.0;
    for (int k = 0; k < nchunk; k++) ss += part[(size_t)blockIdx.y * nchunk + k];
    const float norm = sqrtf((float)ss) + 1e-7f;
    const float inv = 1.0f / norm;
    const size_t len = (size_t)rows * cols;
    float *xi = x + (size_t)blockIdx.y * len;
    const size_t e0 = (size_t)blockIdx.x * NS_CHUNK, e1 = min(len, e0 + NS_CHUNK);
    for (size_t e = e0 + threadIdx.x; e < e1; e += OPT_THREADS) {
        // e indexes X; element (j, i) of X is G[i][j] when transposed
        size_t src = e;
        if (tr) {
            const size_t j = e / rows, i = e - j * rows;
            src = i * cols + j;
        }
        xi[e] = mt.g[src] * inv;
    }
}

// B = b A + c AA, in place in A (optim.rs:103-106).
__global__ void ns_combine_a_kernel(float *a, const float *__restrict__ aa, size_t len) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < len;
         i += (size_t)gridDim.x * blockDim.x)
        a[i] = NS_B * a[i] + NS_C * aa[i];
}

// X = a X + T (optim.rs:118-120).
__global__ void ns_combine_x_kernel(float *x, const float *__restrict__ t, size_t len) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < len;
         i += (size_t)gridDim.x * blockDim.x)
        x[i] = NS_A * x[i] + t[i];
}

// End of a Muon step (optim.rs:191-195), reading the orthogonalised matrix
// straight from X (store_maybe_t folded in): v -= lr (scale x + wd v); g = 0.
// With update = 0, only the store back into g (newton_schulz alone).
__global__ void muon_finish_kernel(const MuonMat *__restrict__ mats, const float *__restrict__ x,
                                   int rows, int cols, int tr, int update, float lr, float scale,
                                   float wdp) {
    const MuonMat mt = mats[blockIdx.y];
    const size_t len = (size_t)rows * cols;
    const float *xi = x + (size_t)blockIdx.y * len;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < len;
         e += (size_t)gridDim.x * blockDim.x) {
        // e indexes G; its X element is (j, i) when transposed
        size_t xs = e;
        if (tr) {
            const size_t i = e / cols, j = e - i * cols;
            xs = j * rows + i;
        }
        const float gx = xi[xs];
        if (update) {
            mt.v[e] -= lr * (scale * gx + wdp * mt.v[e]);
            mt.g[e] = 0.0f;
        } else {
            mt.g[e] = gx;
        }
    }
}

// AdamW over several tensors (Optim::step_adam, optim.rs:207-235): block b
// serves the segment whose block range holds it.
struct AdamSeg {
    float *v, *g, *m, *v2;
    size_t len;
    float wd;  // 0 for tensors that do not decay
    uint32_t blk0, nblk;
};

__global__ void adam_kernel(const AdamSeg *__restrict__ segs, int nseg, float lr, float b1,
                            float b2, float eps, float c1, float c2) {
    int lo = 0, hi = nseg - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (segs[mid].blk0 <= blockIdx.x)
            lo = mid;
        else
            hi = mid - 1;
    }
    const AdamSeg s = segs[lo];
    for (size_t i = (size_t)(blockIdx.x - s.blk0) * blockDim.x + threadIdx.x; i < s.len;
         i += (size_t)s.nblk * blockDim.x) {
        const float g = s.g[i];
        const float m = b1 * s.m[i] + (1.0f - b1) * g;
        const float v2 = b2 * s.v2[i] + (1.0f - b2) * g * g;
        s.m[i] = m;
        s.v2[i] = v2;
        s.v[i] -= lr * ((m / c1) / (sqrtf(v2 / c2) + eps) + s.wd * s.v[i]);
        s.g[i] = 0.0f;
    }
}

// clip_ (optim.rs:237-251) on a flat gradient: block sums of g^2 in f64 ...
__global__ __launch_bounds__(OPT_THREADS) void sumsq_kernel(const float *__restrict__ g,
                                                            size_t len, size_t chunk,
                                                            double *part) {
    __shared__ double red[OPT_THREADS / 64];
    const size_t e0 = (size_t)blockIdx.x * chunk, e1 = min(len, e0 + chunk);
    double s = 0.0;
    for (size_t e = e0 + threadIdx.x; e < e1; e += OPT_THREADS) s += (double)g[e] * (double)g[e];
    for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = red[0];
        for (int w = 1; w < OPT_THREADS / 64; w++) t += red[w];
        part[blockIdx.x] = t;
    }
}

// ... then every block adds the partials in order, and scales its share of g
// by max / norm when the norm is above max (the first block stores the norm).
__global__ __launch_bounds__(OPT_THREADS) void clip_scale_kernel(float *g, size_t len,
                                                                 const double *__restrict__ part,
                                                                 int nparts, float max,
                                                                 float *norm_out) {
    double sq = 0.0;
    for (int k = 0; k < nparts; k++) sq += part[k];
    const float norm = (float)sqrt(sq);
    if (blockIdx.x == 0 && threadIdx.x == 0 && norm_out) *norm_out = norm;
    if (!(norm > max && norm > 0.0f)) return;
    const float sc = max / norm;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < len;
         i += (size_t)gridDim.x * blockDim.x)
        g[i] *= sc;
}

// Ema::update (optim.rs:283-287): w = d w + (1 - d) v.
__global__ void ema_kernel(float *w, const float *__restrict__ v, size_t len, float d) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < len;
         i += (size_t)gridDim.x * blockDim.x)
        w[i] = d * w[i] + (1.0f - d) * v[i];
}

unsigned grid_for(size_t items, unsigned threads) {
    return (unsigned)std::max<size_t>(1, std::min<size_t>(rnn_div_up(items, threads), 8192));
}

}  // namespace

// f32::powi with a run-time exponent, as LLVM lowers it (compiler-rt
// __powisf2: square-and-multiply from the low bit).
static float powi_f32(float a, int b) {
    const bool recip = b < 0;
    float r = 1.0f;
    for (;;) {
        if (b & 1) r *= a;
        b /= 2;
        if (b == 0) break;
        a *= a;
    }
    return recip ? 1.0f / r : r;
}

struct rnn_optim {
    rnn_ctx *ctx = nullptr;
    bool muon = true;
    size_t ns_steps = 3;
    float mom = 0.95f, b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
    size_t t = 0;
    // device scratch: Newton-Schulz buffers, norm partials, tables
    void *scratch = nullptr;
    size_t scratch_bytes = 0;
};

namespace {

int ensure_scratch(rnn_optim *o, size_t bytes) {
    if (bytes <= o->scratch_bytes) return RNN_OK;
    rnn_ctx *ctx = o->ctx;
    if (o->scratch) {
        RNN_HIP(ctx, hipStreamSynchronize(ctx->stream));
        RNN_HIP(ctx, hipFree(o->scratch));
        o->scratch = nullptr;
        o->scratch_bytes = 0;
    }
    const size_t want = std::max(bytes, o->scratch_bytes * 2);
    hipError_t e = hipMalloc(&o->scratch, want);
    if (e != hipSuccess)
        return rnn_fail(ctx, RNN_E_NOMEM, "optim scratch hipMalloc(%zu): %s", want,
                        hipGetErrorString(e));
    o->scratch_bytes = want;
    return RNN_OK;
}

// Newton-Schulz (and, with `update`, the rest of the Muon step) for `mats`
// same-shape matrices whose pointer table sits at the start of the scratch.
int ns_group(rnn_optim *o, const std::vector<MuonMat> &mats, size_t rows, size_t cols,
             size_t steps, int momentum, int update, float lr, float wdp) {
    rnn_ctx *ctx = o->ctx;
    const size_t cnt = mats.size();
    const int tr = rows > cols;
    const size_t m = tr ? cols : rows, n = tr ? rows : cols, len = rows * cols;
    const size_t nchunk = rnn_div_up(len, NS_CHUNK);
    WsCarve cv;
    const size_t o_mats = cv.take(cnt * sizeof(MuonMat));
    const size_t o_part = cv.take(cnt * nchunk * sizeof(double));
    const size_t o_x = cv.take(cnt * m * n * sizeof(float));
    const size_t o_t = cv.take(cnt * m * n * sizeof(float));
    const size_t o_a = cv.take(cnt * m * m * sizeof(float));
    const size_t o_aa = cv.take(cnt * m * m * sizeof(float));
    int rc = ensure_scratch(o, cv.off);
    if (rc) return rc;
    char *base = (char *)o->scratch;
    MuonMat *dm = (MuonMat *)(base + o_mats);
    double *part = (double *)(base + o_part);
    float *x = (float *)(base + o_x), *t = (float *)(base + o_t);
    float *a = (float *)(base + o_a), *aa = (float *)(base + o_aa);
    RNN_HIP(ctx, hipMemcpyAsync(dm, mats.data(), cnt * sizeof(MuonMat), hipMemcpyHostToDevice,
                                ctx->stream));
    const dim3 gchunk((unsigned)nchunk, (unsigned)cnt);
    muon_momentum_kernel<<<gchunk, OPT_THREADS, 0, ctx->stream>>>(dm, len, o->mom, momentum, part);
    RNN_LAUNCHED(ctx);
    ns_load_kernel<<<gchunk, OPT_THREADS, 0, ctx->stream>>>(dm, part, (int)nchunk, (int)rows,
                                                           (int)cols, tr, x);
    RNN_LAUNCHED(ctx);
    for (size_t s = 0; s < steps; s++) {
        // A = X X^T; AA = A A; B = b A + c AA; T = B X; X = a X + T
        rc = rnn_gemm_launch(ctx, cnt, m, m, n, x, m * n, 0, x, m * n, 1, a, m * m, 0, nullptr);
        if (rc) return rc;
        rc = rnn_gemm_launch(ctx, cnt, m, m, m, a, m * m, 0, a, m * m, 0, aa, m * m, 0, nullptr);
        if (rc) return rc;
        ns_combine_a_kernel<<<grid_for(cnt * m * m, OPT_THREADS), OPT_THREADS, 0, ctx->stream>>>(
            a, aa, cnt * m * m);
        RNN_LAUNCHED(ctx);
        rc = rnn_gemm_launch(ctx, cnt, m, n, m, a, m * m, 0, x, m * n, 0, t, m * n, 0, nullptr);
        if (rc) return rc;
        ns_combine_x_kernel<<<grid_for(cnt * m * n, OPT_THREADS), OPT_THREADS, 0, ctx->stream>>>(
            x, t, cnt * m * n);
        RNN_LAUNCHED(ctx);
    }
    const float scale = 0.2f * sqrtf((float)std::max(rows, cols));
    muon_finish_kernel<<<dim3((unsigned)std::min<size_t>(rnn_div_up(len, OPT_THREADS), 1024),
                              (unsigned)cnt),
                         OPT_THREADS, 0, ctx->stream>>>(dm, x, (int)rows, (int)cols, tr, update,
                                                        lr, scale, wdp);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

bool muon_shape_ok(size_t rows, size_t cols) {
    return rows > 0 && cols > 0 && rows * cols < (1ull << 31) &&
           std::min(rows, cols) <= 4096;
}

}  // namespace

extern "C" {

int rnn_newton_schulz(rnn_ctx *ctx, size_t count, size_t rows, size_t cols, size_t steps,
                      float *g, size_t stride) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (count == 0 || rows == 0 || cols == 0) return RNN_OK;
    if (!g) return rnn_fail(ctx, RNN_E_NULL, "newton_schulz: null g");
    if (!muon_shape_ok(rows, cols) || stride < rows * cols || count > 65535)
        return rnn_fail(ctx, RNN_E_INVALID, "newton_schulz: %zu x %zu, stride %zu, count %zu",
                        rows, cols, stride, count);
    // a private optimiser object for the scratch
    rnn_optim o;
    o.ctx = ctx;
    std::vector<MuonMat> mats(count);
    for (size_t i = 0; i < count; i++) mats[i] = {nullptr, g + i * stride, nullptr};
    const int rc = ns_group(&o, mats, rows, cols, steps, 0, 0, 0.0f, 0.0f);
    if (o.scratch) {
        (void)hipStreamSynchronize(ctx->stream);
        (void)hipFree(o.scratch);
    }
    return rc;
}

int rnn_optim_create(rnn_ctx *ctx, int muon, size_t ns_steps, rnn_optim **out) {
    if (!ctx || !out) return RNN_E_NULL;
    rnn_optim *o = new rnn_optim;
    o->ctx = ctx;
    o->muon = muon != 0;
    o->ns_steps = ns_steps;
    *out = o;
    return RNN_OK;
}

int rnn_optim_destroy(rnn_optim *o) {
    if (!o) return RNN_E_NULL;
    if (o->scratch) {
        (void)hipStreamSynchronize(o->ctx->stream);
        (void)hipFree(o->scratch);
    }
    delete o;
    return RNN_OK;
}

int rnn_optim_set(rnn_optim *o, float mom, float b1, float b2, float eps, size_t t) {
    if (!o) return RNN_E_NULL;
    o->mom = mom;
    o->b1 = b1;
    o->b2 = b2;
    o->eps = eps;
    o->t = t;
    return RNN_OK;
}

size_t rnn_optim_t(const rnn_optim *o) { return o ? o->t : 0; }

int rnn_optim_step(rnn_optim *o, size_t nparam, const rnn_param *params, float lr, float wd) {
    if (!o) return RNN_E_NULL;
    rnn_ctx *ctx = o->ctx;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (nparam && !params) return rnn_fail(ctx, RNN_E_NULL, "optim_step: null params");
    // Optim::step_all (optim.rs:177-205): 2-D matrices with both sides > 1 go
    // to Muon (when enabled), everything else to AdamW.
    std::map<std::pair<size_t, size_t>, std::vector<size_t>> groups;
    std::vector<size_t> adam;
    for (size_t i = 0; i < nparam; i++) {
        const rnn_param &p = params[i];
        if (!p.v || !p.g || !p.m)
            return rnn_fail(ctx, RNN_E_NULL, "optim_step: param %zu has a null buffer", i);
        const bool is_muon = o->muon && p.rows > 0 && std::min(p.rows, p.cols) > 1;
        if (is_muon) {
            if (p.rows * p.cols != p.len || !muon_shape_ok(p.rows, p.cols))
                return rnn_fail(ctx, RNN_E_INVALID, "optim_step: param %zu is %zu x %zu, len %zu",
                                i, p.rows, p.cols, p.len);
            groups[{p.rows, p.cols}].push_back(i);
        } else {
            if (!p.v2) return rnn_fail(ctx, RNN_E_NULL, "optim_step: param %zu has no v2", i);
            adam.push_back(i);
        }
    }
    for (auto &gr : groups) {
        // matrices of one shape and one decay setting share a launch sequence
        for (int dec = 0; dec < 2; dec++) {
            std::vector<MuonMat> mats;
            for (size_t i : gr.second)
                if ((params[i].decay != 0) == (dec != 0))
                    mats.push_back({params[i].v, params[i].g, params[i].m});
            for (size_t c0 = 0; c0 < mats.size(); c0 += 65535) {
                std::vector<MuonMat> part(mats.begin() + c0,
                                          mats.begin() + std::min(mats.size(), c0 + 65535));
                const int rc = ns_group(o, part, gr.first.first, gr.first.second, o->ns_steps, 1,
                                        1, lr, dec ? wd : 0.0f);
                if (rc) return rc;
            }
        }
    }
    if (!adam.empty()) {
        std::vector<AdamSeg> segs;
        uint32_t blk = 0;
        for (size_t i : adam) {
            const rnn_param &p = params[i];
            if (p.len == 0) continue;
            AdamSeg s;
            s.v = p.v;
            s.g = p.g;
            s.m = p.m;
            s.v2 = p.v2;
            s.len = p.len;
            s.wd = p.decay ? wd : 0.0f;
            s.blk0 = blk;
            s.nblk = (uint32_t)std::min<size_t>(rnn_div_up(p.len, OPT_THREADS), 1024);
            blk += s.nblk;
            segs.push_back(s);
        }
        if (!segs.empty()) {
            int rc = ensure_scratch(o, segs.size() * sizeof(AdamSeg));
            if (rc) return rc;
            RNN_HIP(ctx, hipMemcpyAsync(o->scratch, segs.data(), segs.size() * sizeof(AdamSeg),
                                        hipMemcpyHostToDevice, ctx->stream));
            const float c1 = 1.0f - powi_f32(o->b1, (int)o->t + 1);
            const float c2 = 1.0f - powi_f32(o->b2, (int)o->t + 1);
            adam_kernel<<<blk, OPT_THREADS, 0, ctx->stream>>>((const AdamSeg *)o->scratch,
                                                             (int)segs.size(), lr, o->b1, o->b2,
                                                             o->eps, c1, c2);
            RNN_LAUNCHED(ctx);
        }
    }
    // after the step, not before: step_adam corrects the bias with t + 1
    o->t += 1;
    return RNN_OK;
}

int rnn_clip_grad_norm(rnn_ctx *ctx, size_t len, float *g, float max, float *norm) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (!g && len) return rnn_fail(ctx, RNN_E_NULL, "clip_grad_norm: null g");
    const size_t chunk = 16384;
    const size_t nparts = std::max<size_t>(1, rnn_div_up(len, chunk));
    double *part = (double *)rnn_workspace(ctx, nparts * sizeof(double));
    if (!part) return rnn_fail(ctx, RNN_E_NOMEM, "clip_grad_norm: workspace");
    sumsq_kernel<<<(unsigned)nparts, OPT_THREADS, 0, ctx->stream>>>(g, len, chunk, part);
    RNN_LAUNCHED(ctx);
    clip_scale_kernel<<<grid_for(len, OPT_THREADS), OPT_THREADS, 0, ctx->stream>>>(
        g, len, part, (int)nparts, max, norm);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_ema_update(rnn_ctx *ctx, size_t len, float *w, const float *v, float d) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (len == 0) return RNN_OK;
    if (!w || !v) return rnn_fail(ctx, RNN_E_NULL, "ema_update: null pointer");
    ema_kernel<<<grid_for(len, OPT_THREADS), OPT_THREADS, 0, ctx->stream>>>(w, v, len, d);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

float rnn_powi_f32(float a, int b) { return powi_f32(a, b); }

}  // extern "C"
