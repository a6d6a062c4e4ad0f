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
// Elements a thread loads before it stores any of them in the elementwise
// passes (a store may alias a later load, so the compiler keeps them in
// order; batching keeps OPT_U loads in flight).
constexpr int OPT_U = 8;
constexpr int NS_CHUNK = 4096;  // elements of one matrix per block in the norm passes

// One matrix of a Newton-Schulz plan.  Its elementwise passes use one block
// per NS_CHUNK elements: blocks blk0 .. blk0 + nchunk - 1 of those launches.
struct NsMat {
    float *v, *g, *m;  // v and m are null when only g is orthogonalised
    float *x;          // X slot [rows x cols] in the scratch
    const float *xf;   // the slot holding X after the last quintic step
    double *part;      // nchunk partial sums of squares
    uint32_t blk0, nchunk;
    int rows, cols, decay;
    float scale;  // 0.2 sqrt(max(rows, cols))
};

__device__ __forceinline__ int mat_of(const NsMat *__restrict__ mats, int nmat, unsigned b) {
    int lo = 0, hi = nmat - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (mats[mid].blk0 <= b)
            lo = mid;
        else
            hi = mid - 1;
    }
    return lo;
}

// Nesterov momentum (optim.rs:186-189: m = mom m + g; g += mom m) and the
// block sums of g^2: in element order per thread, then a fixed tree.
__global__ __launch_bounds__(OPT_THREADS) void muon_momentum_kernel(const NsMat *__restrict__ mats,
                                                                    int nmat, float mom,
                                                                    int momentum) {
    __shared__ double red[OPT_THREADS / 64];
    const NsMat mt = mats[mat_of(mats, nmat, blockIdx.x)];
    const size_t chunk = blockIdx.x - mt.blk0, len = (size_t)mt.rows * mt.cols;
    const size_t e0 = chunk * NS_CHUNK, e1 = min(len, e0 + NS_CHUNK);
    double s = 0.0;
    // OPT_U elements' loads ahead of their stores (the elements, and the
    // adds into s, in the order of a plain strided loop)
    for (size_t b = e0 + threadIdx.x; b < e1; b += OPT_U * OPT_THREADS) {
        float gv[OPT_U], mv[OPT_U];
#pragma unroll
        for (int u = 0; u < OPT_U; u++) {
            const size_t e = min(b + (size_t)u * OPT_THREADS, e1 - 1);
            gv[u] = mt.g[e];
            mv[u] = momentum ? mt.m[e] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < OPT_U; u++) {
            const size_t e = b + (size_t)u * OPT_THREADS;
            if (e >= e1) break;
            float gi = gv[u];
            if (momentum) {
                const float mi = mom * mv[u] + gi;
                mt.m[e] = mi;
                gi += mom * mi;
                mt.g[e] = gi;
            }
            s += (double)gi * (double)gi;
        }
    }
    for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = red[0];
        for (int w = 1; w < OPT_THREADS / 64; w++) t += red[w];
        mt.part[chunk] = t;
    }
}

// X = G / (||G||_F + 1e-7) (optim.rs:133-136); the partial sums are added
// in chunk order.  X keeps G's [rows x cols] layout also when rows > cols: the
// quintic steps then run on X^T's transpose (load_maybe_t, optim.rs:41-53, has
// no counterpart here; see ns_layout).
__global__ __launch_bounds__(OPT_THREADS) void ns_load_kernel(const NsMat *__restrict__ mats,
                                                              int nmat) {
    constexpr uint32_t NS_LDS_PARTS = 2048;
    __shared__ double pl[NS_LDS_PARTS];
    __shared__ double ss_s;
    const NsMat mt = mats[mat_of(mats, nmat, blockIdx.x)];
    // the partials added in chunk order: staged in LDS by the whole block
    // (one round trip), then summed by one thread
    double ss = 0.0;
    if (mt.nchunk <= NS_LDS_PARTS) {
        for (uint32_t k = threadIdx.x; k < mt.nchunk; k += OPT_THREADS) pl[k] = mt.part[k];
        __syncthreads();
        if (threadIdx.x == 0) {
            double t = 0.0;
            for (uint32_t k = 0; k < mt.nchunk; k++) t += pl[k];
            ss_s = t;
        }
        __syncthreads();
        ss = ss_s;
    } else {
        for (uint32_t k0 = 0; k0 < mt.nchunk; k0 += 16) {
            double v[16];
#pragma unroll
            for (int u = 0; u < 16; u++) v[u] = mt.part[min(k0 + u, mt.nchunk - 1)];
#pragma unroll
            for (int u = 0; u < 16; u++)
                if (k0 + u < mt.nchunk) ss += v[u];
        }
    }
    const float norm = sqrtf((float)ss) + 1e-7f;
    const float inv = 1.0f / norm;
    const size_t len = (size_t)mt.rows * mt.cols;
    const size_t e0 = (size_t)(blockIdx.x - mt.blk0) * NS_CHUNK, e1 = min(len, e0 + NS_CHUNK);
    for (size_t b = e0 + threadIdx.x; b < e1; b += OPT_U * OPT_THREADS) {
        float gv[OPT_U];
#pragma unroll
        for (int u = 0; u < OPT_U; u++) gv[u] = mt.g[min(b + (size_t)u * OPT_THREADS, e1 - 1)];
#pragma unroll
        for (int u = 0; u < OPT_U; u++) {
            const size_t e = b + (size_t)u * OPT_THREADS;
            if (e >= e1) break;
            mt.x[e] = gv[u] * inv;
        }
    }
}

// End of a Muon step (optim.rs:191-195), reading the orthogonalised matrix
// from its final slot: v -= lr (scale x + wd v); g = 0.  With update = 0 only
// the store into g (newton_schulz alone).
__global__ __launch_bounds__(OPT_THREADS) void muon_finish_kernel(const NsMat *__restrict__ mats,
                                                                  int nmat, int update, float lr,
                                                                  float wd) {
    const NsMat mt = mats[mat_of(mats, nmat, blockIdx.x)];
    const size_t len = (size_t)mt.rows * mt.cols;
    const size_t e0 = (size_t)(blockIdx.x - mt.blk0) * NS_CHUNK, e1 = min(len, e0 + NS_CHUNK);
    const float wdp = mt.decay ? wd : 0.0f;
    for (size_t b = e0 + threadIdx.x; b < e1; b += OPT_U * OPT_THREADS) {
        float xv[OPT_U], vv[OPT_U];
#pragma unroll
        for (int u = 0; u < OPT_U; u++) {
            const size_t e = min(b + (size_t)u * OPT_THREADS, e1 - 1);
            xv[u] = mt.xf[e];
            vv[u] = update ? mt.v[e] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < OPT_U; u++) {
            const size_t e = b + (size_t)u * OPT_THREADS;
            if (e >= e1) break;
            const float gx = xv[u];
            if (update) {
                mt.v[e] = vv[u] - lr * (mt.scale * gx + wdp * vv[u]);
                mt.g[e] = 0.0f;
            } else {
                mt.g[e] = gx;
            }
        }
    }
}

// AdamW over several tensors (Optim::step_adam, optim.rs:207-235): block b
// serves the segment whose block range holds it.
struct AdamSeg {
    float *v, *g, *m, *v2;
    size_t len;
    int decay;  // 0: no weight decay for this tensor
    uint32_t blk0, nblk;
};

// Index of the segment whose block range [blk0, blk0 + nblk) holds block b
// (segments sorted by blk0, the first at 0).
template <typename Seg>
__device__ int seg_of(const Seg *__restrict__ segs, int nseg, unsigned b) {
    int lo = 0, hi = nseg - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (segs[mid].blk0 <= b)
            lo = mid;
        else
            hi = mid - 1;
    }
    return lo;
}

__global__ void adam_kernel(const AdamSeg *__restrict__ segs, int nseg, float lr, float wd,
                            float b1, float b2, float eps, float c1, float c2) {
    const AdamSeg s = segs[seg_of(segs, nseg, blockIdx.x)];
    const float wdd = s.decay ? wd : 0.0f;
    for (size_t i = (size_t)(blockIdx.x - s.blk0) * blockDim.x + threadIdx.x; i < s.len;
         i += (size_t)s.nblk * blockDim.x) {
        const float g = s.g[i];
        const float m = b1 * s.m[i] + (1.0f - b1) * g;
        const float v2 = b2 * s.v2[i] + (1.0f - b2) * g * g;
        s.m[i] = m;
        s.v2[i] = v2;
        s.v[i] -= lr * ((m / c1) / (sqrtf(v2 / c2) + eps) + wdd * s.v[i]);
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

// ... then one block adds the partials (a fixed order: per thread a strided
// sequence, then a fixed tree), stores the norm and the scale max / norm with
// the flag "norm above max" (sc[0], sc[1]) ...
__global__ __launch_bounds__(OPT_THREADS) void clip_norm_kernel(const double *__restrict__ part,
                                                                int nparts, float max,
                                                                float *norm_out, float *sc) {
    __shared__ double red[OPT_THREADS / 64];
    double s = 0.0;
    for (int k = threadIdx.x; k < nparts; k += OPT_THREADS) s += part[k];
    for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = red[0];
        for (int w = 1; w < OPT_THREADS / 64; w++) t += red[w];
        const float norm = (float)sqrt(t);
        if (norm_out) *norm_out = norm;
        const bool clip = norm > max && norm > 0.0f;
        sc[0] = clip ? max / norm : 1.0f;
        sc[1] = clip ? 1.0f : 0.0f;
    }
}

// ... and every block scales its share of g when the flag is set.
__global__ __launch_bounds__(OPT_THREADS) void clip_scale_kernel(float *g, size_t len,
                                                                 const float *__restrict__ sc) {
    if (sc[1] == 0.0f) return;
    const float f = sc[0];
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < len;
         i += (size_t)gridDim.x * blockDim.x)
        g[i] *= f;
}

// Ema::update (optim.rs:283-287): w = d w + (1 - d) v.
__global__ void ema_kernel(float *w, const float *__restrict__ v, size_t len, float d) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < len;
         i += (size_t)gridDim.x * blockDim.x)
        w[i] = d * w[i] + (1.0f - d) * v[i];
}

// clip_ over a list of gradient tensors (optim.rs:237-251).  Sum pass: block b
// sums the squares of chunk (b - sblk0) of its tensor into part[b]; scale pass:
// block b scales its share (stride cnblk blocks) of its tensor.
struct ClipSeg {
    float *g;
    size_t len;
    uint32_t blk0, nblk;    // sum pass: one block per CLIP_CHUNK elements
    uint32_t cblk0, cnblk;  // scale pass
};
constexpr size_t CLIP_CHUNK = 4096;

__global__ __launch_bounds__(OPT_THREADS) void clip_sumsq_kernel(const ClipSeg *__restrict__ segs,
                                                                 int nseg, double *part) {
    __shared__ double red[OPT_THREADS / 64];
    const ClipSeg sg = segs[seg_of(segs, nseg, blockIdx.x)];
    const size_t e0 = (size_t)(blockIdx.x - sg.blk0) * CLIP_CHUNK;
    const size_t e1 = min(sg.len, e0 + CLIP_CHUNK);
    double s = 0.0;
    for (size_t b = e0 + threadIdx.x; b < e1; b += OPT_U * OPT_THREADS) {
        float gv[OPT_U];
#pragma unroll
        for (int u = 0; u < OPT_U; u++) gv[u] = sg.g[min(b + (size_t)u * OPT_THREADS, e1 - 1)];
#pragma unroll
        for (int u = 0; u < OPT_U; u++) {
            if (b + (size_t)u * OPT_THREADS >= e1) break;
            s += (double)gv[u] * (double)gv[u];
        }
    }
    for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = red[0];
        for (int w = 1; w < OPT_THREADS / 64; w++) t += red[w];
        part[blockIdx.x] = t;
    }
}

struct ClipScaleSeg {
    uint32_t blk0;
    int seg;
};

__global__ __launch_bounds__(OPT_THREADS) void clip_scale_segs_kernel(
    const ClipSeg *__restrict__ segs, const ClipScaleSeg *__restrict__ sidx, int nseg,
    const float *__restrict__ sc) {
    if (sc[1] == 0.0f) return;
    const float f = sc[0];
    const ClipSeg sg = segs[sidx[seg_of(sidx, nseg, blockIdx.x)].seg];
    const size_t st = (size_t)sg.cnblk * OPT_THREADS;
    for (size_t b = (size_t)(blockIdx.x - sg.cblk0) * OPT_THREADS + threadIdx.x; b < sg.len;
         b += OPT_U * st) {
        float gv[OPT_U];
#pragma unroll
        for (int u = 0; u < OPT_U; u++) gv[u] = sg.g[min(b + u * st, sg.len - 1)];
#pragma unroll
        for (int u = 0; u < OPT_U; u++) {
            if (b + u * st >= sg.len) break;
            sg.g[b + u * st] = gv[u] * f;
        }
    }
}

// Stores zeros (a kernel rather than a memset node, for graph capture).
__global__ void zero_kernel(float *p, size_t len) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < len;
         i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0.0f;
}

// Ema::update over a list of tensors (optim.rs:283-287): w = d w + (1 - d) v.
struct EmaSeg {
    float *w;
    const float *v;
    size_t len;
    uint32_t blk0, nblk;
};

__global__ __launch_bounds__(OPT_THREADS) void ema_segs_kernel(const EmaSeg *__restrict__ segs,
                                                               int nseg, float d) {
    const EmaSeg s = segs[seg_of(segs, nseg, blockIdx.x)];
    const size_t st = (size_t)s.nblk * OPT_THREADS;
    for (size_t b = (size_t)(blockIdx.x - s.blk0) * OPT_THREADS + threadIdx.x; b < s.len;
         b += OPT_U * st) {
        float wv[OPT_U], vv[OPT_U];
#pragma unroll
        for (int u = 0; u < OPT_U; u++) {
            const size_t i = min(b + u * st, s.len - 1);
            wv[u] = s.w[i];
            vv[u] = s.v[i];
        }
#pragma unroll
        for (int u = 0; u < OPT_U; u++) {
            if (b + u * st >= s.len) break;
            s.w[b + u * st] = d * wv[u] + (1.0f - d) * vv[u];
        }
    }
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

// A grouped Newton-Schulz plan: every matrix's elementwise passes in one
// launch each, and per quintic step three grouped GEMM launches over all
// shapes (rnn_ns_gemm_launch).  Offsets are bytes into the device table.
struct NsPlan {
    size_t mats = 0, nmat = 0, blocks = 0;  // NsMat table, count, elementwise blocks
    struct Op {
        size_t probs = 0, nprob = 0, tiles = 0;
        int vec = 0;
        float alpha = 0.0f, beta = 0.0f;
    };
    std::vector<Op> ops;  // per quintic step 3, or 6 when some problems need the register tile
};

struct rnn_optim {
    rnn_ctx *ctx = nullptr;
    bool muon = true;
    size_t ns_steps = 3;
    float mom = 0.95f, b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
    size_t t = 0;
    // device scratch: Newton-Schulz buffers and norm partials
    void *scratch = nullptr;
    size_t scratch_bytes = 0;
    // The plan of the last parameter list: Muon matrices, AdamW segments and
    // the device table holding their pointers.  Rebuilt only when the list
    // changes, so a training loop uploads nothing after its first step.
    std::vector<rnn_param> plan_params;
    size_t plan_steps = 0;
    NsPlan ns;
    size_t adam_tab = 0, nseg = 0, adam_blocks = 0;
    RnnDevTable table;
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

// Host-side table under construction; every piece starts 256-byte aligned.
struct TableBuf {
    std::vector<char> b;
    size_t put(const void *src, size_t bytes) {
        const size_t off = rnn_round_up(b.size(), 256);
        b.resize(off + bytes);
        if (bytes) std::memcpy(b.data() + off, src, bytes);
        return off;
    }
};

// One matrix handed to a Newton-Schulz plan.
struct NsIn {
    float *v, *g, *m;
    size_t rows, cols;
    int decay;
};

// Lays out the scratch (offsets from 0) and the tables of a plan over `mats`
// with `steps` quintic steps; the NsMat and problem tables hold offsets from
// the scratch base `base` (known when the plan is built: the scratch is sized
// first).  Returns the scratch bytes needed in *need when base is null.
void ns_layout(const std::vector<NsIn> &mats, size_t steps, char *base, TableBuf &tab,
               NsPlan &plan, size_t *need) {
    // same-shape matrices form a batch of each GEMM
    std::map<std::pair<size_t, size_t>, std::vector<size_t>> shapes;
    for (size_t i = 0; i < mats.size(); i++) shapes[{mats[i].rows, mats[i].cols}].push_back(i);
    WsCarve cv;
    size_t nchunk_all = 0;
    for (const NsIn &mt : mats) nchunk_all += rnn_div_up(mt.rows * mt.cols, NS_CHUNK);
    const size_t o_part = cv.take(nchunk_all * sizeof(double));
    struct Grp {
        size_t rows, cols, m, n, cnt, x, t, a, aa;
    };
    std::vector<Grp> grps;
    for (auto &sh : shapes) {
        Grp g;
        g.rows = sh.first.first;
        g.cols = sh.first.second;
        g.m = std::min(g.rows, g.cols);
        g.n = std::max(g.rows, g.cols);
        g.cnt = sh.second.size();
        g.x = cv.take(g.cnt * g.m * g.n * sizeof(float));
        g.t = cv.take(g.cnt * g.m * g.n * sizeof(float));
        g.a = cv.take(g.cnt * g.m * g.m * sizeof(float));
        g.aa = cv.take(g.cnt * g.m * g.m * sizeof(float));
        grps.push_back(g);
    }
    *need = cv.off;
    if (!base) return;
    auto F = [base](size_t off) { return (float *)(base + off); };
    // the matrices, in shape order (the GEMM batches' order)
    std::vector<NsMat> nm;
    size_t part = 0, gi = 0;
    uint32_t blk = 0;
    for (auto &sh : shapes) {
        const Grp &g = grps[gi++];
        for (size_t k = 0; k < sh.second.size(); k++) {
            const NsIn &in = mats[sh.second[k]];
            NsMat e;
            e.v = in.v;
            e.g = in.g;
            e.m = in.m;
            e.x = F(g.x) + k * g.m * g.n;
            e.xf = (steps & 1 ? F(g.t) : F(g.x)) + k * g.m * g.n;
            e.part = (double *)(base + o_part) + part;
            e.nchunk = (uint32_t)rnn_div_up(g.rows * g.cols, NS_CHUNK);
            e.blk0 = blk;
            e.rows = (int)g.rows;
            e.cols = (int)g.cols;
            e.decay = in.decay;
            e.scale = 0.2f * sqrtf((float)g.n);
            part += e.nchunk;
            blk += e.nchunk;
            nm.push_back(e);
        }
    }
    plan.mats = tab.put(nm.data(), nm.size() * sizeof(NsMat));
    plan.nmat = nm.size();
    plan.blocks = blk;
    // Every X slot keeps G's layout [rows x cols].  For a wide G (rows <= cols,
    // X = G as in the reference) a step is A = X X^T, B = b A + c A A,
    // X' = a X + B X.  For a tall G the reference iterates on X = G^T; here
    // Y = X^T = G is iterated directly: A = Y^T Y, B as before, Y' = a Y + Y B
    // (the transpose of X' = a X + B X, B being symmetric).  A and B are
    // symmetric (each element and its mirror are the same products in the
    // same order), so only their upper tiles are computed, A A is taken as
    // A A^T, and B is read as B^T where that keeps k contiguous.
    std::vector<size_t> order(grps.size());
    for (size_t i = 0; i < order.size(); i++) order[i] = i;
    plan.ops.clear();
    for (size_t s = 0; s < steps; s++) {
        for (int op = 0; op < 3; op++) {
            // longest k first: the long tiles start early
            std::stable_sort(order.begin(), order.end(), [&](size_t p, size_t q) {
                return (op == 0 ? grps[p].n : grps[p].m) > (op == 0 ? grps[q].n : grps[q].m);
            });
            // problems that take the direct-to-LDS tile go in one launch,
            // the others in a second
            std::vector<NsGemmProb> probs, dprobs;
            uint32_t tile = 0, dtile = 0;
            bool vec = true;
            for (size_t k : order) {
                const Grp &g = grps[k];
                const size_t m = g.m, n = g.n;
                const bool tall = g.rows > g.cols;
                float *xs = (s & 1) ? F(g.t) : F(g.x), *xn = (s & 1) ? F(g.x) : F(g.t);
                NsGemmProb p{};
                p.stride_c = (long long)(op == 2 ? m * n : m * m);
                if (op == 0) {
                    // A [m x m] = X X^T (X [m][n]) or Y^T Y (Y [n][m])
                    p.a = xs;
                    p.b = xs;
                    p.c = F(g.a);
                    p.stride_a = p.stride_b = (long long)(m * n);
                    p.M = p.N = (int)m;
                    p.K = (int)n;
                    p.lda = p.ldb = tall ? (int)m : (int)n;
                    p.ldc = (int)m;
                    p.lay = tall ? NS_LAY_TN : NS_LAY_NT;
                    p.sym = 1;
                } else if (op == 1) {
                    // B = b A + c A A^T, into the AA slot
                    p.a = p.b = F(g.a);
                    p.c = F(g.aa);
                    p.e = F(g.a);
                    p.stride_a = p.stride_b = (long long)(m * m);
                    p.M = p.N = p.K = (int)m;
                    p.lda = p.ldb = p.ldc = (int)m;
                    p.lay = NS_LAY_NT;
                    p.sym = 1;
                } else if (!tall) {
                    // X' = a X + B X: [m x m] [m x n]
                    p.a = F(g.aa);
                    p.b = xs;
                    p.c = xn;
                    p.e = xs;
                    p.stride_a = (long long)(m * m);
                    p.stride_b = (long long)(m * n);
                    p.M = (int)m;
                    p.N = (int)n;
                    p.K = (int)m;
                    p.lda = (int)m;
                    p.ldb = p.ldc = (int)n;
                    p.lay = NS_LAY_NN;
                } else {
                    // Y' = a Y + Y B^T: [n x m] [m x m]
                    p.a = xs;
                    p.b = F(g.aa);
                    p.c = xn;
                    p.e = xs;
                    p.stride_a = (long long)(m * n);
                    p.stride_b = (long long)(m * m);
                    p.M = (int)n;
                    p.N = (int)m;
                    p.K = (int)m;
                    p.lda = p.ldb = p.ldc = (int)m;
                    p.lay = NS_LAY_NT;
                }
                p.tn = (uint32_t)rnn_div_up((size_t)p.N, 64);
                p.tmn = p.sym ? p.tn * (p.tn + 1) / 2
                              : (uint32_t)rnn_div_up((size_t)p.M, 64) * p.tn;
                if (ns_dma_ok(p, g.cnt)) {
                    p.tile0 = dtile;
                    dtile += (uint32_t)(g.cnt * p.tmn);
                    dprobs.push_back(p);
                    continue;
                }
                if (op == 0 && !tall) vec = vec && n % 4 == 0;
                if (op != 0) vec = vec && m % 4 == 0;
                p.tile0 = tile;
                tile += (uint32_t)(g.cnt * p.tmn);
                probs.push_back(p);
            }
            for (int d = 0; d < 2; d++) {
                const std::vector<NsGemmProb> &pv = d ? probs : dprobs;
                if (pv.empty()) continue;
                NsPlan::Op o;
                o.probs = tab.put(pv.data(), pv.size() * sizeof(NsGemmProb));
                o.nprob = pv.size();
                o.tiles = d ? tile : dtile;
                o.vec = d ? (int)vec : 2;
                o.alpha = op == 0 ? 0.0f : (op == 1 ? NS_B : NS_A);
                o.beta = op == 0 ? 0.0f : (op == 1 ? NS_C : 1.0f);
                plan.ops.push_back(o);
            }
        }
    }
}

// Runs a plan whose table sits at `tab` (device): momentum (when set), the
// normalised load, the quintic steps, then the update (or the store into g).
int ns_run(rnn_ctx *ctx, const NsPlan &plan, const char *tab, float mom, int momentum,
           int update, float lr, float wd) {
    if (!plan.nmat) return RNN_OK;
    const NsMat *mats = (const NsMat *)(tab + plan.mats);
    const int nmat = (int)plan.nmat;
    const dim3 grid((unsigned)plan.blocks);
    muon_momentum_kernel<<<grid, OPT_THREADS, 0, ctx->stream>>>(mats, nmat, mom, momentum);
    RNN_LAUNCHED(ctx);
    ns_load_kernel<<<grid, OPT_THREADS, 0, ctx->stream>>>(mats, nmat);
    RNN_LAUNCHED(ctx);
    for (const NsPlan::Op &op : plan.ops) {
        const int rc = rnn_ns_gemm_launch(ctx, (const NsGemmProb *)(tab + op.probs), (int)op.nprob,
                                          op.tiles, op.vec, op.alpha, op.beta);
        if (rc) return rc;
    }
    muon_finish_kernel<<<grid, OPT_THREADS, 0, ctx->stream>>>(mats, nmat, update, lr, wd);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

bool same_param(const rnn_param &a, const rnn_param &b) {
    return a.v == b.v && a.g == b.g && a.m == b.m && a.v2 == b.v2 && a.len == b.len &&
           a.rows == b.rows && a.cols == b.cols && (a.decay != 0) == (b.decay != 0);
}

// Builds the plan of `params` (already validated) and uploads its table.
int build_plan(rnn_optim *o, size_t nparam, const rnn_param *params) {
    rnn_ctx *ctx = o->ctx;
    // Optim::step_all (optim.rs:177-205): 2-D matrices with both sides > 1 go
    // to Muon (when enabled), everything else to AdamW.
    std::vector<NsIn> mats;
    std::vector<AdamSeg> segs;
    uint32_t blk = 0;
    for (size_t i = 0; i < nparam; i++) {
        const rnn_param &p = params[i];
        if (o->muon && p.rows > 0 && std::min(p.rows, p.cols) > 1) {
            mats.push_back({p.v, p.g, p.m, p.rows, p.cols, p.decay != 0});
        } else if (p.len) {
            AdamSeg sg;
            sg.v = p.v;
            sg.g = p.g;
            sg.m = p.m;
            sg.v2 = p.v2;
            sg.len = p.len;
            sg.decay = p.decay != 0;
            sg.blk0 = blk;
            sg.nblk = (uint32_t)std::min<size_t>(rnn_div_up(p.len, OPT_THREADS), 1024);
            blk += sg.nblk;
            segs.push_back(sg);
        }
    }
    // the old plan is dropped before anything can fail half-way
    o->plan_params.clear();
    TableBuf tab;
    NsPlan plan;
    size_t need = 0;
    ns_layout(mats, o->ns_steps, nullptr, tab, plan, &need);
    int rc = ensure_scratch(o, need);
    if (rc) return rc;
    ns_layout(mats, o->ns_steps, (char *)o->scratch, tab, plan, &need);
    const size_t adam_tab = segs.empty() ? 0 : tab.put(segs.data(), segs.size() * sizeof(AdamSeg));
    void *dev = nullptr;
    rc = rnn_dev_table(ctx, o->table, tab.b.data(), tab.b.size(), &dev);
    if (rc) return rc;
    o->ns = std::move(plan);
    o->adam_tab = adam_tab;
    o->nseg = segs.size();
    o->adam_blocks = blk;
    o->plan_params.assign(params, params + nparam);
    o->plan_steps = o->ns_steps;
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
    // a private optimiser object for the scratch and the table
    rnn_optim o;
    o.ctx = ctx;
    std::vector<NsIn> mats(count);
    for (size_t i = 0; i < count; i++) mats[i] = {nullptr, g + i * stride, nullptr, rows, cols, 0};
    TableBuf tab;
    NsPlan plan;
    size_t need = 0;
    ns_layout(mats, steps, nullptr, tab, plan, &need);
    int rc = ensure_scratch(&o, need);
    if (!rc) {
        ns_layout(mats, steps, (char *)o.scratch, tab, plan, &need);
        void *dev = nullptr;
        rc = rnn_dev_table(ctx, o.table, tab.b.data(), tab.b.size(), &dev);
        if (!rc) rc = ns_run(ctx, plan, (const char *)dev, 0.0f, 0, 0, 0.0f, 0.0f);
    }
    (void)hipStreamSynchronize(ctx->stream);
    if (o.scratch) (void)hipFree(o.scratch);
    rnn_dev_table_free(o.table);
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
    (void)hipStreamSynchronize(o->ctx->stream);
    if (o->scratch) (void)hipFree(o->scratch);
    rnn_dev_table_free(o->table);
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
    bool same = o->plan_params.size() == nparam && (nparam > 0 || o->table.dev);
    for (size_t i = 0; i < nparam; i++) {
        const rnn_param &p = params[i];
        if (same && same_param(p, o->plan_params[i])) continue;
        same = false;
        if (p.len == 0 && p.rows == 0) continue;  // an empty tensor: nothing to update
        if (!p.v || !p.g || !p.m)
            return rnn_fail(ctx, RNN_E_NULL, "optim_step: param %zu has a null buffer", i);
        const bool is_muon = o->muon && p.rows > 0 && std::min(p.rows, p.cols) > 1;
        if (is_muon) {
            if (p.rows * p.cols != p.len || !muon_shape_ok(p.rows, p.cols))
                return rnn_fail(ctx, RNN_E_INVALID, "optim_step: param %zu is %zu x %zu, len %zu",
                                i, p.rows, p.cols, p.len);
        } else if (!p.v2) {
            return rnn_fail(ctx, RNN_E_NULL, "optim_step: param %zu has no v2", i);
        }
    }
    if (o->plan_steps != o->ns_steps) same = false;
    if (!same) {
        const int rc = build_plan(o, nparam, params);
        if (rc) return rc;
    }
    const char *tab = (const char *)o->table.dev;
    int rc = ns_run(ctx, o->ns, tab, o->mom, 1, 1, lr, wd);
    if (rc) return rc;
    if (o->nseg) {
        const float c1 = 1.0f - powi_f32(o->b1, (int)o->t + 1);
        const float c2 = 1.0f - powi_f32(o->b2, (int)o->t + 1);
        adam_kernel<<<(unsigned)o->adam_blocks, OPT_THREADS, 0, ctx->stream>>>(
            (const AdamSeg *)(tab + o->adam_tab), (int)o->nseg, lr, wd, o->b1, o->b2, o->eps, c1,
            c2);
        RNN_LAUNCHED(ctx);
    }
    // after the step, not before: step_adam corrects the bias with t + 1
    o->t += 1;
    return RNN_OK;
}

int rnn_clip_grad_norm(rnn_ctx *ctx, size_t len, float *g, float max, float *norm) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (!g && len) return rnn_fail(ctx, RNN_E_NULL, "clip_grad_norm: null g");
    const size_t chunk = CLIP_CHUNK;
    const size_t nparts = std::max<size_t>(1, rnn_div_up(len, chunk));
    WsCarve cv;
    const size_t o_sc = cv.take(2 * sizeof(float)), o_part = cv.take(nparts * sizeof(double));
    char *ws = (char *)rnn_workspace(ctx, cv.off);
    if (!ws) return rnn_fail(ctx, RNN_E_NOMEM, "clip_grad_norm: workspace");
    float *sc = (float *)(ws + o_sc);
    double *part = (double *)(ws + o_part);
    sumsq_kernel<<<(unsigned)nparts, OPT_THREADS, 0, ctx->stream>>>(g, len, chunk, part);
    RNN_LAUNCHED(ctx);
    clip_norm_kernel<<<1, OPT_THREADS, 0, ctx->stream>>>(part, (int)nparts, max, norm, sc);
    RNN_LAUNCHED(ctx);
    clip_scale_kernel<<<grid_for(len, OPT_THREADS), OPT_THREADS, 0, ctx->stream>>>(g, len, sc);
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

int rnn_clip_params(rnn_ctx *ctx, size_t nparam, const rnn_param *params, float max,
                    float *norm) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (nparam && !params) return rnn_fail(ctx, RNN_E_NULL, "clip_params: null params");
    std::vector<ClipSeg> segs;
    uint32_t sblk = 0, cblk = 0;
    for (size_t i = 0; i < nparam; i++) {
        if (params[i].len == 0) continue;
        if (!params[i].g)
            return rnn_fail(ctx, RNN_E_NULL, "clip_params: param %zu has a null gradient", i);
        ClipSeg sg;
        sg.g = params[i].g;
        sg.len = params[i].len;
        sg.blk0 = sblk;
        sg.nblk = (uint32_t)rnn_div_up(sg.len, CLIP_CHUNK);
        sg.cblk0 = cblk;
        sg.cnblk = (uint32_t)std::min<size_t>(rnn_div_up(sg.len, OPT_U * OPT_THREADS), 1024);
        sblk += sg.nblk;
        cblk += sg.cnblk;
        segs.push_back(sg);
    }
    if (segs.empty()) {
        // no gradient at all: the norm is 0 and nothing is scaled
        if (norm) {
            zero_kernel<<<1, 64, 0, ctx->stream>>>(norm, 1);
            RNN_LAUNCHED(ctx);
        }
        return RNN_OK;
    }
    std::vector<char> tab(rnn_round_up(segs.size() * sizeof(ClipSeg), 256) +
                          segs.size() * sizeof(ClipScaleSeg));
    std::memcpy(tab.data(), segs.data(), segs.size() * sizeof(ClipSeg));
    ClipScaleSeg *sidx = (ClipScaleSeg *)(tab.data() + rnn_round_up(segs.size() * sizeof(ClipSeg),
                                                                    256));
    for (size_t k = 0; k < segs.size(); k++) sidx[k] = {segs[k].cblk0, (int)k};
    void *dev = nullptr;
    int rc = rnn_dev_table(ctx, ctx->tables[RNN_TABLE_CLIP], tab.data(), tab.size(), &dev);
    if (rc) return rc;
    WsCarve cv;
    const size_t o_sc = cv.take(2 * sizeof(float)), o_part = cv.take(sblk * sizeof(double));
    char *ws = (char *)rnn_workspace(ctx, cv.off);
    if (!ws) return rnn_fail(ctx, RNN_E_NOMEM, "clip_params: workspace");
    float *sc = (float *)(ws + o_sc);
    double *part = (double *)(ws + o_part);
    const ClipSeg *dsegs = (const ClipSeg *)dev;
    const ClipScaleSeg *dsidx = (const ClipScaleSeg *)((char *)dev + ((char *)sidx - tab.data()));
    clip_sumsq_kernel<<<sblk, OPT_THREADS, 0, ctx->stream>>>(dsegs, (int)segs.size(), part);
    RNN_LAUNCHED(ctx);
    clip_norm_kernel<<<1, OPT_THREADS, 0, ctx->stream>>>(part, (int)sblk, max, norm, sc);
    RNN_LAUNCHED(ctx);
    clip_scale_segs_kernel<<<cblk, OPT_THREADS, 0, ctx->stream>>>(dsegs, dsidx, (int)segs.size(),
                                                                  sc);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_ema_update_params(rnn_ctx *ctx, size_t nparam, float *const *w, const rnn_param *params,
                          float d) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (nparam && (!params || !w)) return rnn_fail(ctx, RNN_E_NULL, "ema_update_params: null list");
    std::vector<EmaSeg> segs;
    uint32_t blk = 0;
    for (size_t i = 0; i < nparam; i++) {
        if (params[i].len == 0) continue;
        if (!w[i] || !params[i].v)
            return rnn_fail(ctx, RNN_E_NULL, "ema_update_params: tensor %zu is null", i);
        EmaSeg sg;
        sg.w = w[i];
        sg.v = params[i].v;
        sg.len = params[i].len;
        sg.blk0 = blk;
        sg.nblk = (uint32_t)std::min<size_t>(rnn_div_up(sg.len, OPT_U * OPT_THREADS), 1024);
        blk += sg.nblk;
        segs.push_back(sg);
    }
    if (segs.empty()) return RNN_OK;
    void *dev = nullptr;
    int rc = rnn_dev_table(ctx, ctx->tables[RNN_TABLE_EMA], segs.data(),
                           segs.size() * sizeof(EmaSeg), &dev);
    if (rc) return rc;
    ema_segs_kernel<<<blk, OPT_THREADS, 0, ctx->stream>>>((const EmaSeg *)dev, (int)segs.size(),
                                                         d);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

float rnn_powi_f32(float a, int b) { return powi_f32(a, b); }

// lr_at (train.rs:21-28) in f32 with the C library's cosf, the function the
// reference's f32::cos calls.
float rnn_lr_at(float peak, float lo, size_t step, size_t total, size_t warm) {
    if (warm > 0 && step < warm) return lo + (peak - lo) * (float)(step + 1) / (float)warm;
    const size_t span = total > warm ? total - warm : 1;
    const float t = (float)(step - warm) / (float)span;
    return lo + 0.5f * (peak - lo) * (1.0f + cosf(3.14159265358979323846f * t));
}

}  // extern "C"
