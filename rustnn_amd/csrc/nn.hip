// The ResNet layers around the convolutions, on gfx950: BatchNorm2d train /
// eval forward and backward, ReLU / residual-add helpers, global average
// pooling, the scalar classifier Linear, softmax cross-entropy with label
// smoothing and the Nesterov SGD step.
//
// Reference: nn.rs:102-110 (Param::step), 253-428 (BatchNorm2d), 430-450
// (relu_back_, add_, add_relu_), 452-473 (gap), 475-564 (Linear), 566-637
// (softmax_ce).
//
// Arithmetic is never contracted into FMAs in this file (the reference's Rust
// never fuses a*b + c), so every elementwise formula rounds exactly as the
// reference's does.  Per-channel sums (batch statistics, dgamma / dbeta) are
// accumulated in f64 in a fixed order: partial sums over image ranges, then
// the partials in range order (bit-reproducible).
#pragma clang fp contract(off)

#include "conv_common.h"

#include <algorithm>

namespace {

constexpr int EW_THREADS = 256;
constexpr int BN_PF = 4;  // items a thread of the BN backward loads before the coefficients
constexpr int RED_THREADS = 256;

// ------------------------------------------------------------ reductions

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Sums (a, b) over the block in a fixed order; thread 0 gets the result.
__device__ __forceinline__ void block_sum2(double &a, double &b) {
    __shared__ double red[2][RED_THREADS / 64];
    a = wave_sum(a);
    b = wave_sum(b);
    const int wave = wave_index(), lane = threadIdx.x & 63;
    if (lane == 0) {
        red[0][wave] = a;
        red[1][wave] = b;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        a = red[0][0];
        b = red[1][0];
        for (int w = 1; w < RED_THREADS / 64; w++) {
            a += red[0][w];
            b += red[1][w];
        }
    }
}

// The totals of the P partial pairs part[ci][k][0..1] of channel ci, in
// every thread of the block (all threads must call it).  Up to 64 partials:
// each thread adds them in order (uniform loads).  More (a conv store pass's
// one partial per tile): thread t adds pairs t, t + 256, ... in order, its
// loads issued four at a time, then the waves' fixed-order trees and the
// waves in order.
__device__ __forceinline__ void part_totals(const double *__restrict__ part, int ci, int P,
                                            double &a, double &b) {
    const double *pc = part + (size_t)ci * P * 2;
    if (P <= 64) {
        a = 0.0;
        b = 0.0;
        for (int k = 0; k < P; k++) {
            a += pc[2 * k];
            b += pc[2 * k + 1];
        }
        return;
    }
    __shared__ double red[2][RED_THREADS / 64];
    constexpr int U = 4;
    double sa = 0.0, sb = 0.0;
    for (int k0 = threadIdx.x; k0 < P; k0 += U * RED_THREADS) {
        double2 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int k = k0 + u * RED_THREADS;
            v[u] = k < P ? *reinterpret_cast<const double2 *>(pc + 2 * k) : double2{0.0, 0.0};
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            sa += v[u].x;
            sb += v[u].y;
        }
    }
    sa = wave_sum(sa);
    sb = wave_sum(sb);
    const int wave = wave_index(), lane = threadIdx.x & 63;
    if (lane == 0) {
        red[0][wave] = sa;
        red[1][wave] = sb;
    }
    __syncthreads();
    a = red[0][0];
    b = red[1][0];
    for (int w = 1; w < RED_THREADS / 64; w++) {
        a += red[0][w];
        b += red[1][w];
    }
    __syncthreads();  // red is reused by the next call
}

// Geometry of the per-channel reductions: block (ci, p) sums images
// [p*G, p*G + G) of channel ci.
struct ChanSplit {
    int P, G;
};

static inline ChanSplit chan_split(size_t n, size_t c) {
    size_t p = std::max<size_t>(1, std::min<size_t>(n, rnn_div_up(1024, std::max<size_t>(c, 1))));
    size_t g = rnn_div_up(n, p);
    p = rnn_div_up(n, g);
    return {(int)p, (int)g};
}

// n / d through the multiply-high of `f` when the host found it exact for
// every n of the launch (f.m != 0 or d == 1), else a plain division.
__device__ __forceinline__ uint32_t div_by(uint32_t n, FastDiv f) {
    if (f.m || f.d <= 1) return fdiv(n, f);
    return n / f.d;
}

// BatchNorm2d::batch_stats (nn.rs:272-293), partial sums: part[ci][p] =
// (sum x, sum x^2) over the block's images, f64.
__global__ __launch_bounds__(RED_THREADS) void bn_stats_part_kernel(
    const float *__restrict__ x, int n, int C, int hw, int vec, int G, FastDiv fd_hw4,
    double *part) {
    const int ci = blockIdx.x, p = blockIdx.y, P = gridDim.y;
    const int i0 = p * G, i1 = min(n, i0 + G);
    double s = 0.0, s2 = 0.0;
    if ((hw & 3) == 0 && vec) {
        const int hw4 = hw >> 2, tot = (i1 - i0) * hw4;
        for (int e = threadIdx.x; e < tot; e += RED_THREADS) {
            const int img = (int)div_by((uint32_t)e, fd_hw4), r = e - img * hw4;
            const float4 v = *reinterpret_cast<const float4 *>(
                x + ((size_t)(i0 + img) * C + ci) * hw + 4 * r);
            const double a = v.x, b = v.y, c = v.z, d = v.w;
            s += a;
            s2 += a * a;
            s += b;
            s2 += b * b;
            s += c;
            s2 += c * c;
            s += d;
            s2 += d * d;
        }
    } else {
        const int tot = (i1 - i0) * hw;
        for (int e = threadIdx.x; e < tot; e += RED_THREADS) {
            const int img = e / hw, r = e - img * hw;
            const double a = x[((size_t)(i0 + img) * C + ci) * hw + r];
            s += a;
            s2 += a * a;
        }
    }
    block_sum2(s, s2);
    if (threadIdx.x == 0) {
        part[((size_t)ci * P + p) * 2 + 0] = s;
        part[((size_t)ci * P + p) * 2 + 1] = s2;
    }
}

// Channel coefficients, computed by every thread of a block (uniform loads).
// Train: mean and invstd from the partial sums added in range order -- the
// same values in every block of the channel (batch_stats + run_train,
// nn.rs:272-320: f64 mean and variance clamped at 0, invstd =
// 1/sqrt(var + eps)); thread 0 of the channel's first block also stores them
// and updates the running mean / unbiased running variance.  Eval: the scale
// and shift of run_eval (nn.rs:350-365).
template <bool EVAL>
__device__ __forceinline__ void bn_channel(const RnnBn &s, int ci, bool first, float &a,
                                           float &b) {
    if constexpr (EVAL) {
        const float is = 1.0f / sqrtf(s.rv[ci] + s.eps);
        a = s.gamma[ci] * is;
        b = s.beta[ci] - s.gamma[ci] * is * s.rm[ci];
    } else {
        double sx, sx2;
        part_totals(s.part, ci, s.P, sx, sx2);
        const double mu = sx / (double)s.m;
        const double va = sx2 / (double)s.m - mu * mu;
        const float meanf = (float)mu, varf = (float)(va > 0.0 ? va : 0.0);
        const float is = 1.0f / sqrtf(varf + s.eps);
        a = meanf;
        b = is;
        if (first && threadIdx.x == 0) {
            s.mean[ci] = meanf;
            s.invstd[ci] = is;
            if (s.rm) {
                s.rm[ci] = (1.0f - s.mom) * s.rm[ci] + s.mom * meanf;
                const float den = fmaxf(s.m - 1.0f, 1.0f);
                const float unb = varf * s.m / den;
                s.rv[ci] = (1.0f - s.mom) * s.rv[ci] + s.mom * unb;
            }
        }
    }
}

// Normalisation of one element with the channel coefficients (a, b): train
// (run_train, nn.rs:336-342) g * ((x - mean) * invstd) + beta; eval
// (run_eval) sc * x + sh.
template <bool EVAL>
struct BnFn {
    float a, b, g, be;
    __device__ __forceinline__ float operator()(float x) const {
        if constexpr (EVAL) {
            return a * x + b;
        } else {
            const float h = (x - a) * b;
            return g * h + be;
        }
    }
};

template <bool EVAL>
__device__ __forceinline__ BnFn<EVAL> bn_fn(const RnnBn &s, int ci, bool first) {
    BnFn<EVAL> f;
    bn_channel<EVAL>(s, ci, first, f.a, f.b);
    f.g = EVAL ? 0.0f : s.gamma[ci];
    f.be = EVAL ? 0.0f : s.beta[ci];
    return f;
}

// out = [relu]( bn(x) [+ skip | + bn'(skip)] ) over channel blockIdx.x of
// images [p*G, p*G + G), p = blockIdx.y.  SKIP 0: none; 1: add the tensor
// `skip` (identity shortcut); 2: add bn'(skip) (projection shortcut).  The
// residual add and the ReLU follow add_relu_ (nn.rs:446-450): max(y + s, 0).
template <bool EVAL, bool RELU, int SKIP>
__global__ __launch_bounds__(EW_THREADS) void bn_apply_kernel(const float *x, RnnBn bn,
                                                              const float *skip, RnnBn sbn,
                                                              float *out, int n, int C, int hw,
                                                              int G, FastDiv fd_hw4, int vec) {
    const int ci = blockIdx.x, p = blockIdx.y;
    const bool first = p == 0;
    const BnFn<EVAL> f = bn_fn<EVAL>(bn, ci, first);
    BnFn<EVAL> fs{};
    if constexpr (SKIP == 2) fs = bn_fn<EVAL>(sbn, ci, first);
    const int i0 = p * G, i1 = min(n, i0 + G);
    auto one = [&](float v, float sv) {
        float r = f(v);
        if constexpr (SKIP == 1) r = r + sv;
        if constexpr (SKIP == 2) r = r + fs(sv);
        if constexpr (RELU) r = r > 0.0f ? r : 0.0f;
        return r;
    };
    if (vec) {
        const int hw4 = hw >> 2, tot = (i1 - i0) * hw4;
        for (int e = threadIdx.x; e < tot; e += EW_THREADS) {
            const int img = (int)div_by((uint32_t)e, fd_hw4), r = e - img * hw4;
            const size_t q = ((size_t)(i0 + img) * C + ci) * hw4 + r;
            const float4 v = reinterpret_cast<const float4 *>(x)[q];
            float4 sv = make_float4(0.f, 0.f, 0.f, 0.f);
            if constexpr (SKIP != 0) sv = reinterpret_cast<const float4 *>(skip)[q];
            reinterpret_cast<float4 *>(out)[q] =
                make_float4(one(v.x, sv.x), one(v.y, sv.y), one(v.z, sv.z), one(v.w, sv.w));
        }
    } else {
        const int tot = (i1 - i0) * hw;
        for (int e = threadIdx.x; e < tot; e += EW_THREADS) {
            const int img = e / hw, r = e - img * hw;
            const size_t i = ((size_t)(i0 + img) * C + ci) * hw + r;
            out[i] = one(x[i], SKIP != 0 ? skip[i] : 0.0f);
        }
    }
}

// Upstream gradient with relu_back_ (nn.rs:432-439) folded in: d where the
// ReLU output y is > 0 (or not <= 0), else 0.
template <bool MASK>
__device__ __forceinline__ float masked(float d, const float *mask, size_t i) {
    if constexpr (MASK) return mask[i] <= 0.0f ? 0.0f : d;
    return d;
}

// BatchNorm2d::backward (nn.rs:379-404), partial sums: part[ci][p] =
// (sum dy*xhat, sum dy) with xhat = (x - mean) * invstd recomputed exactly as
// the forward rounded it; the products are f32 as in the reference, the sums
// f64.
template <bool MASK>
__global__ __launch_bounds__(RED_THREADS) void bn_bwd_part_kernel(
    const float *__restrict__ d, const float *__restrict__ mask, const float *__restrict__ x,
    const float *__restrict__ mean, const float *__restrict__ invstd, int n, int C, int hw,
    int vec, int G, FastDiv fd_hw4, double *part) {
    const int ci = blockIdx.x, p = blockIdx.y, P = gridDim.y;
    const int i0 = p * G, i1 = min(n, i0 + G);
    const float mu = mean[ci], is = invstd[ci];
    double a = 0.0, b = 0.0;
    if ((hw & 3) == 0 && vec) {
        const int hw4 = hw >> 2, tot = (i1 - i0) * hw4;
        for (int e = threadIdx.x; e < tot; e += RED_THREADS) {
            const int img = (int)div_by((uint32_t)e, fd_hw4), r = e - img * hw4;
            const size_t i = ((size_t)(i0 + img) * C + ci) * hw + 4 * r;
            const float4 dv = *reinterpret_cast<const float4 *>(d + i);
            const float4 xv = *reinterpret_cast<const float4 *>(x + i);
            float4 mv = make_float4(1.f, 1.f, 1.f, 1.f);
            if constexpr (MASK) mv = *reinterpret_cast<const float4 *>(mask + i);
            const float dd[4] = {dv.x, dv.y, dv.z, dv.w}, xx[4] = {xv.x, xv.y, xv.z, xv.w};
            const float mm[4] = {mv.x, mv.y, mv.z, mv.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float g = (MASK && mm[j] <= 0.0f) ? 0.0f : dd[j];
                const float xh = (xx[j] - mu) * is;
                a += (double)(g * xh);
                b += (double)g;
            }
        }
    } else {
        const int tot = (i1 - i0) * hw;
        for (int e = threadIdx.x; e < tot; e += RED_THREADS) {
            const int img = e / hw, r = e - img * hw;
            const size_t i = ((size_t)(i0 + img) * C + ci) * hw + r;
            const float g = masked<MASK>(d[i], mask, i);
            const float xh = (x[i] - mu) * is;
            a += (double)(g * xh);
            b += (double)g;
        }
    }
    block_sum2(a, b);
    if (threadIdx.x == 0) {
        part[((size_t)ci * P + p) * 2 + 0] = a;
        part[((size_t)ci * P + p) * 2 + 1] = b;
    }
}

// dx = s * (m*dy - dbeta - xhat*dgamma), s = gamma*invstd/m (nn.rs:406-421),
// over channel blockIdx.x of images [p*G, p*G + G).  dgamma / dbeta are the
// partial sums added in range order (the same in every block); thread 0 of
// the channel's first block adds them into g.g / b.g (nn.rs:423-424).
template <bool MASK>
__global__ __launch_bounds__(EW_THREADS) void bn_bwd_apply_kernel(
    const float *__restrict__ d, const float *__restrict__ mask, const float *__restrict__ x,
    RnnBn bn, const double *__restrict__ part, float *dx, int n, int C, int hw, int G,
    FastDiv fd_hw4, int vec) {
    const int ci = blockIdx.x, p = blockIdx.y;
    const int i0 = p * G, i1 = min(n, i0 + G);
    float dg, db, mu, is, m, s;
    auto coefs = [&]() {
        double sa, sb;
        part_totals(part, ci, bn.P, sa, sb);
        dg = (float)sa;
        db = (float)sb;
        if (p == 0 && threadIdx.x == 0) {
            if (bn.dgamma) bn.dgamma[ci] += dg;
            if (bn.dbeta) bn.dbeta[ci] += db;
        }
        mu = bn.mean[ci];
        is = bn.invstd[ci];
        m = bn.m;
        s = bn.gamma[ci] * is / m;
    };
    auto one = [&](float g, float xv) {
        const float xh = (xv - mu) * is;
        return s * (m * g - db - xh * dg);
    };
    const int hw4 = hw >> 2, tot4 = (i1 - i0) * hw4;
    if (vec && tot4 <= BN_PF * EW_THREADS) {
        // the items' loads go out before the partial sums are read
        float4 dv[BN_PF], xv[BN_PF], mv[BN_PF];
        size_t q[BN_PF];
#pragma unroll
        for (int u = 0; u < BN_PF; u++) {
            const int e = min((int)threadIdx.x + u * EW_THREADS, tot4 - 1);
            const int img = (int)div_by((uint32_t)e, fd_hw4), r = e - img * hw4;
            q[u] = ((size_t)(i0 + img) * C + ci) * hw4 + r;
            dv[u] = reinterpret_cast<const float4 *>(d)[q[u]];
            xv[u] = reinterpret_cast<const float4 *>(x)[q[u]];
            mv[u] = make_float4(1.f, 1.f, 1.f, 1.f);
            if constexpr (MASK) mv[u] = reinterpret_cast<const float4 *>(mask)[q[u]];
        }
        coefs();
#pragma unroll
        for (int u = 0; u < BN_PF; u++) {
            if ((int)threadIdx.x + u * EW_THREADS >= tot4) continue;
            const float g0 = (MASK && mv[u].x <= 0.0f) ? 0.0f : dv[u].x;
            const float g1 = (MASK && mv[u].y <= 0.0f) ? 0.0f : dv[u].y;
            const float g2 = (MASK && mv[u].z <= 0.0f) ? 0.0f : dv[u].z;
            const float g3 = (MASK && mv[u].w <= 0.0f) ? 0.0f : dv[u].w;
            reinterpret_cast<float4 *>(dx)[q[u]] = make_float4(
                one(g0, xv[u].x), one(g1, xv[u].y), one(g2, xv[u].z), one(g3, xv[u].w));
        }
        return;
    }
    coefs();
    if (vec) {
        const int hw4 = hw >> 2, tot = (i1 - i0) * hw4;
        for (int e = threadIdx.x; e < tot; e += EW_THREADS) {
            const int img = (int)div_by((uint32_t)e, fd_hw4), r = e - img * hw4;
            const size_t q = ((size_t)(i0 + img) * C + ci) * hw4 + r;
            const float4 dv = reinterpret_cast<const float4 *>(d)[q];
            const float4 xv = reinterpret_cast<const float4 *>(x)[q];
            float4 mv = make_float4(1.f, 1.f, 1.f, 1.f);
            if constexpr (MASK) mv = reinterpret_cast<const float4 *>(mask)[q];
            const float g0 = (MASK && mv.x <= 0.0f) ? 0.0f : dv.x;
            const float g1 = (MASK && mv.y <= 0.0f) ? 0.0f : dv.y;
            const float g2 = (MASK && mv.z <= 0.0f) ? 0.0f : dv.z;
            const float g3 = (MASK && mv.w <= 0.0f) ? 0.0f : dv.w;
            reinterpret_cast<float4 *>(dx)[q] =
                make_float4(one(g0, xv.x), one(g1, xv.y), one(g2, xv.z), one(g3, xv.w));
        }
    } else {
        const int tot = (i1 - i0) * hw;
        for (int e = threadIdx.x; e < tot; e += EW_THREADS) {
            const int img = e / hw, r = e - img * hw;
            const size_t i = ((size_t)(i0 + img) * C + ci) * hw + r;
            dx[i] = one(masked<MASK>(d[i], mask, i), x[i]);
        }
    }
}

// a[i] += [mask] b[i] (add_, nn.rs:441-443, with relu_back_ of b folded in).
template <bool MASK>
__global__ __launch_bounds__(EW_THREADS) void add_kernel(float *a, const float *__restrict__ b,
                                                         const float *__restrict__ mask,
                                                         size_t total, int vec) {
    for (size_t i = (size_t)blockIdx.x * EW_THREADS + threadIdx.x; 4 * i < total;
         i += (size_t)gridDim.x * EW_THREADS) {
        if (vec && 4 * i + 4 <= total) {
            float4 av = reinterpret_cast<float4 *>(a)[i];
            const float4 bv = reinterpret_cast<const float4 *>(b)[i];
            float4 mv = make_float4(1.f, 1.f, 1.f, 1.f);
            if constexpr (MASK) mv = reinterpret_cast<const float4 *>(mask)[i];
            av.x = av.x + ((MASK && mv.x <= 0.0f) ? 0.0f : bv.x);
            av.y = av.y + ((MASK && mv.y <= 0.0f) ? 0.0f : bv.y);
            av.z = av.z + ((MASK && mv.z <= 0.0f) ? 0.0f : bv.z);
            av.w = av.w + ((MASK && mv.w <= 0.0f) ? 0.0f : bv.w);
            reinterpret_cast<float4 *>(a)[i] = av;
        } else {
            for (size_t j = 4 * i; j < total; j++) a[j] = a[j] + masked<MASK>(b[j], mask, j);
        }
    }
}

// The gradient a block's backward starts from, plus the partial sums its
// BN backwards need (BasicBlock::backward, model.rs:59-77), in one pass over
// channel blockIdx.x of images [p*G, p*G + G):
//   d = relu_back_(src, mask) with src = a + add (the previous block's input
//   gradient and its shortcut term) or, for the last block, the GAP backward
//   gsrc[n][c] / hw broadcast over the plane;
//   part1 = (sum d*xhat1, sum d) with xhat1 = (x1 - mean1)*invstd1 for the
//   block's second BN, part2 likewise for its shortcut BN (when x2 is set).
// d is written over a.
struct ResidBn {
    const float *x, *mean, *invstd;
    double *part;
};

__global__ __launch_bounds__(RED_THREADS) void resid_bwd_kernel(
    float *a, const float *__restrict__ add, const float *__restrict__ mask,
    const float *__restrict__ gsrc, ResidBn b1, ResidBn b2, int n, int C, int hw, int G,
    FastDiv fd_hw4, int vec) {
    const int ci = blockIdx.x, p = blockIdx.y, P = gridDim.y;
    const int i0 = p * G, i1 = min(n, i0 + G);
    const float mu1 = b1.mean[ci], is1 = b1.invstd[ci];
    const float mu2 = b2.x ? b2.mean[ci] : 0.f, is2 = b2.x ? b2.invstd[ci] : 0.f;
    double s1 = 0.0, s2 = 0.0, sd = 0.0;
    auto one = [&](float src, float m, float x1, float x2) {
        const float d = m <= 0.0f ? 0.0f : src;
        sd += (double)d;
        s1 += (double)(d * ((x1 - mu1) * is1));
        if (b2.x) s2 += (double)(d * ((x2 - mu2) * is2));
        return d;
    };
    if (vec) {
        const int hw4 = hw >> 2, tot = (i1 - i0) * hw4;
        for (int e = threadIdx.x; e < tot; e += RED_THREADS) {
            const int img = (int)div_by((uint32_t)e, fd_hw4), r = e - img * hw4;
            const size_t q = ((size_t)(i0 + img) * C + ci) * hw4 + r;
            float4 sv;
            if (gsrc) {
                const float g = gsrc[(size_t)(i0 + img) * C + ci] / (float)hw;
                sv = make_float4(g, g, g, g);
            } else {
                sv = reinterpret_cast<const float4 *>(a)[q];
                if (add) {
                    const float4 av = reinterpret_cast<const float4 *>(add)[q];
                    sv.x = sv.x + av.x;
                    sv.y = sv.y + av.y;
                    sv.z = sv.z + av.z;
                    sv.w = sv.w + av.w;
                }
            }
            const float4 mv = reinterpret_cast<const float4 *>(mask)[q];
            const float4 x1 = reinterpret_cast<const float4 *>(b1.x)[q];
            float4 x2 = make_float4(0.f, 0.f, 0.f, 0.f);
            if (b2.x) x2 = reinterpret_cast<const float4 *>(b2.x)[q];
            float4 dv;  // element order fixed: the sums run x, y, z, w
            dv.x = one(sv.x, mv.x, x1.x, x2.x);
            dv.y = one(sv.y, mv.y, x1.y, x2.y);
            dv.z = one(sv.z, mv.z, x1.z, x2.z);
            dv.w = one(sv.w, mv.w, x1.w, x2.w);
            reinterpret_cast<float4 *>(a)[q] = dv;
        }
    } else {
        const int tot = (i1 - i0) * hw;
        for (int e = threadIdx.x; e < tot; e += RED_THREADS) {
            const int img = e / hw, r = e - img * hw;
            const size_t i = ((size_t)(i0 + img) * C + ci) * hw + r;
            float src;
            if (gsrc)
                src = gsrc[(size_t)(i0 + img) * C + ci] / (float)hw;
            else
                src = add ? a[i] + add[i] : a[i];
            a[i] = one(src, mask[i], b1.x[i], b2.x ? b2.x[i] : 0.f);
        }
    }
    block_sum2(s1, sd);
    double s2t = 0.0, dummy = 0.0;
    if (b2.x) {
        __syncthreads();
        s2t = s2;
        block_sum2(s2t, dummy);
    }
    if (threadIdx.x == 0) {
        b1.part[((size_t)ci * P + p) * 2 + 0] = s1;
        b1.part[((size_t)ci * P + p) * 2 + 1] = sd;
        if (b2.x) {
            b2.part[((size_t)ci * P + p) * 2 + 0] = s2t;
            b2.part[((size_t)ci * P + p) * 2 + 1] = sd;
        }
    }
}

// relu_back_ (nn.rs:432-439) and add_relu_ (nn.rs:446-450), elementwise.
__global__ void relu_back_kernel(float *d, const float *__restrict__ y, size_t total) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x)
        if (y[i] <= 0.0f) d[i] = 0.0f;
}

__global__ void add_relu_kernel(float *a, const float *__restrict__ b, size_t total) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const float v = a[i] + b[i];
        a[i] = v > 0.0f ? v : 0.0f;
    }
}

// The same, four elements a thread (16-byte aligned a and b, total % 4 == 0).
__global__ void add_relu4_kernel(float4 *a, const float4 *__restrict__ b, size_t total4) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total4;
         i += (size_t)gridDim.x * blockDim.x) {
        float4 v = a[i];
        const float4 w = b[i];
        v.x = v.x + w.x;
        v.y = v.y + w.y;
        v.z = v.z + w.z;
        v.w = v.w + w.w;
        v.x = v.x > 0.0f ? v.x : 0.0f;
        v.y = v.y > 0.0f ? v.y : 0.0f;
        v.z = v.z > 0.0f ? v.z : 0.0f;
        v.w = v.w > 0.0f ? v.w : 0.0f;
        a[i] = v;
    }
}

// gap_forward (nn.rs:455-463): one thread per plane, the f32 sum in pixel
// order (bit-identical to the reference), divided by hw.
__global__ void gap_fwd_kernel(const float *__restrict__ x, int hw, size_t nc, int vec, float *y) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nc) return;
    const float *p = x + i * hw;
    float s = 0.0f;
    if (vec) {
        // 16 loads in flight ahead of their (pixel-order) adds
        for (int j0 = 0; j0 < hw; j0 += 64) {
            float4 v[16];
#pragma unroll
            for (int u = 0; u < 16; u++)
                v[u] = j0 + 4 * u < hw ? *reinterpret_cast<const float4 *>(p + j0 + 4 * u)
                                       : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int u = 0; u < 16; u++) {
                if (j0 + 4 * u >= hw) break;
                s = s + v[u].x;
                s = s + v[u].y;
                s = s + v[u].z;
                s = s + v[u].w;
            }
        }
    } else {
        for (int j = 0; j < hw; j++) s = s + p[j];
    }
    y[i] = s / (float)hw;
}

// gap_backward (nn.rs:465-473).
__global__ void gap_bwd_kernel(const float *__restrict__ dy, int hw, size_t total, float *dx) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x)
        dx[i] = dy[i / hw] / (float)hw;
}

// nn.rs Linear::forward (nn.rs:500-517): y[i][o] = b[o] + w[o][0]*x[i][0] +
// ... in j order, one thread per output (bit-identical to the reference);
// VEC reads the rows as float4 (the adds stay in j order).
template <bool VEC>
__global__ void fc_fwd_kernel(const float *__restrict__ x, const float *__restrict__ w,
                              const float *__restrict__ b, int rows, int fin, int fout, float *y) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= rows * fout) return;
    const int i = t / fout, o = t - i * fout;
    const float *wr = w + (size_t)o * fin, *xr = x + (size_t)i * fin;
    float s = b[o];
    if constexpr (VEC) {
        for (int j = 0; j < fin; j += 4) {
            const float4 wv = *reinterpret_cast<const float4 *>(wr + j);
            const float4 xv = *reinterpret_cast<const float4 *>(xr + j);
            s = s + wv.x * xv.x;
            s = s + wv.y * xv.y;
            s = s + wv.z * xv.z;
            s = s + wv.w * xv.w;
        }
    } else {
        for (int j = 0; j < fin; j++) s = s + wr[j] * xr[j];
    }
    y[t] = s;
}

// gap then Linear::forward for image blockIdx.x in one launch: thread c <
// fin pools channel c as gap_fwd_kernel does (the same adds in the same
// order, then / hw) into pooled and LDS; thread o < fout then forms y[i][o]
// as fc_fwd_kernel does (b[o], then w[o][j]*x[j] in j order).  The same bits
// as the two launches.
__global__ __launch_bounds__(1024) void gap_fc_fwd_kernel(const float *__restrict__ x, int hw,
                                                          int fin, int fout, int vec,
                                                          const float *__restrict__ w,
                                                          const float *__restrict__ b,
                                                          float *pooled, float *y) {
    extern __shared__ float xs[];  // [fin]
    const int i = blockIdx.x;
    for (int c = threadIdx.x; c < fin; c += blockDim.x) {
        const float *p = x + ((size_t)i * fin + c) * hw;
        float s = 0.0f;
        if (vec) {
            for (int j = 0; j < hw; j += 4) {
                const float4 v = *reinterpret_cast<const float4 *>(p + j);
                s = s + v.x;
                s = s + v.y;
                s = s + v.z;
                s = s + v.w;
            }
        } else {
            for (int j = 0; j < hw; j++) s = s + p[j];
        }
        s = s / (float)hw;
        pooled[(size_t)i * fin + c] = s;
        xs[c] = s;
    }
    __syncthreads();
    for (int o = threadIdx.x; o < fout; o += blockDim.x) {
        const float *wr = w + (size_t)o * fin;
        float s = b[o];
        for (int j = 0; j < fin; j++) s = s + wr[j] * xs[j];
        y[(size_t)i * fout + o] = s;
    }
}

// Linear::backward_w (nn.rs:521-537): w.g[o][j] += dy[i][o]*x[i][j] in row
// order, zero gradients skipped.  Block o; thread j (coalesced over x rows);
// thread j == fin adds the bias: b.g[o] += dy[i][o].
__global__ __launch_bounds__(256) void fc_bwd_w_kernel(const float *__restrict__ dy,
                                                       const float *__restrict__ x, int rows,
                                                       int fin, int fout, float *dw, float *db) {
    constexpr int U = 8;  // loads of U rows go out before their in-order adds
    const int o = blockIdx.x;
    for (int j = threadIdx.x; j <= fin; j += blockDim.x) {
        const bool bias = j == fin;
        float acc = bias ? db[o] : dw[(size_t)o * fin + j];
        int i = 0;
        for (; i + U <= rows; i += U) {
            float g[U], xv[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                g[u] = dy[(size_t)(i + u) * fout + o];
                xv[u] = bias ? 1.0f : x[(size_t)(i + u) * fin + j];
            }
#pragma unroll
            for (int u = 0; u < U; u++)
                if (g[u] != 0.0f) acc = bias ? acc + g[u] : acc + g[u] * xv[u];
        }
        for (; i < rows; i++) {
            const float g = dy[(size_t)i * fout + o];
            if (g != 0.0f) acc = bias ? acc + g : acc + g * x[(size_t)i * fin + j];
        }
        if (bias)
            db[o] = acc;
        else
            dw[(size_t)o * fin + j] = acc;
    }
}

// Linear::backward_x (nn.rs:539-556): dx[i][j] = sum over o (in order, zero
// gradients skipped) of dy[i][o]*w[o][j], from 0.  Block i; thread j.
__global__ __launch_bounds__(256) void fc_bwd_x_kernel(const float *__restrict__ dy,
                                                       const float *__restrict__ w, int rows,
                                                       int fin, int fout, float *dx) {
    constexpr int U = 8;
    const int i = blockIdx.x;
    for (int j = threadIdx.x; j < fin; j += blockDim.x) {
        float acc = 0.0f;
        int o = 0;
        for (; o + U <= fout; o += U) {
            float g[U], wv[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                g[u] = dy[(size_t)i * fout + o + u];
                wv[u] = w[(size_t)(o + u) * fin + j];
            }
#pragma unroll
            for (int u = 0; u < U; u++)
                if (g[u] != 0.0f) acc = acc + g[u] * wv[u];
        }
        for (; o < fout; o++) {
            const float g = dy[(size_t)i * fout + o];
            if (g != 0.0f) acc = acc + g * w[(size_t)o * fin + j];
        }
        dx[(size_t)i * fin + j] = acc;
    }
}

// Max and its first index over a wave (ties keep the lower index, as the
// reference's strict > scan does).
__device__ __forceinline__ void wave_argmax(float &m, int &idx) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float m2 = __shfl_xor(m, o, 64);
        const int i2 = __shfl_xor(idx, o, 64);
        if (m2 > m || (m2 == m && i2 < idx)) {
            m = m2;
            idx = i2;
        }
    }
}

__device__ __forceinline__ float wave_sumf(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// softmax_ce (nn.rs:566-637).  One wave per row (rows wave, wave + NW, ...):
// max / first argmax, sum of exp(z - max), lse, the smoothed loss and the
// gradient (softmax - target) / rows; the wave sums run in a tree order.
// Thread 0 then adds the row losses and hits in row order.  `smooth` comes
// from device memory when `scal` is set (scal[3]), else from the argument.
// One block keeps the row results in LDS.  With `ticket` set, several blocks
// share the rows (one per wave) and keep them in rowbuf [2*rows]; the block
// that takes the last ticket adds them in row order and sets the ticket back
// to 0 for the next launch.
template <int ZR>
__global__ __launch_bounds__(1024) void softmax_ce_kernel(
    const float *__restrict__ logits, const uint32_t *__restrict__ labels, int rows, int nclass,
    float smooth_arg, const float *scal, float *dl, float *loss_out, uint32_t *correct_out,
    uint32_t *ticket, float *rowbuf) {
    extern __shared__ float row_lds[];  // [rows] losses, then [rows] hits
    float *row_loss = ticket ? rowbuf : row_lds;
    const float smooth = scal ? scal[3] : smooth_arg;
    const float inv = 1.0f / (float)rows;
    const float on = 1.0f - smooth, off = smooth / (float)nclass;
    const int wave = wave_index(), lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    for (int r = blockIdx.x * nw + wave; r < rows; r += gridDim.x * nw) {
        const float *z = logits + (size_t)r * nclass;
        float *d = dl + (size_t)r * nclass;
        const uint32_t yl = labels[r];
        // the row, ZR values per lane (class lane + 64*k), loaded once
        float zv[ZR];
#pragma unroll
        for (int k = 0; k < ZR; k++) {
            const int j = lane + 64 * k;
            zv[k] = j < nclass ? z[j] : -INFINITY;
        }
        if (yl >= (uint32_t)nclass) {  // the reference panics on such a label
#pragma unroll
            for (int k = 0; k < ZR; k++)
                if (lane + 64 * k < nclass) d[lane + 64 * k] = NAN;
            if (lane == 0) {
                row_loss[r] = NAN;
                row_loss[rows + r] = 0.0f;
            }
            continue;
        }
        const int y = (int)yl;
        float mx = -INFINITY;
        int arg = 0x7fffffff;
#pragma unroll
        for (int k = 0; k < ZR; k++)
            if (zv[k] > mx) {
                mx = zv[k];
                arg = lane + 64 * k;
            }
        wave_argmax(mx, arg);
        float e[ZR], sum = 0.0f, zs = 0.0f;
#pragma unroll
        for (int k = 0; k < ZR; k++) {
            const bool in = lane + 64 * k < nclass;
            e[k] = in ? expf(zv[k] - mx) : 0.0f;
            sum += e[k];
            zs += in ? zv[k] : 0.0f;
        }
        sum = wave_sumf(sum);
        zs = wave_sumf(zs);
        const float lse = mx + logf(sum);
#pragma unroll
        for (int k = 0; k < ZR; k++) {
            const int j = lane + 64 * k;
            if (j < nclass) {
                const float t = j == y ? on + off : off;
                d[j] = (e[k] / sum - t) * inv;
            }
        }
        // z[y] from the lane that holds it
        float zy = 0.0f;
#pragma unroll
        for (int k = 0; k < ZR; k++)
            if (lane + 64 * k == y) zy = zv[k];
        zy = wave_sumf(zy);
        if (lane == 0) {
            float l = on * (lse - zy);
            // sum_j (lse - z_j) = nclass*lse - sum_j z_j
            if (smooth > 0.0f) l = l + off * ((float)nclass * lse - zs);
            row_loss[r] = l;
            row_loss[rows + r] = arg == y ? 1.0f : 0.0f;
        }
    }
    // every wave releases its own row stores at agent scope before the
    // barrier, so the block's ticket below orders all of them, not only
    // thread 0's
    if (ticket) __threadfence();
    __syncthreads();
    if (ticket) {
        // the last block to finish gathers every block's rows into LDS
        __shared__ int last;
        if (threadIdx.x == 0) {
            __threadfence();
            last = atomicAdd(ticket, 1u) == gridDim.x - 1;
        }
        __syncthreads();
        if (!last) return;
        __threadfence();
        for (int i = threadIdx.x; i < 2 * rows; i += blockDim.x)
            row_lds[i] = __hip_atomic_load(rowbuf + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        float l = 0.0f;
        uint32_t ok = 0;
        for (int r = 0; r < rows; r++) {
            l = l + row_lds[r];
            ok += row_lds[rows + r] != 0.0f;
        }
        if (loss_out) loss_out[0] = l * inv;
        if (correct_out) correct_out[0] = ok;
        if (ticket) __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Param::step (nn.rs:102-110) over a flat parameter array whose first
// `ndecay` elements take weight decay.  (lr, mom, wd) come from scal[0..3]
// when scal is set.
__global__ __launch_bounds__(EW_THREADS) void sgd_kernel(float *v, float *g, float *m, size_t len,
                                                         size_t ndecay, float lr_a, float mom_a,
                                                         float wd_a, const float *scal) {
    const float lr = scal ? scal[0] : lr_a, mom = scal ? scal[1] : mom_a;
    const float wdv = scal ? scal[2] : wd_a;
    for (size_t i = (size_t)blockIdx.x * EW_THREADS + threadIdx.x; i < len;
         i += (size_t)gridDim.x * EW_THREADS) {
        const float wd = i < ndecay ? wdv : 0.0f;
        const float gi = g[i] + wd * v[i];
        const float mi = mom * m[i] + gi;
        m[i] = mi;
        v[i] = v[i] - lr * (gi + mom * mi);
        g[i] = 0.0f;
    }
}

// Gradient finalisation over a flat parameter layout: block b belongs to the
// segment with the last blk0 <= b and takes its 32 elements [32*(b - blk0),
// +32).  Slab sums follow the dW reduction exactly (8 thread groups each sum
// a contiguous run of slabs with 16 loads in flight, then the 8 partials in
// order), so g ends as it would after a separate reduce; the SGD step is
// Param::step (nn.rs:102-110) on that g.
__global__ __launch_bounds__(256) void grad_finalize_kernel(const GradSeg *__restrict__ segs,
                                                            int nseg, float *v, float *g,
                                                            float *m, const float *scal,
                                                            int do_sgd) {
    constexpr int PARTS = 8;
    __shared__ float red[PARTS][32];
    int lo = 0, hi = nseg - 1;
    while (lo < hi) {  // last segment with blk0 <= blockIdx.x
        const int mid = (lo + hi + 1) >> 1;
        if (segs[mid].blk0 <= (long long)blockIdx.x)
            lo = mid;
        else
            hi = mid - 1;
    }
    const GradSeg sg = segs[lo];
    const int el = threadIdx.x & 31, j = threadIdx.x >> 5;
    const long long e = ((long long)blockIdx.x - sg.blk0) * 32 + el;
    const bool in = e < sg.len;
    if (sg.nz > 0) {
        const int G = (sg.nz + PARTS - 1) / PARTS;
        const int z0 = j * G, z1 = min(sg.nz, z0 + G);
        float s = 0.f;
        if (in) {
            for (int b = z0; b < z1; b += 16) {
                float t[16];
#pragma unroll
                for (int u = 0; u < 16; u++)
                    t[u] = b + u < z1 ? sg.slabs[(long long)(b + u) * sg.len + e] : 0.f;
#pragma unroll
                for (int u = 0; u < 16; u++)
                    if (b + u < z1) s = (b + u == z0) ? t[u] : s + t[u];
            }
        }
        red[j][el] = s;
    }
    __syncthreads();
    if (j != 0 || !in) return;
    const long long i = sg.off + e;
    float gi = g[i];
    if (sg.nz > 0) {
        float t = red[0][el];
        for (int q = 1; q < PARTS && q * ((sg.nz + PARTS - 1) / PARTS) < sg.nz; q++) t += red[q][el];
        gi += t;
    }
    if (!do_sgd) {
        g[i] = gi;
        return;
    }
    const float lr = scal[0], mom = scal[1], wd = sg.decay ? scal[2] : 0.0f;
    const float gg = gi + wd * v[i];
    const float mi = mom * m[i] + gg;
    m[i] = mi;
    v[i] = v[i] - lr * (gg + mom * mi);
    g[i] = 0.0f;
}

__global__ void set_scalars_kernel(float *scal, float a, float b, float c, float d) {
    scal[0] = a;
    scal[1] = b;
    scal[2] = c;
    scal[3] = d;
}

// Divider for indices n < limit: the multiply-high form when it is exact
// there (n * d < 2^32), else marked for plain division.
static inline FastDiv divider(size_t d, size_t limit) {
    FastDiv f = make_fastdiv((uint32_t)std::max<size_t>(d, 1));
    if (d > 1 && (unsigned __int128)limit * d >= ((unsigned __int128)1 << 32)) f.m = 0;
    return f;
}

static inline bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

static inline unsigned ew_grid(rnn_ctx *ctx, size_t items, int threads = EW_THREADS) {
    size_t g = rnn_div_up(std::max<size_t>(items, 1), threads);
    return (unsigned)std::min<size_t>(g, (size_t)ctx->num_cus * 16);
}

}  // namespace

// ---------------------------------------------------------------- launchers

size_t rnn_bn_scratch_doubles(size_t n, size_t c) {
    ChanSplit s = chan_split(n, c);
    return 2 * c * (size_t)s.P;
}

int rnn_bn_stats_launch(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *x,
                        double *part) {
    ChanSplit s = chan_split(n, c);
    bn_stats_part_kernel<<<dim3((unsigned)c, (unsigned)s.P), RED_THREADS, 0, ctx->stream>>>(
        x, (int)n, (int)c, (int)hw, aligned16(x), s.G, divider(hw / 4, (size_t)s.G * (hw / 4)),
        part);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

template <bool EVAL, bool RELU, int SKIP>
static void bn_apply_t(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *x,
                       const RnnBn &bn, const float *skip, const RnnBn &sbn, float *out) {
    ChanSplit s = chan_split(n, c);
    const int vec = (hw & 3) == 0 && aligned16(x) && aligned16(out) &&
                    (SKIP == 0 || aligned16(skip));
    bn_apply_kernel<EVAL, RELU, SKIP><<<dim3((unsigned)c, (unsigned)s.P), EW_THREADS, 0,
                                        ctx->stream>>>(
        x, bn, skip, sbn, out, (int)n, (int)c, (int)hw, s.G,
        divider(hw / 4, (size_t)s.G * (hw / 4)), vec);
}

int rnn_bn_apply_launch(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *x, RnnBn bn,
                        bool eval, int relu, int skip_mode, const float *skip, const RnnBn *sbn,
                        float *out) {
    if (n * c * hw == 0) return RNN_OK;
    ChanSplit s = chan_split(n, c);
    if (bn.P <= 0) bn.P = s.P;  // else the partials come from a conv's store pass
    bn.m = (float)(n * hw);
    RnnBn sb = sbn ? *sbn : bn;
    if (sb.P <= 0) sb.P = s.P;
    sb.m = bn.m;
    if (eval) {
        if (skip_mode == 0) {
            if (relu)
                bn_apply_t<true, true, 0>(ctx, n, c, hw, x, bn, skip, sb, out);
            else
                bn_apply_t<true, false, 0>(ctx, n, c, hw, x, bn, skip, sb, out);
        } else if (skip_mode == 1) {
            bn_apply_t<true, true, 1>(ctx, n, c, hw, x, bn, skip, sb, out);
        } else {
            bn_apply_t<true, true, 2>(ctx, n, c, hw, x, bn, skip, sb, out);
        }
    } else {
        if (skip_mode == 0) {
            if (relu)
                bn_apply_t<false, true, 0>(ctx, n, c, hw, x, bn, skip, sb, out);
            else
                bn_apply_t<false, false, 0>(ctx, n, c, hw, x, bn, skip, sb, out);
        } else if (skip_mode == 1) {
            bn_apply_t<false, true, 1>(ctx, n, c, hw, x, bn, skip, sb, out);
        } else {
            bn_apply_t<false, true, 2>(ctx, n, c, hw, x, bn, skip, sb, out);
        }
    }
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_bn_backward_apply_launch(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *dy,
                                 const float *mask, const float *x, RnnBn bn,
                                 const double *part, float *dx) {
    if (n * c * hw == 0) return RNN_OK;
    ChanSplit s = chan_split(n, c);
    if (bn.P <= 0) bn.P = s.P;  // else the partials come from a conv's store pass
    bn.m = (float)(n * hw);
    const FastDiv fd_hw4 = divider(hw / 4, (size_t)s.G * (hw / 4));
    const dim3 grid((unsigned)c, (unsigned)s.P);
    const int vec = (hw & 3) == 0 && aligned16(dy) && aligned16(x) && aligned16(dx) &&
                    (!mask || aligned16(mask));
    if (mask)
        bn_bwd_apply_kernel<true><<<grid, EW_THREADS, 0, ctx->stream>>>(
            dy, mask, x, bn, part, dx, (int)n, (int)c, (int)hw, s.G, fd_hw4, vec);
    else
        bn_bwd_apply_kernel<false><<<grid, EW_THREADS, 0, ctx->stream>>>(
            dy, mask, x, bn, part, dx, (int)n, (int)c, (int)hw, s.G, fd_hw4, vec);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_bn_backward_launch(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *dy,
                           const float *mask, const float *x, RnnBn bn, double *part, float *dx) {
    if (n * c * hw == 0) return RNN_OK;
    ChanSplit s = chan_split(n, c);
    const FastDiv fd_hw4 = divider(hw / 4, (size_t)s.G * (hw / 4));
    const dim3 grid((unsigned)c, (unsigned)s.P);
    const int vec = (hw & 3) == 0 && aligned16(dy) && aligned16(x) && (!mask || aligned16(mask));
    if (mask)
        bn_bwd_part_kernel<true><<<grid, RED_THREADS, 0, ctx->stream>>>(
            dy, mask, x, bn.mean, bn.invstd, (int)n, (int)c, (int)hw, vec, s.G, fd_hw4, part);
    else
        bn_bwd_part_kernel<false><<<grid, RED_THREADS, 0, ctx->stream>>>(
            dy, mask, x, bn.mean, bn.invstd, (int)n, (int)c, (int)hw, vec, s.G, fd_hw4, part);
    RNN_LAUNCHED(ctx);
    bn.P = s.P;  // the partials just taken
    return rnn_bn_backward_apply_launch(ctx, n, c, hw, dy, mask, x, bn, part, dx);
}

int rnn_resid_bwd_launch(rnn_ctx *ctx, size_t n, size_t c, size_t hw, float *a, const float *add,
                         const float *mask, const float *gsrc, const RnnBn &bn1, const float *x1,
                         double *part1, const RnnBn *bn2, const float *x2, double *part2) {
    if (n * c * hw == 0) return RNN_OK;
    ChanSplit s = chan_split(n, c);
    ResidBn b1{x1, bn1.mean, bn1.invstd, part1};
    ResidBn b2{bn2 ? x2 : nullptr, bn2 ? bn2->mean : nullptr, bn2 ? bn2->invstd : nullptr,
               bn2 ? part2 : nullptr};
    const int vec = (hw & 3) == 0 && aligned16(a) && (!add || aligned16(add)) &&
                    aligned16(mask) && aligned16(x1) && (!b2.x || aligned16(b2.x));
    resid_bwd_kernel<<<dim3((unsigned)c, (unsigned)s.P), RED_THREADS, 0, ctx->stream>>>(
        a, add, mask, gsrc, b1, b2, (int)n, (int)c, (int)hw, s.G,
        divider(hw / 4, (size_t)s.G * (hw / 4)), vec);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_add_launch(rnn_ctx *ctx, size_t len, float *a, const float *b, const float *mask) {
    if (len == 0) return RNN_OK;
    const size_t items = rnn_div_up(len, 4);
    const int vec = aligned16(a) && aligned16(b) && (!mask || aligned16(mask));
    if (mask)
        add_kernel<true><<<ew_grid(ctx, items), EW_THREADS, 0, ctx->stream>>>(a, b, mask, len,
                                                                               vec);
    else
        add_kernel<false><<<ew_grid(ctx, items), EW_THREADS, 0, ctx->stream>>>(a, b, mask, len,
                                                                                vec);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_relu_back_launch(rnn_ctx *ctx, size_t len, float *d, const float *y) {
    if (len == 0) return RNN_OK;
    relu_back_kernel<<<ew_grid(ctx, len), EW_THREADS, 0, ctx->stream>>>(d, y, len);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_gap_forward_launch(rnn_ctx *ctx, size_t nc, size_t hw, const float *x, float *y) {
    if (nc == 0) return RNN_OK;
    const int vec = (hw & 3) == 0 && aligned16(x);
    gap_fwd_kernel<<<(unsigned)rnn_div_up(nc, 128), 128, 0, ctx->stream>>>(x, (int)hw, nc, vec, y);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_gap_backward_launch(rnn_ctx *ctx, size_t nc, size_t hw, const float *dy, float *dx) {
    if (nc * hw == 0) return RNN_OK;
    gap_bwd_kernel<<<ew_grid(ctx, nc * hw), EW_THREADS, 0, ctx->stream>>>(dy, (int)hw, nc * hw,
                                                                         dx);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_gap_fc_forward_launch(rnn_ctx *ctx, size_t rows, size_t fin, size_t hw, size_t fout,
                              const float *x, const float *w, const float *b, float *pooled,
                              float *y) {
    if (rows == 0 || fin == 0) return RNN_OK;
    if (fin > 8192 || rows > 0x7fffffff) {
        const int rc = rnn_gap_forward_launch(ctx, rows * fin, hw, x, pooled);
        return rc ? rc : rnn_fc_forward_launch(ctx, rows, fin, fout, pooled, w, b, y);
    }
    const int vec = (hw & 3) == 0 && aligned16(x);
    const unsigned threads =
        (unsigned)std::min<size_t>(1024, rnn_round_up(std::max(fin, fout), 64));
    gap_fc_fwd_kernel<<<(unsigned)rows, threads, fin * sizeof(float), ctx->stream>>>(
        x, (int)hw, (int)fin, (int)fout, vec, w, b, pooled, y);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_fc_forward_launch(rnn_ctx *ctx, size_t rows, size_t fin, size_t fout, const float *x,
                          const float *w, const float *b, float *y) {
    const size_t t = rows * fout;
    if (t == 0) return RNN_OK;
    if ((fin & 3) == 0 && aligned16(x) && aligned16(w))
        fc_fwd_kernel<true><<<(unsigned)rnn_div_up(t, 128), 128, 0, ctx->stream>>>(
            x, w, b, (int)rows, (int)fin, (int)fout, y);
    else
        fc_fwd_kernel<false><<<(unsigned)rnn_div_up(t, 128), 128, 0, ctx->stream>>>(
            x, w, b, (int)rows, (int)fin, (int)fout, y);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_fc_backward_launch(rnn_ctx *ctx, size_t rows, size_t fin, size_t fout, const float *dy,
                           const float *x, const float *w, float *dw, float *db, float *dx) {
    const unsigned tb = (unsigned)std::min<size_t>(256, rnn_round_up(fin + 1, 64));
    if (fout && dw && db) {
        fc_bwd_w_kernel<<<(unsigned)fout, tb, 0, ctx->stream>>>(dy, x, (int)rows, (int)fin,
                                                                (int)fout, dw, db);
        RNN_LAUNCHED(ctx);
    }
    if (rows && fin && dx) {
        fc_bwd_x_kernel<<<(unsigned)rows, tb, 0, ctx->stream>>>(dy, w, (int)rows, (int)fin,
                                                                (int)fout, dx);
        RNN_LAUNCHED(ctx);
    }
    return RNN_OK;
}

int rnn_softmax_ce_launch(rnn_ctx *ctx, size_t rows, size_t nclass, const float *logits,
                          const uint32_t *labels, float smooth, const float *scal, float *dl,
                          float *loss, uint32_t *correct, uint32_t *ticket, float *rowbuf) {
    if (rows == 0) return RNN_OK;
    // with a ticket: one row per wave, four waves a block
    const bool multi = ticket && rowbuf && rows > 4;
    const unsigned threads = multi ? 256u : (unsigned)std::min<size_t>(64 * rows, 1024);
    const unsigned blocks = multi ? (unsigned)rnn_div_up(rows, 4) : 1u;
    const size_t lds = 2 * rows * sizeof(float);
    auto go = [&](auto kern) {
        kern<<<blocks, threads, lds, ctx->stream>>>(logits, labels, (int)rows, (int)nclass, smooth,
                                                    scal, dl, loss, correct,
                                                    multi ? ticket : nullptr, rowbuf);
    };
    if (nclass <= 64)
        go(softmax_ce_kernel<1>);
    else if (nclass <= 128)
        go(softmax_ce_kernel<2>);
    else if (nclass <= 256)
        go(softmax_ce_kernel<4>);
    else if (nclass <= 1024)
        go(softmax_ce_kernel<16>);
    else
        return rnn_fail(ctx, RNN_E_UNSUPPORTED, "softmax_ce: nclass %zu > 1024", nclass);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_sgd_launch(rnn_ctx *ctx, size_t len, size_t ndecay, float *v, float *g, float *m, float lr,
                   float mom, float wd, const float *scal) {
    if (len == 0) return RNN_OK;
    sgd_kernel<<<ew_grid(ctx, len), EW_THREADS, 0, ctx->stream>>>(v, g, m, len, ndecay, lr, mom,
                                                                  wd, scal);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_grad_finalize_launch(rnn_ctx *ctx, const GradSeg *segs, int nseg, long long nblocks,
                             float *v, float *g, float *m, const float *scal, int do_sgd) {
    if (nblocks <= 0) return RNN_OK;
    grad_finalize_kernel<<<(unsigned)nblocks, 256, 0, ctx->stream>>>(segs, nseg, v, g, m, scal,
                                                                     do_sgd);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_set_scalars_launch(rnn_ctx *ctx, float *scal, float a, float b, float c, float d) {
    set_scalars_kernel<<<1, 1, 0, ctx->stream>>>(scal, a, b, c, d);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

// ---------------------------------------------------------------- C ABI

namespace {

// BN partial sums in the workspace.
double *bn_scratch(rnn_ctx *ctx, size_t n, size_t c) {
    return (double *)rnn_workspace(ctx, rnn_bn_scratch_doubles(n, c) * sizeof(double));
}

bool dims_ok(size_t n, size_t c, size_t hw) {
    return n * c * hw < (1ull << 34) && n * c < (1ull << 31) && c < (1u << 20) && hw < (1u << 30);
}

}  // namespace

extern "C" {

int rnn_bn_forward_train(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *x, float *y,
                         const float *gamma, const float *beta, float *running_mean,
                         float *running_var, float *mean, float *invstd, float momentum, float eps,
                         int relu) {
    if (!ctx) return RNN_E_NULL;
    if (n * c * hw == 0) return RNN_OK;
    if (!x || !y || !gamma || !beta || !mean || !invstd)
        return rnn_fail(ctx, RNN_E_NULL, "bn_forward_train: null pointer");
    if ((running_mean == nullptr) != (running_var == nullptr))
        return rnn_fail(ctx, RNN_E_NULL, "bn_forward_train: running mean/var must both be set");
    if (!dims_ok(n, c, hw)) return rnn_fail(ctx, RNN_E_INVALID, "bn_forward_train: too large");
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    double *part = bn_scratch(ctx, n, c);
    if (!part) return RNN_E_NOMEM;
    int st = rnn_bn_stats_launch(ctx, n, c, hw, x, part);
    if (st) return st;
    RnnBn bn;
    bn.part = part;
    bn.mom = momentum;
    bn.eps = eps;
    bn.mean = mean;
    bn.invstd = invstd;
    bn.rm = running_mean;
    bn.rv = running_var;
    bn.gamma = gamma;
    bn.beta = beta;
    return rnn_bn_apply_launch(ctx, n, c, hw, x, bn, false, relu, 0, nullptr, nullptr, y);
}

int rnn_bn_forward_eval(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *x, float *y,
                        const float *gamma, const float *beta, const float *running_mean,
                        const float *running_var, float eps, int relu) {
    if (!ctx) return RNN_E_NULL;
    if (n * c * hw == 0) return RNN_OK;
    if (!x || !y || !gamma || !beta || !running_mean || !running_var)
        return rnn_fail(ctx, RNN_E_NULL, "bn_forward_eval: null pointer");
    if (!dims_ok(n, c, hw)) return rnn_fail(ctx, RNN_E_INVALID, "bn_forward_eval: too large");
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    RnnBn bn;
    bn.eps = eps;
    bn.rm = const_cast<float *>(running_mean);  // read only in eval mode
    bn.rv = const_cast<float *>(running_var);
    bn.gamma = gamma;
    bn.beta = beta;
    return rnn_bn_apply_launch(ctx, n, c, hw, x, bn, true, relu, 0, nullptr, nullptr, y);
}

int rnn_bn_backward(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *dy,
                    const float *relu_out, const float *x, const float *mean, const float *invstd,
                    const float *gamma, float *dx, float *dgamma, float *dbeta) {
    if (!ctx) return RNN_E_NULL;
    if (n * c * hw == 0) return RNN_OK;
    if (!dy || !x || !mean || !invstd || !gamma || !dx || !dgamma || !dbeta)
        return rnn_fail(ctx, RNN_E_NULL, "bn_backward: null pointer");
    if (!dims_ok(n, c, hw)) return rnn_fail(ctx, RNN_E_INVALID, "bn_backward: too large");
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    double *part = bn_scratch(ctx, n, c);
    if (!part) return RNN_E_NOMEM;
    RnnBn bn;
    bn.mean = const_cast<float *>(mean);
    bn.invstd = const_cast<float *>(invstd);
    bn.gamma = gamma;
    bn.dgamma = dgamma;
    bn.dbeta = dbeta;
    return rnn_bn_backward_launch(ctx, n, c, hw, dy, relu_out, x, bn, part, dx);
}

int rnn_relu_back(rnn_ctx *ctx, size_t len, float *d, const float *y) {
    if (!ctx) return RNN_E_NULL;
    if (len == 0) return RNN_OK;
    if (!d || !y) return rnn_fail(ctx, RNN_E_NULL, "relu_back: null pointer");
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    return rnn_relu_back_launch(ctx, len, d, y);
}

int rnn_add(rnn_ctx *ctx, size_t len, float *a, const float *b) {
    if (!ctx) return RNN_E_NULL;
    if (len == 0) return RNN_OK;
    if (!a || !b) return rnn_fail(ctx, RNN_E_NULL, "add: null pointer");
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    return rnn_add_launch(ctx, len, a, b, nullptr);
}

int rnn_add_relu_back(rnn_ctx *ctx, size_t len, float *a, const float *b, const float *y) {
    if (!ctx) return RNN_E_NULL;
    if (len == 0) return RNN_OK;
    if (!a || !b || !y) return rnn_fail(ctx, RNN_E_NULL, "add_relu_back: null pointer");
    if (a == b) return rnn_fail(ctx, RNN_E_INVALID, "add_relu_back: a is b");
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    return rnn_add_launch(ctx, len, a, b, y);
}

int rnn_add_relu(rnn_ctx *ctx, size_t len, float *a, const float *b) {
    if (!ctx) return RNN_E_NULL;
    if (len == 0) return RNN_OK;
    if (!a || !b) return rnn_fail(ctx, RNN_E_NULL, "add_relu: null pointer");
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (len % 4 == 0 && aligned16(a) && aligned16(b))
        add_relu4_kernel<<<ew_grid(ctx, len / 4), EW_THREADS, 0, ctx->stream>>>(
            (float4 *)a, (const float4 *)b, len / 4);
    else
        add_relu_kernel<<<ew_grid(ctx, len), EW_THREADS, 0, ctx->stream>>>(a, b, len);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_gap_forward(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *x, float *y) {
    if (!ctx) return RNN_E_NULL;
    if (n * c * hw == 0) return RNN_OK;
    if (!x || !y) return rnn_fail(ctx, RNN_E_NULL, "gap_forward: null pointer");
    if (!dims_ok(n, c, hw)) return rnn_fail(ctx, RNN_E_INVALID, "gap_forward: too large");
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    return rnn_gap_forward_launch(ctx, n * c, hw, x, y);
}

int rnn_gap_backward(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *dy, float *dx) {
    if (!ctx) return RNN_E_NULL;
    if (n * c * hw == 0) return RNN_OK;
    if (!dy || !dx) return rnn_fail(ctx, RNN_E_NULL, "gap_backward: null pointer");
    if (!dims_ok(n, c, hw)) return rnn_fail(ctx, RNN_E_INVALID, "gap_backward: too large");
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    return rnn_gap_backward_launch(ctx, n * c, hw, dy, dx);
}

int rnn_fc_forward(rnn_ctx *ctx, size_t rows, size_t fin, size_t fout, const float *x,
                   const float *w, const float *b, float *y) {
    if (!ctx) return RNN_E_NULL;
    if (rows * fout == 0) return RNN_OK;
    if (!x || !w || !b || !y) return rnn_fail(ctx, RNN_E_NULL, "fc_forward: null pointer");
    if (rows * fout >= (1ull << 31) || rows * fin >= (1ull << 31))
        return rnn_fail(ctx, RNN_E_INVALID, "fc_forward: too large");
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    return rnn_fc_forward_launch(ctx, rows, fin, fout, x, w, b, y);
}

int rnn_fc_backward(rnn_ctx *ctx, size_t rows, size_t fin, size_t fout, const float *dy,
                    const float *x, const float *w, float *dw, float *db, float *dx) {
    if (!ctx) return RNN_E_NULL;
    if (!dy || !x || !w || !dw || !db) return rnn_fail(ctx, RNN_E_NULL, "fc_backward: null pointer");
    if (rows * fout >= (1ull << 31) || rows * fin >= (1ull << 31) ||
        fout * (fin + 1) >= (1ull << 31))
        return rnn_fail(ctx, RNN_E_INVALID, "fc_backward: too large");
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    return rnn_fc_backward_launch(ctx, rows, fin, fout, dy, x, w, dw, db, dx);
}

int rnn_softmax_ce(rnn_ctx *ctx, size_t rows, size_t nclass, const float *logits,
                   const uint32_t *labels, float smooth, float *dlogits, float *loss,
                   uint32_t *correct) {
    if (!ctx) return RNN_E_NULL;
    if (rows == 0) return RNN_OK;
    if (!logits || !labels || !dlogits) return rnn_fail(ctx, RNN_E_NULL, "softmax_ce: null pointer");
    if (nclass == 0 || rows > 8192 || rows * nclass >= (1ull << 31))
        return rnn_fail(ctx, RNN_E_INVALID, "softmax_ce: rows %zu x nclass %zu unsupported", rows,
                        nclass);
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    return rnn_softmax_ce_launch(ctx, rows, nclass, logits, labels, smooth, nullptr, dlogits, loss,
                                 correct);
}

int rnn_sgd_step(rnn_ctx *ctx, size_t len, float *v, float *g, float *m, float lr, float momentum,
                 float wd) {
    if (!ctx) return RNN_E_NULL;
    if (len == 0) return RNN_OK;
    if (!v || !g || !m) return rnn_fail(ctx, RNN_E_NULL, "sgd_step: null pointer");
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    return rnn_sgd_launch(ctx, len, len, v, g, m, lr, momentum, wd, nullptr);
}

}  // extern "C"
