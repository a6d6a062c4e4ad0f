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

// batch_stats + the per-channel part of run_train (nn.rs:272-320): mean, var
// (f64, clamped at 0), invstd = 1/sqrt(var + eps), running mean / unbiased
// running variance.
__global__ void bn_stats_final_kernel(const double *__restrict__ part, int P, int C, float m,
                                      float mom, float eps, float *mean, float *invstd, float *rm,
                                      float *rv) {
    const int ci = blockIdx.x * blockDim.x + threadIdx.x;
    if (ci >= C) return;
    double s = 0.0, s2 = 0.0;
    for (int p = 0; p < P; p++) {
        s += part[((size_t)ci * P + p) * 2 + 0];
        s2 += part[((size_t)ci * P + p) * 2 + 1];
    }
    const double mu = s / (double)m;
    const double va = s2 / (double)m - mu * mu;
    const float meanf = (float)mu, varf = (float)(va > 0.0 ? va : 0.0);
    const float is = 1.0f / sqrtf(varf + eps);
    mean[ci] = meanf;
    invstd[ci] = is;
    if (rm) {
        rm[ci] = (1.0f - mom) * rm[ci] + mom * meanf;
        const float den = fmaxf(m - 1.0f, 1.0f);
        const float unb = varf * m / den;
        rv[ci] = (1.0f - mom) * rv[ci] + mom * unb;
    }
}

// run_eval (nn.rs:350-365): per-channel scale and shift.
__global__ void bn_eval_prep_kernel(const float *__restrict__ gamma, const float *__restrict__ beta,
                                    const float *__restrict__ rm, const float *__restrict__ rv,
                                    float eps, int C, float *sc, float *sh) {
    const int ci = blockIdx.x * blockDim.x + threadIdx.x;
    if (ci >= C) return;
    const float is = 1.0f / sqrtf(rv[ci] + eps);
    sc[ci] = gamma[ci] * is;
    sh[ci] = beta[ci] - gamma[ci] * is * rm[ci];
}

// Per-channel normalisation of one element.  Train (run_train, nn.rs:336-342):
// g * ((x - mean) * invstd) + b.  Eval (run_eval): sc * x + sh, with sc / sh
// passed in the mean / invstd slots.
template <bool EVAL>
struct BnCoef {
    const float *a, *b, *g, *be;
    __device__ __forceinline__ float apply(int ci, float x) const {
        if constexpr (EVAL) {
            return a[ci] * x + b[ci];
        } else {
            const float h = (x - a[ci]) * b[ci];
            return g[ci] * h + be[ci];
        }
    }
};

// out = [relu]( bn(x) [+ skip | + bn'(skip)] ), elementwise over [n][C][hw].
// SKIP 0: none; 1: add the tensor `skip` (identity shortcut); 2: add
// bn'(skip) (projection shortcut).  The residual add and the ReLU follow
// add_relu_ (nn.rs:446-450): max(y + s, 0).
template <bool EVAL, bool RELU, int SKIP>
__global__ __launch_bounds__(EW_THREADS) void bn_apply_kernel(
    const float *x, BnCoef<EVAL> bn, const float *skip, BnCoef<EVAL> sbn, float *out,
    size_t total4, FastDiv fd_hw4, FastDiv fd_c) {
    for (size_t q = (size_t)blockIdx.x * EW_THREADS + threadIdx.x; q < total4;
         q += (size_t)gridDim.x * EW_THREADS) {
        const uint32_t plane = div_by((uint32_t)q, fd_hw4);
        const int ci = (int)(plane - div_by(plane, fd_c) * fd_c.d);
        float4 v = reinterpret_cast<const float4 *>(x)[q];
        float r[4] = {bn.apply(ci, v.x), bn.apply(ci, v.y), bn.apply(ci, v.z), bn.apply(ci, v.w)};
        if constexpr (SKIP != 0) {
            const float4 s = reinterpret_cast<const float4 *>(skip)[q];
            float t[4] = {s.x, s.y, s.z, s.w};
            if constexpr (SKIP == 2) {
#pragma unroll
                for (int j = 0; j < 4; j++) t[j] = sbn.apply(ci, t[j]);
            }
#pragma unroll
            for (int j = 0; j < 4; j++) r[j] = r[j] + t[j];
        }
        if constexpr (RELU) {
#pragma unroll
            for (int j = 0; j < 4; j++) r[j] = r[j] > 0.0f ? r[j] : 0.0f;
        }
        reinterpret_cast<float4 *>(out)[q] = make_float4(r[0], r[1], r[2], r[3]);
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

// dgamma / dbeta of BatchNorm2d::backward: g.g += dgamma, b.g += dbeta
// (nn.rs:423-424); the values are kept in dgdb[2*C] for the dx pass.
__global__ void bn_bwd_final_kernel(const double *__restrict__ part, int P, int C, float *dgamma,
                                    float *dbeta, float *dgdb) {
    const int ci = blockIdx.x * blockDim.x + threadIdx.x;
    if (ci >= C) return;
    double a = 0.0, b = 0.0;
    for (int p = 0; p < P; p++) {
        a += part[((size_t)ci * P + p) * 2 + 0];
        b += part[((size_t)ci * P + p) * 2 + 1];
    }
    const float dg = (float)a, db = (float)b;
    dgdb[ci] = dg;
    dgdb[C + ci] = db;
    if (dgamma) dgamma[ci] += dg;
    if (dbeta) dbeta[ci] += db;
}

// dx = s * (m*dy - dbeta - xhat*dgamma), s = gamma*invstd/m (nn.rs:406-421).
template <bool MASK>
__global__ __launch_bounds__(EW_THREADS) void bn_bwd_apply_kernel(
    const float *__restrict__ d, const float *__restrict__ mask, const float *__restrict__ x,
    const float *__restrict__ mean, const float *__restrict__ invstd,
    const float *__restrict__ gamma, const float *__restrict__ dgdb, float m, float *dx,
    size_t total4, FastDiv fd_hw4, FastDiv fd_c) {
    const int C = (int)fd_c.d;
    for (size_t q = (size_t)blockIdx.x * EW_THREADS + threadIdx.x; q < total4;
         q += (size_t)gridDim.x * EW_THREADS) {
        const uint32_t plane = div_by((uint32_t)q, fd_hw4);
        const int ci = (int)(plane - div_by(plane, fd_c) * fd_c.d);
        const float mu = mean[ci], is = invstd[ci];
        const float s = gamma[ci] * is / m;
        const float dg = dgdb[ci], db = dgdb[C + ci];
        const float4 dv = reinterpret_cast<const float4 *>(d)[q];
        const float4 xv = reinterpret_cast<const float4 *>(x)[q];
        float4 mv = make_float4(1.f, 1.f, 1.f, 1.f);
        if constexpr (MASK) mv = reinterpret_cast<const float4 *>(mask)[q];
        const float dd[4] = {dv.x, dv.y, dv.z, dv.w}, xx[4] = {xv.x, xv.y, xv.z, xv.w};
        const float mm[4] = {mv.x, mv.y, mv.z, mv.w};
        float r[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float g = (MASK && mm[j] <= 0.0f) ? 0.0f : dd[j];
            const float xh = (xx[j] - mu) * is;
            r[j] = s * (m * g - db - xh * dg);
        }
        reinterpret_cast<float4 *>(dx)[q] = make_float4(r[0], r[1], r[2], r[3]);
    }
}

// Scalar-tail variants of the elementwise kernels (hw not a multiple of 4).
template <bool MASK>
__global__ void bn_bwd_apply_scalar_kernel(const float *__restrict__ d,
                                           const float *__restrict__ mask,
                                           const float *__restrict__ x,
                                           const float *__restrict__ mean,
                                           const float *__restrict__ invstd,
                                           const float *__restrict__ gamma,
                                           const float *__restrict__ dgdb, float m, float *dx,
                                           size_t total, int hw, int C) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const int ci = (int)((i / hw) % C);
        const float mu = mean[ci], is = invstd[ci];
        const float s = gamma[ci] * is / m;
        const float g = masked<MASK>(d[i], mask, i);
        const float xh = (x[i] - mu) * is;
        dx[i] = s * (m * g - dgdb[C + ci] - xh * dgdb[ci]);
    }
}

template <bool EVAL, bool RELU, int SKIP>
__global__ void bn_apply_scalar_kernel(const float *x, BnCoef<EVAL> bn, const float *skip,
                                       BnCoef<EVAL> sbn, float *out, size_t total, int hw, int C) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const int ci = (int)((i / hw) % C);
        float r = bn.apply(ci, x[i]);
        if constexpr (SKIP == 1) r = r + skip[i];
        if constexpr (SKIP == 2) r = r + sbn.apply(ci, skip[i]);
        if constexpr (RELU) r = r > 0.0f ? r : 0.0f;
        out[i] = r;
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

// gap_forward (nn.rs:455-463): one thread per plane, the f32 sum in pixel
// order (bit-identical to the reference), divided by hw.
__global__ void gap_fwd_kernel(const float *__restrict__ x, int hw, size_t nc, int vec, float *y) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nc) return;
    const float *p = x + i * hw;
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
    y[i] = s / (float)hw;
}

// gap_backward (nn.rs:465-473).
__global__ void gap_bwd_kernel(const float *__restrict__ dy, int hw, size_t total, float *dx) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x)
        dx[i] = dy[i / hw] / (float)hw;
}

// nn.rs Linear::forward (nn.rs:500-517): y[i][o] = b[o] + w[o][0]*x[i][0] +
// ... in j order, one thread per output (bit-identical to the reference).
__global__ void fc_fwd_kernel(const float *__restrict__ x, const float *__restrict__ w,
                              const float *__restrict__ b, int rows, int fin, int fout, float *y) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= rows * fout) return;
    const int i = t / fout, o = t - i * fout;
    const float *wr = w + (size_t)o * fin, *xr = x + (size_t)i * fin;
    float s = b[o];
    for (int j = 0; j < fin; j++) s = s + wr[j] * xr[j];
    y[t] = s;
}

// Linear::backward_w (nn.rs:521-537): w.g[o][j] += dy[i][o]*x[i][j] in row
// order, zero gradients skipped; thread (o, j).  Threads with j == fin do the
// bias: b.g[o] += dy[i][o].
__global__ void fc_bwd_w_kernel(const float *__restrict__ dy, const float *__restrict__ x, int rows,
                                int fin, int fout, float *dw, float *db) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    const int fin1 = fin + 1;
    if (t >= fout * fin1) return;
    const int o = t / fin1, j = t - o * fin1;
    if (j == fin) {
        float acc = db[o];
        for (int i = 0; i < rows; i++) {
            const float g = dy[(size_t)i * fout + o];
            if (g != 0.0f) acc = acc + g;
        }
        db[o] = acc;
        return;
    }
    float acc = dw[(size_t)o * fin + j];
    for (int i = 0; i < rows; i++) {
        const float g = dy[(size_t)i * fout + o];
        if (g != 0.0f) acc = acc + g * x[(size_t)i * fin + j];
    }
    dw[(size_t)o * fin + j] = acc;
}

// Linear::backward_x (nn.rs:539-556): dx[i][j] = sum over o (in order, zero
// gradients skipped) of dy[i][o]*w[o][j], from 0.
__global__ void fc_bwd_x_kernel(const float *__restrict__ dy, const float *__restrict__ w, int rows,
                                int fin, int fout, float *dx) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= rows * fin) return;
    const int i = t / fin, j = t - i * fin;
    float acc = 0.0f;
    for (int o = 0; o < fout; o++) {
        const float g = dy[(size_t)i * fout + o];
        if (g != 0.0f) acc = acc + g * w[(size_t)o * fin + j];
    }
    dx[t] = acc;
}

// softmax_ce (nn.rs:566-637).  Thread r handles rows r, r + blockDim, ...;
// thread 0 then adds the row losses and hits in row order.  `smooth` comes
// from device memory when `scal` is set (scal[3]), else from the argument.
__global__ void softmax_ce_kernel(const float *__restrict__ logits,
                                  const uint32_t *__restrict__ labels, int rows, int nclass,
                                  float smooth_arg, const float *scal, float *dl, float *loss_out,
                                  uint32_t *correct_out) {
    extern __shared__ float row_loss[];  // [rows] losses, then [rows] hits
    const float smooth = scal ? scal[3] : smooth_arg;
    const float inv = 1.0f / (float)rows;
    for (int r = threadIdx.x; r < rows; r += blockDim.x) {
        const float *z = logits + (size_t)r * nclass;
        float *d = dl + (size_t)r * nclass;
        const uint32_t yl = labels[r];
        if (yl >= (uint32_t)nclass) {  // the reference panics on such a label
            for (int j = 0; j < nclass; j++) d[j] = NAN;
            row_loss[r] = NAN;
            row_loss[rows + r] = 0.0f;
            continue;
        }
        const int y = (int)yl;
        float mx = -INFINITY;
        int arg = 0;
        for (int j = 0; j < nclass; j++)
            if (z[j] > mx) {
                mx = z[j];
                arg = j;
            }
        float sum = 0.0f;
        for (int j = 0; j < nclass; j++) {
            const float e = expf(z[j] - mx);
            d[j] = e;
            sum = sum + e;
        }
        const float lse = mx + logf(sum);
        const float on = 1.0f - smooth, off = smooth / (float)nclass;
        float l = on * (lse - z[y]);
        if (smooth > 0.0f) {
            float s = 0.0f;
            for (int j = 0; j < nclass; j++) s = s + (lse - z[j]);
            l = l + off * s;
        }
        for (int j = 0; j < nclass; j++) {
            const float t = j == y ? on + off : off;
            d[j] = (d[j] / sum - t) * inv;
        }
        row_loss[r] = l;
        row_loss[rows + r] = arg == y ? 1.0f : 0.0f;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float l = 0.0f;
        uint32_t ok = 0;
        for (int r = 0; r < rows; r++) {
            l = l + row_loss[r];
            ok += row_loss[rows + r] != 0.0f;
        }
        if (loss_out) loss_out[0] = l * inv;
        if (correct_out) correct_out[0] = ok;
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

int rnn_bn_stats_launch(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *x, double *part,
                        float *mean, float *invstd, float *rm, float *rv, float mom, float eps) {
    ChanSplit s = chan_split(n, c);
    bn_stats_part_kernel<<<dim3((unsigned)c, (unsigned)s.P), RED_THREADS, 0, ctx->stream>>>(
        x, (int)n, (int)c, (int)hw, aligned16(x), s.G, divider(hw / 4, (size_t)s.G * (hw / 4)),
        part);
    RNN_LAUNCHED(ctx);
    bn_stats_final_kernel<<<(unsigned)rnn_div_up(c, 64), 64, 0, ctx->stream>>>(
        part, s.P, (int)c, (float)(n * hw), mom, eps, mean, invstd, rm, rv);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

template <bool EVAL, bool RELU, int SKIP>
static int bn_apply_t(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *x,
                      BnCoef<EVAL> bn, const float *skip, BnCoef<EVAL> sbn, float *out) {
    const size_t total = n * c * hw;
    if (total == 0) return RNN_OK;
    if ((hw & 3) == 0 && total / 4 < (1ull << 31) && aligned16(x) && aligned16(out) &&
        (SKIP == 0 || aligned16(skip))) {
        const size_t t4 = total / 4;
        bn_apply_kernel<EVAL, RELU, SKIP><<<ew_grid(ctx, t4), EW_THREADS, 0, ctx->stream>>>(
            x, bn, skip, sbn, out, t4, divider(hw / 4, t4), divider(c, n * c));
    } else {
        bn_apply_scalar_kernel<EVAL, RELU, SKIP><<<ew_grid(ctx, total), EW_THREADS, 0,
                                                   ctx->stream>>>(x, bn, skip, sbn, out, total,
                                                                  (int)hw, (int)c);
    }
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_bn_apply_launch(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *x,
                        const RnnBnCoef &bn, int relu, int skip_mode, const float *skip,
                        const RnnBnCoef &sbn, float *out) {
    if (bn.eval) {
        BnCoef<true> a{bn.mean, bn.invstd, bn.gamma, bn.beta};
        BnCoef<true> b{sbn.mean, sbn.invstd, sbn.gamma, sbn.beta};
        if (skip_mode == 0)
            return relu ? bn_apply_t<true, true, 0>(ctx, n, c, hw, x, a, skip, b, out)
                        : bn_apply_t<true, false, 0>(ctx, n, c, hw, x, a, skip, b, out);
        if (skip_mode == 1) return bn_apply_t<true, true, 1>(ctx, n, c, hw, x, a, skip, b, out);
        return bn_apply_t<true, true, 2>(ctx, n, c, hw, x, a, skip, b, out);
    }
    BnCoef<false> a{bn.mean, bn.invstd, bn.gamma, bn.beta};
    BnCoef<false> b{sbn.mean, sbn.invstd, sbn.gamma, sbn.beta};
    if (skip_mode == 0)
        return relu ? bn_apply_t<false, true, 0>(ctx, n, c, hw, x, a, skip, b, out)
                    : bn_apply_t<false, false, 0>(ctx, n, c, hw, x, a, skip, b, out);
    if (skip_mode == 1) return bn_apply_t<false, true, 1>(ctx, n, c, hw, x, a, skip, b, out);
    return bn_apply_t<false, true, 2>(ctx, n, c, hw, x, a, skip, b, out);
}

int rnn_bn_eval_prep_launch(rnn_ctx *ctx, size_t c, const float *gamma, const float *beta,
                            const float *rm, const float *rv, float eps, float *sc, float *sh) {
    bn_eval_prep_kernel<<<(unsigned)rnn_div_up(c, 64), 64, 0, ctx->stream>>>(gamma, beta, rm, rv,
                                                                             eps, (int)c, sc, sh);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_bn_backward_launch(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *dy,
                           const float *mask, const float *x, const float *mean,
                           const float *invstd, const float *gamma, float *dx, float *dgamma,
                           float *dbeta, double *part, float *dgdb) {
    ChanSplit s = chan_split(n, c);
    const FastDiv fd_hw4 = divider(hw / 4, (size_t)s.G * (hw / 4));
    const dim3 grid((unsigned)c, (unsigned)s.P);
    const int vec = aligned16(dy) && aligned16(x) && (!mask || aligned16(mask));
    if (mask)
        bn_bwd_part_kernel<true><<<grid, RED_THREADS, 0, ctx->stream>>>(
            dy, mask, x, mean, invstd, (int)n, (int)c, (int)hw, vec, s.G, fd_hw4, part);
    else
        bn_bwd_part_kernel<false><<<grid, RED_THREADS, 0, ctx->stream>>>(
            dy, mask, x, mean, invstd, (int)n, (int)c, (int)hw, vec, s.G, fd_hw4, part);
    RNN_LAUNCHED(ctx);
    bn_bwd_final_kernel<<<(unsigned)rnn_div_up(c, 64), 64, 0, ctx->stream>>>(part, s.P, (int)c,
                                                                             dgamma, dbeta, dgdb);
    RNN_LAUNCHED(ctx);
    const size_t total = n * c * hw;
    const float m = (float)(n * hw);
    if ((hw & 3) == 0 && total / 4 < (1ull << 31) && aligned16(dy) && aligned16(x) &&
        aligned16(dx) && (!mask || aligned16(mask))) {
        const size_t t4 = total / 4;
        const FastDiv fq = divider(hw / 4, t4), fc = divider(c, n * c);
        if (mask)
            bn_bwd_apply_kernel<true><<<ew_grid(ctx, t4), EW_THREADS, 0, ctx->stream>>>(
                dy, mask, x, mean, invstd, gamma, dgdb, m, dx, t4, fq, fc);
        else
            bn_bwd_apply_kernel<false><<<ew_grid(ctx, t4), EW_THREADS, 0, ctx->stream>>>(
                dy, mask, x, mean, invstd, gamma, dgdb, m, dx, t4, fq, fc);
    } else {
        if (mask)
            bn_bwd_apply_scalar_kernel<true><<<ew_grid(ctx, total), EW_THREADS, 0, ctx->stream>>>(
                dy, mask, x, mean, invstd, gamma, dgdb, m, dx, total, (int)hw, (int)c);
        else
            bn_bwd_apply_scalar_kernel<false><<<ew_grid(ctx, total), EW_THREADS, 0,
                                                ctx->stream>>>(dy, mask, x, mean, invstd, gamma,
                                                               dgdb, m, dx, total, (int)hw, (int)c);
    }
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

int rnn_fc_forward_launch(rnn_ctx *ctx, size_t rows, size_t fin, size_t fout, const float *x,
                          const float *w, const float *b, float *y) {
    const size_t t = rows * fout;
    if (t == 0) return RNN_OK;
    fc_fwd_kernel<<<(unsigned)rnn_div_up(t, 128), 128, 0, ctx->stream>>>(x, w, b, (int)rows,
                                                                        (int)fin, (int)fout, y);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_fc_backward_launch(rnn_ctx *ctx, size_t rows, size_t fin, size_t fout, const float *dy,
                           const float *x, const float *w, float *dw, float *db, float *dx) {
    const size_t tw = fout * (fin + 1), tx = rows * fin;
    if (tw) {
        fc_bwd_w_kernel<<<(unsigned)rnn_div_up(tw, 128), 128, 0, ctx->stream>>>(
            dy, x, (int)rows, (int)fin, (int)fout, dw, db);
        RNN_LAUNCHED(ctx);
    }
    if (tx && dx) {
        fc_bwd_x_kernel<<<(unsigned)rnn_div_up(tx, 128), 128, 0, ctx->stream>>>(
            dy, w, (int)rows, (int)fin, (int)fout, dx);
        RNN_LAUNCHED(ctx);
    }
    return RNN_OK;
}

int rnn_softmax_ce_launch(rnn_ctx *ctx, size_t rows, size_t nclass, const float *logits,
                          const uint32_t *labels, float smooth, const float *scal, float *dl,
                          float *loss, uint32_t *correct) {
    if (rows == 0) return RNN_OK;
    const unsigned threads = (unsigned)std::min<size_t>(rnn_round_up(rows, 64), 1024);
    softmax_ce_kernel<<<1, threads, 2 * rows * sizeof(float), ctx->stream>>>(
        logits, labels, (int)rows, (int)nclass, smooth, scal, dl, loss, correct);
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

int rnn_set_scalars_launch(rnn_ctx *ctx, float *scal, float a, float b, float c, float d) {
    set_scalars_kernel<<<1, 1, 0, ctx->stream>>>(scal, a, b, c, d);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

// ---------------------------------------------------------------- C ABI

namespace {

// Carves BN scratch (partials + dgamma/dbeta values) out of the workspace.
struct BnScratch {
    double *part;
    float *f;
};

bool bn_scratch(rnn_ctx *ctx, size_t n, size_t c, BnScratch &s) {
    WsCarve cv;
    size_t o1 = cv.take(rnn_bn_scratch_doubles(n, c) * sizeof(double));
    size_t o2 = cv.take(2 * c * sizeof(float));
    char *ws = (char *)rnn_workspace(ctx, cv.off);
    if (!ws) return false;
    s.part = (double *)(ws + o1);
    s.f = (float *)(ws + o2);
    return true;
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
    BnScratch s;
    if (!bn_scratch(ctx, n, c, s)) return RNN_E_NOMEM;
    int st = rnn_bn_stats_launch(ctx, n, c, hw, x, s.part, mean, invstd, running_mean,
                                 running_var, momentum, eps);
    if (st) return st;
    RnnBnCoef bn{false, mean, invstd, gamma, beta};
    return rnn_bn_apply_launch(ctx, n, c, hw, x, bn, relu, 0, nullptr, bn, y);
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
    BnScratch s;
    if (!bn_scratch(ctx, n, c, s)) return RNN_E_NOMEM;
    float *sc = s.f, *sh = s.f + c;
    int st = rnn_bn_eval_prep_launch(ctx, c, gamma, beta, running_mean, running_var, eps, sc, sh);
    if (st) return st;
    RnnBnCoef bn{true, sc, sh, nullptr, nullptr};
    return rnn_bn_apply_launch(ctx, n, c, hw, x, bn, relu, 0, nullptr, bn, y);
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
    BnScratch s;
    if (!bn_scratch(ctx, n, c, s)) return RNN_E_NOMEM;
    return rnn_bn_backward_launch(ctx, n, c, hw, dy, relu_out, x, mean, invstd, gamma, dx, dgamma,
                                  dbeta, s.part, s.f);
}

int rnn_relu_back(rnn_ctx *ctx, size_t len, float *d, const float *y) {
    if (!ctx) return RNN_E_NULL;
    if (len == 0) return RNN_OK;
    if (!d || !y) return rnn_fail(ctx, RNN_E_NULL, "relu_back: null pointer");
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    relu_back_kernel<<<ew_grid(ctx, len), EW_THREADS, 0, ctx->stream>>>(d, y, len);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_add(rnn_ctx *ctx, size_t len, float *a, const float *b) {
    if (!ctx) return RNN_E_NULL;
    if (len == 0) return RNN_OK;
    if (!a || !b) return rnn_fail(ctx, RNN_E_NULL, "add: null pointer");
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    return rnn_add_launch(ctx, len, a, b, nullptr);
}

int rnn_add_relu(rnn_ctx *ctx, size_t len, float *a, const float *b) {
    if (!ctx) return RNN_E_NULL;
    if (len == 0) return RNN_OK;
    if (!a || !b) return rnn_fail(ctx, RNN_E_NULL, "add_relu: null pointer");
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
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
