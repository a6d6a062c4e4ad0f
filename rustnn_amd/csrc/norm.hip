// norm.rs on the device: LayerNorm, LayerScale, the SwiGLU gate, the
// channel-last depthwise 3x3 convolution and SeqPool, over token tensors
// [n, t, c] (tok.rs: rows = n*t, channel fastest).
//
// Reference: LayerNorm (norm.rs:17-143) with f64 row statistics; LayerScale
// (norm.rs:147-217); SwiGlu's gate (norm.rs:221-294; its two projections are
// Linear calls through the GEMM core); DwConv3 (norm.rs:296-457); SeqPool
// (norm.rs:459-586).  Each reference layer runs rayon over rows or images.
//
// HBM-bound work: every kernel reads its inputs once and writes its outputs
// once, except the channel reductions (dgamma / dbeta, dlambda, the depthwise
// dW / db, dp), which read their operands once more in a column pass:
// column partials per row block in f64, then one fixed-order pass over the
// blocks (deterministic, like every reduction in this library).
//
// Operation order.  Where the reference's per-element arithmetic is a fixed
// sequence (the depthwise taps, SeqPool's sums over tokens, the LayerNorm
// output, SwiGLU's products) the kernels keep it, with contraction off, so
// those outputs round as the reference does; row sums that the reference
// makes sequentially in f32 (LayerNorm backward's m1 / m2) are summed in f64
// here.  exp is the device's expf.
#include "rnn_internal.h"

#include <algorithm>
#include <cmath>

#pragma clang fp contract(off)

namespace {

constexpr int NT = 256;  // threads per block


// ------------------------------------------------------------ LayerNorm
// One wave per row: f64 sums of x and x^2 (norm.rs:56-62), mu, var =
// max(s2/c - mu^2, 0) as f32, invstd = 1 / sqrt(var + eps) in f32; then
// xhat = (x - mu) invstd and y = g xhat + b (norm.rs:63-69).  NV > 0: the
// row's c <= 64 NV values stay in registers (lane l holds columns l, l + 64,
// ...; every load issued before the sums), the wave sums take a DPP tree;
// NV = 0: any c, strided loops.
template <int NV>
__global__ __launch_bounds__(NT) void ln_fwd_kernel(size_t rows, int c, const float *__restrict__ x,
                                                    const float *__restrict__ g,
                                                    const float *__restrict__ b, float eps,
                                                    float *__restrict__ y, float *__restrict__ xhat,
                                                    float *__restrict__ invstd) {
    const int lane = threadIdx.x & 63;
    const size_t r = (size_t)blockIdx.x * (NT / 64) + wave_index();
    if (r >= rows) return;
    const float *xr = x + r * c;
    float *yr = y + r * c;
    float *hr = xhat ? xhat + r * c : nullptr;
    const double m = (double)c;
    if constexpr (NV > 0) {
        float xv[NV], gv[NV], bv[NV];
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int j = min(lane + 64 * i, c - 1);
            xv[i] = xr[j];
            gv[i] = g[j];
            bv[i] = b[j];
        }
        double s = 0.0, s2 = 0.0;
#pragma unroll
        for (int i = 0; i < NV; i++)
            if (lane + 64 * i < c) {
                const double v = xv[i];
                s += v;
                s2 += v * v;
            }
        s = rnn_wave_sum_d(s);
        s2 = rnn_wave_sum_d(s2);
        const double mu = s / m;
        const float var = (float)fmax(s2 / m - mu * mu, 0.0);
        const float inv = 1.0f / sqrtf(var + eps);
        const float muf = (float)mu;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int j = lane + 64 * i;
            if (j >= c) break;
            const float h = (xv[i] - muf) * inv;
            if (hr) hr[j] = h;
            yr[j] = gv[i] * h + bv[i];
        }
        if (invstd && lane == 0) invstd[r] = inv;
    } else {
        double s = 0.0, s2 = 0.0;
        for (int j = lane; j < c; j += 64) {
            const double v = xr[j];
            s += v;
            s2 += v * v;
        }
        s = rnn_wave_sum_d(s);
        s2 = rnn_wave_sum_d(s2);
        const double mu = s / m;
        const float var = (float)fmax(s2 / m - mu * mu, 0.0);
        const float inv = 1.0f / sqrtf(var + eps);
        const float muf = (float)mu;
        for (int j = lane; j < c; j += 64) {
            const float h = (xr[j] - muf) * inv;
            if (hr) hr[j] = h;
            yr[j] = g[j] * h + b[j];
        }
        if (invstd && lane == 0) invstd[r] = inv;
    }
}

// dx per row (norm.rs:121-135): d = dy g; m1 = sum d, m2 = sum d xhat;
// dx = invstd (d - m1/c - xhat m2/c).  NV as in the forward.
template <int NV>
__global__ __launch_bounds__(NT) void ln_bwd_kernel(size_t rows, int c, const float *__restrict__ dy,
                                                    const float *__restrict__ xhat,
                                                    const float *__restrict__ invstd,
                                                    const float *__restrict__ g,
                                                    float *__restrict__ dx) {
    const int lane = threadIdx.x & 63;
    const size_t r = (size_t)blockIdx.x * (NT / 64) + wave_index();
    if (r >= rows) return;
    const float *dr = dy + r * c, *hr = xhat + r * c;
    const float inv = 1.0f / (float)c;
    const float is = invstd[r];
    float *xr = dx + r * c;
    if constexpr (NV > 0) {
        float dv[NV], hv[NV], gv[NV];
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int j = min(lane + 64 * i, c - 1);
            dv[i] = dr[j];
            hv[i] = hr[j];
            gv[i] = g[j];
        }
        double m1 = 0.0, m2 = 0.0;
#pragma unroll
        for (int i = 0; i < NV; i++)
            if (lane + 64 * i < c) {
                const float d = dv[i] * gv[i];
                m1 += d;
                m2 += (double)(d * hv[i]);
            }
        const float s1 = (float)rnn_wave_sum_d(m1), s2 = (float)rnn_wave_sum_d(m2);
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int j = lane + 64 * i;
            if (j >= c) break;
            const float d = dv[i] * gv[i];
            xr[j] = is * (d - s1 * inv - hv[i] * s2 * inv);
        }
    } else {
        double m1 = 0.0, m2 = 0.0;
        for (int j = lane; j < c; j += 64) {
            const float d = dr[j] * g[j];
            m1 += d;
            m2 += (double)(d * hr[j]);
        }
        const float s1 = (float)rnn_wave_sum_d(m1), s2 = (float)rnn_wave_sum_d(m2);
        for (int j = lane; j < c; j += 64) {
            const float d = dr[j] * g[j];
            xr[j] = is * (d - s1 * inv - hr[j] * s2 * inv);
        }
    }
}

// ------------------------------------------- row kernels with column sums
// A block of 4 waves takes RB_ROWS consecutive rows, wave w the rows w,
// w + 4, ... of them in order, each lane columns lane + 64 i (i < NV).  Its
// lanes keep f64 column sums over their rows, and the block stores the four
// waves' sums, added in wave order, as partial row blockIdx.x of
// part[nblk][NO * c] -- the stage-1 layout of colsum_red_kernel.
constexpr int RB_ROWS = 16;

template <int NV, int NO>
__device__ __forceinline__ void store_col_partials(const double (&p)[NO][NV], int c,
                                                   double *__restrict__ part) {
    __shared__ double red[NO][NT / 64][NV * 64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int o = 0; o < NO; o++)
#pragma unroll
        for (int i = 0; i < NV; i++) red[o][w][lane + 64 * i] = p[o][i];
    __syncthreads();
    double *row = part + (size_t)blockIdx.x * NO * c;
    for (int j = threadIdx.x; j < c; j += NT)
#pragma unroll
        for (int o = 0; o < NO; o++) {
            double t = red[o][0][j];
#pragma unroll
            for (int q = 1; q < NT / 64; q++) t += red[o][q][j];
            row[(size_t)o * c + j] = t;
        }
}

// LayerNorm backward (ln_bwd_kernel per row) with dgamma's and dbeta's
// partials: sums of (double)(dy xhat) and of dy.  A wave loads all its rows'
// dy and xhat before the first row's reductions.  With `add` set, dx = the
// row's gradient + add (Block::backward's add_ after the norm; add may be
// dx: each element is read, then written, by one lane).
// With LS, the DropPath + LayerScale backward that reads dx next
// (ls_bwd_cs_kernel's values): t = dx m, lsdx = t l, dl's partials
// (double)(t lsx) into lspart.
struct LnLs {
    const float *x, *l, *mask;
    size_t rpi;
    float *dx;
    double *part;
};

template <int NV, bool LS = false>
__global__ __launch_bounds__(NT) void ln_bwd_cs_kernel(size_t rows, int c,
                                                       const float *dy,
                                                       const float *__restrict__ xhat,
                                                       const float *__restrict__ invstd,
                                                       const float *__restrict__ g,
                                                       const float *add, float *dx,
                                                       double *__restrict__ part, LnLs ls = {}) {
    constexpr int RPW = RB_ROWS / 4;
    const int lane = threadIdx.x & 63, w = wave_index();
    const size_t r0 = (size_t)blockIdx.x * RB_ROWS + w;
    const int nr = r0 < rows ? (int)min((size_t)RPW, (rows - r0 + 3) / 4) : 0;
    const float inv = 1.0f / (float)c;
    double p[2][NV], pl[1][NV];
    float gv[NV], dv[RPW][NV], hv[RPW][NV], ad[RPW][NV];
    float lv[NV], lx[RPW][NV], lm[RPW];
    if constexpr (LS) {
#pragma unroll
        for (int k = 0; k < RPW; k++) {
            const size_t r = min(r0 + 4 * (size_t)k, rows - 1);
            lm[k] = ls.mask ? ls.mask[r / ls.rpi] : 1.0f;
        }
    }
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int j = min(lane + 64 * i, c - 1);
        gv[i] = g[j];
        p[0][i] = p[1][i] = 0.0;
        if constexpr (LS) {
            lv[i] = ls.l[j];
            pl[0][i] = 0.0;
        }
#pragma unroll
        for (int k = 0; k < RPW; k++) {
            const size_t r = min(r0 + 4 * (size_t)k, rows - 1);
            dv[k][i] = dy[r * c + j];
            hv[k][i] = xhat[r * c + j];
            // add's values too, before any store (add may be dx)
            ad[k][i] = add ? add[r * c + j] : 0.0f;
            if constexpr (LS) lx[k][i] = ls.x[r * c + j];
        }
    }
#pragma unroll
    for (int k = 0; k < RPW; k++) {
        if (k >= nr) break;
        const size_t r = r0 + 4 * (size_t)k;
        double m1 = 0.0, m2 = 0.0;
#pragma unroll
        for (int i = 0; i < NV; i++)
            if (lane + 64 * i < c) {
                const float d = dv[k][i] * gv[i];
                m1 += d;
                m2 += (double)(d * hv[k][i]);
                p[0][i] += (double)(dv[k][i] * hv[k][i]);
                p[1][i] += dv[k][i];
            }
        const float s1 = (float)rnn_wave_sum_d(m1), s2 = (float)rnn_wave_sum_d(m2);
        const float is = invstd[r];
        float *xr = dx + r * c;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int j = lane + 64 * i;
            if (j >= c) break;
            const float d = dv[k][i] * gv[i];
            const float v = is * (d - s1 * inv - hv[k][i] * s2 * inv);
            const float o = add ? v + ad[k][i] : v;
            xr[j] = o;
            if constexpr (LS) {
                const float t = ls.mask ? o * lm[k] : o;
                pl[0][i] += (double)(t * lx[k][i]);
                ls.dx[r * c + j] = t * lv[i];
            }
        }
    }
    store_col_partials<NV, 2>(p, c, part);
    if constexpr (LS) {
        __syncthreads();  // the partials' LDS staging is reused
        store_col_partials<NV, 1>(pl, c, ls.part);
    }
}

// DropPath + LayerScale backward (scale_cols_masked_kernel per row) with
// dl's partials: sums of (double)((dy m) x), m = mask[r / rpi] (1 without a
// mask).  dx may be dy: each element is read, then written, by one lane.
template <int NV>
__global__ __launch_bounds__(NT) void ls_bwd_cs_kernel(size_t rows, int c, const float *dy,
                                                       const float *__restrict__ x,
                                                       const float *__restrict__ l,
                                                       const float *__restrict__ mask, size_t rpi,
                                                       float *dx, double *__restrict__ part) {
    constexpr int RPW = RB_ROWS / 4;
    const int lane = threadIdx.x & 63, w = wave_index();
    const size_t r0 = (size_t)blockIdx.x * RB_ROWS + w;
    const int nr = r0 < rows ? (int)min((size_t)RPW, (rows - r0 + 3) / 4) : 0;
    double p[1][NV];
    float lv[NV], dv[RPW][NV], xv[RPW][NV], m[RPW];
#pragma unroll
    for (int k = 0; k < RPW; k++) {
        const size_t r = min(r0 + 4 * (size_t)k, rows - 1);
        m[k] = mask ? mask[r / rpi] : 1.0f;
    }
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int j = min(lane + 64 * i, c - 1);
        lv[i] = l[j];
        p[0][i] = 0.0;
#pragma unroll
        for (int k = 0; k < RPW; k++) {
            const size_t r = min(r0 + 4 * (size_t)k, rows - 1);
            dv[k][i] = dy[r * c + j];
            xv[k][i] = x[r * c + j];
        }
    }
#pragma unroll
    for (int k = 0; k < RPW; k++) {
        if (k >= nr) break;
        float *xr = dx + (r0 + 4 * (size_t)k) * c;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int j = lane + 64 * i;
            if (j >= c) break;
            const float a = mask ? dv[k][i] * m[k] : dv[k][i];
            p[0][i] += (double)(a * xv[k][i]);
            xr[j] = a * lv[i];
        }
    }
    store_col_partials<NV, 1>(p, c, part);
}

// The first residual's branch gradients of a Block backward in one pass
// over dy, each value as ls_bwd_cs_kernel computes it: t1 = dy m1,
// da = t1 l1, p1 += (double)(t1 a); then the gamma gate, ddw = da gamma,
// pg += (double)(da dwo); with CROSS, t2 = dy m2, dc = t2 lm,
// pm += (double)(t2 cm).  m1 / m2 = mask[r / rpi] when the mask is set.
// part1 / partg / partm: [nblk][c] each, in store_col_partials' order.
struct BranchBwd {
    const float *dy, *a, *l1, *m1, *dwo, *gamma, *cm, *lm, *m2;
    float *da, *ddw, *dc;
    double *part1, *partg, *partm;
    size_t rows, rpi;
    int c;
};

template <int NV, bool CROSS>
__global__ __launch_bounds__(NT) void branch_bwd_cs_kernel(BranchBwd g) {
    constexpr int RPW = RB_ROWS / 4;
    const int lane = threadIdx.x & 63, w = wave_index(), c = g.c;
    const size_t rows = g.rows;
    const size_t r0 = (size_t)blockIdx.x * RB_ROWS + w;
    const int nr = r0 < rows ? (int)min((size_t)RPW, (rows - r0 + 3) / 4) : 0;
    double p1[1][NV], pg[1][NV], pm[1][NV];
    float l1v[NV], gv[NV], lmv[NV], m1[RPW], m2[RPW];
    float dv[RPW][NV], av[RPW][NV], wv[RPW][NV], cv[RPW][NV];
#pragma unroll
    for (int k = 0; k < RPW; k++) {
        const size_t r = min(r0 + 4 * (size_t)k, rows - 1);
        m1[k] = g.m1 ? g.m1[r / g.rpi] : 1.0f;
        m2[k] = CROSS && g.m2 ? g.m2[r / g.rpi] : 1.0f;
    }
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int j = min(lane + 64 * i, c - 1);
        l1v[i] = g.l1[j];
        gv[i] = g.gamma[j];
        lmv[i] = CROSS ? g.lm[j] : 0.0f;
        p1[0][i] = 0.0;
        pg[0][i] = 0.0;
        pm[0][i] = 0.0;
#pragma unroll
        for (int k = 0; k < RPW; k++) {
            const size_t e = min(r0 + 4 * (size_t)k, rows - 1) * c + j;
            dv[k][i] = g.dy[e];
            av[k][i] = g.a[e];
            wv[k][i] = g.dwo[e];
            cv[k][i] = CROSS ? g.cm[e] : 0.0f;
        }
    }
#pragma unroll
    for (int k = 0; k < RPW; k++) {
        if (k >= nr) break;
        const size_t rb = (r0 + 4 * (size_t)k) * c;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int j = lane + 64 * i;
            if (j >= c) break;
            const float t1 = g.m1 ? dv[k][i] * m1[k] : dv[k][i];
            p1[0][i] += (double)(t1 * av[k][i]);
            const float da = t1 * l1v[i];
            g.da[rb + j] = da;
            pg[0][i] += (double)(da * wv[k][i]);
            g.ddw[rb + j] = da * gv[i];
            if (CROSS) {
                const float t2 = g.m2 ? dv[k][i] * m2[k] : dv[k][i];
                pm[0][i] += (double)(t2 * cv[k][i]);
                g.dc[rb + j] = t2 * lmv[i];
            }
        }
    }
    store_col_partials<NV, 1>(p1, c, g.part1);
    __syncthreads();  // the partials' LDS staging is reused
    store_col_partials<NV, 1>(pg, c, g.partg);
    if (CROSS) {
        __syncthreads();
        store_col_partials<NV, 1>(pm, c, g.partm);
    }
}

// Column sums in two fixed-order stages.  Stage 1, block (x, y): columns
// [64x, 64x + 64), rows [CS_ROWS y, CS_ROWS (y + 1)); wave g sums the rows
// g, g + 4, ... of the block in order (8 loads ahead of their adds), and the
// four wave sums are added in wave order.  part: [block row][nout * c], the
// sums of a*b (b set) first, then those of a.  With rs set, a's row r is
// first multiplied by rs[r / rpi].
constexpr int CS_ROWS = 64;
constexpr int CS_RED_COLS = 16;  // columns per stage-2 block (16 groups each)

__global__ __launch_bounds__(NT) void colsum_part_kernel(size_t rows, int c,
                                                         const float *__restrict__ a,
                                                         const float *__restrict__ b, int want_a,
                                                         const float *__restrict__ rs, size_t rpi,
                                                         double *__restrict__ part) {
    __shared__ double red[2][NT / 64][64];
    const int lane = threadIdx.x & 63, g = threadIdx.x >> 6;
    const int j = blockIdx.x * 64 + lane, jc = min(j, c - 1);
    const size_t r0 = (size_t)blockIdx.y * CS_ROWS, r1 = min(rows, r0 + CS_ROWS);
    double sab = 0.0, sa = 0.0;
    for (size_t r = r0 + g; r < r1; r += 8 * (NT / 64)) {
        float av[8], bv[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const size_t rr = min(r + (size_t)(NT / 64) * u, r1 - 1);
            av[u] = a[rr * c + jc];
            if (rs) av[u] = av[u] * rs[rr / rpi];
            bv[u] = b ? b[rr * c + jc] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            if (r + (size_t)(NT / 64) * u >= r1) break;
            if (b) sab += (double)(av[u] * bv[u]);
            sa += av[u];
        }
    }
    red[0][g][lane] = sab;
    red[1][g][lane] = sa;
    __syncthreads();
    if (g != 0 || j >= c) return;
    double tab = red[0][0][lane], ta = red[1][0][lane];
#pragma unroll
    for (int w = 1; w < NT / 64; w++) {
        tab += red[0][w][lane];
        ta += red[1][w][lane];
    }
    const size_t len = (size_t)((b ? 1 : 0) + (want_a ? 1 : 0)) * c;
    double *row = part + (size_t)blockIdx.y * len;
    if (b) row[j] = tab;
    if (want_a) row[(b ? c : 0) + j] = ta;
}

// Stage 2: column j of part ([nblk][len]) summed over the block rows in
// order -- 16 consecutive groups of rows, each summed in order, then the 16
// group sums in order -- and added into out0[j] (j < split) or
// out1[j - split].
__global__ __launch_bounds__(NT) void colsum_red_kernel(int nblk, size_t len, size_t split,
                                                        const double *__restrict__ part,
                                                        float *__restrict__ out0,
                                                        float *__restrict__ out1) {
    static_assert(NT == 256 && CS_RED_COLS == 16, "rnn_colsum_red_block's shape");
    rnn_colsum_red_block(nblk, len, split, part, out0, out1, blockIdx.x);
}

// ------------------------------------------------------------ LayerScale
// y = x l (norm.rs:168-180); backward dx = dy l (norm.rs:205-211).  y may be x.
__global__ void scale_cols_kernel(size_t len, int c, const float *x, const float *__restrict__ l,
                                  float *y) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < len;
         i += (size_t)gridDim.x * blockDim.x)
        y[i] = x[i] * l[i % c];
}

// dx = (dy m) l with m = mask[i / per] (DropPath::backward, vit.rs:61-73,
// then LayerScale's, norm.rs:205-211).
__global__ void scale_cols_masked_kernel(size_t len, int c, size_t per, const float *dy,
                                         const float *__restrict__ l,
                                         const float *__restrict__ mask, float *dx) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < len;
         i += (size_t)gridDim.x * blockDim.x)
        dx[i] = (dy[i] * mask[i / per]) * l[i % c];
}

// y = x + (a l) m with m = mask[r / rpi] (1 without a mask): a residual
// branch of Block::forward, x + DropPath(LayerScale(a)) (vit.rs:155-176 over
// norm.rs:168-180, vit.rs:40-57 and add_, nn.rs:441-443), in one pass with
// the reference's rounding order.  y may be x.  VEC: c % 4 == 0, 16-byte
// aligned rows.
template <bool VEC>
__global__ void residual_add_scaled_kernel(size_t len, int c, size_t per, const float *x,
                                           const float *__restrict__ a,
                                           const float *__restrict__ l,
                                           const float *__restrict__ mask, float *y) {
    const size_t step = (size_t)gridDim.x * blockDim.x;
    if constexpr (VEC) {
        for (size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4; i < len; i += 4 * step) {
            const float4 xv = *reinterpret_cast<const float4 *>(x + i);
            const float4 av = *reinterpret_cast<const float4 *>(a + i);
            const float4 lv = *reinterpret_cast<const float4 *>(l + i % c);
            float4 t = make_float4(av.x * lv.x, av.y * lv.y, av.z * lv.z, av.w * lv.w);
            if (mask) {
                const float m = mask[i / per];
                t = make_float4(t.x * m, t.y * m, t.z * m, t.w * m);
            }
            *reinterpret_cast<float4 *>(y + i) =
                make_float4(xv.x + t.x, xv.y + t.y, xv.z + t.z, xv.w + t.w);
        }
    } else {
        for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < len; i += step) {
            float t = a[i] * l[i % c];
            if (mask) t = t * mask[i / per];
            y[i] = x[i] + t;
        }
    }
}

// y = a + b (y may be b).
__global__ void sum2_kernel(size_t len, const float *__restrict__ a, const float *b, float *y) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < len;
         i += (size_t)gridDim.x * blockDim.x)
        y[i] = a[i] + b[i];
}

// ------------------------------------------------------------ SwiGLU gate
__device__ __forceinline__ float sigmoid(float z) { return 1.0f / (1.0f + expf(-z)); }

// u = a sigmoid(a) b with a = ab[r][j], b = ab[r][h + j] (norm.rs:255-262).
__global__ void swiglu_fwd_kernel(size_t rows, int h, const float *__restrict__ ab,
                                  float *__restrict__ u) {
    const size_t len = rows * h;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < len;
         i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / h, j = i - r * h;
        const float a = ab[r * 2 * h + j];
        u[i] = a * sigmoid(a) * ab[r * 2 * h + h + j];
    }
}

// dab[r][j] = du b s (1 + a (1 - s)), dab[r][h + j] = du a s (norm.rs:276-287).
__global__ void swiglu_bwd_kernel(size_t rows, int h, const float *__restrict__ du,
                                  const float *__restrict__ ab, float *__restrict__ dab) {
    const size_t len = rows * h;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < len;
         i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / h, j = i - r * h;
        const float a = ab[r * 2 * h + j], b = ab[r * 2 * h + h + j];
        const float s = sigmoid(a);
        const float sa = a * s;
        const float d = du[i];
        dab[r * 2 * h + j] = d * b * s * (1.0f + a * (1.0f - s));
        dab[r * 2 * h + h + j] = d * sa;
    }
}

// The same two passes four columns a thread (h % 4 == 0, 16-byte aligned
// tensors): each element computed as above, with 16-byte loads and stores
// and one division per four elements.
__global__ void swiglu_fwd4_kernel(size_t rows, int hq, const float4 *__restrict__ ab,
                                   float4 *__restrict__ u) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * hq) return;
    const size_t r = i / hq, j = i - r * hq;
    const float4 a = ab[r * 2 * hq + j], b = ab[r * 2 * hq + hq + j];
    float4 o;
    o.x = a.x * sigmoid(a.x) * b.x;
    o.y = a.y * sigmoid(a.y) * b.y;
    o.z = a.z * sigmoid(a.z) * b.z;
    o.w = a.w * sigmoid(a.w) * b.w;
    u[i] = o;
}

__device__ __forceinline__ void swiglu_bwd1(float d, float a, float b, float &da, float &db) {
    const float s = sigmoid(a);
    const float sa = a * s;
    da = d * b * s * (1.0f + a * (1.0f - s));
    db = d * sa;
}

__global__ void swiglu_bwd4_kernel(size_t rows, int hq, const float4 *__restrict__ du,
                                   const float4 *__restrict__ ab, float4 *__restrict__ dab) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * hq) return;
    const size_t r = i / hq, j = i - r * hq;
    const float4 a = ab[r * 2 * hq + j], b = ab[r * 2 * hq + hq + j], d = du[i];
    float4 ga, gb;
    swiglu_bwd1(d.x, a.x, b.x, ga.x, gb.x);
    swiglu_bwd1(d.y, a.y, b.y, ga.y, gb.y);
    swiglu_bwd1(d.z, a.z, b.z, ga.z, gb.z);
    swiglu_bwd1(d.w, a.w, b.w, ga.w, gb.w);
    dab[r * 2 * hq + j] = ga;
    dab[r * 2 * hq + hq + j] = gb;
}

// ------------------------------------------------------------ DwConv3
// y = b, then the in-bounds taps in (ky, kx) order: y += w[tap] x[src]
// (norm.rs:344-369).  One thread per output element.
__global__ void dw3_fwd_kernel(size_t n, int th, int tw, int c, const float *__restrict__ x,
                               const float *__restrict__ w, const float *__restrict__ b,
                               float *__restrict__ y) {
    const size_t len = n * th * tw * c;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < len;
         i += (size_t)gridDim.x * blockDim.x) {
        const int ch = (int)(i % c);
        const size_t pos = i / c;
        const int ox = (int)(pos % tw), oy = (int)((pos / tw) % th);
        const size_t img = pos / ((size_t)th * tw);
        const float *xi = x + img * th * tw * c;
        float acc = b[ch];
        for (int ky = 0; ky < 3; ky++) {
            const int sy = oy + ky - 1;
            if (sy < 0 || sy >= th) continue;
            for (int kx = 0; kx < 3; kx++) {
                const int sx = ox + kx - 1;
                if (sx < 0 || sx >= tw) continue;
                acc += w[(ky * 3 + kx) * c + ch] * xi[((size_t)sy * tw + sx) * c + ch];
            }
        }
        y[i] = acc;
    }
}

// dx[src] = sum over the outputs that read src of w[tap] dy[out], in the
// order the reference's scatter visits them (output raster order, i.e. taps
// 8, 7, ..., 0; norm.rs:423-450).
__global__ void dw3_bwd_x_kernel(size_t n, int th, int tw, int c, const float *__restrict__ dy,
                                 const float *__restrict__ w, float *__restrict__ dx, int acc_dx) {
    const size_t len = n * th * tw * c;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < len;
         i += (size_t)gridDim.x * blockDim.x) {
        const int ch = (int)(i % c);
        const size_t pos = i / c;
        const int sx = (int)(pos % tw), sy = (int)((pos / tw) % th);
        const size_t img = pos / ((size_t)th * tw);
        const float *di = dy + img * th * tw * c;
        float acc = 0.0f;
        for (int ky = 2; ky >= 0; ky--) {
            const int oy = sy - ky + 1;
            if (oy < 0 || oy >= th) continue;
            for (int kx = 2; kx >= 0; kx--) {
                const int ox = sx - kx + 1;
                if (ox < 0 || ox >= tw) continue;
                acc += w[(ky * 3 + kx) * c + ch] * di[((size_t)oy * tw + ox) * c + ch];
            }
        }
        dx[i] = acc_dx ? dx[i] + acc : acc;
    }
}

// The same two passes for c % 4 == 0 with 16-byte rows: block (x, oy, img)
// covers output row oy of image img, one thread per (column, channel quad),
// 32-bit indexing.  The nine taps' inputs load unconditionally from clamped
// addresses before the adds, which skip the taps outside the image in the
// reference's order, so the sums are the ones above bit for bit.
__device__ __forceinline__ float4 fma4(float4 acc, float4 w, float4 x) {
    return make_float4(acc.x + w.x * x.x, acc.y + w.y * x.y, acc.z + w.z * x.z, acc.w + w.w * x.w);
}

// Output (oy, ox) of image img, channel quad cq (x: that image's first quad).
__device__ __forceinline__ float4 dw3_out4(int th, int tw, int c4, int oy, int ox, int cq,
                                           const float4 *__restrict__ xi,
                                           const float4 *__restrict__ w,
                                           const float4 *__restrict__ b) {
#pragma clang fp contract(off)
    float4 xv[9], wv[9];
#pragma unroll
    for (int t = 0; t < 9; t++) {
        const int sy = min(max(oy + t / 3 - 1, 0), th - 1), sx = min(max(ox + t % 3 - 1, 0), tw - 1);
        xv[t] = xi[(sy * tw + sx) * c4 + cq];
        wv[t] = w[t * c4 + cq];
    }
    float4 acc = b[cq];
#pragma unroll
    for (int t = 0; t < 9; t++) {
        const int sy = oy + t / 3 - 1, sx = ox + t % 3 - 1;
        if (sy >= 0 && sy < th && sx >= 0 && sx < tw) acc = fma4(acc, wv[t], xv[t]);
    }
    return acc;
}

__global__ __launch_bounds__(NT) void dw3_fwd4_kernel(int th, int tw, int c4,
                                                      const float4 *__restrict__ x,
                                                      const float4 *__restrict__ w,
                                                      const float4 *__restrict__ b,
                                                      float4 *__restrict__ y) {
    const int e = blockIdx.x * NT + threadIdx.x;
    if (e >= tw * c4) return;
    const int oy = blockIdx.y, img = blockIdx.z;
    const int ox = e / c4, cq = e - ox * c4;
    const size_t o = ((size_t)img * th * tw + (size_t)oy * tw + ox) * c4 + cq;
    y[o] = dw3_out4(th, tw, c4, oy, ox, cq, x + (size_t)img * th * tw * c4, w, b);
}

// Block::forward's first branch after the attention (vit.rs:150-160) in one
// pass: d = DwConv3(h) (as dw3_fwd4_kernel), a += gamma d (axpy_cols_kernel's
// rounding), y = x + (a l) m with m = mask[img] (1 without a mask;
// residual_add_scaled_kernel's rounding).  a is updated in place; y may be x.
__global__ __launch_bounds__(NT) void dw3_branch4_kernel(
    int th, int tw, int c4, const float4 *__restrict__ h, const float4 *__restrict__ w,
    const float4 *__restrict__ b, float4 *__restrict__ d, float4 *a,
    const float4 *__restrict__ gamma, const float4 *x, const float4 *__restrict__ l,
    const float *__restrict__ mask, float4 *y) {
#pragma clang fp contract(off)
    const int e = blockIdx.x * NT + threadIdx.x;
    if (e >= tw * c4) return;
    const int oy = blockIdx.y, img = blockIdx.z;
    const int ox = e / c4, cq = e - ox * c4;
    const size_t o = ((size_t)img * th * tw + (size_t)oy * tw + ox) * c4 + cq;
    const float4 dv = dw3_out4(th, tw, c4, oy, ox, cq, h + (size_t)img * th * tw * c4, w, b);
    d[o] = dv;
    const float4 g = gamma[cq];
    float4 av = a[o];
    av = make_float4(av.x + g.x * dv.x, av.y + g.y * dv.y, av.z + g.z * dv.z, av.w + g.w * dv.w);
    a[o] = av;
    const float4 lv = l[cq];
    float4 t = make_float4(av.x * lv.x, av.y * lv.y, av.z * lv.z, av.w * lv.w);
    if (mask) {
        const float m = mask[img];
        t = make_float4(t.x * m, t.y * m, t.z * m, t.w * m);
    }
    const float4 xv = x[o];
    y[o] = make_float4(xv.x + t.x, xv.y + t.y, xv.z + t.z, xv.w + t.w);
}

// ACC: dx += the input gradient (old value first, rnn_add's order).
template <bool ACC>
__global__ __launch_bounds__(NT) void dw3_bwd_x4_kernel(int th, int tw, int c4,
                                                        const float4 *__restrict__ dy,
                                                        const float4 *__restrict__ w,
                                                        float4 *__restrict__ dx) {
#pragma clang fp contract(off)
    const int e = blockIdx.x * NT + threadIdx.x;
    if (e >= tw * c4) return;
    const int sy = blockIdx.y, img = blockIdx.z;
    const int sx = e / c4, cq = e - sx * c4;
    const float4 *di = dy + (size_t)img * th * tw * c4;
    // tap t = 8 - u, u = 0..8: output (sy - ky + 1, sx - kx + 1)
    float4 dv[9], wv[9];
#pragma unroll
    for (int u = 0; u < 9; u++) {
        const int t = 8 - u;
        const int oy = min(max(sy - t / 3 + 1, 0), th - 1), ox = min(max(sx - t % 3 + 1, 0), tw - 1);
        dv[u] = di[(oy * tw + ox) * c4 + cq];
        wv[u] = w[t * c4 + cq];
    }
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < 9; u++) {
        const int t = 8 - u;
        const int oy = sy - t / 3 + 1, ox = sx - t % 3 + 1;
        if (oy >= 0 && oy < th && ox >= 0 && ox < tw) acc = fma4(acc, wv[u], dv[u]);
    }
    float4 *o = dx + ((size_t)img * th * tw + (size_t)sy * tw + sx) * c4 + cq;
    if constexpr (ACC) {
        const float4 v = *o;
        acc = make_float4(v.x + acc.x, v.y + acc.y, v.z + acc.z, v.w + acc.w);
    }
    *o = acc;
}

// dW [9][c] and db [c] partials over output rows [rb*RB, rb*RB + RB) of
// image im (block y = im * nrb + rb): thread = channel, f64 sums in (output
// row, output column, tap) order (norm.rs:377-418).  The 3x3 input window
// slides along the row in registers (3 loads per output position); taps
// outside the image hold 0 and add nothing.  part: [n * nrb][10][c] (taps
// 0-8, then db).
__global__ __launch_bounds__(NT) void dw3_bwd_w_kernel(int th, int tw, int c, int RB, int nrb,
                                                       const float *__restrict__ dy,
                                                       const float *__restrict__ x,
                                                       double *__restrict__ part) {
    const int ch = blockIdx.x * NT + threadIdx.x;
    if (ch >= c) return;
    const size_t im = blockIdx.y / nrb;
    const int rb = blockIdx.y % nrb, oy0 = rb * RB, oy1 = min(th, oy0 + RB);
    double aw[9], ab = 0.0;
#pragma unroll
    for (int k = 0; k < 9; k++) aw[k] = 0.0;
    const size_t img = (size_t)th * tw * c;
    const float *di = dy + im * img + ch, *xi = x + im * img + ch;
    auto xat = [&](int sy, int sx) {
        return (sy >= 0 && sy < th && sx >= 0 && sx < tw) ? xi[((size_t)sy * tw + sx) * c] : 0.0f;
    };
    for (int oy = oy0; oy < oy1; oy++) {
        float win[3][3];
#pragma unroll
        for (int ky = 0; ky < 3; ky++) {
            win[ky][0] = 0.0f;
            win[ky][1] = xat(oy + ky - 1, 0);
            win[ky][2] = xat(oy + ky - 1, 1);
        }
        for (int ox = 0; ox < tw; ox++) {
            const float d = di[((size_t)oy * tw + ox) * c];
            float nxt[3];
#pragma unroll
            for (int ky = 0; ky < 3; ky++) nxt[ky] = xat(oy + ky - 1, ox + 2);
            ab += d;
#pragma unroll
            for (int ky = 0; ky < 3; ky++)
#pragma unroll
                for (int kx = 0; kx < 3; kx++) aw[ky * 3 + kx] += (double)(d * win[ky][kx]);
#pragma unroll
            for (int ky = 0; ky < 3; ky++) {
                win[ky][0] = win[ky][1];
                win[ky][1] = win[ky][2];
                win[ky][2] = nxt[ky];
            }
        }
    }
    double *pb = part + (size_t)blockIdx.y * 10 * c;
#pragma unroll
    for (int k = 0; k < 9; k++) pb[(size_t)k * c + ch] = aw[k];
    pb[(size_t)9 * c + ch] = ab;
}

// ------------------------------------------------------------ SeqPool
// One block per image (norm.rs:488-519): s_j = sum_k x[j][k] p[k] in k order;
// w = softmax(s) with a sequential sum and a multiply by 1/sum;
// z[k] = sum_j w_j x[j][k] in j order.  s, w live in LDS (t <= SP_MAXT).
// XL: the image's x [t][c] is first staged into LDS by the whole block
// (coalesced float4 loads) with a row stride of c + 1 floats, so the
// per-token chains (thread j reading row j) fall in distinct banks and the
// per-channel chains read consecutive words; the sums keep the orders above.
// The softmax's max and exps run one token a thread (the max is exact in any
// order), its sum in token order on one thread.
constexpr int SP_MAXT = 1024;
constexpr size_t SP_XL_BYTES = 96 * 1024;  // x staged in LDS up to this size

__host__ __device__ constexpr size_t seqpool_xl_bytes(size_t t, size_t c) {
    return t * (c + 1) * sizeof(float);
}

// The image's x into xl ([t][c + 1], dynamic LDS), 16-byte global loads when
// c % 4 == 0, eight of them in flight a thread before their LDS stores.
__device__ __forceinline__ void seqpool_stage(const float *__restrict__ xi, int t, int c,
                                              float *xl) {
    const int tot = t * c;
    if ((c & 3) == 0 && ((uintptr_t)xi & 15) == 0) {
        constexpr int U = 8;
        for (int e0 = threadIdx.x * 4; e0 < tot; e0 += NT * 4 * U) {
            float4 v[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int e = e0 + u * NT * 4;
                if (e < tot) v[u] = *reinterpret_cast<const float4 *>(xi + e);
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int e = e0 + u * NT * 4;
                if (e >= tot) break;
                const int j = e / c, k = e - j * c;  // the four stay in row j
                float *d = xl + j * (c + 1) + k;
                d[0] = v[u].x;
                d[1] = v[u].y;
                d[2] = v[u].z;
                d[3] = v[u].w;
            }
        }
    } else {
        for (int e = threadIdx.x; e < tot; e += NT) {
            const int j = e / c;
            xl[e + j] = xi[e];
        }
    }
    __syncthreads();
}

// w[0..t) = softmax(w) in place (the forward's order: max, exps, the sum in
// token order, a multiply by 1/sum).  All NT threads call it.
__device__ __forceinline__ void seqpool_softmax(float *w, int t) {
    __shared__ float red[NT / 64];
    __shared__ float inv_s;
    float mx = -INFINITY;
    for (int j = threadIdx.x; j < t; j += NT) mx = w[j] > mx ? w[j] : mx;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float v = __shfl_xor(mx, o);
        mx = v > mx ? v : mx;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int q = 1; q < NT / 64; q++) mx = red[q] > mx ? red[q] : mx;
    for (int j = threadIdx.x; j < t; j += NT) w[j] = expf(w[j] - mx);
    __syncthreads();
    if (threadIdx.x == 0) {
        float sum = 0.0f;
        for (int j = 0; j < t; j++) sum += w[j];
        inv_s = 1.0f / sum;
    }
    __syncthreads();
    const float inv = inv_s;
    for (int j = threadIdx.x; j < t; j += NT) w[j] *= inv;
    __syncthreads();
}

template <bool XL>
__global__ __launch_bounds__(NT) void seqpool_fwd_kernel(int t, int c, const float *__restrict__ x,
                                                         const float *__restrict__ p,
                                                         float *__restrict__ z,
                                                         float *__restrict__ wout) {
    __shared__ float w[SP_MAXT];
    extern __shared__ float xl[];
    const size_t im = blockIdx.x;
    const float *xi = x + im * t * c;
    size_t ld = c;
    if constexpr (XL) {
        seqpool_stage(xi, t, c, xl);
        xi = xl;
        ld = c + 1;
    }
    for (int j = threadIdx.x; j < t; j += NT) {
        float s = 0.0f;
        for (int k = 0; k < c; k++) s += xi[(size_t)j * ld + k] * p[k];
        w[j] = s;
    }
    __syncthreads();
    seqpool_softmax(w, t);
    for (int j = threadIdx.x; j < t; j += NT) wout[im * t + j] = w[j];
    for (int k = threadIdx.x; k < c; k += NT) {
        float acc = 0.0f;
        for (int j = 0; j < t; j++) acc += w[j] * xi[(size_t)j * ld + k];
        z[im * c + k] = acc;
    }
}

// Backward, one block per image (norm.rs:530-572): dw_j = sum_k dz_k x[j][k];
// dot = sum_j dw_j w_j; ds_j = w_j (dw_j - dot); dx[j][k] = w_j dz_k +
// ds_j p_k; the image's share of dp, sum_j ds_j x[j][k], into part[image][k].
template <bool XL>
__global__ __launch_bounds__(NT) void seqpool_bwd_kernel(int t, int c, const float *__restrict__ dz,
                                                         const float *__restrict__ wsave,
                                                         const float *__restrict__ x,
                                                         const float *__restrict__ p,
                                                         float *__restrict__ dx,
                                                         float *__restrict__ part) {
    __shared__ float dw[SP_MAXT], wi[SP_MAXT];
    __shared__ float dot_s;
    extern __shared__ float xl[];
    const size_t im = blockIdx.x;
    const float *xi = x + im * t * c, *dzi = dz + im * c;
    // the image's softmax weights in LDS (read by every channel's loop)
    for (int j = threadIdx.x; j < t; j += NT) wi[j] = wsave[im * t + j];
    size_t ld = c;
    if constexpr (XL) {
        seqpool_stage(xi, t, c, xl);  // (its barrier also covers wi)
        xi = xl;
        ld = c + 1;
    } else {
        __syncthreads();
    }
    for (int j = threadIdx.x; j < t; j += NT) {
        float s = 0.0f;
        for (int k = 0; k < c; k++) s += dzi[k] * xi[(size_t)j * ld + k];
        dw[j] = s;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float dot = 0.0f;
        for (int j = 0; j < t; j++) dot += dw[j] * wi[j];
        dot_s = dot;
    }
    __syncthreads();
    const float dot = dot_s;
    for (int j = threadIdx.x; j < t; j += NT) dw[j] = wi[j] * (dw[j] - dot);  // ds_j
    __syncthreads();
    float *dxi = dx + im * t * c;
    for (int k = threadIdx.x; k < c; k += NT) {
        const float dzk = dzi[k], pk = p[k];
        float adp = 0.0f;
        for (int j = 0; j < t; j++) {
            const float ds = dw[j];
            dxi[(size_t)j * c + k] = wi[j] * dzk + ds * pk;
            adp += ds * xi[(size_t)j * ld + k];
        }
        part[im * c + k] = adp;
    }
}

// out[k] += sum over images of part[image][k] (image order, f64; 64 loads
// ahead of their adds).  Launched with 64-thread blocks, so a few hundred
// channels spread over several CUs.
constexpr int RS_NT = 64;
__global__ __launch_bounds__(RS_NT) void rowsum_add_kernel(size_t n, int c,
                                                           const float *__restrict__ part,
                                                           float *__restrict__ out) {
    const int k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= c) return;
    double s = 0.0;
    for (size_t i0 = 0; i0 < n; i0 += 64) {
        float v[64];
#pragma unroll
        for (int u = 0; u < 64; u++) v[u] = part[min(i0 + u, n - 1) * c + k];
#pragma unroll
        for (int u = 0; u < 64; u++)
            if (i0 + u < n) s += v[u];
    }
    out[k] += (float)s;
}

unsigned ew_grid(size_t len) {
    return (unsigned)std::max<size_t>(1, std::min<size_t>(rnn_div_up(len, NT), 16384));
}

}  // namespace

// The float4 depthwise passes: channels a multiple of 4, 16-byte aligned
// tensors, images within the grid's z range.
static bool dw3_vec(const void *a, const void *w, const void *out, size_t c, size_t n) {
    return c % 4 == 0 && n <= 65535 && ((uintptr_t)a & 15) == 0 && ((uintptr_t)w & 15) == 0 &&
           ((uintptr_t)out & 15) == 0;
}

// Partial rows of a column reduction: in the workspace, or -- when the
// context defers parameter-gradient reductions -- in its arena until the
// flush.
static double *col_part(rnn_ctx *ctx, size_t bytes) {
    return (double *)(ctx->defer ? rnn_defer_take(ctx, bytes) : rnn_workspace(ctx, bytes));
}

// Stage 2 of a column reduction (colsum_red_kernel), launched now or queued.
static int col_reduce(rnn_ctx *ctx, size_t nblk, size_t len, size_t split, const double *part,
                      float *out0, float *out1) {
    if (ctx->defer) {
        RnnDeferSeg sg{};
        sg.part = part;
        sg.out0 = out0;
        sg.out1 = out1;
        sg.len = (long long)len;
        sg.split = (long long)split;
        sg.nrow = (int)nblk;
        sg.kind = RNN_DEFER_COLS;
        rnn_defer_push(ctx, sg);
        return RNN_OK;
    }
    colsum_red_kernel<<<(unsigned)rnn_div_up(len, (size_t)CS_RED_COLS), NT, 0, ctx->stream>>>(
        (int)nblk, len, split, part, out0, out1);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

// Column sums of a*b (b set) and of a over rows, added into outab / outa.
// Many short chains: blocks of CS_ROWS rows x 64 columns (colsum_part_kernel),
// then the blocks' partials in order, 16 groups per column (colsum_red_kernel).
int rnn_colsum_f64(rnn_ctx *ctx, size_t rows, int c, const float *a, const float *b,
                   float *outab, float *outa, const float *rs, size_t rpi) {
    if (rows == 0 || c == 0) return RNN_OK;
    const size_t nblk = rnn_div_up(rows, (size_t)CS_ROWS);
    if (nblk > 65535) return rnn_fail(ctx, RNN_E_UNSUPPORTED, "column sums: too many rows");
    const int nout = (b ? 1 : 0) + (outa ? 1 : 0);
    const size_t len = (size_t)nout * c;
    double *part = col_part(ctx, nblk * len * sizeof(double));
    if (!part) return RNN_E_NOMEM;
    colsum_part_kernel<<<dim3((unsigned)rnn_div_up((size_t)c, (size_t)64), (unsigned)nblk), NT, 0,
                         ctx->stream>>>(rows, c, a, b, outa != nullptr, rs, rpi, part);
    RNN_LAUNCHED(ctx);
    return col_reduce(ctx, nblk, len, (size_t)(b ? c : len), part, b ? outab : outa,
                      b ? outa : nullptr);
}

namespace {

int colsum_add(rnn_ctx *ctx, size_t rows, int c, const float *a, const float *b, float *outab,
               float *outa) {
    return rnn_colsum_f64(ctx, rows, c, a, b, outab, outa, nullptr, 1);
}

bool dims_ok(size_t rows, size_t c) { return c <= (1u << 20) && rows <= ((size_t)1 << 40); }

}  // namespace

extern "C" {

int rnn_ln_forward(rnn_ctx *ctx, size_t rows, size_t c, const float *x, const float *g,
                   const float *b, float eps, float *y, float *xhat, float *invstd) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (rows == 0 || c == 0) return RNN_OK;
    if (!x || !g || !b || !y) return rnn_fail(ctx, RNN_E_NULL, "ln_forward: null operand");
    if ((xhat == nullptr) != (invstd == nullptr))
        return rnn_fail(ctx, RNN_E_INVALID, "ln_forward: xhat and invstd go together");
    if (!dims_ok(rows, c)) return rnn_fail(ctx, RNN_E_INVALID, "ln_forward: %zu x %zu", rows, c);
    const unsigned grid = (unsigned)rnn_div_up(rows, NT / 64);
    const int nv = (int)rnn_div_up(c, (size_t)64);
    auto fwd = [&](auto kern) {
        kern<<<grid, NT, 0, ctx->stream>>>(rows, (int)c, x, g, b, eps, y, xhat, invstd);
    };
    switch (nv) {
        case 1: fwd(ln_fwd_kernel<1>); break;
        case 2: fwd(ln_fwd_kernel<2>); break;
        case 3: fwd(ln_fwd_kernel<3>); break;
        case 4: fwd(ln_fwd_kernel<4>); break;
        case 5: fwd(ln_fwd_kernel<5>); break;
        case 6: fwd(ln_fwd_kernel<6>); break;
        case 7: fwd(ln_fwd_kernel<7>); break;
        case 8: fwd(ln_fwd_kernel<8>); break;
        case 16: fwd(ln_fwd_kernel<16>); break;
        default: fwd(ln_fwd_kernel<0>); break;
    }
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

// rnn_ln_backward, then dx += add where add is set (in one pass up to 512
// columns).
static int ln_backward(rnn_ctx *ctx, size_t rows, size_t c, const float *dy, const float *xhat,
                       const float *invstd, const float *g, const float *add, float *dx,
                       float *dg, float *db, const LnLs *ls = nullptr, float *dl = nullptr) {
    if (rows == 0 || c == 0) return RNN_OK;
    if (!dy || !xhat || !invstd || !g || !dx || !dg || !db)
        return rnn_fail(ctx, RNN_E_NULL, "ln_backward: null operand");
    if (!dims_ok(rows, c)) return rnn_fail(ctx, RNN_E_INVALID, "ln_backward: %zu x %zu", rows, c);
    // dgamma += sum dy xhat, dbeta += sum dy (norm.rs:94-119)
    const int nv = (int)rnn_div_up(c, (size_t)64);
    if (nv <= 8) {
        // one pass: dx and the column sums' partials, then their reduction
        const size_t nblk = rnn_div_up(rows, (size_t)RB_ROWS);
        if (nblk > 0x7fffffff) return rnn_fail(ctx, RNN_E_UNSUPPORTED, "ln_backward: rows");
        const size_t pb = nblk * 2 * c * sizeof(double);
        double *part = col_part(ctx, pb + (ls ? nblk * c * sizeof(double) : 0));
        if (!part) return RNN_E_NOMEM;
        LnLs l{};
        if (ls) {
            l = *ls;
            l.part = part + nblk * 2 * c;
        }
        auto cs = [&](auto kern) {
            kern<<<(unsigned)nblk, NT, 0, ctx->stream>>>(rows, (int)c, dy, xhat, invstd, g, add,
                                                         dx, part, l);
        };
#define RNN_LN_CS(NV)                                                                     \
    ls ? cs(ln_bwd_cs_kernel<NV, true>) : cs(ln_bwd_cs_kernel<NV, false>);               \
    break;
        switch (nv) {
            case 1: RNN_LN_CS(1)
            case 2: RNN_LN_CS(2)
            case 3: RNN_LN_CS(3)
            case 4: RNN_LN_CS(4)
            case 5: RNN_LN_CS(5)
            case 6: RNN_LN_CS(6)
            case 7: RNN_LN_CS(7)
            default: RNN_LN_CS(8)
        }
#undef RNN_LN_CS
        RNN_LAUNCHED(ctx);
        int rc = col_reduce(ctx, nblk, 2 * c, c, part, dg, db);
        if (!rc && ls) rc = col_reduce(ctx, nblk, c, c, l.part, dl, nullptr);
        return rc;
    }
    if (ls) {
        // the two passes
        int rc = ln_backward(ctx, rows, c, dy, xhat, invstd, g, add, dx, dg, db);
        if (!rc) rc = rnn_drop_layerscale_backward(ctx, rows, c, dx, ls->x, ls->l, ls->mask,
                                                   ls->rpi, ls->dx, dl);
        return rc;
    }
    int rc = colsum_add(ctx, rows, (int)c, dy, xhat, dg, db);
    if (rc) return rc;
    // with `add`, the row gradients go to a workspace copy first, then
    // dx = that + add (add may be dx or dy)
    float *out = dx;
    if (add) {
        out = (float *)rnn_workspace(ctx, rows * c * sizeof(float));
        if (!out) return RNN_E_NOMEM;
    }
    const unsigned grid = (unsigned)rnn_div_up(rows, NT / 64);
    auto bwd = [&](auto kern) {
        kern<<<grid, NT, 0, ctx->stream>>>(rows, (int)c, dy, xhat, invstd, g, out);
    };
    switch (nv) {
        case 1: bwd(ln_bwd_kernel<1>); break;
        case 2: bwd(ln_bwd_kernel<2>); break;
        case 3: bwd(ln_bwd_kernel<3>); break;
        case 4: bwd(ln_bwd_kernel<4>); break;
        case 5: bwd(ln_bwd_kernel<5>); break;
        case 6: bwd(ln_bwd_kernel<6>); break;
        case 7: bwd(ln_bwd_kernel<7>); break;
        case 8: bwd(ln_bwd_kernel<8>); break;
        case 16: bwd(ln_bwd_kernel<16>); break;
        default: bwd(ln_bwd_kernel<0>); break;
    }
    RNN_LAUNCHED(ctx);
    if (add) {
        sum2_kernel<<<ew_grid(rows * c), NT, 0, ctx->stream>>>(rows * c, out, add, dx);
        RNN_LAUNCHED(ctx);
    }
    return RNN_OK;
}

int rnn_ln_backward_add_ls(rnn_ctx *ctx, size_t rows, size_t c, const float *dy,
                           const float *xhat, const float *invstd, const float *g,
                           const float *add, float *dx, float *dg, float *db, const float *lsx,
                           const float *l, const float *mask, size_t rpi, float *lsdx,
                           float *dl) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (rows == 0 || c == 0) return RNN_OK;
    if (!add || !lsx || !l || !lsdx || !dl)
        return rnn_fail(ctx, RNN_E_NULL, "ln_backward_add_ls: null operand");
    if (mask && (rpi == 0 || rows % rpi))
        return rnn_fail(ctx, RNN_E_INVALID, "ln_backward_add_ls: %zu rows per image of %zu", rpi,
                        rows);
    if (lsdx == dx || lsdx == dy || lsdx == add || lsdx == lsx)
        return rnn_fail(ctx, RNN_E_INVALID, "ln_backward_add_ls: lsdx overlaps an operand");
    const LnLs ls{lsx, l, mask, mask ? rpi : 1, lsdx, nullptr};
    return ln_backward(ctx, rows, c, dy, xhat, invstd, g, add, dx, dg, db, &ls, dl);
}

int rnn_ln_backward(rnn_ctx *ctx, size_t rows, size_t c, const float *dy, const float *xhat,
                    const float *invstd, const float *g, float *dx, float *dg, float *db) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    return ln_backward(ctx, rows, c, dy, xhat, invstd, g, nullptr, dx, dg, db);
}

int rnn_ln_backward_add(rnn_ctx *ctx, size_t rows, size_t c, const float *dy, const float *xhat,
                        const float *invstd, const float *g, const float *add, float *dx,
                        float *dg, float *db) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (!add) return rnn_fail(ctx, RNN_E_NULL, "ln_backward_add: add is null");
    return ln_backward(ctx, rows, c, dy, xhat, invstd, g, add, dx, dg, db);
}

int rnn_layerscale_forward(rnn_ctx *ctx, size_t rows, size_t c, const float *x, const float *l,
                           float *y) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (rows == 0 || c == 0) return RNN_OK;
    if (!x || !l || !y) return rnn_fail(ctx, RNN_E_NULL, "layerscale_forward: null operand");
    if (!dims_ok(rows, c)) return rnn_fail(ctx, RNN_E_INVALID, "layerscale: %zu x %zu", rows, c);
    scale_cols_kernel<<<ew_grid(rows * c), NT, 0, ctx->stream>>>(rows * c, (int)c, x, l, y);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

// LayerScale backward (c <= 512) in one pass -- dx and dl's partials -- then
// their reduction: dl += sum (dy m) x, dx = (dy m) l, m = mask[r / rpi] or 1.
static int ls_backward_cs(rnn_ctx *ctx, size_t rows, size_t c, const float *dy, const float *x,
                          const float *l, const float *mask, size_t rpi, float *dx, float *dl) {
    const size_t nblk = rnn_div_up(rows, (size_t)RB_ROWS);
    if (nblk > 0x7fffffff) return rnn_fail(ctx, RNN_E_UNSUPPORTED, "layerscale: rows");
    double *part = col_part(ctx, nblk * c * sizeof(double));
    if (!part) return RNN_E_NOMEM;
    auto cs = [&](auto kern) {
        kern<<<(unsigned)nblk, NT, 0, ctx->stream>>>(rows, (int)c, dy, x, l, mask, rpi, dx, part);
    };
    switch ((int)rnn_div_up(c, (size_t)64)) {
        case 1: cs(ls_bwd_cs_kernel<1>); break;
        case 2: cs(ls_bwd_cs_kernel<2>); break;
        case 3: cs(ls_bwd_cs_kernel<3>); break;
        case 4: cs(ls_bwd_cs_kernel<4>); break;
        case 5: cs(ls_bwd_cs_kernel<5>); break;
        case 6: cs(ls_bwd_cs_kernel<6>); break;
        case 7: cs(ls_bwd_cs_kernel<7>); break;
        default: cs(ls_bwd_cs_kernel<8>); break;
    }
    RNN_LAUNCHED(ctx);
    return col_reduce(ctx, nblk, c, c, part, dl, nullptr);
}

int rnn_layerscale_backward(rnn_ctx *ctx, size_t rows, size_t c, const float *dy, const float *x,
                            const float *l, float *dx, float *dl) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (rows == 0 || c == 0) return RNN_OK;
    if (!dy || !x || !l || !dx || !dl)
        return rnn_fail(ctx, RNN_E_NULL, "layerscale_backward: null operand");
    if (!dims_ok(rows, c)) return rnn_fail(ctx, RNN_E_INVALID, "layerscale: %zu x %zu", rows, c);
    // dl += sum dy x (norm.rs:183-204), before dx may overwrite dy
    if (c <= 512) return ls_backward_cs(ctx, rows, c, dy, x, l, nullptr, 1, dx, dl);
    int rc = colsum_add(ctx, rows, (int)c, dy, x, dl, nullptr);
    if (rc) return rc;
    scale_cols_kernel<<<ew_grid(rows * c), NT, 0, ctx->stream>>>(rows * c, (int)c, dy, l, dx);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_drop_layerscale_backward(rnn_ctx *ctx, size_t rows, size_t c, const float *dy,
                                 const float *x, const float *l, const float *mask, size_t rpi,
                                 float *dx, float *dl) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (rows == 0 || c == 0) return RNN_OK;
    if (!dy || !x || !l || !dx || !dl)
        return rnn_fail(ctx, RNN_E_NULL, "drop_layerscale_backward: null operand");
    if (!dims_ok(rows, c)) return rnn_fail(ctx, RNN_E_INVALID, "layerscale: %zu x %zu", rows, c);
    if (dx == dy) return rnn_fail(ctx, RNN_E_INVALID, "drop_layerscale_backward: dx is dy");
    if (mask && (rpi == 0 || rows % rpi))
        return rnn_fail(ctx, RNN_E_INVALID, "drop_layerscale_backward: %zu rows per image of %zu",
                        rpi, rows);
    // dl += sum (dy m) x, then dx = (dy m) l
    if (c <= 512) return ls_backward_cs(ctx, rows, c, dy, x, l, mask, mask ? rpi : 1, dx, dl);
    int rc = rnn_colsum_f64(ctx, rows, (int)c, dy, x, dl, nullptr, mask, mask ? rpi : 1);
    if (rc) return rc;
    if (mask)
        scale_cols_masked_kernel<<<ew_grid(rows * c), NT, 0, ctx->stream>>>(rows * c, (int)c,
                                                                           rpi * c, dy, l, mask, dx);
    else
        scale_cols_kernel<<<ew_grid(rows * c), NT, 0, ctx->stream>>>(rows * c, (int)c, dy, l, dx);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_block_branch_backward(rnn_ctx *ctx, size_t rows, size_t c, const float *dy,
                              const float *a, const float *l1, const float *m1, const float *dwo,
                              const float *gamma, const float *cm, const float *lm,
                              const float *m2, size_t rpi, float *da, float *dl1, float *ddw,
                              float *dgamma, float *dc, float *dlm) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (rows == 0 || c == 0) return RNN_OK;
    if (!dy || !a || !l1 || !dwo || !gamma || !da || !dl1 || !ddw || !dgamma)
        return rnn_fail(ctx, RNN_E_NULL, "block_branch_backward: null operand");
    const bool cross = cm != nullptr;
    if (cross && (!lm || !dc || !dlm))
        return rnn_fail(ctx, RNN_E_NULL, "block_branch_backward: cm without lm, dc or dlm");
    if (!dims_ok(rows, c))
        return rnn_fail(ctx, RNN_E_INVALID, "block_branch_backward: %zu x %zu", rows, c);
    if ((m1 || m2) && (rpi == 0 || rows % rpi))
        return rnn_fail(ctx, RNN_E_INVALID, "block_branch_backward: %zu rows per image of %zu",
                        rpi, rows);
    if (da == dy || ddw == dy || ddw == da || (cross && (dc == dy || dc == da || dc == ddw)))
        return rnn_fail(ctx, RNN_E_INVALID, "block_branch_backward: outputs overlap");
    if (c > 512) {
        // the separate passes, in the reference's order
        int rc = RNN_OK;
        if (cross) rc = rnn_drop_layerscale_backward(ctx, rows, c, dy, cm, lm, m2, rpi, dc, dlm);
        if (!rc) rc = rnn_drop_layerscale_backward(ctx, rows, c, dy, a, l1, m1, rpi, da, dl1);
        if (!rc) rc = rnn_layerscale_backward(ctx, rows, c, da, dwo, gamma, ddw, dgamma);
        return rc;
    }
    const size_t nblk = rnn_div_up(rows, (size_t)RB_ROWS);
    if (nblk > 0x7fffffff) return rnn_fail(ctx, RNN_E_UNSUPPORTED, "block_branch_backward: rows");
    const size_t pb = nblk * c * sizeof(double);
    double *part = col_part(ctx, (cross ? 3 : 2) * pb);
    if (!part) return RNN_E_NOMEM;
    BranchBwd g{dy, a, l1, m1, dwo, gamma, cm, lm, m2, da, ddw, dc,
                part, part + nblk * c, cross ? part + 2 * nblk * c : nullptr,
                rows, (m1 || m2) ? rpi : 1, (int)c};
    auto go = [&](auto kern) { kern<<<(unsigned)nblk, NT, 0, ctx->stream>>>(g); };
    const int nv = (int)rnn_div_up(c, (size_t)64);
#define RNN_BRANCH_NV(NV)                                         \
    case NV:                                                       \
        cross ? go(branch_bwd_cs_kernel<NV, true>) : go(branch_bwd_cs_kernel<NV, false>); \
        break;
    switch (nv) {
        RNN_BRANCH_NV(1)
        RNN_BRANCH_NV(2)
        RNN_BRANCH_NV(3)
        RNN_BRANCH_NV(4)
        RNN_BRANCH_NV(5)
        RNN_BRANCH_NV(6)
        RNN_BRANCH_NV(7)
        default:
            cross ? go(branch_bwd_cs_kernel<8, true>) : go(branch_bwd_cs_kernel<8, false>);
            break;
    }
#undef RNN_BRANCH_NV
    RNN_LAUNCHED(ctx);
    int rc = RNN_OK;
    if (cross) rc = col_reduce(ctx, nblk, c, c, g.partm, dlm, nullptr);
    if (!rc) rc = col_reduce(ctx, nblk, c, c, g.part1, dl1, nullptr);
    if (!rc) rc = col_reduce(ctx, nblk, c, c, g.partg, dgamma, nullptr);
    return rc;
}

int rnn_residual_add_scaled(rnn_ctx *ctx, size_t rows, size_t c, const float *x, const float *a,
                            const float *l, const float *mask, size_t rpi, float *y) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (rows == 0 || c == 0) return RNN_OK;
    if (!x || !a || !l || !y) return rnn_fail(ctx, RNN_E_NULL, "residual_add_scaled: null operand");
    if (!dims_ok(rows, c)) return rnn_fail(ctx, RNN_E_INVALID, "residual_add_scaled: %zu x %zu",
                                           rows, c);
    if (mask && (rpi == 0 || rows % rpi))
        return rnn_fail(ctx, RNN_E_INVALID, "residual_add_scaled: %zu rows per image of %zu", rpi,
                        rows);
    if (a == y) return rnn_fail(ctx, RNN_E_INVALID, "residual_add_scaled: y is a");
    const size_t len = rows * c, per = (mask ? rpi : rows) * c;
    const bool vec = c % 4 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)a & 15) == 0 &&
                     ((uintptr_t)l & 15) == 0 && ((uintptr_t)y & 15) == 0;
    if (vec)
        residual_add_scaled_kernel<true><<<ew_grid(rnn_div_up(len, (size_t)4)), NT, 0, ctx->stream>>>(
            len, (int)c, per, x, a, l, mask, y);
    else
        residual_add_scaled_kernel<false><<<ew_grid(len), NT, 0, ctx->stream>>>(len, (int)c, per, x,
                                                                                a, l, mask, y);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

// The float4 SwiGLU passes: h a multiple of 4, 16-byte aligned tensors.
static bool swiglu_vec(size_t h, const void *a, const void *b, const void *c) {
    return h % 4 == 0 && (((uintptr_t)a | (uintptr_t)b | (uintptr_t)c) & 15) == 0;
}

int rnn_swiglu_forward(rnn_ctx *ctx, size_t rows, size_t h, const float *ab, float *u) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (rows == 0 || h == 0) return RNN_OK;
    if (!ab || !u) return rnn_fail(ctx, RNN_E_NULL, "swiglu_forward: null operand");
    if (!dims_ok(rows, h)) return rnn_fail(ctx, RNN_E_INVALID, "swiglu: %zu x %zu", rows, h);
    if (swiglu_vec(h, ab, u, u) && rows * h / 4 < ((size_t)1 << 31))
        swiglu_fwd4_kernel<<<(unsigned)rnn_div_up(rows * h / 4, (size_t)NT), NT, 0,
                             ctx->stream>>>(rows, (int)(h / 4), (const float4 *)ab, (float4 *)u);
    else
        swiglu_fwd_kernel<<<ew_grid(rows * h), NT, 0, ctx->stream>>>(rows, (int)h, ab, u);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_swiglu_backward(rnn_ctx *ctx, size_t rows, size_t h, const float *du, const float *ab,
                        float *dab) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (rows == 0 || h == 0) return RNN_OK;
    if (!du || !ab || !dab) return rnn_fail(ctx, RNN_E_NULL, "swiglu_backward: null operand");
    if (!dims_ok(rows, h)) return rnn_fail(ctx, RNN_E_INVALID, "swiglu: %zu x %zu", rows, h);
    if (swiglu_vec(h, du, ab, dab) && rows * h / 4 < ((size_t)1 << 31))
        swiglu_bwd4_kernel<<<(unsigned)rnn_div_up(rows * h / 4, (size_t)NT), NT, 0,
                             ctx->stream>>>(rows, (int)(h / 4), (const float4 *)du,
                                            (const float4 *)ab, (float4 *)dab);
    else
        swiglu_bwd_kernel<<<ew_grid(rows * h), NT, 0, ctx->stream>>>(rows, (int)h, du, ab, dab);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_dwconv3_forward(rnn_ctx *ctx, size_t n, size_t th, size_t tw, size_t c, const float *x,
                        const float *w, const float *b, float *y) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (n == 0 || th == 0 || tw == 0 || c == 0) return RNN_OK;
    if (!x || !w || !b || !y) return rnn_fail(ctx, RNN_E_NULL, "dwconv3_forward: null operand");
    if (th > 65536 || tw > 65536 || !dims_ok(n * th * tw, c))
        return rnn_fail(ctx, RNN_E_INVALID, "dwconv3: %zu x %zu x %zu x %zu", n, th, tw, c);
    const size_t len = n * th * tw * c;
    if (dw3_vec(x, w, y, c, n) && b && ((uintptr_t)b & 15) == 0) {
        const int c4 = (int)(c / 4);
        dw3_fwd4_kernel<<<dim3((unsigned)rnn_div_up(tw * c4, (size_t)NT), (unsigned)th, (unsigned)n),
                          NT, 0, ctx->stream>>>((int)th, (int)tw, c4, (const float4 *)x,
                                                (const float4 *)w, (const float4 *)b, (float4 *)y);
    } else {
        dw3_fwd_kernel<<<ew_grid(len), NT, 0, ctx->stream>>>(n, (int)th, (int)tw, (int)c, x, w, b,
                                                             y);
    }
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_dwconv3_branch_forward(rnn_ctx *ctx, size_t n, size_t th, size_t tw, size_t c,
                               const float *h, const float *w, const float *b, float *d, float *a,
                               const float *gamma, const float *x, const float *l,
                               const float *mask, float *y) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (n == 0 || th == 0 || tw == 0 || c == 0) return RNN_OK;
    if (!h || !w || !b || !d || !a || !gamma || !x || !l || !y)
        return rnn_fail(ctx, RNN_E_NULL, "dwconv3_branch_forward: null operand");
    if (th > 65536 || tw > 65536 || !dims_ok(n * th * tw, c))
        return rnn_fail(ctx, RNN_E_INVALID, "dwconv3: %zu x %zu x %zu x %zu", n, th, tw, c);
    if (y == a || x == a || d == a || d == h || d == x || d == y || a == h || y == h)
        return rnn_fail(ctx, RNN_E_INVALID, "dwconv3_branch_forward: aliased operands");
    auto al = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
    if (dw3_vec(h, w, d, c, n) && al(b) && al(a) && al(gamma) && al(x) && al(l) && al(y)) {
        const int c4 = (int)(c / 4);
        dw3_branch4_kernel<<<dim3((unsigned)rnn_div_up(tw * c4, (size_t)NT), (unsigned)th,
                                  (unsigned)n),
                             NT, 0, ctx->stream>>>(
            (int)th, (int)tw, c4, (const float4 *)h, (const float4 *)w, (const float4 *)b,
            (float4 *)d, (float4 *)a, (const float4 *)gamma, (const float4 *)x,
            (const float4 *)l, mask, (float4 *)y);
        RNN_LAUNCHED(ctx);
        return RNN_OK;
    }
    // the same three steps as separate passes
    const size_t rows = n * th * tw;
    int rc = rnn_dwconv3_forward(ctx, n, th, tw, c, h, w, b, d);
    if (!rc) rc = rnn_axpy_cols(ctx, rows, c, a, gamma, d);
    if (!rc) rc = rnn_residual_add_scaled(ctx, rows, c, x, a, l, mask, th * tw, y);
    return rc;
}

int rnn_dwconv3_backward(rnn_ctx *ctx, size_t n, size_t th, size_t tw, size_t c, const float *dy,
                         const float *x, const float *w, float *dx, float *dw, float *db) {
    return rnn_dwconv3_backward_ex(ctx, n, th, tw, c, dy, x, w, dx, dw, db, 0);
}

int rnn_dwconv3_backward_ex(rnn_ctx *ctx, size_t n, size_t th, size_t tw, size_t c,
                            const float *dy, const float *x, const float *w, float *dx, float *dw,
                            float *db, uint32_t flags) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (n == 0 || th == 0 || tw == 0 || c == 0) return RNN_OK;
    if (!dy || !x || !w || !dx || !dw || !db)
        return rnn_fail(ctx, RNN_E_NULL, "dwconv3_backward: null operand");
    if (flags & ~RNN_DW3_ACC_DX)
        return rnn_fail(ctx, RNN_E_INVALID, "dwconv3_backward: flags 0x%x", flags);
    if (dx == dy) return rnn_fail(ctx, RNN_E_INVALID, "dwconv3_backward: dx is dy");
    if (th > 65536 || tw > 65536 || !dims_ok(n * th * tw, c))
        return rnn_fail(ctx, RNN_E_INVALID, "dwconv3: %zu x %zu x %zu x %zu", n, th, tw, c);
    const bool acc = (flags & RNN_DW3_ACC_DX) != 0;
    // dW and db partials per block of output rows (about 512 blocks), then
    // the block-order sum (1024 blocks: more partial rows to sum, 0.02 ms
    // slower in the rustvit step; 256: the dW pass too serial)
    const size_t cblk = rnn_div_up(c, (size_t)NT);
    const size_t want = std::max<size_t>(1, 512 / (cblk * n));
    const size_t nrb = std::min(th, want), RB = rnn_div_up(th, nrb);
    const size_t nrb_used = rnn_div_up(th, RB), nblk = n * nrb_used;
    if (nblk > 65535) return rnn_fail(ctx, RNN_E_UNSUPPORTED, "dwconv3: too many images");
    double *part = col_part(ctx, nblk * 10 * c * sizeof(double));
    if (!part) return RNN_E_NOMEM;
    dw3_bwd_w_kernel<<<dim3((unsigned)cblk, (unsigned)nblk), NT, 0, ctx->stream>>>(
        (int)th, (int)tw, (int)c, (int)RB, (int)nrb_used, dy, x, part);
    RNN_LAUNCHED(ctx);
    // part is [nblk][10c]: taps 0-8 (dW's [9][c] order), then db
    int rc = col_reduce(ctx, nblk, 10 * c, 9 * c, part, dw, db);
    if (rc) return rc;
    const size_t len = n * th * tw * c;
    if (dw3_vec(dy, w, dx, c, n)) {
        const int c4 = (int)(c / 4);
        const dim3 grid((unsigned)rnn_div_up(tw * c4, (size_t)NT), (unsigned)th, (unsigned)n);
        if (acc)
            dw3_bwd_x4_kernel<true><<<grid, NT, 0, ctx->stream>>>(
                (int)th, (int)tw, c4, (const float4 *)dy, (const float4 *)w, (float4 *)dx);
        else
            dw3_bwd_x4_kernel<false><<<grid, NT, 0, ctx->stream>>>(
                (int)th, (int)tw, c4, (const float4 *)dy, (const float4 *)w, (float4 *)dx);
    } else {
        dw3_bwd_x_kernel<<<ew_grid(len), NT, 0, ctx->stream>>>(n, (int)th, (int)tw, (int)c, dy, w,
                                                               dx, acc ? 1 : 0);
    }
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_seqpool_forward(rnn_ctx *ctx, size_t n, size_t t, size_t c, const float *x,
                        const float *p, float *z, float *w) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (n == 0 || c == 0) return RNN_OK;
    if (!x || !p || !z || !w) return rnn_fail(ctx, RNN_E_NULL, "seqpool_forward: null operand");
    if (t == 0 || t > SP_MAXT || n > 0x7fffffff || !dims_ok(n * t, c))
        return rnn_fail(ctx, RNN_E_INVALID, "seqpool: n %zu, t %zu (1..%d), c %zu", n, t, SP_MAXT,
                        c);
    const size_t xl = seqpool_xl_bytes(t, c);
    if (xl <= SP_XL_BYTES) {
        static bool attr = false;
        if (!attr) {
            attr = true;
            (void)hipFuncSetAttribute((const void *)seqpool_fwd_kernel<true>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      (int)SP_XL_BYTES);
        }
        seqpool_fwd_kernel<true><<<(unsigned)n, NT, xl, ctx->stream>>>((int)t, (int)c, x, p, z, w);
    } else {
        seqpool_fwd_kernel<false><<<(unsigned)n, NT, 0, ctx->stream>>>((int)t, (int)c, x, p, z, w);
    }
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_seqpool_backward(rnn_ctx *ctx, size_t n, size_t t, size_t c, const float *dz,
                         const float *w, const float *x, const float *p, float *dx, float *dp) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (n == 0 || c == 0) return RNN_OK;
    if (!dz || !w || !x || !p || !dx || !dp)
        return rnn_fail(ctx, RNN_E_NULL, "seqpool_backward: null operand");
    if (t == 0 || t > SP_MAXT || n > 0x7fffffff || !dims_ok(n * t, c))
        return rnn_fail(ctx, RNN_E_INVALID, "seqpool: n %zu, t %zu (1..%d), c %zu", n, t, SP_MAXT,
                        c);
    float *part = (float *)rnn_workspace(ctx, n * c * sizeof(float));
    if (!part) return RNN_E_NOMEM;
    const size_t xl = seqpool_xl_bytes(t, c);
    if (xl <= SP_XL_BYTES) {
        static bool attr = false;
        if (!attr) {
            attr = true;
            (void)hipFuncSetAttribute((const void *)seqpool_bwd_kernel<true>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      (int)SP_XL_BYTES);
        }
        seqpool_bwd_kernel<true><<<(unsigned)n, NT, xl, ctx->stream>>>((int)t, (int)c, dz, w, x,
                                                                       p, dx, part);
    } else {
        seqpool_bwd_kernel<false><<<(unsigned)n, NT, 0, ctx->stream>>>((int)t, (int)c, dz, w, x,
                                                                        p, dx, part);
    }
    RNN_LAUNCHED(ctx);
    rowsum_add_kernel<<<(unsigned)rnn_div_up(c, (size_t)RS_NT), RS_NT, 0, ctx->stream>>>(
        n, (int)c, part, dp);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

}  // extern "C"
