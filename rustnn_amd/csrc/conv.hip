// Implicit-GEMM convolution on gfx950 fp32 MFMA: forward, dX (col2im in
// gather form, no atomics) and dW (deterministic split-K).
//
// Reference: conv.rs (per-image W * im2col(X) through the 6x16 AVX2
// micro-kernel, im2col fused into B-panel packing by gather_span, col2im
// fused into the tile write-back by scatter_span) and the Conv2d batch
// drivers (nn.rs:166-250).  No im2col or dcol matrix exists here either: a
// workgroup stages a zero-padded halo tile of the source image(s) in LDS once
// per channel chunk, and every (channel, kh, kw) row of the implicit im2col
// matrix is an LDS read at a per-tap constant offset from a per-lane base.
//
// MFMA mapping (v_mfma_f32_32x32x2f32): M = output channels (32 per block),
// N = output pixels (32 per group), K = (channel pair, tap).  Lane half h of a
// K step carries channel cp + h*CH/2 so both halves read the same tap offset.
//
// This file holds the C entry points, the generic per-class tile kernel used
// for (k, stride, pad) combinations without a specialisation in
// conv_fast.hip, and the im2col debug export.  Forward and dX share
// conv_tile_kernel.  A launch computes an output "class
// grid" (a, b) -> dst(a*OS + py, b*OS + px) from source positions
// (a*IS + dy_t, b*IS + dx_t) over its tap list t:
//   forward:          one class, IS = stride, OS = 1, taps (kh-pad, kw-pad)
//   dX, stride s:     s*s classes (py, px), IS = 1, OS = s, taps = the (kh, kw)
//                     with (p + pad - k) % s == 0, offset (p + pad - k) / s.
// Each dX element is written once (gather form), so no col2im accumulation.
#include "rnn_internal.h"

#include <algorithm>

namespace {

constexpr int MAXT = 9;

struct TileArgs {
    const float *src;  // [N][CS][HS][WS]
    const float *w;    // weights; element (m, ch, tap t) at w[m*sm + ch*sc + wtap[t]]
    float *dst;        // [N][CD][HD][WD]
    int sm, sc;        // weight strides of output row m and source channel ch
    int ch_inner;      // staging order: 1 = channel before row (sc < sm)
    int N, CS, HS, WS;
    int CD, HD, WD;
    int GA, GB;
    int OS, py, px, IS;
    int dy_min, dx_min;
    int TR, IMGS, TIH, TIW, TIWP, HALF, deint;
    int CH, nchunks, nmblk, tiles_a;
    int tapoff[MAXT];
    int wtap[MAXT];
};

// LDS column of tile column tx (de-interleaved by parity when IS == 2 so a
// 32-pixel group reads 32 consecutive words).
__device__ __forceinline__ int tile_col(int tx, int deint, int half) {
    return deint ? (tx & 1) * half + (tx >> 1) : tx;
}

// Stages the channel chunk [c0, c0+CH) of the source tile: rows
// a0*IS + dy_min + ty, columns dx_min + tx, zero outside the image.
__device__ __forceinline__ void load_src_tile(const TileArgs &g, float *xs, int n0, int a0, int c0,
                                              int tid, int nthreads) {
    const int tih = g.TIH, tiw = g.TIW, per_img = tih * tiw, per_ch = g.IMGS * per_img;
    const int total = g.CH * per_ch;
    const int chs = g.IMGS * tih * g.TIWP, imgs = tih * g.TIWP;
    const int y0 = a0 * g.IS + g.dy_min;
    for (int idx = tid; idx < total; idx += nthreads) {
        int ch = idx / per_ch, rem = idx - ch * per_ch;
        int img = rem / per_img;
        rem -= img * per_img;
        int ty = rem / tiw, tx = rem - ty * tiw;
        int n = n0 + img, c = c0 + ch, y = y0 + ty, x = g.dx_min + tx;
        float v = 0.f;
        if (n < g.N && c < g.CS && y >= 0 && y < g.HS && x >= 0 && x < g.WS)
            v = g.src[(((long long)n * g.CS + c) * g.HS + y) * g.WS + x];
        xs[ch * chs + img * imgs + ty * g.TIWP + tile_col(tx, g.deint, g.HALF)] = v;
    }
}

template <int NTAPS, int NPW, int MB>
__global__ __launch_bounds__(256) void conv_tile_kernel(TileArgs g) {
    extern __shared__ float smem[];
    const int nthreads = blockDim.x, tid = threadIdx.x, lane = tid & 63, wave = wave_index();
    const int tile = blockIdx.x;
    const int ta = tile % g.tiles_a, tn = tile / g.tiles_a;
    const int a0 = ta * g.TR, n0 = tn * g.IMGS;
    const int mb0 = blockIdx.y * MB;
    const int CP = g.CH >> 1;
    const int chs = g.IMGS * g.TIH * g.TIWP, imgs = g.TIH * g.TIWP;
    float *xs = smem;
    float *ws = smem + ((g.CH * chs + 3) & ~3);  // 16-byte aligned weight slab
    const int npix = g.IMGS * g.TR * g.GB;
    const int h = lane >> 5;

    // Per-lane LDS base of each pixel group (channel half h included).
    int vb[NPW];
    bool pv[NPW];
#pragma unroll
    for (int j = 0; j < NPW; j++) {
        int p = (wave * NPW + j) * 32 + (lane & 31);
        pv[j] = p < npix;
        if (!pv[j]) p = 0;
        int img = p / (g.TR * g.GB), rem = p - img * (g.TR * g.GB);
        int r = rem / g.GB, c = rem - r * g.GB;
        vb[j] = h * CP * chs + img * imgs + r * g.IS * g.TIWP + (g.deint ? c : c * g.IS);
    }

    f32x16 acc[MB][NPW];
#pragma unroll
    for (int mb = 0; mb < MB; mb++)
#pragma unroll
        for (int j = 0; j < NPW; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[mb][j][v] = 0.f;

    const int wchunk = CP * NTAPS * 64;  // floats per m-block of a chunk
    for (int chunk = 0; chunk < g.nchunks; chunk++) {
        __syncthreads();
        load_src_tile(g, xs, n0, a0, chunk * g.CH, tid, nthreads);
        // Weight slab in MFMA fragment order: ws[mb][cp][t][lane] with lane
        // l -> row m = (mb0+mb)*32 + l%32, channel chunk*CH + cp + (l/32)*CP.
        // Consecutive threads walk taps, then the operand with the smaller
        // global stride, so the gather from w stays coalesced.
        for (int idx = tid; idx < MB * 32 * g.CH * NTAPS; idx += nthreads) {
            const int t = idx % NTAPS;
            int r = idx / NTAPS, chl, ml;
            if (g.ch_inner) {
                chl = r % g.CH;
                r /= g.CH;
                ml = r % 32;
            } else {
                ml = r % 32;
                r /= 32;
                chl = r % g.CH;
            }
            const int mb = r / (g.ch_inner ? 32 : g.CH);
            const int m = (mb0 + mb) * 32 + ml, ch = chunk * g.CH + chl;
            float v = 0.f;
            if (m < g.CD && ch < g.CS) v = g.w[(long long)m * g.sm + (long long)ch * g.sc + g.wtap[t]];
            const int cp = chl % CP, hh = chl / CP;
            ws[mb * wchunk + (cp * NTAPS + t) * 64 + ml + 32 * hh] = v;
        }
        __syncthreads();
        const float *wl = ws + lane;
        for (int cp = 0; cp < CP; cp++) {
            const int coff = cp * chs;
#pragma unroll
            for (int t = 0; t < NTAPS; t++) {
                float a[MB], b[NPW];
#pragma unroll
                for (int mb = 0; mb < MB; mb++) a[mb] = wl[mb * wchunk + (cp * NTAPS + t) * 64];
#pragma unroll
                for (int j = 0; j < NPW; j++) b[j] = xs[vb[j] + coff + g.tapoff[t]];
#pragma unroll
                for (int mb = 0; mb < MB; mb++)
#pragma unroll
                    for (int j = 0; j < NPW; j++)
                        acc[mb][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[mb], b[j], acc[mb][j],
                                                                          0, 0, 0);
            }
        }
    }

    // Write-back: acc row 8*(v/4) + 4*h + v%4 = output channel, column = pixel.
#pragma unroll
    for (int j = 0; j < NPW; j++) {
        if (!pv[j]) continue;
        int p = (wave * NPW + j) * 32 + (lane & 31);
        int img = p / (g.TR * g.GB), rem = p - img * (g.TR * g.GB);
        int r = rem / g.GB, c = rem - r * g.GB;
        int n = n0 + img, a = a0 + r;
        if (n >= g.N || a >= g.GA) continue;
        long long pix = (long long)(a * g.OS + g.py) * g.WD + (c * g.OS + g.px);
#pragma unroll
        for (int mb = 0; mb < MB; mb++) {
            int mbase = (mb0 + mb) * 32;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                int m = mbase + 8 * (v >> 2) + 4 * h + (v & 3);
                if (m < g.CD) g.dst[((long long)n * g.CD + m) * g.HD * g.WD + pix] = acc[mb][j][v];
            }
        }
    }
}

// Zero-fills the class (py, px) positions of dst (dX classes with no tap).
__global__ void zero_class_kernel(float *dst, int N, int CD, int HD, int WD, int GA, int GB, int OS,
                                  int py, int px) {
    long long total = (long long)N * CD * GA * GB;
    long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= total) return;
    int b = (int)(e % GB);
    long long r = e / GB;
    int a = (int)(r % GA);
    long long nc = r / GA;
    dst[nc * HD * WD + (long long)(a * OS + py) * WD + (b * OS + px)] = 0.f;
}

__global__ void im2col_kernel(const float *x, float *col, int CI, int H, int W, int K, int S,
                              int pad, int OH, int OW) {
    long long total = (long long)CI * K * K * OH * OW;
    long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= total) return;
    int hw = OH * OW;
    int r = (int)(e / hw), p = (int)(e % hw);
    int ci = r / (K * K), kh = (r / K) % K, kw = r % K;
    int oy = p / OW, ox = p % OW;
    // the same source coordinate the staging loads use: (a*IS + dy, b*IS + dx)
    int y = oy * S + (kh - pad), xx = ox * S + (kw - pad);
    float v = 0.f;
    if (y >= 0 && y < H && xx >= 0 && xx < W) v = x[((long long)ci * H + y) * W + xx];
    col[e] = v;
}

// ---------------------------------------------------------------- host side

struct Tap {
    int kh, kw, dy, dx;
};

struct Plan {
    int NPW, MB, NW, TR, IMGS, TIH, TIW, TIWP, HALF, deint, CH, nchunks, nmblk;
    size_t lds;
};

constexpr size_t LDS_HALF = 80 * 1024;  // two workgroups per CU
constexpr size_t LDS_FULL = 160 * 1024;

// Picks tile rows / images per tile for the tile kernel: up to 256 output
// pixels per workgroup (whole images first, then fewer rows) within the LDS
// budget of two workgroups per CU, else of one.
static bool plan_tile(int CS, int CD, int GA, int GB, int IS, int ntaps, int dyr, int dxr,
                      Plan &p) {
    p.deint = IS == 2;
    p.CH = std::min(32, (CS + 1) & ~1);
    p.nchunks = (CS + p.CH - 1) / p.CH;
    p.nmblk = (CD + 31) / 32;
    p.MB = 1;
    if (GB > 256) return false;
    const int target = 256;
    for (size_t budget : {LDS_HALF, LDS_FULL}) {
        int tr, imgs;
        if (GA * GB <= target) {
            tr = GA;
            imgs = std::max(1, target / (GA * GB));
        } else {
            tr = std::max(1, std::min(GA, target / GB));
            imgs = 1;
        }
        for (;;) {
            int tih = (tr - 1) * IS + dyr + 1, tiw = (GB - 1) * IS + dxr + 1;
            int half = (tiw + 1) / 2, tiwp = p.deint ? 2 * half : tiw;
            size_t xsf = ((size_t)p.CH * imgs * tih * tiwp + 3) & ~(size_t)3;
            size_t wsf = (size_t)p.MB * (p.CH / 2) * ntaps * 64;
            size_t lds = (xsf + wsf) * 4;
            if (lds <= budget) {
                int npix = imgs * tr * GB;
                p.NPW = npix > 128 ? 2 : 1;
                p.NW = std::max(1, (npix + 32 * p.NPW - 1) / (32 * p.NPW));
                p.TR = tr;
                p.IMGS = imgs;
                p.TIH = tih;
                p.TIW = tiw;
                p.TIWP = tiwp;
                p.HALF = half;
                p.lds = lds;
                return true;
            }
            if (imgs > 1)
                imgs /= 2;
            else if (tr > 1)
                tr = (tr + 1) / 2;
            else
                break;
        }
    }
    return false;
}

template <int NTAPS>
static int launch_tile_t(rnn_ctx *ctx, const TileArgs &a, const Plan &p) {
    dim3 grid((unsigned)(a.tiles_a * ((a.N + a.IMGS - 1) / a.IMGS)),
              (unsigned)((p.nmblk + p.MB - 1) / p.MB));
    dim3 block(64 * p.NW);
    if (p.NPW == 2)
        hipLaunchKernelGGL((conv_tile_kernel<NTAPS, 2, 1>), grid, block, p.lds, ctx->stream, a);
    else
        hipLaunchKernelGGL((conv_tile_kernel<NTAPS, 1, 1>), grid, block, p.lds, ctx->stream, a);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

static bool lds_attr_done = false;

static void set_lds_limits() {
    if (lds_attr_done) return;
    lds_attr_done = true;
    const void *ks[] = {
        (const void *)conv_tile_kernel<1, 1, 1>, (const void *)conv_tile_kernel<1, 2, 1>,
        (const void *)conv_tile_kernel<2, 1, 1>, (const void *)conv_tile_kernel<2, 2, 1>,
        (const void *)conv_tile_kernel<4, 1, 1>, (const void *)conv_tile_kernel<4, 2, 1>,
        (const void *)conv_tile_kernel<9, 1, 1>, (const void *)conv_tile_kernel<9, 2, 1>,
    };
    for (const void *k : ks)
        (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDS_FULL);
}

// One tile-kernel launch: dst class (py, px) of an OS-strided output grid
// GA x GB computed from src through `taps`.  W element of tap t for output
// row m and source channel ch: w[m*sm + ch*sc + kh*K + kw].
static int run_tile(rnn_ctx *ctx, const float *src, int N, int CS, int HS, int WS, float *dst,
                    int CD, int HD, int WD, int GA, int GB, int OS, int py, int px, int IS,
                    const Tap *taps, int ntaps, const float *w, int sm, int sc, int K) {
    if (GA <= 0 || GB <= 0) return RNN_OK;
    if (ntaps == 0) {
        long long total = (long long)N * CD * GA * GB;
        hipLaunchKernelGGL(zero_class_kernel, dim3((unsigned)rnn_div_up(total, 256)), dim3(256), 0,
                           ctx->stream, dst, N, CD, HD, WD, GA, GB, OS, py, px);
        RNN_LAUNCHED(ctx);
        return RNN_OK;
    }
    int dy_min = 1 << 30, dy_max = -(1 << 30), dx_min = 1 << 30, dx_max = -(1 << 30);
    for (int t = 0; t < ntaps; t++) {
        dy_min = std::min(dy_min, taps[t].dy);
        dy_max = std::max(dy_max, taps[t].dy);
        dx_min = std::min(dx_min, taps[t].dx);
        dx_max = std::max(dx_max, taps[t].dx);
    }
    Plan p;
    if (!plan_tile(CS, CD, GA, GB, IS, ntaps, dy_max - dy_min, dx_max - dx_min, p))
        return rnn_fail(ctx, RNN_E_UNSUPPORTED, "conv: no LDS tiling for %dx%d grid", GA, GB);
    TileArgs a;
    a.src = src;
    a.w = w;
    a.dst = dst;
    a.sm = sm;
    a.sc = sc;
    a.ch_inner = sc < sm ? 1 : 0;
    a.N = N;
    a.CS = CS;
    a.HS = HS;
    a.WS = WS;
    a.CD = CD;
    a.HD = HD;
    a.WD = WD;
    a.GA = GA;
    a.GB = GB;
    a.OS = OS;
    a.py = py;
    a.px = px;
    a.IS = IS;
    a.dy_min = dy_min;
    a.dx_min = dx_min;
    a.TR = p.TR;
    a.IMGS = p.IMGS;
    a.TIH = p.TIH;
    a.TIW = p.TIW;
    a.TIWP = p.TIWP;
    a.HALF = p.HALF;
    a.deint = p.deint;
    a.CH = p.CH;
    a.nchunks = p.nchunks;
    a.nmblk = p.nmblk;
    a.tiles_a = (GA + p.TR - 1) / p.TR;
    for (int t = 0; t < MAXT; t++) {
        a.tapoff[t] = 0;
        a.wtap[t] = t < ntaps ? taps[t].kh * K + taps[t].kw : 0;
        if (t < ntaps) {
            int dyp = taps[t].dy - dy_min, dxp = taps[t].dx - dx_min;
            a.tapoff[t] = dyp * p.TIWP + (p.deint ? (dxp & 1) * p.HALF + (dxp >> 1) : dxp);
        }
    }
    switch (ntaps) {
        case 1: return launch_tile_t<1>(ctx, a, p);
        case 2: return launch_tile_t<2>(ctx, a, p);
        case 4: return launch_tile_t<4>(ctx, a, p);
        case 9: return launch_tile_t<9>(ctx, a, p);
        default: return rnn_fail(ctx, RNN_E_UNSUPPORTED, "conv: %d taps per class", ntaps);
    }
}

static int check_spec(rnn_ctx *ctx, const rnn_conv_spec *sp) {
    if (!sp) return rnn_fail(ctx, RNN_E_NULL, "conv: spec is null");
    if (!sp->cin || !sp->cout || !sp->k || !sp->stride || !sp->h || !sp->w)
        return rnn_fail(ctx, RNN_E_INVALID, "conv: zero dimension in spec");
    if (sp->oh != (sp->h + 2 * sp->pad - sp->k) / sp->stride + 1 ||
        sp->ow != (sp->w + 2 * sp->pad - sp->k) / sp->stride + 1 || sp->k > sp->h + 2 * sp->pad)
        return rnn_fail(ctx, RNN_E_INVALID, "conv: oh/ow do not match Conv2d::out_dim");
    if (sp->k * sp->k > MAXT) return rnn_fail(ctx, RNN_E_UNSUPPORTED, "conv: k > 3");
    return RNN_OK;
}

}  // namespace

extern "C" {

int rnn_conv2d_forward(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *x,
                       const float *w, float *y) {
    return rnn_conv2d_forward_wp(ctx, sp, n, x, w, nullptr, y);
}

int rnn_conv2d_backward_x(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *dy,
                          const float *w, float *dx) {
    return rnn_conv2d_backward_x_wp(ctx, sp, n, dy, w, nullptr, dx);
}

}  // extern "C"

int rnn_conv2d_forward_wp(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *x,
                          const float *w, const float *wp, float *y) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    int rc = check_spec(ctx, sp);
    if (rc) return rc;
    if (n == 0) return RNN_OK;
    if (!x || !w || !y) return rnn_fail(ctx, RNN_E_NULL, "conv2d_forward: null operand");
    rc = rnn_conv_fast(ctx, 0, sp, n, x, w, wp, y);
    if (rc != RNN_E_UNSUPPORTED) return rc;
    set_lds_limits();
    const int K = sp->k, KK = K * K;
    Tap taps[MAXT];
    for (int kh = 0; kh < K; kh++)
        for (int kw = 0; kw < K; kw++)
            taps[kh * K + kw] = {kh, kw, kh - (int)sp->pad, kw - (int)sp->pad};
    // A = W[cout][cin][kh][kw]: m = cout (stride cin*KK), ch = cin (stride KK)
    return run_tile(ctx, x, (int)n, sp->cin, sp->h, sp->w, y, sp->cout, sp->oh, sp->ow, sp->oh,
                    sp->ow, 1, 0, 0, sp->stride, taps, KK, w, sp->cin * KK, KK, K);
}

int rnn_conv2d_forward_stats(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *x,
                             const float *w, const float *wp, float *y, double *part) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    int rc = check_spec(ctx, sp);
    if (rc) return rc;
    if (n == 0) return RNN_OK;
    if (!x || !w || !y || !part)
        return rnn_fail(ctx, RNN_E_NULL, "conv2d_forward_stats: null operand");
    ConvStats st;
    st.part = part;
    rc = rnn_conv_fast(ctx, 0, sp, n, x, w, wp, y, &st);
    if (rc == RNN_E_UNSUPPORTED)
        return rnn_fail(ctx, rc, "conv2d_forward_stats: no specialised kernel for k%u s%u p%u",
                        sp->k, sp->stride, sp->pad);
    return rc;
}

int rnn_conv2d_backward_x_wp(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *dy,
                             const float *w, const float *wp, float *dx) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    int rc = check_spec(ctx, sp);
    if (rc) return rc;
    if (n == 0) return RNN_OK;
    if (!dy || !w || !dx) return rnn_fail(ctx, RNN_E_NULL, "conv2d_backward_x: null operand");
    rc = rnn_conv_fast(ctx, 1, sp, n, dy, w, wp, dx);
    if (rc != RNN_E_UNSUPPORTED) return rc;
    set_lds_limits();
    const int K = sp->k, S = sp->stride, P = sp->pad, KK = K * K;
    for (int py = 0; py < S; py++)
        for (int px = 0; px < S; px++) {
            // dX[iy][ix] with iy = a*S + py gathers dY[a + (py + P - kh)/S] over
            // the kh with (py + P - kh) divisible by S (same for columns).
            Tap taps[MAXT];
            int nt = 0;
            for (int kh = 0; kh < K; kh++) {
                int ry = py + P - kh;
                if (((ry % S) + S) % S) continue;
                for (int kw = 0; kw < K; kw++) {
                    int rx = px + P - kw;
                    if (((rx % S) + S) % S) continue;
                    taps[nt++] = {kh, kw, (ry - ((ry % S) + S) % S) / S, (rx - ((rx % S) + S) % S) / S};
                }
            }
            int GA = ((int)sp->h - py + S - 1) / S, GB = ((int)sp->w - px + S - 1) / S;
            // A = W^T: m = cin (stride KK), ch = cout (stride cin*KK)
            rc = run_tile(ctx, dy, (int)n, sp->cout, sp->oh, sp->ow, dx, sp->cin, sp->h, sp->w, GA,
                          GB, S, py, px, 1, taps, nt, w, KK, sp->cin * KK, K);
            if (rc) return rc;
        }
    return RNN_OK;
}

extern "C" {

int rnn_conv_packed_floats(const rnn_conv_spec *sp, int dx, size_t *floats) {
    if (!sp || !floats) return RNN_E_NULL;
    PackGeo pg;
    const int rc = rnn_conv_pack_geo(sp, dx, &pg);
    *floats = rc ? 0 : pg.floats();
    return rc;
}

int rnn_conv_pack_weights(rnn_ctx *ctx, const rnn_conv_spec *sp, int dx, const float *w,
                          float *wp) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    int rc = check_spec(ctx, sp);
    if (rc) return rc;
    if (!w || !wp) return rnn_fail(ctx, RNN_E_NULL, "conv_pack_weights: null operand");
    rc = rnn_conv_pack(ctx, sp, dx, w, wp);
    if (rc == RNN_E_UNSUPPORTED)
        return rnn_fail(ctx, rc, "conv_pack_weights: no packed form for k %u stride %u pad %u",
                        sp->k, sp->stride, sp->pad);
    return rc;
}

int rnn_conv2d_forward_packed(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *x,
                              const float *w, const float *wp, float *y) {
    if (!wp) return ctx ? rnn_fail(ctx, RNN_E_NULL, "conv2d_forward_packed: null wp") : RNN_E_NULL;
    return rnn_conv2d_forward_wp(ctx, sp, n, x, w, wp, y);
}

int rnn_conv2d_backward_x_packed(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *dy,
                                 const float *w, const float *wp, float *dx) {
    if (!wp)
        return ctx ? rnn_fail(ctx, RNN_E_NULL, "conv2d_backward_x_packed: null wp") : RNN_E_NULL;
    return rnn_conv2d_backward_x_wp(ctx, sp, n, dy, w, wp, dx);
}

int rnn_conv2d_backward_w(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *dy,
                          const float *x, float *dw) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    int rc = check_spec(ctx, sp);
    if (rc) return rc;
    if (n == 0) return RNN_OK;
    if (!dy || !x || !dw) return rnn_fail(ctx, RNN_E_NULL, "conv2d_backward_w: null operand");
    return rnn_conv_dw(ctx, sp, n, dy, x, dw);
}

int rnn_conv2d_backward_w_noalloc(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n,
                                  const float *dy, const float *x, float *dw) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    int rc = check_spec(ctx, sp);
    if (rc) return rc;
    if (n == 0) return RNN_OK;
    if (!dy || !x || !dw)
        return rnn_fail(ctx, RNN_E_NULL, "conv2d_backward_w_noalloc: null operand");
    float *scr = nullptr;
    rc = rnn_noalloc_scratch(ctx, &scr);
    if (rc) return rc;
    return rnn_noalloc_run(ctx, [&] {
        return rnn_conv_dw(ctx, sp, n, dy, x, dw, scr, RNN_NOALLOC_SCRATCH_BYTES / sizeof(float));
    });
}

size_t rnn_conv2d_backward_w_slab_floats(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n) {
    if (!ctx || !sp || n == 0) return 0;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (check_spec(ctx, sp)) return 0;
    return rnn_conv_dw_slab_floats(ctx, sp, n);
}

int rnn_conv2d_backward_w_slabs(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *dy,
                                const float *x, float *slabs, int *nz) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    int rc = check_spec(ctx, sp);
    if (rc) return rc;
    if (n == 0) return rnn_fail(ctx, RNN_E_INVALID, "conv2d_backward_w_slabs: empty batch");
    if (!dy || !x || !slabs)
        return rnn_fail(ctx, RNN_E_NULL, "conv2d_backward_w_slabs: null operand");
    return rnn_conv_dw_slabs(ctx, sp, n, dy, x, slabs, nz);
}

int rnn_dbg_im2col(rnn_ctx *ctx, const rnn_conv_spec *sp, const float *x_img, float *col) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    int rc = check_spec(ctx, sp);
    if (rc) return rc;
    if (!x_img || !col) return RNN_E_NULL;
    long long total = (long long)sp->cin * sp->k * sp->k * sp->oh * sp->ow;
    hipLaunchKernelGGL(im2col_kernel, dim3((unsigned)rnn_div_up(total, 256)), dim3(256), 0,
                       ctx->stream, x_img, col, sp->cin, sp->h, sp->w, sp->k, sp->stride, sp->pad,
                       sp->oh, sp->ow);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

}  // extern "C"
