// Specialised implicit-GEMM forward / dX convolution for the (k, stride, pad)
// pairs rustnn uses: 3x3/s1/p1, 3x3/s2/p1, 1x1/s2/p0 (and 1x1/s1/p0).
//
// One launch per call.  A workgroup owns a tile of output positions (TR rows
// of IMGS images, full width) for MB blocks of 32 output channels.  Per chunk
// of CH source channels it stages
//   * the zero-padded source window in LDS (x for forward, dY for dX), and
//   * the weight slab in MFMA fragment order ws[mb][cp][tap][lane],
// then runs v_mfma_f32_32x32x2f32 over K = (channel pair, tap): lane half h
// carries channel cp + h*CH/2, so one per-tap LDS offset serves the whole
// wave.  For dX with stride s the workgroup computes all s*s parity classes
// of its block positions from the same dY window, each tap feeding exactly
// one class accumulator (gather-form col2im: no atomics, each dX element
// written once).
//
// Reference: conv.rs forward_image (168-203), dx_image (205-246) and the
// Conv2d batch drivers (nn.rs:166-250).
#include "conv_common.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>

namespace {

struct FastArgs {
    const float *src;  // [N][CS][HS][WS]
    const float *w;    // [cout][cin][k][k]
    const float *wf;   // weights in fragment order [mblk][chunk][cp][tap][64]
    float *dst;        // [N][CD][HD][WD]
    int xregion;       // LDS words of the source window region (64-word rows)
    int N, CS, HS, WS;
    int CD, HD, WD;
    int GA, GB;        // output block grid per image
    int TR, tiles_a, ntiles, ngroups;
    int stage;         // LDS words of one stage buffer (window + MB weight slabs)
    int CH, nchunks;
    int sm, sc;        // weight strides of output row m and source channel ch
    int dymin, dxmin;  // smallest tap offsets (tile origin)
    int lrow, lcol;    // LDS rows / columns per output row / column step
    TileGeo geo;
    int tapoff[9];
};

// Weights in MFMA fragment order: wf[mblk][chunk][cp][tap][lane], lane l ->
// row m = mblk*32 + l%32, channel ch = chunk*CH + cp + (l/32)*CH/2; element
// w[m*sm + ch*sc + tap], 0 outside [0, M) x [0, C).  One small kernel per call;
// every workgroup then stages its slab with one contiguous DMA.
__global__ void prep_fragments_kernel(const float *__restrict__ w, float *__restrict__ wf, int M,
                                      int C, int CH, int nchunks, int nmblk, int KK, int sm,
                                      int sc) {
    const int CP = CH >> 1;
    const long long total = (long long)nmblk * nchunks * CP * KK * 64;
    const long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= total) return;
    const int lane = (int)(e & 63);
    long long r = e >> 6;
    const int t = (int)(r % KK);
    r /= KK;
    const int cp = (int)(r % CP);
    r /= CP;
    const int chunk = (int)(r % nchunks), mblk = (int)(r / nchunks);
    const int m = mblk * 32 + (lane & 31), ch = chunk * CH + cp + (lane >> 5) * CP;
    float v = 0.f;
    if (m < M && ch < C) v = w[(long long)m * sm + (long long)ch * sc + t];
    wf[e] = v;
}

template <int K, int S, int P, bool DX, int NPW, int MB>
__global__ __launch_bounds__(256) void conv_fast_kernel(FastArgs g) {
    using T = ConvTaps<K, S, P, DX>;
    constexpr int KK = T::KK, NCLS = T::NCLS;
    extern __shared__ float smem[];
    const int nthreads = blockDim.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nw = nthreads >> 6, h = lane >> 5, l32 = lane & 31;
    const int CP = g.CH >> 1, chs = g.geo.chs;
    const int wchunk = CP * KK * 64;
    const int nmblk = (g.CD + 31) / 32;
    const int tpix = g.TR * g.GB, npix = g.geo.IMGS * tpix;
    const int nitems = g.ntiles * g.ngroups;
    const long long img_elems = (long long)g.CS * g.HS * g.WS;
    const __amdgpu_buffer_rsrc_t rs_w =
        make_rsrc(g.wf, (uint32_t)((long long)nmblk * g.nchunks * wchunk * 4));

    // Per-lane LDS base of each position group (channel half h included);
    // tile-relative, so the same for every work item.
    int vb[NPW];
#pragma unroll
    for (int j = 0; j < NPW; j++) {
        int p = (wave * NPW + j) * 32 + l32;
        if (p >= npix) p = 0;
        const int img = p / tpix, rem = p - img * tpix, r = rem / g.GB, c = rem - r * g.GB;
        vb[j] = h * CP * chs + img * g.geo.imgs + r * g.lrow * g.geo.TIWP + c * g.lcol;
    }

    // Stage = (work item, channel chunk); a work item = (tile, group of MB
    // output-channel blocks).  Stage data lives in one of two LDS buffers.
    auto issue = [&](int item, int chunk, float *buf) {
        const int tile = item % g.ntiles, grp = item / g.ntiles;
        const int ta = tile % g.tiles_a, tn = tile / g.tiles_a;
        const int a0 = ta * g.TR, n0 = tn * g.geo.IMGS;
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(
            g.src + (long long)n0 * img_elems, (uint32_t)(min(g.N - n0, g.geo.IMGS) * img_elems * 4));
        dma_tile(rs, g.N, g.CS, g.HS, g.WS, n0, chunk * g.CH, g.CH, a0 * T::IS + g.dymin, g.dxmin,
                 g.geo, buf, wave, nw, lane);
#pragma unroll
        for (int mb = 0; mb < MB; mb++) {
            const int mblk = min(grp * MB + mb, nmblk - 1);
            dma_copy(rs_w, (uint32_t)(((long long)mblk * g.nchunks + chunk) * wchunk * 4),
                     buf + g.xregion + mb * wchunk, wchunk, wave, nw, lane);
        }
    };

    f32x16 acc[NCLS][MB][NPW];
    int s = 0;
    if ((int)blockIdx.x < nitems) issue(blockIdx.x, 0, smem);
    for (int item = blockIdx.x; item < nitems; item += gridDim.x) {
#pragma unroll
        for (int c = 0; c < NCLS; c++)
#pragma unroll
            for (int mb = 0; mb < MB; mb++)
#pragma unroll
                for (int j = 0; j < NPW; j++)
#pragma unroll
                    for (int v = 0; v < 16; v++) acc[c][mb][j][v] = 0.f;
        for (int chunk = 0; chunk < g.nchunks; chunk++, s++) {
            // Stage s has landed and every wave is done with stage s-1, whose
            // buffer now receives stage s+1 while stage s is computed.
            dma_wait_barrier();
            float *cur = smem + (s & 1) * g.stage;
            if (chunk + 1 < g.nchunks)
                issue(item, chunk + 1, smem + ((s + 1) & 1) * g.stage);
            else if (item + (int)gridDim.x < nitems)
                issue(item + gridDim.x, 0, smem + ((s + 1) & 1) * g.stage);
            const float *xs = cur, *ws = cur + g.xregion;
            // Operands of channel pair cp+1 are fetched from LDS while the
            // MFMAs of cp run (register double buffer), so no MFMA waits on a
            // just-issued LDS read.
            float av[2][KK][MB], bv[2][KK][NPW];
            auto fetch = [&](int cp, int slot) {
                const float *xc = xs + cp * chs;
                const float *wl = ws + cp * KK * 64 + lane;
                static_for<0, KK>([&](auto tc) {
                    constexpr int t = decltype(tc)::value;
#pragma unroll
                    for (int mb = 0; mb < MB; mb++) av[slot][t][mb] = wl[mb * wchunk + t * 64];
#pragma unroll
                    for (int j = 0; j < NPW; j++) bv[slot][t][j] = xc[vb[j] + g.tapoff[t]];
                });
            };
            auto mma = [&](int slot) {
                static_for<0, KK>([&](auto tc) {
                    constexpr int t = decltype(tc)::value;
                    constexpr int c = T::cls(t);
#pragma unroll
                    for (int mb = 0; mb < MB; mb++)
#pragma unroll
                        for (int j = 0; j < NPW; j++)
                            acc[c][mb][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                                av[slot][t][mb], bv[slot][t][j], acc[c][mb][j], 0, 0, 0);
                });
            };
            fetch(0, 0);
            int cp = 0;
            for (; cp + 2 <= CP; cp += 2) {
                fetch(cp + 1, 1);
                mma(0);
                if (cp + 2 < CP) fetch(cp + 2, 0);
                mma(1);
            }
            if (cp < CP) mma(0);
        }
        // acc row 8*(v/4) + 4*h + v%4 = output channel in the block, column = position.
        const int tile = item % g.ntiles, grp = item / g.ntiles;
        const int a0 = (tile % g.tiles_a) * g.TR, n0 = (tile / g.tiles_a) * g.geo.IMGS;
#pragma unroll
        for (int j = 0; j < NPW; j++) {
            const int p = (wave * NPW + j) * 32 + l32;
            if (p >= npix) continue;
            const int img = p / tpix, rem = p - img * tpix, r = rem / g.GB, cb = rem - r * g.GB;
            const int n = n0 + img, a = a0 + r;
            if (n >= g.N || a >= g.GA) continue;
#pragma unroll
            for (int c = 0; c < NCLS; c++) {
                const int y = a * T::OS + (DX ? c / S : 0), x = cb * T::OS + (DX ? c % S : 0);
                if (y >= g.HD || x >= g.WD) continue;
                float *dp = g.dst + ((long long)n * g.CD * g.HD + y) * g.WD + x;
                const long long cst = (long long)g.HD * g.WD;
#pragma unroll
                for (int mb = 0; mb < MB; mb++) {
#pragma unroll
                    for (int v = 0; v < 16; v++) {
                        const int m = (grp * MB + mb) * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                        if (m < g.CD) dp[m * cst] = acc[c][mb][j][v];
                    }
                }
            }
        }
    }
}

struct FastPlan {
    int TR, IMGS, CH, NPW, MB;
    int wpc;  // cap on resident workgroups per CU (0 = occupancy limit)
    size_t lds;
};

// LDS bytes of a plan and the tile geometry it implies.
template <int K, int S, int P, bool DX>
static size_t plan_geometry(const FastPlan &p, int GB, int CS, FastArgs &a) {
    using T = ConvTaps<K, S, P, DX>;
    int dymin = 1 << 20, dymax = -(1 << 20), dxmin = 1 << 20, dxmax = -(1 << 20);
    for (int t = 0; t < T::KK; t++) {
        dymin = std::min(dymin, T::dy(t));
        dymax = std::max(dymax, T::dy(t));
        dxmin = std::min(dxmin, T::dx(t));
        dxmax = std::max(dxmax, T::dx(t));
    }
    const int IS = T::IS;
    const int step = (T::KK == 1) ? IS : 1;  // 1x1: only every IS-th source row/column
    TileGeo &t = a.geo;
    t.IMGS = p.IMGS;
    t.rowstep = step;
    t.colstep = step;
    a.lrow = IS / step;
    t.TIH = (p.TR - 1) * a.lrow + (dymax - dymin) + 1;
    t.TIW = (GB - 1) * (IS / step) + (dxmax - dxmin) + 1;
    t.deint = (IS / step) == 2;
    t.HALF = (t.TIW + 1) / 2;
    t.TIWP = t.deint ? 2 * t.HALF : t.TIW;
    a.lcol = t.deint ? 1 : IS / step;
    t.imgs = t.TIH * t.TIWP;
    t.chs = p.IMGS * t.imgs;
    tilegeo_finish(t);
    a.dymin = dymin;
    a.dxmin = dxmin;
    for (int i = 0; i < 9; i++) {
        a.tapoff[i] = 0;
        if (i < T::KK) {
            int dyp = T::dy(i) - dymin, dxp = T::dx(i) - dxmin;
            a.tapoff[i] = dyp * t.TIWP + (t.deint ? (dxp & 1) * t.HALF + (dxp >> 1) : dxp);
        }
    }
    size_t xsf = dma_region((size_t)p.CH * t.chs);
    size_t wsf = (size_t)p.MB * (p.CH / 2) * T::KK * 64;
    a.xregion = (int)xsf;
    a.stage = (int)(xsf + wsf);
    (void)CS;
    return 2 * (xsf + wsf) * 4;  // double-buffered stages
}

// Tile choice: RNN_CONV_PLAN="TR,IMGS,CH,NPW,MB[,WPC]" overrides (tuning
// sweeps); otherwise up to 256 positions per workgroup, whole images first,
// within 80 KB of LDS (two workgroups per CU) when possible.
template <int K, int S, int P, bool DX>
static bool choose_plan(int CS, int CD, int GA, int GB, FastPlan &best, FastArgs &a) {
    const int CSe = (CS + 1) & ~1;
    if (const char *env = getenv("RNN_CONV_PLAN")) {
        FastPlan p{};
        if (sscanf(env, "%d,%d,%d,%d,%d,%d", &p.TR, &p.IMGS, &p.CH, &p.NPW, &p.MB, &p.wpc) >= 5 &&
            p.TR > 0 &&
            p.IMGS > 0 && p.CH >= 2 && p.CH % 2 == 0 && (p.NPW == 1 || p.NPW == 2) &&
            (p.MB == 1 || p.MB == 2)) {
            p.CH = std::min(p.CH, CSe);
            p.TR = std::min(p.TR, GA);
            p.lds = plan_geometry<K, S, P, DX>(p, GB, CS, a);
            if (p.lds <= 160 * 1024 && p.IMGS * p.TR * GB <= 4 * p.NPW * 32) {
                best = p;
                return true;
            }
        }
    }
    if (GB > 256) return false;
    const int mbs[2] = {1, 2};
    for (size_t budget : {(size_t)80 * 1024, (size_t)160 * 1024}) {
        for (int npw : {2, 1}) {
            for (int mb : mbs) {
                if (mb == 2 && CD <= 32) continue;
                // stride-2 dX keeps 4 class accumulators per (mb, group)
                if (ConvTaps<K, S, P, DX>::NCLS * npw * mb > 4) continue;
                const int target = 4 * npw * 32;
                for (int ch : {32, 16, 8, 4, 2}) {
                    if (ch > CSe && ch != std::min(32, CSe)) continue;
                    FastPlan p{};
                    p.CH = std::min(ch, CSe);
                    p.NPW = npw;
                    p.MB = mb;
                    if (GA * GB <= target) {
                        p.TR = GA;
                        p.IMGS = std::max(1, target / (GA * GB));
                    } else {
                        p.TR = std::max(1, std::min(GA, target / GB));
                        p.IMGS = 1;
                    }
                    for (;;) {
                        p.lds = plan_geometry<K, S, P, DX>(p, GB, CS, a);
                        if (p.lds <= budget) {
                            best = p;
                            plan_geometry<K, S, P, DX>(p, GB, CS, a);
                            return true;
                        }
                        if (p.IMGS > 1)
                            p.IMGS /= 2;
                        else if (p.TR > 1)
                            p.TR = (p.TR + 1) / 2;
                        else
                            break;
                    }
                }
            }
        }
    }
    return false;
}

template <int K, int S, int P, bool DX, int NPW, int MB>
static void set_attr() {
    (void)hipFuncSetAttribute((const void *)conv_fast_kernel<K, S, P, DX, NPW, MB>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
}

template <int K, int S, int P, bool DX>
static int launch(rnn_ctx *ctx, const rnn_conv_spec *sp, int n, const float *src, const float *w,
                  float *dst) {
    using T = ConvTaps<K, S, P, DX>;
    static bool attr = false;
    if (!attr) {
        attr = true;
        set_attr<K, S, P, DX, 1, 1>();
        set_attr<K, S, P, DX, 2, 1>();
        set_attr<K, S, P, DX, 1, 2>();
        set_attr<K, S, P, DX, 2, 2>();
    }
    FastArgs a;
    std::memset(&a, 0, sizeof(a));
    a.src = src;
    a.w = w;
    a.dst = dst;
    a.N = n;
    const int cin = sp->cin, cout = sp->cout;
    if (!DX) {
        a.CS = cin;
        a.HS = sp->h;
        a.WS = sp->w;
        a.CD = cout;
        a.HD = sp->oh;
        a.WD = sp->ow;
        a.GA = sp->oh;
        a.GB = sp->ow;
        a.sm = cin * T::KK;  // W[m = cout][ch = cin][tap]
        a.sc = T::KK;
    } else {
        a.CS = cout;
        a.HS = sp->oh;
        a.WS = sp->ow;
        a.CD = cin;
        a.HD = sp->h;
        a.WD = sp->w;
        a.GA = (sp->h + S - 1) / S;
        a.GB = (sp->w + S - 1) / S;
        a.sm = T::KK;  // W^T: m = cin, ch = cout
        a.sc = cin * T::KK;
    }
    FastPlan p;
    if (!choose_plan<K, S, P, DX>(a.CS, a.CD, a.GA, a.GB, p, a))
        return rnn_fail(ctx, RNN_E_UNSUPPORTED, "conv: no LDS tiling for a %dx%d grid", a.GA, a.GB);
    a.TR = p.TR;
    a.tiles_a = (a.GA + p.TR - 1) / p.TR;
    a.CH = p.CH;
    a.nchunks = (a.CS + p.CH - 1) / p.CH;
    const int nmblk_all = (a.CD + 31) / 32;
    const size_t wf_len = (size_t)nmblk_all * a.nchunks * (p.CH / 2) * T::KK * 64;
    if ((long long)p.IMGS * a.CS * a.HS * a.WS * 4 >= 0x7FFFFFF0ll || wf_len * 4 >= (1ull << 31))
        return rnn_fail(ctx, RNN_E_UNSUPPORTED, "conv: tile source or weights beyond 2 GiB");
    float *wf = (float *)rnn_workspace(ctx, wf_len * sizeof(float));
    if (!wf) return RNN_E_NOMEM;
    a.wf = wf;
    hipLaunchKernelGGL(prep_fragments_kernel, dim3((unsigned)rnn_div_up(wf_len, 256)), dim3(256), 0,
                       ctx->stream, w, wf, a.CD, a.CS, p.CH, a.nchunks, nmblk_all, T::KK, a.sm,
                       a.sc);
    RNN_LAUNCHED(ctx);
    const int nw = std::max(1, std::min(4, (p.IMGS * p.TR * a.GB + 32 * p.NPW - 1) / (32 * p.NPW)));
    const int nmblk = (a.CD + 31) / 32;
    a.ntiles = a.tiles_a * ((n + p.IMGS - 1) / p.IMGS);
    a.ngroups = (nmblk + p.MB - 1) / p.MB;
    const long long nitems = (long long)a.ntiles * a.ngroups;
    if (nitems > 0x7fffffffll) return rnn_fail(ctx, RNN_E_UNSUPPORTED, "conv: too many tiles");
    // Persistent grid: as many workgroups as fit on the chip at once.
    auto run = [&](auto kern) -> int {
        int occ = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, 64 * nw, p.lds) != hipSuccess ||
            occ < 1)
            occ = 1;
        if (p.wpc > 0) occ = std::min(occ, p.wpc);
        const long long grid = std::min<long long>(nitems, (long long)ctx->num_cus * occ);
        hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * nw), p.lds, ctx->stream, a);
        RNN_LAUNCHED(ctx);
        return RNN_OK;
    };
    if (p.NPW == 2 && p.MB == 1) return run(conv_fast_kernel<K, S, P, DX, 2, 1>);
    if (p.NPW == 1 && p.MB == 1) return run(conv_fast_kernel<K, S, P, DX, 1, 1>);
    if (p.NPW == 2 && p.MB == 2) return run(conv_fast_kernel<K, S, P, DX, 2, 2>);
    return run(conv_fast_kernel<K, S, P, DX, 1, 2>);
}

}  // namespace

// Forward (dx = 0) or dX (dx = 1) through the specialised kernels; returns
// RNN_E_UNSUPPORTED (without recording an error) when (k, stride, pad) has no
// specialisation, so the caller can take the generic per-class path.
int rnn_conv_fast(rnn_ctx *ctx, int dx, const rnn_conv_spec *sp, size_t n, const float *src,
                  const float *w, float *dst) {
    if (getenv("RNN_CONV_GENERIC")) return RNN_E_UNSUPPORTED;
    const int k = sp->k, s = sp->stride, p = sp->pad;
    const int ni = (int)n;
#define RNN_CONV_CASE(K_, S_, P_)                                                               \
    if (k == K_ && s == S_ && p == P_)                                                          \
        return dx ? launch<K_, S_, P_, true>(ctx, sp, ni, src, w, dst)                          \
                  : launch<K_, S_, P_, false>(ctx, sp, ni, src, w, dst);
    RNN_CONV_CASE(3, 1, 1)
    RNN_CONV_CASE(3, 2, 1)
    RNN_CONV_CASE(1, 2, 0)
    RNN_CONV_CASE(1, 1, 0)
#undef RNN_CONV_CASE
    return RNN_E_UNSUPPORTED;
}
