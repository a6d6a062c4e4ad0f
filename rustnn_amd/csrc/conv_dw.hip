// Convolution weight gradient, deterministic split-K on fp32 MFMA.
//
// dW[co][ci][kh][kw] += sum over (n, oy, ox) of dY[n][co][oy][ox] *
//                       X[n][ci][oy*s + kh - pad][ox*s + kw - pad]
//
// Reference: conv.rs dw_image (277-322) folded per image and reduced over
// rayon workers in Conv2d::backward_w (nn.rs:193-227).  Here GEMM M = co
// (32 per block), N = ci (32 per block) for each tap, K = output pixels.  A
// workgroup owns a (co block, ci block) pair and a strided set of pixel tiles
// (TR output rows of IMGS images).  Per tile it stages the X halo window and
// the dY window in LDS with odd channel strides (lanes index channels, so an
// odd stride keeps every 32-lane b32 read conflict-free), then each wave takes
// whole tile rows: one K step = pixel pair (2q, 2q+1) of a row, lane half h
// carrying pixel 2q+h, one 32x32 accumulator per tap.  The waves' sums are
// added in LDS in wave order and the workgroup writes one partial slab; slabs
// are added in slab order by a two-level reduction (no atomics: the result is
// bit-reproducible).
#include "conv_common.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>

namespace {

struct DwArgs {
    const float *dy;  // [N][CO][OH][OW]
    const float *x;   // [N][CI][H][W]
    float *part;      // [nz][CO][CI*KK]
    int N, CO, CI, H, W, OH, OW;
    int IS, pad;
    int TR, GBP, tiles_a, ntiles, nz;
    int xlrow, xlcol;  // X-window rows / columns per output row / column step
    int xregion;       // LDS words of the X window region (64-word rows)
    int stage;         // LDS words of one stage buffer (X window + dY window)
    TileGeo xg, dg;    // X window [32 ci][IMGS][TIH][TIWP]; dY window [32 co][IMGS][TR][GBP]
    int tapoff[9];
};

template <int K>
__global__ __launch_bounds__(256, 2) void conv_dw_kernel(DwArgs g) {
    constexpr int KK = K * K;
    extern __shared__ float smem[];
    const int nthreads = blockDim.x, nw = nthreads >> 6;
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_index(), h = lane >> 5, l32 = lane & 31;
    const int z = blockIdx.x, cob = blockIdx.y, cib = blockIdx.z;
    const int rows = g.xg.IMGS * g.TR;
    const int npairs = g.GBP >> 1;
    const long long ximg = (long long)g.CI * g.H * g.W, dyimg = (long long)g.CO * g.OH * g.OW;

    f32x16 acc[KK];
#pragma unroll
    for (int t = 0; t < KK; t++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[t][v] = 0.f;

    const int abase = l32 * g.dg.chs + h;
    const int bbase = l32 * g.xg.chs + h * g.xlcol;

    // Stage = one pixel tile (X window + dY window) in one of two LDS buffers;
    // the next tile is staged while the current one is computed.
    auto issue = [&](int tile, float *buf) {
        const int ta = tile % g.tiles_a, tn = tile / g.tiles_a;
        const int a0 = ta * g.TR, n0 = tn * g.xg.IMGS;
        const int nimg = min(g.N - n0, g.xg.IMGS);
        const __amdgpu_buffer_rsrc_t rs_x =
            make_rsrc(g.x + (long long)n0 * ximg, (uint32_t)(nimg * ximg * 4));
        const __amdgpu_buffer_rsrc_t rs_dy =
            make_rsrc(g.dy + (long long)n0 * dyimg, (uint32_t)(nimg * dyimg * 4));
        dma_tile(rs_x, g.N, g.CI, g.H, g.W, n0, cib * 32, 32, a0 * g.IS - g.pad, -g.pad, g.xg, buf,
                 wave, nw, lane);
        dma_tile(rs_dy, g.N, g.CO, g.OH, g.OW, n0, cob * 32, 32, a0, 0, g.dg, buf + g.xregion,
                 wave, nw, lane);
    };

    int s = 0;
    if (z < g.ntiles) issue(z, smem);
    for (int tile = z; tile < g.ntiles; tile += g.nz, s++) {
        dma_wait_barrier();
        const float *xs = smem + (s & 1) * g.stage;
        const float *dys = xs + g.xregion;
        if (tile + g.nz < g.ntiles) issue(tile + g.nz, smem + ((s + 1) & 1) * g.stage);
        for (int row = wave; row < rows; row += nw) {
            const int img = row / g.TR, r = row - img * g.TR;
            const float *arow = dys + abase + img * g.dg.imgs + r * g.GBP;
            const float *xrow = xs + bbase + img * g.xg.imgs + r * g.xlrow * g.xg.TIWP;
            // operands of pixel pair q+1 are fetched while pair q's MFMAs run
            float av[2], bv[2][KK];
            auto fetch = [&](int q, int slot) {
                av[slot] = arow[2 * q];
                const float *xb = xrow + 2 * q * g.xlcol;
                static_for<0, KK>([&](auto tc) {
                    constexpr int t = decltype(tc)::value;
                    bv[slot][t] = xb[g.tapoff[t]];
                });
            };
            auto mma = [&](int slot) {
                static_for<0, KK>([&](auto tc) {
                    constexpr int t = decltype(tc)::value;
                    acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[slot], bv[slot][t], acc[t], 0,
                                                                  0, 0);
                });
            };
            fetch(0, 0);
            int q = 0;
            for (; q + 2 <= npairs; q += 2) {
                fetch(q + 1, 1);
                mma(0);
                if (q + 2 < npairs) fetch(q + 2, 0);
                mma(1);
            }
            if (q < npairs) mma(0);
        }
    }
    // Sum the waves in wave order through LDS, then write the slab.
    dma_wait_barrier();
    float *red = smem;  // KK*1024 floats
    for (int w = 0; w < nw; w++) {
        if (wave == w) {
#pragma unroll
            for (int t = 0; t < KK; t++)
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int i = 8 * (v >> 2) + 4 * h + (v & 3);  // co
                    const int e = t * 1024 + i * 32 + l32;          // l32 = ci
                    red[e] = (w == 0) ? acc[t][v] : red[e] + acc[t][v];
                }
        }
        __syncthreads();
    }
    const int ckk = g.CI * KK;
    float *slab = g.part + (long long)z * g.CO * ckk;
    for (int e = tid; e < KK * 1024; e += nthreads) {
        const int t = e >> 10, i = (e >> 5) & 31, c = e & 31;
        const int co = cob * 32 + i, ci = cib * 32 + c;
        if (co < g.CO && ci < g.CI) slab[(long long)co * ckk + ci * KK + t] = red[e];
    }
}

// tmp[gz][e] = sum of slabs [gz*G, min(nz, gz*G + G)) in slab order.
__global__ void slab_sum_kernel(const float *part, int nz, int G, long long len, float *tmp) {
    const long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const int gz = blockIdx.y;
    if (e >= len) return;
    const int z0 = gz * G, z1 = min(nz, z0 + G);
    float s = part[(long long)z0 * len + e];
    for (int z = z0 + 1; z < z1; z++) s += part[(long long)z * len + e];
    tmp[(long long)gz * len + e] = s;
}

// out[e] += sum_g tmp[g][e] in order.
__global__ void slab_final_kernel(const float *tmp, int ng, long long len, float *out) {
    const long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= len) return;
    float s = tmp[e];
    for (int gz = 1; gz < ng; gz++) s += tmp[(long long)gz * len + e];
    out[e] += s;
}

template <int K>
void dw_attr() {
    (void)hipFuncSetAttribute((const void *)conv_dw_kernel<K>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
}

// Geometry for (TR, IMGS); returns LDS bytes.
size_t dw_geometry(DwArgs &g, int K, int TR, int IMGS) {
    const int S = g.IS;
    const int step = (K == 1) ? S : 1;
    g.TR = TR;
    TileGeo &x = g.xg;
    x.IMGS = IMGS;
    x.rowstep = step;
    x.colstep = step;
    g.xlrow = S / step;
    x.TIH = (TR - 1) * g.xlrow + K;
    x.TIW = (g.GBP - 1) * (S / step) + K;
    x.deint = (S / step) == 2;
    x.HALF = (x.TIW + 1) / 2;
    x.TIWP = x.deint ? 2 * x.HALF : x.TIW;
    g.xlcol = x.deint ? 1 : S / step;
    x.imgs = x.TIH * x.TIWP;
    x.chs = IMGS * x.imgs;
    x.chs += (x.chs & 1) ? 0 : 1;
    tilegeo_finish(x);
    TileGeo &d = g.dg;
    d.IMGS = IMGS;
    d.rowstep = 1;
    d.colstep = 1;
    d.TIH = TR;
    d.TIW = g.GBP;
    d.deint = 0;
    d.HALF = 0;
    d.TIWP = g.GBP;
    d.imgs = TR * g.GBP;
    d.chs = IMGS * d.imgs;
    d.chs += (d.chs & 1) ? 0 : 1;
    tilegeo_finish(d);
    for (int t = 0; t < 9; t++) {
        g.tapoff[t] = 0;
        if (t < K * K) {
            const int kh = t / K, kw = t % K;
            g.tapoff[t] = kh * x.TIWP + (x.deint ? (kw & 1) * x.HALF + (kw >> 1) : kw);
        }
    }
    const size_t xsf = dma_region((size_t)32 * x.chs), dsf = dma_region((size_t)32 * d.chs);
    g.xregion = (int)xsf;
    g.stage = (int)(xsf + dsf);
    return std::max(2 * (xsf + dsf) * 4, (size_t)K * K * 1024 * 4);  // double-buffered
}

}  // namespace

// dW += sum over images (see above).  k must be 1 or 3.
int rnn_conv_dw(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *dy, const float *x,
                float *dw) {
    const int K = sp->k;
    if (K != 1 && K != 3) return rnn_fail(ctx, RNN_E_UNSUPPORTED, "conv dW: k must be 1 or 3");
    static bool attr = false;
    if (!attr) {
        attr = true;
        dw_attr<1>();
        dw_attr<3>();
    }
    DwArgs g;
    std::memset(&g, 0, sizeof(g));
    g.dy = dy;
    g.x = x;
    g.N = (int)n;
    g.CO = sp->cout;
    g.CI = sp->cin;
    g.H = sp->h;
    g.W = sp->w;
    g.OH = sp->oh;
    g.OW = sp->ow;
    g.IS = sp->stride;
    g.pad = sp->pad;
    g.GBP = (sp->ow + 1) & ~1;
    if (g.GBP > 512) return rnn_fail(ctx, RNN_E_UNSUPPORTED, "conv dW: output row too wide");
    int TR = 0, IMGS = 0, NZ = 0;
    if (const char *env = getenv("RNN_DW_PLAN"))
        if (sscanf(env, "%d,%d,%d", &TR, &IMGS, &NZ) != 3) TR = IMGS = NZ = 0;
    size_t lds = 0;
    if (TR > 0 && IMGS > 0) {
        TR = std::min(TR, g.OH);
        lds = dw_geometry(g, K, TR, IMGS);
        if (lds > 160 * 1024) TR = 0;
    }
    if (TR <= 0 || IMGS <= 0) {
        const int target = 256;
        if (g.OH * g.GBP <= target) {
            TR = g.OH;
            IMGS = std::max(1, target / (g.OH * g.GBP));
        } else {
            TR = std::max(1, target / g.GBP);
            IMGS = 1;
        }
        const int TR0 = TR, IMGS0 = IMGS;
        bool ok = false;
        for (size_t budget : {(size_t)80 * 1024, (size_t)160 * 1024}) {
            TR = TR0;
            IMGS = IMGS0;
            for (;;) {
                lds = dw_geometry(g, K, TR, IMGS);
                if (lds <= budget) {
                    ok = true;
                    break;
                }
                if (IMGS > 1)
                    IMGS /= 2;
                else if (TR > 1)
                    TR = (TR + 1) / 2;
                else
                    break;
            }
            if (ok) break;
        }
        if (!ok) return rnn_fail(ctx, RNN_E_UNSUPPORTED, "conv dW: tile exceeds LDS");
    }
    if ((long long)IMGS * std::max((long long)g.CI * g.H * g.W, (long long)g.CO * g.OH * g.OW) * 4 >=
        0x7FFFFFF0ll)
        return rnn_fail(ctx, RNN_E_UNSUPPORTED, "conv dW: tile source beyond 2 GiB");
    g.tiles_a = (g.OH + g.TR - 1) / g.TR;
    g.ntiles = g.tiles_a * (int)((n + IMGS - 1) / IMGS);
    const int ncb = (g.CO + 31) / 32, ncib = (g.CI + 31) / 32;
    if (NZ <= 0) {
        // persistent: as many workgroups as fit on the chip at once
        int occ = 0;
        const void *kern = K == 3 ? (const void *)conv_dw_kernel<3> : (const void *)conv_dw_kernel<1>;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, 256, lds) != hipSuccess ||
            occ < 1)
            occ = 1;
        NZ = std::max(1, occ * ctx->num_cus / (ncb * ncib));
    }
    NZ = std::min(NZ, g.ntiles);
    g.nz = NZ;
    const size_t ckk = (size_t)g.CI * K * K, len = (size_t)g.CO * ckk;
    const int G = 16, ng = (NZ + G - 1) / G;
    float *ws = (float *)rnn_workspace(ctx, ((size_t)NZ + (ng > 1 ? ng : 0)) * len * sizeof(float));
    if (!ws) return RNN_E_NOMEM;
    g.part = ws;
    dim3 grid(NZ, ncb, ncib), block(256);
    if (K == 3)
        hipLaunchKernelGGL(conv_dw_kernel<3>, grid, block, lds, ctx->stream, g);
    else
        hipLaunchKernelGGL(conv_dw_kernel<1>, grid, block, lds, ctx->stream, g);
    RNN_LAUNCHED(ctx);
    const unsigned eb = (unsigned)rnn_div_up(len, 256);
    if (ng > 1) {
        float *tmp = ws + (size_t)NZ * len;
        hipLaunchKernelGGL(slab_sum_kernel, dim3(eb, ng), dim3(256), 0, ctx->stream, ws, NZ, G,
                           (long long)len, tmp);
        RNN_LAUNCHED(ctx);
        hipLaunchKernelGGL(slab_final_kernel, dim3(eb), dim3(256), 0, ctx->stream, tmp, ng,
                           (long long)len, dw);
    } else {
        hipLaunchKernelGGL(slab_final_kernel, dim3(eb), dim3(256), 0, ctx->stream, ws, NZ,
                           (long long)len, dw);
    }
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}
