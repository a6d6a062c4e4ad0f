// Specialised implicit-GEMM forward / dX convolution for the (k, stride, pad)
// pairs rustnn uses: 3x3/s1/p1, 3x3/s2/p1, 1x1/s2/p0 (and 1x1/s1/p0).
//
// Persistent workgroups walk a list of work items -- (tile of output
// positions, group of MB blocks of 32 output channels) -- and, per item, the
// source channels in chunks of CH.  Each (item, chunk) stage is staged into
// one of two LDS buffers by DMA (buffer_load ... lds, no registers) while the
// previous stage is computed:
//   * the zero-padded source window (x for forward, dY for dX), stored
//     [channel quad][position][4]: the 4 channels of a quad are adjacent, so
//     one ds_read_b128 gives a lane the B operand of 4 MFMA k-steps;
//   * the weight slab, gathered straight from W into MFMA fragment order
//     [mb][quad][tap][lane][4] (one ds_read_b128 per 4 k-steps for A).
// MFMA mapping (v_mfma_f32_32x32x2f32): M = output channels, N = output
// positions (32 per group), K = (channel, tap) with lane half h carrying
// channel h*CH/2 + 4q + i, so one per-tap offset serves all 64 lanes.  The
// operands of the next (quad, tap) step are read while the MFMAs of the
// current one run.
//
// For dX with stride s the workgroup computes all s*s parity classes of its
// block positions from the same dY window, each tap feeding exactly one class
// accumulator (gather-form col2im: no atomics, every dX element written once).
//
// Reference: conv.rs forward_image (168-203), dx_image (205-246) and the
// Conv2d batch drivers (nn.rs:166-250).
#include "conv_common.h"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>

namespace {

constexpr int FAST_NW = 4;  // waves per workgroup

// Window DMA rows of 16 positions that one wave stages per channel quad:
// row u of wave w covers window positions (w + 4u)*16 .. +16.  Row u is issued
// at tap u % KK of a step, so its per-lane source offsets sit in a register
// table indexed at compile time.
template <int KK>
struct WinRows {
    static constexpr int MAX = KK == 1 ? 4 : KK;
};

struct FastArgs {
    const float *src;  // [N][CS][HS][WS]
    const float *w;    // [cout][cin][k][k]
    const float *wp;   // the same weights packed in slab order (conv_pack), or null
    int wpbytes;       // bytes of wp
    float *dst;        // [N][CD][HD][WD]
    int N, CS, HS, WS;
    int CD, HD, WD;
    int GA, GB;        // output block grid per image
    int TR, tiles_a, ntiles, ngroups;
    int CH, nchunks;   // source channels per stage (multiple of 8)
    int sm, sc;        // weight strides of output row m and source channel ch
    int wbytes;        // bytes of W
    int dymin, dxmin;  // smallest tap offsets (window origin)
    int lrow, lcol;    // window rows / columns per output row / column step
    int plane;         // window positions per channel quad (multiple of 64)
    int ppw;           // plane / 64: window rows per quad and wave
    int xwords;        // LDS words of the window: CH * plane
    int stage;         // LDS words of one stage: window, then weight slabs
    TileGeo geo;       // window geometry in positions (chs unused)
    int tapoff[9];     // window-position offset of each tap
    uint32_t m_imgs, m_tiwp;  // FastDiv multipliers of geo.imgs and geo.TIWP
    int npart;         // store-pass statistics: partials per channel (= ntiles)
    ConvStats stats;   // store-pass statistics (forward with EPI = 1)
};

// Wave-uniform description of the stage being staged by DMA.
struct StageDMA {
    __amdgpu_buffer_rsrc_t rs;  // source images n0 .. n0 + IMGS
    float *buf;                 // stage buffer
    int c0, grp;                // first source channel, output-channel group
    int ebase;                  // element offset of window row 0 in image n0 (may be < 0)
    int ylo, yhi;               // window rows inside the source image
    int nimg;                   // images of the tile inside the batch
    int mlim;                   // output rows of the group inside [0, CD)
};

template <int K, int S, int P, bool DX, int SL>
__device__ __forceinline__ StageDMA stage_dma(const FastArgs &g, int item, int chunk,
                                              float *buf) {
    using T = ConvTaps<K, S, P, DX>;
    StageDMA d;
    const int tile = item % g.ntiles;
    d.grp = item / g.ntiles;
    const int n0 = (tile / g.tiles_a) * g.geo.IMGS;
    const int y0 = (tile % g.tiles_a) * g.TR * T::IS + g.dymin;
    const int rowstep = g.geo.rowstep;
    const long long img_elems = (long long)g.CS * g.HS * g.WS;
    d.rs = make_rsrc(g.src + (long long)n0 * img_elems,
                     (uint32_t)(min(g.N - n0, g.geo.IMGS) * img_elems * 4));
    d.buf = buf;
    d.c0 = chunk * g.CH;
    d.ebase = y0 * g.WS;
    d.ylo = y0 >= 0 ? 0 : (-y0 + rowstep - 1) / rowstep;
    d.yhi = min(g.geo.TIH, (g.HS - y0 + rowstep - 1) / rowstep);
    if (d.yhi < d.ylo) d.yhi = d.ylo;
    d.nimg = min(g.N - n0, g.geo.IMGS);
    d.mlim = g.CD - d.grp * SL * 32;
    return d;
}

// Per-lane constants of the DMA rows (computed once per workgroup).
template <int KK>
struct LaneDMA {
    int toff[WinRows<KK>::MAX];   // window row u: element offset in the tile, channel lane&3
    int tmeta[WinRows<KK>::MAX];  // window row ty | img << 8 (ty = 255: no source element)
    int wl;                       // weight row: (lane/4)*sm + (lane%4)*sc
    // Per work item: byte offset of window row u for channel lane&3 of
    // channel 0, or an offset >= 2^31 (beyond any buffer) when the row has
    // no source data.  A stage adds its channel's byte offset.
    uint32_t roff[WinRows<KK>::MAX];
};

template <int KK>
__device__ __forceinline__ void lane_dma_init(const FastArgs &g, LaneDMA<KK> &L, int wave,
                                              int lane) {
    const TileGeo &t = g.geo;
    const int i = lane & 3;
#pragma unroll
    for (int u = 0; u < WinRows<KK>::MAX; u++) {
        const int pos = (wave + FAST_NW * u) * 16 + (lane >> 2);
        const uint32_t mi = g.m_imgs, mt = g.m_tiwp;  // FastDiv magic multipliers
        const int img = (int)(mi ? __umulhi((uint32_t)pos, mi) : (uint32_t)pos);
        const int rem = pos - img * t.imgs;
        const int ty = (int)(mt ? __umulhi((uint32_t)rem, mt) : (uint32_t)rem);
        const int col = rem - ty * t.TIWP;
        const int tx = t.deint ? (col < t.HALF ? 2 * col : 2 * (col - t.HALF) + 1) : col;
        const int x = g.dxmin + tx * t.colstep;
        const bool ok = u < g.ppw && img < t.IMGS && ty < t.TIH && tx < t.TIW && x >= 0 &&
                        x < g.WS;
        L.toff[u] = ((img * g.CS + i) * g.HS + ty * t.rowstep) * g.WS + x;
        L.tmeta[u] = ok ? (ty | (img << 8)) : 255;
    }
    L.wl = (lane >> 2) * g.sm + i * g.sc;
}

// Weight rows (mb, q, TT) of stage d gathered from W in [cout][cin][k][k]
// order: 64-word row `wave` of each slab, lane l = wave*16 + lane/4.
template <int KK, int SL, int TT>
__device__ __forceinline__ void issue_w_gather(const FastArgs &g, const StageDMA &d,
                                               const LaneDMA<KK> &L, __amdgpu_buffer_rsrc_t rs_w,
                                               int q, int wave, int lane) {
    const int CP = g.CH >> 1, cq = g.CH >> 3;
#pragma unroll
    for (int mb = 0; mb < SL; mb++) {
        const int mrel = mb * 32 + (wave & 1) * 16;
        const int cbase = d.c0 + (wave >> 1) * CP + 4 * q;
        const bool ok = (lane >> 2) < d.mlim - mrel && (lane & 3) < g.CS - cbase;
        const int e = L.wl + (d.grp * SL * 32 + mrel) * g.sm + cbase * g.sc + TT;
        const uint32_t off = max((uint32_t)e * 4u, ok ? 0u : DMA_OOB);
        float *dst = d.buf + g.xwords + ((mb * cq + q) * KK + TT) * 256 + wave * 64;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_w, (lds_ptr_t)dst, 4, off, 0, 0, 0);
    }
}

// The per-item window row offsets (LaneDMA::roff) of stage d's work item.
template <int KK>
__device__ __forceinline__ void item_rows(const FastArgs &g, const StageDMA &d, LaneDMA<KK> &L) {
#pragma unroll
    for (int u = 0; u < WinRows<KK>::MAX; u++) {
        const int ty = L.tmeta[u] & 255, img = L.tmeta[u] >> 8;
        const bool rowok = (unsigned)(ty - d.ylo) < (unsigned)(d.yhi - d.ylo) && img < d.nimg;
        L.roff[u] = rowok ? (uint32_t)(L.toff[u] + d.ebase) * 4u : 0x80000000u;
    }
}

// One stage of the GEMM on the MFMA waves: (quad q, tap t) steps over the
// window `xs` and the weight slabs of the current buffer, the operands of the
// next step read from LDS while the MFMAs of the current one run.
template <int K, int S, int P, bool DX, int NPW, int MB, int WM, int NACC>
__device__ __forceinline__ void compute_stage(
    const FastArgs &g, const float *__restrict__ xs, const int (&vb)[NPW],
    f32x16 (&acc)[ConvTaps<K, S, P, DX>::NCLS][MB][NPW][NACC], int wave, int lane) {
    using T = ConvTaps<K, S, P, DX>;
    constexpr int KK = T::KK;
    const int CQ = g.CH >> 3;
    const int wslab = CQ * KK * 256;
    const float *ws = xs + g.xwords + lane * 4;
    constexpr int WP = FAST_NW / WM;  // waves along positions
    const float *wsw = ws + (wave / WP) * MB * wslab;  // this wave's m-blocks

    auto fetch = [&](int q, int t, float4 *fa, float4 *fb) {
#pragma unroll
        for (int mb = 0; mb < MB; mb++)
            fa[mb] = *reinterpret_cast<const float4 *>(wsw + mb * wslab + (q * KK + t) * 256);
        const float *xq = xs + (q * g.plane + g.tapoff[t]) * 4;
#pragma unroll
        for (int j = 0; j < NPW; j++) fb[j] = *reinterpret_cast<const float4 *>(xq + vb[j]);
    };
    float4 ca[MB], cb[NPW];
    fetch(0, 0, ca, cb);
    for (int q = 0; q < CQ; q++) {
        static_for<0, KK>([&](auto tc) {
            constexpr int t = decltype(tc)::value;
            constexpr int c = T::cls(t);
            float4 na[MB], nb[NPW];
            if (t + 1 < KK)
                fetch(q, t + 1 < KK ? t + 1 : 0, na, nb);
            else if (q + 1 < CQ)
                fetch(q + 1, 0, na, nb);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int mb = 0; mb < MB; mb++)
#pragma unroll
                    for (int j = 0; j < NPW; j++)
                        acc[c][mb][j][i % NACC] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                            ca[mb][i], cb[j][i], acc[c][mb][j][i % NACC], 0, 0, 0);
#pragma unroll
            for (int mb = 0; mb < MB; mb++) ca[mb] = na[mb];
#pragma unroll
            for (int j = 0; j < NPW; j++) cb[j] = nb[j];
        });
    }
}

// All DMA of stage `chunk` of the work item described by d (its window
// rows in L.roff) into `buf`, issued by producer wave `dw`: the window rows
// u = dw, dw + 4, ... of every channel quad, then the weights -- contiguous
// 1 KiB slabs of the packed copy, 16 bytes a lane, or gathered from W.
template <int K, int S, int P, bool DX, int SL>
__device__ __forceinline__ void issue_stage(const FastArgs &g, StageDMA d, float *buf, int chunk,
                                            const LaneDMA<ConvTaps<K, S, P, DX>::KK> &L,
                                            __amdgpu_buffer_rsrc_t rs_w, int dw, int lane) {
    constexpr int KK = ConvTaps<K, S, P, DX>::KK;
    const int cq = g.CH >> 3;
    d.buf = buf;
    d.c0 = chunk * g.CH;
    const uint32_t hsws4 = (uint32_t)(g.HS * g.WS) * 4u;
    for (int hq = 0; hq < 2 * cq; hq++) {
        const int cb = d.c0 + 4 * hq;
        const uint32_t cbytes = (uint32_t)cb * hsws4;
        // lanes whose channel cb + lane%4 is beyond the source get no data
        const uint32_t chbad = g.CS - cb >= 4 ? 0u : ((lane & 3) >= g.CS - cb ? 0x80000000u : 0u);
        float *row0 = buf + (hq * g.plane + dw * 16) * 4;
#pragma unroll
        for (int u = 0; u < WinRows<KK>::MAX; u++)
            if (u < g.ppw)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    d.rs, (lds_ptr_t)(row0 + FAST_NW * u * 64), 4, (L.roff[u] + cbytes) | chbad, 0,
                    0, 0);
    }
    if (g.wp) {
        const int per = cq * KK;
        const __amdgpu_buffer_rsrc_t rs_p = make_rsrc(g.wp, (uint32_t)g.wpbytes);
        for (int k = dw; k < SL * per; k += FAST_NW) {
            const int mb = k / per, r = k - mb * per;
            const uint32_t src =
                (uint32_t)(((d.grp * SL + mb) * g.nchunks + chunk) * per + r) * 1024u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_p, (lds_ptr_t)(buf + g.xwords + k * 256),
                                                     16, src + (uint32_t)lane * 16u, 0, 0, 0);
        }
    } else {
        for (int q = 0; q < cq; q++)
            static_for<0, KK>([&](auto tc) {
                issue_w_gather<KK, SL, decltype(tc)::value>(g, d, L, rs_w, q, dw, lane);
            });
    }
}

// Sums 4 values per lane over the 32 lanes of each half-wave: offsets 16 and
// 8 each keep half of the values, offsets 4, 2, 1 add the rest; lane l ends
// with the total of value 2*b4 + b3 (b = bits of l), the 8 lanes that share
// those bits holding the same total.  The order is fixed.
__device__ __forceinline__ double half_reduce4(const double (&x)[4], int l32) {
    const bool b4 = l32 & 16, b3 = l32 & 8;
    double a2[2];
#pragma unroll
    for (int i = 0; i < 2; i++)
        a2[i] = (b4 ? x[i + 2] : x[i]) + __shfl_xor(b4 ? x[i] : x[i + 2], 16, 64);
    double a1 = (b3 ? a2[1] : a2[0]) + __shfl_xor(b3 ? a2[0] : a2[1], 8, 64);
    a1 = a1 + __shfl_xor(a1, 4, 64);
    a1 = a1 + __shfl_xor(a1, 2, 64);
    return a1 + __shfl_xor(a1, 1, 64);
}

// The forward's store pass with the batch statistics' sums (see ConvStats):
// the same stores as the plain pass, with the accumulator registers taken 4
// at a time so that only 4 (sum y, sum y^2) pairs are live; each wave's
// totals over the item's positions, reduced over its lanes, are left in red
// (LDS) for the workgroup's fixed-order sum over its waves.
template <int K, int S, int P, int NPW, int MB, int WM, int NACC>
__device__ __forceinline__ void store_stats(
    const FastArgs &g, const f32x16 (&acc)[1][MB][NPW][NACC], int wave, int lane, int grp,
    int a0, int n0, double *__restrict__ red) {
    constexpr int VG = 4, WP = FAST_NW / WM, SL = WM * MB;
    const int h = lane >> 5, l32 = lane & 31;
    const int tpix = g.TR * g.GB, npix = g.geo.IMGS * tpix;
    const long long cst = (long long)g.HD * g.WD;
    static_for<0, 16 / VG>([&](auto gc) {
        constexpr int vbase = decltype(gc)::value * VG;
        double es[MB][2][VG];
#pragma unroll
        for (int mb = 0; mb < MB; mb++)
#pragma unroll
            for (int u = 0; u < VG; u++) es[mb][0][u] = es[mb][1][u] = 0.0;
#pragma unroll
        for (int j = 0; j < NPW; j++) {
            const int p = ((wave % WP) * NPW + j) * 32 + l32;
            const int img = p / tpix, rem = p - img * tpix, r = rem / g.GB, cb = rem - r * g.GB;
            const int n = n0 + img, a = a0 + r;
            if (p >= npix || n >= g.N || a >= g.GA) continue;
            const long long o = ((long long)n * g.CD * g.HD + a) * g.WD + cb;
#pragma unroll
            for (int mb = 0; mb < MB; mb++) {
                f32x16 v16 = acc[0][mb][j][0];
                if constexpr (NACC == 2) v16 += acc[0][mb][j][1];
                static_for<0, VG>([&](auto uc) {
                    constexpr int u = decltype(uc)::value, v = vbase + u;
                    const int m = (grp * SL + (wave / WP) * MB + mb) * 32 + 8 * (v >> 2) + 4 * h +
                                  (v & 3);
                    if (m >= g.CD) return;
                    const float y = v16[v];
                    g.dst[o + m * cst] = y;
                    es[mb][0][u] += (double)y;
                    es[mb][1][u] += (double)y * (double)y;
                });
            }
        }
        // this wave's totals into red[wave % WP][channel of the group][kind]
        const int v = vbase + ((l32 >> 4) & 1) * 2 + ((l32 >> 3) & 1);
#pragma unroll
        for (int mb = 0; mb < MB; mb++) {
            const double t0 = half_reduce4(es[mb][0], l32), t1 = half_reduce4(es[mb][1], l32);
            const int cl = ((wave / WP) * MB + mb) * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
            if ((l32 & 7) == 0) {
                red[((wave % WP) * 32 * SL + cl) * 2] = t0;
                red[((wave % WP) * 32 * SL + cl) * 2 + 1] = t1;
            }
        }
    });
}

// Waves 0..3 compute: WP = 4 / WM along positions (NPW groups of 32 each)
// times WM along output channels (MB blocks of 32 each).  Waves 4..7 only
// move data: producer wave 4 + w issues the DMA rows that the row tables
// assign to wave w, a whole stage at a time, so that the memory pipeline's
// back-pressure stalls a producer and never the MFMA issue of a compute
// wave.  One barrier per stage: when it completes, stage s has landed (each
// producer waited for its own DMA) and stage s - 1's buffer is free.
// EPI = 1: the forward's store pass also takes the batch statistics
// (store_stats, ConvStats), with one more barrier per work item that the
// producers match.
template <int K, int S, int P, bool DX, int NPW, int MB, int WM, int EPI>
__global__ __launch_bounds__(64 * FAST_NW * 2)
__attribute__((amdgpu_waves_per_eu(EPI ? 4 : 1))) void conv_fast_kernel(FastArgs g) {
    using T = ConvTaps<K, S, P, DX>;
    constexpr int NCLS = T::NCLS;
    // A wave with a single output block alternates two accumulators so that
    // consecutive MFMAs do not depend on each other.
    constexpr int NACC = NCLS * NPW * MB == 1 ? 2 : 1;
    constexpr int WP = FAST_NW / WM, SL = WM * MB;
    extern __shared__ float smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_index();
    const int h = lane >> 5, l32 = lane & 31;
    const int CQ = g.CH >> 3;
    const int tpix = g.TR * g.GB, npix = g.geo.IMGS * tpix;
    const int nitems = g.ntiles * g.ngroups;
    if ((int)blockIdx.x >= nitems) return;

    if (wave >= FAST_NW) {
        // producer
        const int dw = wave - FAST_NW;
        const __amdgpu_buffer_rsrc_t rs_w = make_rsrc(g.w, (uint32_t)g.wbytes);
        LaneDMA<T::KK> L;
        lane_dma_init<T::KK>(g, L, dw, lane);
        StageDMA d = stage_dma<K, S, P, DX, SL>(g, blockIdx.x, 0, smem);
        item_rows<T::KK>(g, d, L);
        issue_stage<K, S, P, DX, SL>(g, d, smem, 0, L, rs_w, dw, lane);
        int s = 0;
        for (int item = blockIdx.x; item < nitems; item += gridDim.x) {
            for (int chunk = 0; chunk < g.nchunks; chunk++, s++) {
                dma_wait_barrier();
                float *nbuf = smem + ((s + 1) & 1) * g.stage;
                if (chunk + 1 < g.nchunks) {
                    issue_stage<K, S, P, DX, SL>(g, d, nbuf, chunk + 1, L, rs_w, dw, lane);
                } else if (item + (int)gridDim.x < nitems) {
                    d = stage_dma<K, S, P, DX, SL>(g, item + gridDim.x, 0, nbuf);
                    item_rows<T::KK>(g, d, L);
                    issue_stage<K, S, P, DX, SL>(g, d, nbuf, 0, L, rs_w, dw, lane);
                }
            }
            if constexpr (EPI != 0) __syncthreads();  // the compute waves' store-pass sums
        }
        return;
    }

    // LDS word offset of this lane's channel half and window position for
    // each 32-position group (tile-relative: the same for every work item).
    int vb[NPW];
#pragma unroll
    for (int j = 0; j < NPW; j++) {
        int p = ((wave % WP) * NPW + j) * 32 + l32;
        if (p >= npix) p = 0;
        const int img = p / tpix, rem = p - img * tpix, r = rem / g.GB, c = rem - r * g.GB;
        vb[j] = (h * CQ * g.plane + img * g.geo.imgs + r * g.lrow * g.geo.TIWP + c * g.lcol) * 4;
    }

    f32x16 acc[NCLS][MB][NPW][NACC];
    int s = 0;
    for (int item = blockIdx.x; item < nitems; item += gridDim.x) {
#pragma unroll
        for (int c = 0; c < NCLS; c++)
#pragma unroll
            for (int mb = 0; mb < MB; mb++)
#pragma unroll
                for (int j = 0; j < NPW; j++)
#pragma unroll
                    for (int a = 0; a < NACC; a++)
#pragma unroll
                        for (int v = 0; v < 16; v++) acc[c][mb][j][a][v] = 0.f;
        for (int chunk = 0; chunk < g.nchunks; chunk++, s++) {
            // Stage s has landed and every wave is done with stage s-1, whose
            // buffer the producers fill with stage s+1 while stage s is computed.
            dma_wait_barrier();
            compute_stage<K, S, P, DX, NPW, MB, WM, NACC>(g, smem + (s & 1) * g.stage, vb, acc,
                                                          wave, lane);
        }
        // acc row 8*(v/4) + 4*h + v%4 = output channel in the block, column = position.
        const int tile = item % g.ntiles, grp = item / g.ntiles;
        const int a0 = (tile % g.tiles_a) * g.TR, n0 = (tile / g.tiles_a) * g.geo.IMGS;
        if constexpr (EPI != 0) {
            // Store pass with the statistics' sums; then the WP position
            // waves' totals of each channel, summed in wave order, make partial
            // `tile` of the channel.  The barrier pairs with the producers'
            // one after the item.
            constexpr int NCH = 32 * SL;
            double *red = reinterpret_cast<double *>(smem + 2 * g.stage);
            store_stats<K, S, P, NPW, MB, WM, NACC>(g, acc, wave, lane, grp, a0, n0, red);
            __syncthreads();
            for (int t = tid; t < 2 * NCH; t += 64 * FAST_NW) {
                const int cl = t >> 1, m = grp * NCH + cl;
                if (m >= g.CD) continue;
                double tot = red[t];
                for (int w = 1; w < WP; w++) tot += red[w * 2 * NCH + t];
                g.stats.part[((long long)m * g.npart + tile) * 2 + (t & 1)] = tot;
            }
            continue;
        }
#pragma unroll
        for (int j = 0; j < NPW; j++) {
            const int p = ((wave % WP) * NPW + j) * 32 + l32;
            if (p >= npix) continue;
            const int img = p / tpix, rem = p - img * tpix, r = rem / g.GB, cb = rem - r * g.GB;
            const int n = n0 + img, a = a0 + r;
            if (n >= g.N || a >= g.GA) continue;
            const long long cst = (long long)g.HD * g.WD;
            if constexpr (NCLS == 4) {
                // stride-2 dX: the two column classes of a row are adjacent in
                // dX, so one 8-byte store writes both (each line written once)
#pragma unroll
                for (int py = 0; py < 2; py++) {
                    const int y = 2 * a + py, x = 2 * cb;
                    if (y >= g.HD || x >= g.WD) continue;
                    float *dp = g.dst + ((long long)n * g.CD * g.HD + y) * g.WD + x;
                    const bool pair = (g.WD & 1) == 0;  // x + 1 < WD and 8-byte aligned
#pragma unroll
                    for (int mb = 0; mb < MB; mb++) {
                        f32x16 v0 = acc[2 * py][mb][j][0], v1 = acc[2 * py + 1][mb][j][0];
                        if constexpr (NACC == 2) {
                            v0 += acc[2 * py][mb][j][1];
                            v1 += acc[2 * py + 1][mb][j][1];
                        }
#pragma unroll
                        for (int v = 0; v < 16; v++) {
                            const int m = (grp * SL + (wave / WP) * MB + mb) * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                            if (m >= g.CD) continue;
                            if (pair) {
                                *reinterpret_cast<float2 *>(dp + m * cst) = float2{v0[v], v1[v]};
                            } else {
                                dp[m * cst] = v0[v];
                                if (x + 1 < g.WD) dp[m * cst + 1] = v1[v];
                            }
                        }
                    }
                }
            } else {
#pragma unroll
                for (int c = 0; c < NCLS; c++) {
                    const int y = a * T::OS + (DX ? c / S : 0), x = cb * T::OS + (DX ? c % S : 0);
                    if (y >= g.HD || x >= g.WD) continue;
                    float *dp = g.dst + ((long long)n * g.CD * g.HD + y) * g.WD + x;
#pragma unroll
                    for (int mb = 0; mb < MB; mb++) {
                        f32x16 v16 = acc[c][mb][j][0];
                        if constexpr (NACC == 2) v16 += acc[c][mb][j][1];
#pragma unroll
                        for (int v = 0; v < 16; v++) {
                            const int m = (grp * SL + (wave / WP) * MB + mb) * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                            if (m < g.CD) dp[m * cst] = v16[v];
                        }
                    }
                }
            }
        }
    }
}

struct FastPlan {
    int TR, IMGS, CH, NPW, MB, WM;
    int wpc;  // cap on resident workgroups per CU (0 = occupancy limit)
    size_t lds;
};

// Window geometry of a plan; returns the LDS bytes (two stage buffers), or
// 0 when the window does not fit the per-wave DMA row tables.
template <int K, int S, int P, bool DX>
static size_t plan_geometry(const FastPlan &p, int GB, FastArgs &a) {
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
    t.chs = 0;
    tilegeo_finish(t);
    a.plane = (p.IMGS * t.imgs + 16 * FAST_NW - 1) / (16 * FAST_NW) * (16 * FAST_NW);
    a.ppw = a.plane / (16 * FAST_NW);
    if (a.ppw > WinRows<T::KK>::MAX || t.TIH > 254 || p.IMGS > 255) return 0;
    a.dymin = dymin;
    a.dxmin = dxmin;
    for (int i = 0; i < 9; i++) {
        a.tapoff[i] = 0;
        if (i < T::KK) {
            const int dyp = T::dy(i) - dymin, dxp = T::dx(i) - dxmin;
            a.tapoff[i] = dyp * t.TIWP + (t.deint ? (dxp & 1) * t.HALF + (dxp >> 1) : dxp);
        }
    }
    a.m_imgs = t.fd_imgstr.m;
    a.m_tiwp = t.fd_tiwp.m;
    a.xwords = p.CH * a.plane;
    a.stage = a.xwords + p.WM * p.MB * p.CH * T::KK * 32;
    return (size_t)2 * a.stage * 4;
}

template <int K, int S, int P, bool DX>
static bool plan_ok(FastPlan &p, int CS, int GA, int GB, FastArgs &a) {
    using T = ConvTaps<K, S, P, DX>;
    const int CSe = std::max(8, (CS + 7) & ~7);
    p.CH = std::min(p.CH, std::min(32, CSe));
    p.TR = std::min(p.TR, GA);
    if (p.TR <= 0 || p.IMGS <= 0 || p.CH < 8 || p.CH % 8) return false;
    if (p.WM <= 0) p.WM = 1;
    const int nwm = p.NPW * 100 + p.MB * 10 + p.WM;
    const bool shape_ok = T::NCLS == 1 ? (nwm == 211 || nwm == 111 || nwm == 121 || nwm == 112)
                                       : (nwm == 111 || nwm == 112);
    if (!shape_ok || p.IMGS * p.TR * GB > (FAST_NW / p.WM) * p.NPW * 32) return false;
    p.lds = plan_geometry<K, S, P, DX>(p, GB, a);
    return p.lds > 0 && p.lds <= 160 * 1024;
}

// Tile choice.  RNN_CONV_PLAN="TR,IMGS,CH,NPW,MB[,WM[,WPC]]" overrides
// (tuning sweeps).  Otherwise rules fitted to measured sweeps on MI355X:
// channel chunks of a quarter of the source channels (8..32; 32 for 1x1);
// stride-1 3x3 and 1x1 forward take 256 positions in two 32-position groups
// per wave when an image has 256 or more positions, else 128 positions (whole
// images); strided 3x3 forward takes 64 positions with the waves split two
// ways along output channels, so every wave has a 32x32 block.  A plan that
// does not fit falls back to shrinking the tile; a strided 3x3 forward gives
// up channels per chunk before positions (at 96 source channels, 24-channel
// chunks with 32 positions ran at half the rate of 8-channel chunks with 64).
template <int K, int S, int P, bool DX>
static bool choose_plan(int CS, int CD, int GA, int GB, FastPlan &best, FastArgs &a) {
    using T = ConvTaps<K, S, P, DX>;
    if (const char *env = getenv("RNN_CONV_PLAN")) {
        FastPlan p{};
        const int got = sscanf(env, "%d,%d,%d,%d,%d,%d,%d", &p.TR, &p.IMGS, &p.CH, &p.NPW, &p.MB,
                               &p.WM, &p.wpc);
        if (got >= 5 && plan_ok<K, S, P, DX>(p, CS, GA, GB, a)) {
            best = p;
            return true;
        }
    }
    if (GB > 256) return false;
    const int ch = T::KK == 1 ? 32 : std::max(8, std::min(32, (CS / 4 + 7) & ~7));
    const bool strided = T::KK == 9 && T::IS == 2;
    FastPlan r{};
    r.CH = ch;
    r.NPW = 1;
    r.MB = 1;
    r.WM = 1;
    int npos = 128;
    if (T::KK == 9 && T::NCLS == 1 && T::IS == 1) {
        if (GA * GB >= 256) {
            r.NPW = 2;
            npos = 256;
        }
    } else if (strided) {
        npos = 64;
        if (CD > 32) r.WM = 2;
    } else if (T::KK == 1 && T::NCLS == 1 && GA * GB >= 256) {
        r.NPW = 2;
        npos = 256;
    }
    if (GA * GB <= npos) {
        r.TR = GA;
        r.IMGS = std::max(1, npos / (GA * GB));
    } else {
        r.TR = std::max(1, npos / GB);
        r.IMGS = 1;
    }
    for (;;) {
        FastPlan q = r;
        if (plan_ok<K, S, P, DX>(q, CS, GA, GB, a)) {
            best = q;
            return true;
        }
        if (r.IMGS > 1)
            r.IMGS /= 2;
        else if (strided && r.CH > 8)
            r.CH = std::max(8, (r.CH / 2) & ~7);
        else if (r.TR > 1)
            r.TR = (r.TR + 1) / 2;
        else if (r.CH > 8)
            r.CH /= 2;
        else if (r.WM > 1)
            r.WM = 1;
        else
            return false;
    }
}

// LDS after the two stage buffers for the store-pass sums: per position wave,
// channel of the group and kind, one double.
static size_t epi_lds(const FastPlan &p) {
    return (size_t)(FAST_NW / p.WM) * 32 * p.WM * p.MB * 2 * sizeof(double);
}

template <int K, int S, int P, bool DX, int NPW, int MB, int WM>
static void set_attr() {
    (void)hipFuncSetAttribute((const void *)conv_fast_kernel<K, S, P, DX, NPW, MB, WM, 0>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if constexpr (!DX)
        (void)hipFuncSetAttribute((const void *)conv_fast_kernel<K, S, P, DX, NPW, MB, WM, 1>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
}

// Operand roles, geometry and tile plan of a (k, stride, pad) forward / dX
// convolution; false when no plan fits.
template <int K, int S, int P, bool DX>
static bool setup(const rnn_conv_spec *sp, FastArgs &a, FastPlan &p) {
    using T = ConvTaps<K, S, P, DX>;
    std::memset(&a, 0, sizeof(a));
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
    if (!choose_plan<K, S, P, DX>(a.CS, a.CD, a.GA, a.GB, p, a)) return false;
    if (getenv("RNN_CONV_DEBUG"))
        fprintf(stderr, "conv k%d s%d p%d %s %dx%d->%d: plan %d,%d,%d,%d,%d,%d lds %zu\n", K, S, P,
                DX ? "dx" : "fwd", a.CS, a.GA, a.CD, p.TR, p.IMGS, p.CH, p.NPW, p.MB, p.WM, p.lds);
    a.TR = p.TR;
    a.tiles_a = (a.GA + p.TR - 1) / p.TR;
    a.CH = p.CH;
    a.nchunks = (a.CS + p.CH - 1) / p.CH;
    return true;
}

template <int K, int S, int P, bool DX>
static PackGeo pack_geo(const FastArgs &a) {
    PackGeo pg;
    pg.CS = a.CS;
    pg.CD = a.CD;
    pg.KK = ConvTaps<K, S, P, DX>::KK;
    pg.CH = a.CH;
    pg.nchunks = a.nchunks;
    pg.nmblk = (a.CD + 31) / 32;
    pg.sm = a.sm;
    pg.sc = a.sc;
    return pg;
}

template <int K, int S, int P, bool DX>
static int launch(rnn_ctx *ctx, const rnn_conv_spec *sp, int n, const float *src, const float *w,
                  const float *wp, float *dst, const ConvStats *cs) {
    using T = ConvTaps<K, S, P, DX>;
    static bool attr = false;
    if (!attr) {
        attr = true;
        set_attr<K, S, P, DX, 1, 1, 1>();
        set_attr<K, S, P, DX, 1, 1, 2>();
        if constexpr (T::NCLS == 1) {
            set_attr<K, S, P, DX, 2, 1, 1>();
            set_attr<K, S, P, DX, 1, 2, 1>();
        }
    }
    FastArgs a;
    FastPlan p;
    if (!setup<K, S, P, DX>(sp, a, p))
        return rnn_fail(ctx, RNN_E_UNSUPPORTED, "conv: no LDS tiling for a %dx%d grid", a.GA, a.GB);
    a.src = src;
    a.w = w;
    a.dst = dst;
    a.N = n;
    const long long wbytes = (long long)sp->cout * sp->cin * T::KK * 4;
    const long long pbytes = (long long)pack_geo<K, S, P, DX>(a).floats() * 4;
    if ((long long)p.IMGS * a.CS * a.HS * a.WS * 4 >= 0x7FFFFFF0ll || wbytes >= 0x7FFFFFF0ll ||
        pbytes >= 0x7FFFFFF0ll)
        return rnn_fail(ctx, RNN_E_UNSUPPORTED, "conv: tile source or weights beyond 2 GiB");
    a.wbytes = (int)wbytes;
    a.wp = wp;
    a.wpbytes = (int)pbytes;
    const int nmblk = (a.CD + 31) / 32;
    a.ntiles = a.tiles_a * ((n + p.IMGS - 1) / p.IMGS);
    a.ngroups = (nmblk + p.MB * p.WM - 1) / (p.MB * p.WM);
    const long long nitems = (long long)a.ntiles * a.ngroups;
    if (nitems > 0x7fffffffll) return rnn_fail(ctx, RNN_E_UNSUPPORTED, "conv: too many tiles");
    const bool stats = cs != nullptr;
    if (stats) {
        if (DX || !cs->part)
            return rnn_fail(ctx, RNN_E_INVALID, "conv: store-pass statistics need a forward");
        a.stats = *cs;
        a.npart = a.ntiles;
        p.lds += epi_lds(p);
        if (p.lds > 160 * 1024)
            return rnn_fail(ctx, RNN_E_UNSUPPORTED, "conv: no LDS for the store-pass sums");
    }
    // Persistent grid: as many workgroups as fit on the chip at once.
    auto run = [&](auto kern) -> int {
        int occ = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, 64 * FAST_NW * 2, p.lds) !=
                hipSuccess ||
            occ < 1)
            occ = 1;
        if (p.wpc > 0) occ = std::min(occ, p.wpc);
        const long long grid = std::min<long long>(nitems, (long long)ctx->num_cus * occ);
        hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * FAST_NW * 2), p.lds, ctx->stream,
                           a);
        RNN_LAUNCHED(ctx);
        return RNN_OK;
    };
    auto pick = [&](auto ec) -> int {
        constexpr int E = decltype(ec)::value;
        if constexpr (T::NCLS == 1) {
            if (p.NPW == 2) return run(conv_fast_kernel<K, S, P, DX, 2, 1, 1, E>);
            if (p.MB == 2) return run(conv_fast_kernel<K, S, P, DX, 1, 2, 1, E>);
        }
        if (p.WM == 2) return run(conv_fast_kernel<K, S, P, DX, 1, 1, 2, E>);
        return run(conv_fast_kernel<K, S, P, DX, 1, 1, 1, E>);
    };
    if constexpr (!DX)
        if (stats) return pick(std::integral_constant<int, 1>{});
    return pick(std::integral_constant<int, 0>{});
}

template <int K, int S, int P>
static int parts_of(const rnn_conv_spec *sp, size_t n) {
    FastArgs a;
    FastPlan p;
    if (!setup<K, S, P, false>(sp, a, p)) return -1;
    if (p.lds + epi_lds(p) > 160 * 1024) return -1;
    const long long np = (long long)a.tiles_a * (((long long)n + p.IMGS - 1) / p.IMGS);
    return np > 0x3fffffffll ? -1 : (int)np;
}


// Packs W for the forward (dx = 0) or dX (dx = 1) kernel: slab order
// [m-block][chunk][quad][tap][lane][4], the layout the kernel's LDS weight
// slabs take, zero-filled beyond the channels, so that a stage's weights are
// one contiguous copy.  Lane L of slab (q, t) holds rows m = 32*mblk + L%32
// and channels c = chunk*CH + (L/32)*CH/2 + 4q + i.
__global__ __launch_bounds__(256) void conv_pack_kernel(const float *__restrict__ w, PackGeo g,
                                                        float *wp) {
    for (int r = blockIdx.x; r < g.slabs(); r += gridDim.x)
        wp[(size_t)r * 256 + threadIdx.x] = g.value(w, r, threadIdx.x);
}

// Several packs in one launch: block b serves the segment whose block range
// holds it, one 256-float slab at a time.
__global__ __launch_bounds__(256) void conv_pack_multi_kernel(const float *__restrict__ src,
                                                              const PackSeg *__restrict__ segs,
                                                              int nseg, float *dst) {
    int lo = 0, hi = nseg - 1;
    while (lo < hi) {  // last segment with blk0 <= blockIdx.x
        const int mid = (lo + hi + 1) >> 1;
        if (segs[mid].blk0 <= blockIdx.x)
            lo = mid;
        else
            hi = mid - 1;
    }
    const PackSeg sg = segs[lo];
    const float *w = src + sg.src;
    float *wp = dst + sg.dst;
    for (int r = blockIdx.x - sg.blk0; r < sg.geo.slabs(); r += sg.nblk)
        wp[(size_t)r * 256 + threadIdx.x] = sg.geo.value(w, r, threadIdx.x);
}

template <int K, int S, int P, bool DX>
static int geo_of(const rnn_conv_spec *sp, PackGeo *pg) {
    FastArgs a;
    FastPlan p;
    if (!setup<K, S, P, DX>(sp, a, p)) return RNN_E_UNSUPPORTED;
    *pg = pack_geo<K, S, P, DX>(a);
    return RNN_OK;
}

}  // namespace

// Forward (dx = 0) or dX (dx = 1) through the specialised kernels; returns
// RNN_E_UNSUPPORTED (without recording an error) when (k, stride, pad) has no
// specialisation, so the caller can take the generic per-class path.  wp:
// the weights packed by rnn_conv_pack for this direction, or null.
int rnn_conv_fast(rnn_ctx *ctx, int dx, const rnn_conv_spec *sp, size_t n, const float *src,
                  const float *w, const float *wp, float *dst, const ConvStats *stats) {
    if (getenv("RNN_CONV_GENERIC")) return RNN_E_UNSUPPORTED;
    const int k = sp->k, s = sp->stride, p = sp->pad;
    const int ni = (int)n;
#define RNN_CONV_CASE(K_, S_, P_)                                                               \
    if (k == K_ && s == S_ && p == P_)                                                          \
        return dx ? launch<K_, S_, P_, true>(ctx, sp, ni, src, w, wp, dst, stats)               \
                  : launch<K_, S_, P_, false>(ctx, sp, ni, src, w, wp, dst, stats);
    RNN_CONV_CASE(3, 1, 1)
    RNN_CONV_CASE(3, 2, 1)
    RNN_CONV_CASE(1, 2, 0)
    RNN_CONV_CASE(1, 1, 0)
#undef RNN_CONV_CASE
    return RNN_E_UNSUPPORTED;
}

int rnn_conv_fast_parts(const rnn_conv_spec *sp, size_t n) {
    if (getenv("RNN_CONV_GENERIC") || n == 0 || n > 0x7fffffff) return -1;
    const int k = sp->k, s = sp->stride, p = sp->pad;
#define RNN_CONV_CASE(K_, S_, P_) \
    if (k == K_ && s == S_ && p == P_) return parts_of<K_, S_, P_>(sp, n);
    RNN_CONV_CASE(3, 1, 1)
    RNN_CONV_CASE(3, 2, 1)
    RNN_CONV_CASE(1, 2, 0)
    RNN_CONV_CASE(1, 1, 0)
#undef RNN_CONV_CASE
    return -1;
}

int rnn_conv_pack_geo(const rnn_conv_spec *sp, int dx, PackGeo *pg) {
    if (getenv("RNN_CONV_GENERIC")) return RNN_E_UNSUPPORTED;
    const int k = sp->k, s = sp->stride, p = sp->pad;
#define RNN_CONV_CASE(K_, S_, P_)                                                               \
    if (k == K_ && s == S_ && p == P_)                                                          \
        return dx ? geo_of<K_, S_, P_, true>(sp, pg) : geo_of<K_, S_, P_, false>(sp, pg);
    RNN_CONV_CASE(3, 1, 1)
    RNN_CONV_CASE(3, 2, 1)
    RNN_CONV_CASE(1, 2, 0)
    RNN_CONV_CASE(1, 1, 0)
#undef RNN_CONV_CASE
    return RNN_E_UNSUPPORTED;
}

int rnn_conv_pack(rnn_ctx *ctx, const rnn_conv_spec *sp, int dx, const float *w, float *wp) {
    PackGeo pg;
    const int rc = rnn_conv_pack_geo(sp, dx, &pg);
    if (rc) return rc;
    const unsigned grid = (unsigned)std::min(pg.slabs(), 4096);
    conv_pack_kernel<<<grid, 256, 0, ctx->stream>>>(w, pg, wp);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_conv_pack_multi_launch(rnn_ctx *ctx, const PackSeg *segs, int nseg, int nblocks,
                               const float *src, float *dst) {
    if (nseg <= 0) return RNN_OK;
    conv_pack_multi_kernel<<<nblocks, 256, 0, ctx->stream>>>(src, segs, nseg, dst);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

// Packed copies of several convolutions' weights in one device block: the
// data (each copy a whole number of 256-float slabs), then the segment table
// that conv_pack_multi_kernel walks.  Sources are addressed from the lowest
// W pointer, so a segment's source offset is its W's distance from it.
struct rnn_conv_packs {
    void *mem = nullptr;
    PackSeg *segs = nullptr;
    int nseg = 0, nblk = 0;
    const float *src = nullptr;
    float *data = nullptr;
    std::vector<const float *> wp[2];
};

int rnn_conv_packs_create(rnn_ctx *ctx, size_t count, const rnn_conv_spec *specs, const float **w,
                          rnn_conv_packs **out) {
    if (!ctx || !out) return RNN_E_NULL;
    *out = nullptr;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (count == 0 || !specs || !w) return rnn_fail(ctx, RNN_E_NULL, "conv_packs: no convolutions");
    uintptr_t lo = UINTPTR_MAX;
    for (size_t i = 0; i < count; i++) {
        if (!w[i]) return rnn_fail(ctx, RNN_E_NULL, "conv_packs: null weights %zu", i);
        if ((uintptr_t)w[i] & 3) return rnn_fail(ctx, RNN_E_INVALID, "conv_packs: unaligned W");
        lo = std::min(lo, (uintptr_t)w[i]);
    }
    std::vector<PackSeg> segs;
    std::vector<std::pair<size_t, int>> who;  // (conv, direction) of each segment
    size_t floats = 0;
    uint32_t blk = 0;
    for (size_t i = 0; i < count; i++) {
        for (int dx = 0; dx < 2; dx++) {
            PackSeg sg;
            if (rnn_conv_pack_geo(&specs[i], dx, &sg.geo) != RNN_OK) continue;
            sg.src = ((uintptr_t)w[i] - lo) / sizeof(float);
            sg.dst = floats;
            sg.blk0 = blk;
            sg.nblk = (uint32_t)std::min(sg.geo.slabs(), 512);
            blk += sg.nblk;
            floats += sg.geo.floats();
            segs.push_back(sg);
            who.push_back({i, dx});
        }
    }
    if (blk > 0x7fffffffu) return rnn_fail(ctx, RNN_E_UNSUPPORTED, "conv_packs: too many slabs");
    auto *p = new (std::nothrow) rnn_conv_packs();
    if (!p) return rnn_fail(ctx, RNN_E_NOMEM, "conv_packs: host allocation");
    p->wp[0].assign(count, nullptr);
    p->wp[1].assign(count, nullptr);
    p->src = (const float *)lo;
    p->nseg = (int)segs.size();
    p->nblk = (int)blk;
    if (!segs.empty()) {
        const size_t dbytes = floats * sizeof(float), tbytes = segs.size() * sizeof(PackSeg);
        hipError_t e = hipMalloc(&p->mem, dbytes + tbytes);
        if (e != hipSuccess) {
            delete p;
            return rnn_fail(ctx, RNN_E_NOMEM, "conv_packs hipMalloc(%zu): %s", dbytes + tbytes,
                            hipGetErrorString(e));
        }
        p->data = (float *)p->mem;
        p->segs = (PackSeg *)((char *)p->mem + dbytes);
        e = hipMemcpy(p->segs, segs.data(), tbytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            (void)hipFree(p->mem);
            delete p;
            return rnn_fail(ctx, RNN_E_HIP, "conv_packs table upload: %s", hipGetErrorString(e));
        }
        for (size_t k = 0; k < segs.size(); k++)
            p->wp[who[k].second][who[k].first] = p->data + segs[k].dst;
    }
    const int rc = rnn_conv_pack_multi_launch(ctx, p->segs, p->nseg, p->nblk, p->src, p->data);
    if (rc) {
        rnn_conv_packs_destroy(p);
        return rc;
    }
    *out = p;
    return RNN_OK;
}

int rnn_conv_packs_update(rnn_ctx *ctx, rnn_conv_packs *p) {
    if (!ctx || !p) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    return rnn_conv_pack_multi_launch(ctx, p->segs, p->nseg, p->nblk, p->src, p->data);
}

const float *rnn_conv_packs_get(const rnn_conv_packs *p, size_t i, int dx) {
    if (!p || (dx != 0 && dx != 1) || i >= p->wp[0].size()) return nullptr;
    return p->wp[dx][i];
}

void rnn_conv_packs_destroy(rnn_conv_packs *p) {
    if (!p) return;
    if (p->mem) (void)hipFree(p->mem);
    delete p;
}
