// Convolution weight gradient, deterministic split-K on fp32 MFMA.
//
// dW[co][ci][kh][kw] += sum over (n, oy, ox) of dY[n][co][oy][ox] *
//                       X[n][ci][oy*s + kh - pad][ox*s + kw - pad]
//
// Reference: conv.rs dw_image (277-322) folded per image and reduced over
// rayon workers in Conv2d::backward_w (nn.rs:193-227).  GEMM M = co (32 per
// block), N = ci (32 per block) for each tap, K = output pixels.
//
// A workgroup owns a (co block, ci block) pair and walks a strided set of
// pixel tiles (TR output rows of IMGS images, full width).  Four producer
// waves stage each tile by DMA into one of two LDS buffers while the MFMA
// waves (eight for 3x3: two per SIMD, each set owning half of the taps; four
// for 1x1) compute the previous one (the memory pipeline's back-pressure
// stalls only the producers):
//   * the dY window [co][img][r][OWP] and the X halo window [ci][img][ty][TIWP]
//     (stride 2: even columns then odd columns), one LDS channel every 64m+4
//     words so that the 32 lanes of a b128 read hit distinct banks while no
//     64-word DMA row straddles two channels;
//   * per-lane DMA source offsets come from small register tables built once
//     per workgroup, so a DMA row costs a few integer ops.
// Compute: a wave takes 8-pixel groups of a tile row; lane half h reads the 4
// pixels 4h..4h+3 of the group with one ds_read_b128 for dY and, per kernel
// row kh, the 6 (or 5 + 4) X values those pixels touch, so the three kw taps
// are register offsets into the same read.  MFMA k-step i takes pixels i and
// 4 + i; a wave's tap accumulators (5 or 4) are independent chains.  The 4
// waves of a tap set add their sums through LDS in a fixed pairwise order and the workgroup
// writes one partial slab; slabs are added in slab order by one reduction
// launch (no atomics: the result is bit-reproducible).
#include "conv_common.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>

namespace {

constexpr int DW_NW = 4;  // MFMA waves per tap group (one workgroup per CU, one per SIMD)
constexpr int DW_NP = 4;  // DMA producer waves per workgroup (one per SIMD)

// Tap groups: a 3x3 kernel's 9 taps are split over two sets of DW_NW MFMA
// waves (taps 0-4 and 5-8), so every SIMD runs two MFMA waves that cover
// each other's operand waits and loop overhead; a 1x1 kernel keeps one set.
// Each tap is still summed by the same wave sequence over the same groups.
template <int K>
constexpr int dw_tap_groups() {
    return K == 3 ? 2 : 1;
}
template <int K>
constexpr int dw_threads() {
    return 64 * (DW_NW * dw_tap_groups<K>() + DW_NP);
}
inline int dw_threads_of(int k) { return k == 3 ? dw_threads<3>() : dw_threads<1>(); }

struct DwArgs {
    const float *dy;  // [N][CO][OH][OW]
    const float *x;   // [N][CI][H][W]
    float *part;      // [nz][CO][CI*KK]
    int N, CO, CI, H, W, OH, OW;
    int S, pad;
    int TR, IMGS, OWP;       // tile: TR output rows of IMGS images, rows padded to OWP
    int tiles_a, ntiles, nz;
    int TIH, TIWP, HE;       // X window rows, row length, even-column part (stride-2 3x3)
    int xrow, xstep;         // X window rows per output row; source rows per window row
    int ximg, dimg;          // window positions per image (X, dY)
    int mx, md;              // 64-word DMA rows per channel (X, dY)
    int chsx, chsd;          // LDS channel strides: 64*m + 4
    int xwords;              // LDS words of the X region (32 * chsx)
    int stage;               // LDS words of one stage: X, dY, 64-word sink
    int ngroups;             // 8-pixel groups per tile
    int gpr;                 // groups per tile row (OWP / 8)
    int hw, ohw, cihw, cohw; // H*W, OH*OW, CI*H*W, CO*OH*OW
    FastDiv fd_gpr, fd_tr, fd_ximg, fd_tiwp, fd_dimg, fd_owp;
    int nbuf;                // stage buffers (1 or 2)
    // 16-byte staging (3x3 stride 1 pad 1, whole tiles; the plan's MT = 0):
    // X window rows of rch 16-byte chunks, x = -4 .. OW + 3 at row column
    // x + 4 (the first and last chunk stay zero: the left and right padding);
    // dY rows as they lie in memory.  Channels sit an odd number of chunks
    // apart, as the 4-byte layout's 64m + 4 words do.
    int rch;                 // chunks of an X window row: OW / 4 + 2
    int xdata, xchunks;      // X data chunks per channel (IMGS * TIH * rch), LDS chunks (odd)
    int ddata, dchunks;      // dY data chunks per channel (IMGS * TR * OW / 4), LDS chunks (odd)
    int nix, nid;            // 64-lane 16-byte DMA instructions per tile (X, dY)
};

// Per-lane DMA table entry: (element offset in the image plane, 16 bits) |
// window row << 16 | image << 24; window row 255 marks a position without
// source data (padding or outside the image columns).
constexpr int DW_NOROW = 255 << 16;

template <int MT>
struct DwLane {
    int tx[MT];  // X window rows
    int td[MT];  // dY window rows
};

template <int K, int S, int MT>
__device__ __forceinline__ void dw_lane_init(const DwArgs &g, DwLane<MT> &L, int lane) {
#pragma unroll
    for (int j = 0; j < MT; j++) {
        // X window position p = 64j + lane of a channel plane
        {
            const int p = 64 * j + lane;
            const int img = (int)fdiv((uint32_t)p, g.fd_ximg), rem = p - img * g.ximg;
            const int ty = (int)fdiv((uint32_t)rem, g.fd_tiwp), wc = rem - ty * g.TIWP;
            int x;
            if (K == 1)
                x = wc * S - g.pad;
            else if (S == 1)
                x = wc - g.pad;
            else
                x = wc < g.HE ? 2 * wc - g.pad : 2 * (wc - g.HE) + 1 - g.pad;
            const bool ok = j < g.mx && img < g.IMGS && x >= 0 && x < g.W;
            L.tx[j] = ok ? ((ty * g.xstep * g.W + x) | (ty << 16) | (img << 24)) : DW_NOROW;
        }
        // dY window position
        {
            const int p = 64 * j + lane;
            const int img = (int)fdiv((uint32_t)p, g.fd_dimg), rem = p - img * g.dimg;
            const int r = (int)fdiv((uint32_t)rem, g.fd_owp), col = rem - r * g.OWP;
            const bool ok = j < g.md && img < g.IMGS && col < g.OW;
            L.td[j] = ok ? ((r * g.OW + col) | (r << 16) | (img << 24)) : DW_NOROW;
        }
    }
}

// Wave-uniform description of the tile being staged plus, per lane, the
// byte offset of each DMA row's element for the block's first channel (or
// DMA_OOB when the position has no source data).  A channel adds c*H*W*4;
// min() with DMA_OOB keeps out-of-range positions out of range.
template <int MT>
struct DwStage {
    __amdgpu_buffer_rsrc_t rx, rd;  // X / dY images n0 .. n0 + IMGS
    float *buf, *sink;
    int valid;
    uint32_t xo[MT], dof[MT];
};

template <int MT>
__device__ __forceinline__ DwStage<MT> dw_stage(const DwArgs &g, const DwLane<MT> &L, int tile,
                                                int cob, int cib, float *buf) {
    DwStage<MT> d;
    d.valid = tile < g.ntiles;
    if (!d.valid) tile = 0;
    const int n0 = (tile / g.tiles_a) * g.IMGS, a0 = (tile % g.tiles_a) * g.TR;
    const int nimg0 = min(g.N - n0, g.IMGS);
    d.rx = make_rsrc(g.x + (long long)n0 * g.cihw, (uint32_t)(nimg0 * (long long)g.cihw * 4));
    d.rd = make_rsrc(g.dy + (long long)n0 * g.cohw, (uint32_t)(nimg0 * (long long)g.cohw * 4));
    d.buf = buf;
    d.sink = buf + g.stage - 64;
    const int y0 = a0 * g.S - g.pad;
    int ylo = y0 >= 0 ? 0 : (-y0 + g.xstep - 1) / g.xstep;
    int yhi = min(g.TIH, (g.H - y0 + g.xstep - 1) / g.xstep);
    if (yhi < ylo) yhi = ylo;
    const int rhi = min(g.TR, g.OH - a0);
    const int nimg = d.valid ? nimg0 : 0;
    const int xb = cib * 32 * g.hw + y0 * g.W, db = cob * 32 * g.ohw + a0 * g.OW;
#pragma unroll
    for (int j = 0; j < MT; j++) {
        {
            const int e = L.tx[j];
            const int ty = (e >> 16) & 255, img = e >> 24;
            const bool ok = (unsigned)(ty - ylo) < (unsigned)(yhi - ylo) && img < nimg;
            d.xo[j] = ok ? (uint32_t)(img * g.cihw + xb + (e & 0xFFFF)) * 4u : DMA_OOB;
        }
        {
            const int e = L.td[j];
            const int r = (e >> 16) & 255, img = e >> 24;
            const bool ok = r < rhi && img < nimg;
            d.dof[j] = ok ? (uint32_t)(img * g.cohw + db + (e & 0xFFFF)) * 4u : DMA_OOB;
        }
    }
    return d;
}

// DMA of all rows of block channel c (X and dY) of stage d.
template <int MT>
__device__ __forceinline__ void dw_issue_channel(const DwArgs &g, const DwStage<MT> &d, int c,
                                                 int cob, int cib, float *__restrict__ buf) {
    if (!d.valid) return;
    const uint32_t cx = cib * 32 + c < g.CI ? (uint32_t)(c * g.hw) * 4u : DMA_OOB;
    const uint32_t cd = cob * 32 + c < g.CO ? (uint32_t)(c * g.ohw) * 4u : DMA_OOB;
#pragma unroll
    for (int j = 0; j < MT; j++) {
        if (j < g.mx)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(d.rx, (lds_ptr_t)(buf + c * g.chsx + 64 * j), 4,
                                                     min(d.xo[j] + cx, DMA_OOB), 0, 0, 0);
        if (j < g.md)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                d.rd, (lds_ptr_t)(buf + g.xwords + c * g.chsd + 64 * j), 4,
                min(d.dof[j] + cd, DMA_OOB), 0, 0, 0);
    }
}

// Operands of one 8-pixel group.
template <int K, int S, bool X4 = false>
struct DwOps {
    float4 a;                                   // dY: pixels 4h .. 4h+3
    float4 x0[K];                               // X: 4 values from 4h (even part for S = 2)
    float2 x1[K];                               // X: the 2 values after them (X4: before them)
    float4 xo[(K == 3 && S == 2) ? K : 1];      // X odd columns (stride-2 3x3; X4: next 4)
    float xr[X4 ? K : 1];                       // X4: one more value (see dw_fetch)
};

template <int K, int S, bool X4>
__device__ __forceinline__ void dw_fetch(const DwArgs &g, const float *__restrict__ xs,
                                         const float *__restrict__ ds, int grp, int lane,
                                         DwOps<K, S, X4> &o) {
    const int h = lane >> 5, l32 = lane & 31;
    // group -> (tile row rr = img*TR + r, column group cq); the dY window is
    // dense in groups, so its offset is 8*grp
    const int rr = (int)fdiv((uint32_t)grp, g.fd_gpr), cq = grp - rr * g.gpr;
    const int img = (int)fdiv((uint32_t)rr, g.fd_tr), r = rr - img * g.TR;
    o.a = *reinterpret_cast<const float4 *>(ds + l32 * g.chsd + 8 * grp + 4 * h);
    const float *xr = xs + l32 * g.chsx + img * g.ximg + r * g.xrow * g.TIWP +
                      (X4 && S == 2 ? 16 * cq + 8 * h : 8 * cq + 4 * h);
#pragma unroll
    for (int kh = 0; kh < K; kh++) {
        if constexpr (X4 && S == 1) {
            // pixels ox0 = 8cq + 4h .. +3 read x = ox0 - 1 .. ox0 + 4, stored
            // at row column x + 4: x = ox0 - 2, ox0 - 1 / ox0 .. ox0 + 3 / ox0 + 4
            o.x1[kh] = *reinterpret_cast<const float2 *>(xr + kh * g.TIWP + 2);
            o.x0[kh] = *reinterpret_cast<const float4 *>(xr + kh * g.TIWP + 4);
            o.xr[kh] = xr[kh * g.TIWP + 8];
        } else if constexpr (X4) {
            // stride 2: pixels ox0 .. ox0 + 3 read x = 2ox0 - 1 .. 2ox0 + 7:
            // 2ox0 - 1 / 2ox0 .. +3 / 2ox0 + 4 .. +7 at row column x + 4
            o.xr[kh] = xr[kh * g.TIWP + 3];
            o.x0[kh] = *reinterpret_cast<const float4 *>(xr + kh * g.TIWP + 4);
            o.xo[kh] = *reinterpret_cast<const float4 *>(xr + kh * g.TIWP + 8);
        } else {
            o.x0[kh] = *reinterpret_cast<const float4 *>(xr + kh * g.TIWP);
            if constexpr (K == 3) {
                // 2 more values: b64 read of the next 4-aligned group
                o.x1[kh] = *reinterpret_cast<const float2 *>(xr + kh * g.TIWP + 4);
            }
            if constexpr (K == 3 && S == 2)
                o.xo[kh] = *reinterpret_cast<const float4 *>(xr + kh * g.TIWP + g.HE);
        }
    }
}

// B value of tap (kh, kw) for k-step i.
template <int K, int S, bool X4>
__device__ __forceinline__ float dw_bval(const DwOps<K, S, X4> &o, int kh, int kw, int i) {
    if constexpr (K == 1) {
        return o.x0[0][i];
    } else if constexpr (X4 && S == 1) {
        const int v = kw + i;  // x = ox0 - 1 + v
        return v == 0 ? o.x1[kh].y : (v < 5 ? o.x0[kh][v - 1] : o.xr[kh]);
    } else if constexpr (X4) {
        const int t = 2 * i + kw - 1;  // x = 2ox0 + t, t = -1 .. 7
        return t < 0 ? o.xr[kh] : (t < 4 ? o.x0[kh][t] : o.xo[kh][t - 4]);
    } else if constexpr (S == 1) {
        const int v = kw + i;  // compile-time after unrolling
        return v < 4 ? o.x0[kh][v] : (v == 4 ? o.x1[kh].x : o.x1[kh].y);
    } else {
        if (kw == 1) return o.xo[kh][i];
        const int v = i + (kw >> 1);
        return v < 4 ? o.x0[kh][v] : o.x1[kh].x;
    }
}

// DMA of a whole tile by producer wave pw: channels pw, pw + DW_NP, ...
template <int MT>
__device__ __forceinline__ void dw_issue_tile(const DwArgs &g, const DwLane<MT> &L, int tile,
                                              int cob, int cib, float *__restrict__ buf,
                                              int pw) {
    const DwStage<MT> d = dw_stage<MT>(g, L, tile, cob, cib, buf);
    for (int k = 0; k < 32 / DW_NP; k++)
        dw_issue_channel<MT>(g, d, pw + DW_NP * k, cob, cib, buf);
}

// 16-byte staging.  A 64-lane DMA instruction fills 64 consecutive 16-byte
// LDS chunks (1 KiB), lane i chunk i; instruction k of a tile's X (dY)
// region fills chunks 64k .. 64k + 63 of [channel][xchunks] ([channel]
// [dchunks]).  Which source chunk a lane loads depends only on k, the lane,
// the conv and its (co, ci) blocks, so each producer lane keeps its byte
// offsets for the whole job in registers -- one set per window kind, the
// first row (top padding) and / or the last row (bottom padding) left out --
// and a tile costs one buffer descriptor and the DMA instructions, with no
// per-row address arithmetic.  Chunks without source data (padding columns,
// padding rows, the odd-stride filler, channels past the convolution's) take
// an offset past every buffer and are written as zeros.
// X instructions per producer wave, at most: stride-2 windows hold about
// twice the rows (fewer table registers for stride 1 measured faster)
template <int S>
constexpr int dw4_xk() {
    return S == 1 ? 11 : 13;
}
constexpr int DW4_DK = 5;   // dY instructions per producer wave, at most

template <int S>
struct DwLane4 {
    static constexpr int XK = dw4_xk<S>();
    uint32_t xo[4][XK];  // window kind (bit 0: no first row, bit 1: no last row)
    uint32_t dof[DW4_DK];
};

template <int S>
__device__ __forceinline__ void dw_lane4_init(const DwArgs &g, DwLane4<S> &L, int pw, int lane,
                                              int cob, int cib) {
    const int rpi = g.TIH * g.rch;  // X chunks of one image's window
#pragma unroll
    for (int kk = 0; kk < DwLane4<S>::XK; kk++) {
        const int k = pw + DW_NP * kk;
        const int q = 64 * k + lane;
        const int c = q / g.xchunks, r = q - c * g.xchunks;
        const int img = r / rpi, rem = r - img * rpi;
        const int ty = rem / g.rch, m = rem - ty * g.rch;
        const bool ok = k < g.nix && c < 32 && cib * 32 + c < g.CI && r < g.xdata && m > 0 &&
                        m < g.rch - 1;
        const int e = img * g.cihw + c * g.hw + 4 * (m - 1);
#pragma unroll
        for (int w = 0; w < 4; w++) {
            // rows lo .. hi of the window hold image rows; offsets are taken
            // from the window's first such row
            const int lo = w & 1, hi = g.TIH - 1 - (w >> 1);
            const bool v = ok && ty >= lo && ty <= hi;
            L.xo[w][kk] = v ? (uint32_t)(e + (ty - lo) * g.W) * 4u : DMA_OOB;
        }
    }
    const int dpi = g.TR * (g.OW >> 2);  // dY chunks of one image's tile
#pragma unroll
    for (int kk = 0; kk < DW4_DK; kk++) {
        const int k = pw + DW_NP * kk;
        const int q = 64 * k + lane;
        const int c = q / g.dchunks, r = q - c * g.dchunks;
        const int img = r / dpi, rem = r - img * dpi;
        const bool ok = k < g.nid && c < 32 && cob * 32 + c < g.CO && r < g.ddata;
        L.dof[kk] = ok ? (uint32_t)(img * g.cohw + c * g.ohw + 4 * rem) * 4u : DMA_OOB;
    }
}

// All DMA of one tile by producer wave pw (whole tiles: n0 + IMGS <= N and
// a0 + TR <= OH).  The descriptors start at the tile's first image row that
// the window reads (X) and at its first output row (dY) and end with the
// tile's last image, so every chunk with source data lies inside them.
template <int S>
__device__ __forceinline__ void dw_issue_tile4(const DwArgs &g, const DwLane4<S> &L, int tile,
                                               int cob, int cib, float *__restrict__ buf, int pw) {
    if (tile >= g.ntiles) return;
    const int n0 = (tile / g.tiles_a) * g.IMGS, a0 = (tile % g.tiles_a) * g.TR;
    const int y0 = a0 * g.S - g.pad;
    const int kind = (y0 < 0 ? 1 : 0) | (y0 + g.TIH - 1 >= g.H ? 2 : 0);
    const long long xend = (long long)(n0 + g.IMGS) * g.cihw;
    const long long xo = (long long)n0 * g.cihw + (long long)cib * 32 * g.hw +
                         (long long)max(y0, 0) * g.W;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(g.x + xo, (uint32_t)((xend - xo) * 4));
    const long long dend = (long long)(n0 + g.IMGS) * g.cohw;
    const long long dq = (long long)n0 * g.cohw + (long long)cob * 32 * g.ohw + (long long)a0 * g.OW;
    const __amdgpu_buffer_rsrc_t rd = make_rsrc(g.dy + dq, (uint32_t)((dend - dq) * 4));
    auto issue_x = [&](auto wc) {
        constexpr int w = decltype(wc)::value;
#pragma unroll
        for (int kk = 0; kk < DwLane4<S>::XK; kk++)
            if (pw + DW_NP * kk < g.nix)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rx, (lds_ptr_t)(buf + (pw + DW_NP * kk) * 256), 16, L.xo[w][kk], 0, 0, 0);
    };
    switch (kind) {
        case 0: issue_x(std::integral_constant<int, 0>()); break;
        case 1: issue_x(std::integral_constant<int, 1>()); break;
        case 2: issue_x(std::integral_constant<int, 2>()); break;
        default: issue_x(std::integral_constant<int, 3>()); break;
    }
#pragma unroll
    for (int kk = 0; kk < DW4_DK; kk++)
        if (pw + DW_NP * kk < g.nid)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rd, (lds_ptr_t)(buf + g.xwords + (pw + DW_NP * kk) * 256), 16, L.dof[kk], 0, 0, 0);
}

// MFMAs of one 8-pixel group for taps T0 .. T0 + NT - 1 (a 1x1 kernel: the
// four k-steps into four accumulators): k-step i takes pixels i and 4 + i.
template <int K, int S, bool X4, int T0, int NT>
__device__ __forceinline__ void dw_mma(const DwOps<K, S, X4> &o, f32x16 (&acc)[NT]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if constexpr (K == 1) {
            acc[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(o.a[i], dw_bval<K, S, X4>(o, 0, 0, i),
                                                          acc[i], 0, 0, 0);
        } else {
#pragma unroll
            for (int j = 0; j < NT; j++)
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                    o.a[i], dw_bval<K, S, X4>(o, (T0 + j) / K, (T0 + j) % K, i), acc[j], 0, 0, 0);
        }
    }
}

// Scheduling hint for one step: the LDS reads of the next group go out
// among the first MFMAs of this one, so their latency hides under the rest.
template <int K, int S, bool X4, int NT>
__device__ __forceinline__ void dw_step_schedule() {
    constexpr int NMF = K == 1 ? 4 : 4 * NT;
    constexpr int NRD = 1 + (K == 1 ? 1 : K * (S == 2 || X4 ? 3 : 2));
    static_for<0, NRD>([&](auto) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 LDS read
    });
    __builtin_amdgcn_sched_group_barrier(0x008, NMF - NRD, 0);
}

// The GEMM steps of one staged tile: 8-pixel groups wave, wave + NW, ...;
// two operand sets alternate so that the reads of group n+1 overlap the
// MFMAs of group n.  Reads past the tile's last group are clamped to group
// `wave` (in range; their values are not used).
template <int K, int S, bool X4, int T0, int NT>
__device__ __forceinline__ void dw_compute(const DwArgs &g, const float *__restrict__ cur,
                                           int wave, int lane, f32x16 (&acc)[NT]) {
    const float *xs = cur, *ds = cur + g.xwords;
    const int nsteps = (g.ngroups - wave + DW_NW - 1) / DW_NW;
    auto grp = [&](int s) {
        const int gi = wave + DW_NW * s;
        return gi < g.ngroups ? gi : min(wave, g.ngroups - 1);
    };
    DwOps<K, S, X4> oa, ob;
    dw_fetch<K, S, X4>(g, xs, ds, grp(0), lane, oa);
#pragma unroll 1
    for (int s = 0; s < nsteps; s += 2) {
        dw_fetch<K, S, X4>(g, xs, ds, grp(s + 1), lane, ob);
        dw_mma<K, S, X4, T0, NT>(oa, acc);
        dw_step_schedule<K, S, X4, NT>();
        if (s + 1 >= nsteps) break;
        dw_fetch<K, S, X4>(g, xs, ds, grp(s + 2), lane, oa);
        dw_mma<K, S, X4, T0, NT>(ob, acc);
        dw_step_schedule<K, S, X4, NT>();
    }
}

// Accumulator v of tap t (accumulator j = t - T0 of this wave) of this lane
// lives at slab-order slot ((8*(v/4) + 4*h + v%4)*32 + l32)*KK + t =
// (lbase + 32*(8*(v/4) + v%4))*KK + t.
template <int KK, int T0, int NT>
__device__ __forceinline__ void dw_red_store(float *dst, int lbase, const f32x16 *acc) {
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
        for (int v = 0; v < 16; v++)
            dst[(lbase + 32 * (8 * (v >> 2) + (v & 3))) * KK + T0 + j] = acc[j][v];
}

template <int KK, int T0, int NT>
__device__ __forceinline__ void dw_red_add(const float *src, int lbase, f32x16 *acc) {
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
        for (int v = 0; v < 16; v++)
            acc[j][v] += src[(lbase + 32 * (8 * (v >> 2) + (v & 3))) * KK + T0 + j];
}

// An MFMA wave of tap group (T0, NT): tiles z, z + nz, ... (the same
// barriers as the producers, one per tile, two with a single buffer), then
// the sum of the DW_NW waves of the group in a fixed order, (w0 + w2) + (w1
// + w3), through two LDS slices in slab order [co][ci][tap]
// (bit-reproducible).  The groups' taps are disjoint, so both groups use
// the same slices at once.
template <int K, int S, bool X4, int NB, int T0, int NT>
__device__ __forceinline__ void dw_mfma_wave(const DwArgs &g, float *smem, float *red, int z,
                                             int wq, int lane) {
    constexpr int KK = K * K, SL = KK * 1024, NR = K == 1 ? 1 : NT;
    f32x16 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[t][v] = 0.f;
    int s = 0;
    for (int tile = z; tile < g.ntiles; tile += g.nz, s++) {
        dma_wait_barrier();
        if constexpr (NB == 2) {
            dw_compute<K, S, X4, T0, NT>(g, smem + (s & 1) * g.stage, wq, lane, acc);
        } else {
            dw_compute<K, S, X4, T0, NT>(g, smem, wq, lane, acc);
            __syncthreads();
        }
    }
    if constexpr (K == 1) {
#pragma unroll
        for (int v = 0; v < 16; v++)
            acc[0][v] = (acc[0][v] + acc[1][v]) + (acc[2][v] + acc[3][v]);
    }
    static_assert(DW_NW == 4, "reduction order written for four MFMA waves per group");
    dma_wait_barrier();
    const int lbase = 4 * (lane >> 5) * 32 + (lane & 31);  // slot of (v = 0, t = 0)
    if (wq >= 2) dw_red_store<KK, T0, NR>(red + (wq - 2) * SL, lbase, acc);
    __syncthreads();
    if (wq < 2) dw_red_add<KK, T0, NR>(red + wq * SL, lbase, acc);
    __syncthreads();
    if (wq < 2) dw_red_store<KK, T0, NR>(red + wq * SL, lbase, acc);
    __syncthreads();
}

// Waves 0 .. 4*NG-1 compute: wave w takes the pixel groups w%4, w%4 + 4, ...
// of every tile for the taps of group w/4 (3x3: taps 0-4, then 5-8); the
// last 4 waves only stage tiles by DMA, so that the memory pipeline's
// back-pressure never stalls an MFMA wave.  Double-buffered plans (NB = 2)
// stage the next tile while this one is computed (one barrier per tile);
// single-buffered plans stage it after the compute barrier.
// MT = 0: the 16-byte staging of a 3x3 pad-1 plan (whole tiles).
template <int K, int S, int MT, int NB>
__device__ __forceinline__ void dw_body(const DwArgs &g, int z, int cob, int cib) {
    constexpr int KK = K * K, NG = dw_tap_groups<K>(), NMW = DW_NW * NG;
    constexpr bool X4 = MT == 0;
    static_assert(!X4 || (K == 3 && NB == 2), "16-byte staging: 3x3, two buffers");
    extern __shared__ float smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_index();
    float *red = smem;  // after the tiles: 2 slices of [32][32][KK]
    const int SL = KK * 1024;
    if (wave >= NMW) {
        // producer: the same barriers as the MFMA waves, one per tile (two
        // with a single buffer), then those of the reduction
        const int pw = wave - NMW;
        if constexpr (X4) {
            DwLane4<S> L;
            dw_lane4_init<S>(g, L, pw, lane, cob, cib);
            dw_issue_tile4<S>(g, L, z, cob, cib, smem, pw);
            int s = 0;
            for (int tile = z; tile < g.ntiles; tile += g.nz, s++) {
                dma_wait_barrier();
                if (tile + g.nz < g.ntiles)
                    dw_issue_tile4<S>(g, L, tile + g.nz, cob, cib, smem + ((s + 1) & 1) * g.stage,
                                      pw);
            }
        } else {
            DwLane<MT> L;
            dw_lane_init<K, S, MT>(g, L, lane);
            dw_issue_tile<MT>(g, L, z, cob, cib, smem, pw);
            int s = 0;
            for (int tile = z; tile < g.ntiles; tile += g.nz, s++) {
                dma_wait_barrier();
                const bool more = tile + g.nz < g.ntiles;
                if constexpr (NB == 2) {
                    if (more)
                        dw_issue_tile<MT>(g, L, tile + g.nz, cob, cib,
                                          smem + ((s + 1) & 1) * g.stage, pw);
                } else {
                    __syncthreads();
                    if (more) dw_issue_tile<MT>(g, L, tile + g.nz, cob, cib, smem, pw);
                }
            }
        }
        dma_wait_barrier();
        __syncthreads();
        __syncthreads();
        __syncthreads();
    } else if constexpr (K == 1) {
        dw_mfma_wave<K, S, X4, NB, 0, 4>(g, smem, red, z, wave, lane);
    } else if (wave < DW_NW) {
        dw_mfma_wave<K, S, X4, NB, 0, 5>(g, smem, red, z, wave, lane);
    } else {
        dw_mfma_wave<K, S, X4, NB, 5, KK - 5>(g, smem, red, z, wave - DW_NW, lane);
    }
    const int ckk = g.CI * KK, rowlen = 32 * KK;
    float *slab = g.part + (long long)z * g.CO * ckk + cib * 32 * KK;
    const int rlim = min(32, g.CI - cib * 32) * KK;
    for (int e = tid; e < SL; e += dw_threads<K>()) {
        const int co = e / rowlen, rem = e - co * rowlen;
        const float v = red[e] + red[SL + e];
        if (cob * 32 + co < g.CO && rem < rlim) slab[(long long)(cob * 32 + co) * ckk + rem] = v;
    }
}

template <int K, int S, int MT, int NB>
__global__ __launch_bounds__(dw_threads<K>()) void conv_dw_kernel(DwArgs g) {
    dw_body<K, S, MT, NB>(g, blockIdx.x, blockIdx.y, blockIdx.z);
}

// The weight gradients of several convolutions of one kernel shape in one
// launch (a network's backward, once every output gradient exists): a
// workgroup takes job blockIdx.x = (conv, slab z, co block, ci block),
// packed conv | z << 8 | cob << 20 | cib << 26, and runs that conv's plan
// tab[conv] exactly as conv_dw_kernel runs workgroup (z, cob, cib).  One
// launch pays the ramp, the first tile's DMA and the epilogue once instead
// of once per conv, and each conv can take far fewer, longer slabs.
template <int K, int S, int MT, int NB>
__global__ __launch_bounds__(dw_threads<K>()) void conv_dw_group_kernel(
    const DwArgs *__restrict__ tab, const uint32_t *__restrict__ jobs) {
    const uint32_t j = jobs[blockIdx.x];
    dw_body<K, S, MT, NB>(tab[j & 255u], (int)((j >> 8) & 4095u), (int)((j >> 20) & 63u),
                          (int)(j >> 26));
}

// out[e] += sum over slabs z of part[z][e], in slab order, in one launch: a
// block takes 32 elements; thread (j, e) sums slabs [j*G, j*G + G) with its
// loads issued ahead of the in-order adds, then the 8 partials are added in
// j order (a fixed order: bit-reproducible).
constexpr int DW_RED_PARTS = 8;
__global__ __launch_bounds__(256) void slab_reduce_kernel(const float *part, int nz, long long len,
                                                          float *out) {
    __shared__ float red[DW_RED_PARTS][32];
    const int el = threadIdx.x & 31, j = threadIdx.x >> 5;
    const long long e = (long long)blockIdx.x * 32 + el;
    const int G = (nz + DW_RED_PARTS - 1) / DW_RED_PARTS;
    const int z0 = j * G, z1 = min(nz, z0 + G);
    float s = 0.f;
    if (e < len) {
        for (int b = z0; b < z1; b += 16) {
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; u++) v[u] = b + u < z1 ? part[(long long)(b + u) * len + e] : 0.f;
#pragma unroll
            for (int u = 0; u < 16; u++)
                if (b + u < z1) s = (b + u == z0) ? v[u] : s + v[u];
        }
    }
    red[j][el] = s;
    __syncthreads();
    if (j == 0 && e < len) {
        float t = red[0][el];
        for (int q = 1; q < DW_RED_PARTS && q * G < nz; q++) t += red[q][el];
        out[e] += t;
    }
}

// Weight gradient of a 3x3 stride-1 convolution with few input channels
// (cin * 9 <= 32, the network stem): the im2col rows (ci, kh, kw), numbered
// r = ci*9 + kh*3 + kw as conv.rs's RowMap numbers them, make up a single
// 32-wide MFMA N block, so a pixel pair costs one MFMA where the tap kernel
// above spends nine 32x32 taps on zero-padded channels.
//   * a workgroup (4 waves) takes the tiles z, z + nz, ... : SMC_R output
//     rows of one image, full width; it stages dY [32 co][pixels] and the
//     zero-padded X window [ci][R + 2][OW + 2] in LDS with plain loads;
//   * MFMA k-step = a pixel pair: lane l reads dY[co = l%32][p] and
//     X[ci][r + kh][c + kw] for column n = l%32 (0 for n >= cin*9), where
//     p = 2q + l/32 is pixel (r, c) of the tile; wave w takes the pairs
//     w, w + 4, ... into two alternating accumulators;
//   * the 4 waves are added through LDS in the order (w0 + w1) + (w2 + w3),
//     and the workgroup writes slab z; slabs are summed in slab order as for
//     the tap kernel (bit-reproducible).
constexpr int SMC_THREADS = 256;
constexpr int SMC_PIX = 256;             // pixels per tile (at most; = SMC_THREADS)
constexpr int SMC_DS = SMC_PIX + 1;      // LDS row stride of dY (conflict-free reads)
constexpr int SMC_XMAX = 3 * 1300;       // LDS floats of the X window
constexpr int SMC_RS = 33;               // row stride of the reduction slices

struct DwSmallArgs {
    const float *dy, *x;
    float *part;  // [nz][CO][CI*9]
    int N, CO, CI, H, W, OH, OW, pad;
    int R, tiles_a, ntiles;
    int vec;                   // OW % 4 == 0 and dY 16-byte aligned: float4 dY loads
    FastDiv fd_xplane, fd_xw;  // X window plane (R + 2) * (OW + 2) and row OW + 2
};

__global__ __launch_bounds__(SMC_THREADS) void conv_dw_smallc_kernel(DwSmallArgs g) {
    __shared__ float sdy[32 * SMC_DS];
    __shared__ float sx[SMC_XMAX];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int z = blockIdx.x, nz = gridDim.x, cob = blockIdx.y;
    const int n = lane & 31, kidx = lane >> 5;
    const int NV = g.CI * 9, XW = g.OW + 2, XR = g.R + 2;
    // this lane's B column: (ci, kh, kw) of im2col row n
    const int bci = n < NV ? n / 9 : 0, bkh = n < NV ? (n % 9) / 3 : 0,
              bkw = n < NV ? n % 3 : 0;
    const int boff = (bci * XR + bkh) * XW + bkw;
    const int tpix = g.R * g.OW;
    f32x16 acc0, acc1;
#pragma unroll
    for (int v = 0; v < 16; v++) acc0[v] = acc1[v] = 0.f;
    for (int tile = z; tile < g.ntiles; tile += nz) {
        const int img = tile / g.tiles_a, a0 = (tile % g.tiles_a) * g.R;
        const int rows = min(g.R, g.OH - a0), npix = rows * g.OW;
        __syncthreads();  // the previous tile's reads are done
        const float *dsrc = g.dy + ((long long)img * g.CO + cob * 32) * g.OH * g.OW +
                            (long long)a0 * g.OW;
        // all loads of the tile are issued before the first LDS store
        const long long cst = (long long)g.OH * g.OW;
        if (g.vec) {
            // 16-byte loads: thread (co4 = tid / 64, j = tid % 64) takes
            // pixels 4j .. 4j+3 of output channels co4, co4 + 4, ...
            const int j = tid & 63, co4 = tid >> 6, p = 4 * j;
            float4 v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int co = co4 + 4 * k;
                v[k] = float4{0.f, 0.f, 0.f, 0.f};
                if (p < npix && cob * 32 + co < g.CO)
                    v[k] = *reinterpret_cast<const float4 *>(dsrc + co * cst + p);
            }
            if (p < tpix) {
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    float *d = sdy + (co4 + 4 * k) * SMC_DS + p;
                    d[0] = v[k].x;
                    d[1] = v[k].y;
                    d[2] = v[k].z;
                    d[3] = v[k].w;
                }
            }
        } else if (tid < tpix) {  // tpix <= SMC_PIX = SMC_THREADS
            const bool okp = tid < npix;
            float v[32];
#pragma unroll
            for (int co = 0; co < 32; co++) {
                v[co] = 0.f;
                if (okp && cob * 32 + co < g.CO) v[co] = dsrc[co * cst + tid];
            }
#pragma unroll
            for (int co = 0; co < 32; co++) sdy[co * SMC_DS + tid] = v[co];
        }
        const float *xsrc = g.x + (long long)img * g.CI * g.H * g.W;
        const int xtot = g.CI * XR * XW;
        float xv[SMC_XMAX / SMC_THREADS + 1];
#pragma unroll
        for (int k = 0; k <= SMC_XMAX / SMC_THREADS; k++) {
            const int e = tid + k * SMC_THREADS;
            const int ci = (int)fdiv((uint32_t)e, g.fd_xplane), rem = e - ci * (XR * XW);
            const int t = (int)fdiv((uint32_t)rem, g.fd_xw), u = rem - t * XW;
            const int y = a0 - g.pad + t, x = u - g.pad;
            xv[k] = 0.f;
            if (e < xtot && y >= 0 && y < g.H && x >= 0 && x < g.W)
                xv[k] = xsrc[((long long)ci * g.H + y) * g.W + x];
        }
#pragma unroll
        for (int k = 0; k <= SMC_XMAX / SMC_THREADS; k++) {
            const int e = tid + k * SMC_THREADS;
            if (e < xtot) sx[e] = xv[k];
        }
        __syncthreads();
        const int npairs = (npix + 1) >> 1;
        for (int q = wave; q < npairs; q += 8) {
#pragma unroll
            for (int h2 = 0; h2 < 2; h2++) {
                const int qq = q + 4 * h2;
                const int p = 2 * qq + kidx;
                const bool ok = qq < npairs && p < npix;
                const int pc = ok ? p : 0;
                const int r = pc / g.OW, c = pc - r * g.OW;
                const float a = ok ? sdy[n * SMC_DS + pc] : 0.f;
                const float b = n < NV ? sx[boff + r * XW + c] : 0.f;
                if (h2 == 0)
                    acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc0, 0, 0, 0);
                else
                    acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc1, 0, 0, 0);
            }
        }
    }
    // acc register v of lane l: D row (co) 8*(v/4) + 4*(l/32) + v%4, column n = l%32
    __syncthreads();
    float *red = sdy;  // 4 slices of [32][SMC_RS]
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const int co = 8 * (v >> 2) + 4 * kidx + (v & 3);
        red[(wave * 32 + co) * SMC_RS + n] = acc0[v] + acc1[v];
    }
    __syncthreads();
    float *slab = g.part + (long long)z * g.CO * NV;
    for (int e = tid; e < 32 * NV; e += SMC_THREADS) {
        const int co = e / NV, col = e - co * NV;
        if (cob * 32 + co >= g.CO) continue;
        const float v = (red[co * SMC_RS + col] + red[(32 + co) * SMC_RS + col]) +
                        (red[(64 + co) * SMC_RS + col] + red[(96 + co) * SMC_RS + col]);
        slab[(long long)(cob * 32 + co) * NV + col] = v;
    }
}

constexpr int DW_MT[3] = {2, 4, 8};

// Geometry of a (TR, IMGS) tile; returns LDS bytes, 0 if the tile does not
// fit the kernel's tables and formats.
size_t dw_geometry(DwArgs &g, int K, int TR, int IMGS, int nbuf) {
    g.nbuf = nbuf;
    const int S = g.S;
    g.TR = TR;
    g.IMGS = IMGS;
    g.gpr = g.OWP / 8;
    g.ngroups = IMGS * TR * g.gpr;
    if (K == 1) {
        g.xrow = 1;
        g.xstep = S;
        g.TIH = TR;
        g.TIWP = g.OWP;
        g.HE = 0;
    } else {
        g.xrow = S;
        g.xstep = 1;
        g.TIH = (TR - 1) * S + K;
        if (S == 1) {
            g.TIWP = g.OWP + 4;
            g.HE = 0;
        } else {
            g.HE = g.OWP + 4;
            g.TIWP = g.HE + g.OWP;
        }
    }
    g.fd_gpr = make_fastdiv(g.gpr);
    g.fd_tr = make_fastdiv(TR);
    g.ximg = g.TIH * g.TIWP;
    g.dimg = TR * g.OWP;
    g.fd_ximg = make_fastdiv(g.ximg);
    g.fd_tiwp = make_fastdiv(g.TIWP);
    g.fd_dimg = make_fastdiv(g.dimg);
    g.fd_owp = make_fastdiv(g.OWP);
    g.mx = (IMGS * g.ximg + 63) / 64;
    g.md = (IMGS * g.dimg + 63) / 64;
    if (std::max(g.mx, g.md) > DW_MT[2] || g.TIH > 254 || IMGS > 127) return 0;
    if ((long long)g.TIH * g.xstep * g.W > 0xFFFF || (long long)TR * g.OW > 0xFFFF) return 0;
    g.chsx = 64 * g.mx + 4;
    g.chsd = 64 * g.md + 4;
    g.xwords = 32 * g.chsx;
    g.stage = g.xwords + 32 * g.chsd + 64;
    return std::max((size_t)nbuf * g.stage * 4, (size_t)(DW_NW / 2) * K * K * 1024 * 4);
}

// Geometry of a (TR, IMGS) tile of the 16-byte staging (3x3 pad 1, stride 1
// or 2 with W = S*OW and H = S*OH, OW a multiple of 8, whole tiles); returns
// LDS bytes, 0 if the shape or tile does not qualify.  A stride-2 window
// holds 2 TR + 1 image rows (the last one always inside the image).
size_t dw_geometry4(DwArgs &g, int TR, int IMGS, size_t n) {
    if ((g.S != 1 && g.S != 2) || g.pad != 1 || g.W != g.S * g.OW || g.H != g.S * g.OH ||
        (g.OW & 7) || (g.W & 3) || g.OH % TR || (long long)n % IMGS)
        return 0;
    g.nbuf = 2;
    g.TR = TR;
    g.IMGS = IMGS;
    g.OWP = g.OW;
    g.gpr = g.OW / 8;
    g.ngroups = IMGS * TR * g.gpr;
    g.xrow = g.S;
    g.xstep = 1;
    g.TIH = (TR - 1) * g.S + 3;
    g.HE = 0;
    g.rch = g.W / 4 + 2;
    g.TIWP = 4 * g.rch;
    g.ximg = g.TIH * g.TIWP;
    g.dimg = TR * g.OW;
    g.fd_gpr = make_fastdiv(g.gpr);
    g.fd_tr = make_fastdiv(TR);
    g.fd_ximg = make_fastdiv(g.ximg);
    g.fd_tiwp = make_fastdiv(g.TIWP);
    g.fd_dimg = make_fastdiv(g.dimg);
    g.fd_owp = make_fastdiv(g.OWP);
    g.xdata = IMGS * g.TIH * g.rch;
    g.xchunks = g.xdata | 1;
    g.ddata = IMGS * TR * g.OW / 4;
    g.dchunks = g.ddata | 1;
    g.nix = (32 * g.xchunks + 63) / 64;
    g.nid = (32 * g.dchunks + 63) / 64;
    const int xk = g.S == 1 ? dw4_xk<1>() : dw4_xk<2>();
    if (g.nix > DW_NP * xk || g.nid > DW_NP * DW4_DK || IMGS > 127) return 0;
    g.mx = g.md = 0;
    g.chsx = 4 * g.xchunks;
    g.chsd = 4 * g.dchunks;
    g.xwords = g.nix * 256;
    g.stage = g.xwords + g.nid * 256;
    return std::max((size_t)2 * g.stage * 4, (size_t)(DW_NW / 2) * 9 * 1024 * 4);
}

template <int K, int S, int MT, int NB>
const void *dw_kernel_ptr() {
    static bool attr = false;
    const void *k = (const void *)conv_dw_kernel<K, S, MT, NB>;
    if (!attr) {
        attr = true;
        (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    }
    return k;
}

template <int K, int S, int NB>
const void *dw_pick_mt(int mt) {
    if (mt <= DW_MT[0]) return dw_kernel_ptr<K, S, DW_MT[0], NB>();
    if (mt <= DW_MT[1]) return dw_kernel_ptr<K, S, DW_MT[1], NB>();
    return dw_kernel_ptr<K, S, DW_MT[2], NB>();
}

template <int K, int S>
const void *dw_pick(int mt, int nb) {
    return nb == 2 ? dw_pick_mt<K, S, 2>(mt) : dw_pick_mt<K, S, 1>(mt);
}

template <int S, int MT>
const void *dw_group_ptr() {
    static bool attr = false;
    const void *k = (const void *)conv_dw_group_kernel<3, S, MT, 2>;
    if (!attr) {
        attr = true;
        (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    }
    return k;
}

// The grouped kernel (3x3, double-buffered tiles) for stride s and tables of
// mt DMA rows (mt = 0: the 16-byte staging).
const void *dw_group_pick(int s, int mt) {
    if (s == 1) {
        if (mt == 0) return dw_group_ptr<1, 0>();
        if (mt <= DW_MT[0]) return dw_group_ptr<1, DW_MT[0]>();
        if (mt <= DW_MT[1]) return dw_group_ptr<1, DW_MT[1]>();
        return dw_group_ptr<1, DW_MT[2]>();
    }
    if (mt == 0) return dw_group_ptr<2, 0>();
    if (mt <= DW_MT[0]) return dw_group_ptr<2, DW_MT[0]>();
    if (mt <= DW_MT[1]) return dw_group_ptr<2, DW_MT[1]>();
    return dw_group_ptr<2, DW_MT[2]>();
}

}  // namespace

// dW += sum over images (see above).  k must be 1 or 3, stride 1 or 2.
// Plan of one dW launch: kernel arguments (slab pointer unset), kernel, LDS
// bytes and the grid (NZ slabs x output-channel blocks x input-channel blocks).
struct DwLaunch {
    DwArgs g;
    DwSmallArgs gs;  // the few-input-channel kernel's arguments (small)
    bool small = false;
    const void *kern;
    size_t lds;
    dim3 grid;
    int threads;
    int nz;      // slabs
    size_t len;  // floats of one slab: cout * cin * k * k
    void set_part(float *p) {
        if (small)
            gs.part = p;
        else
            g.part = p;
    }
    void *arg() { return small ? (void *)&gs : (void *)&g; }
};

// Plan of the few-input-channel kernel (3x3, stride 1, cin * 9 <= 32), or
// false when the shape is not one.
static bool dw_small_plan(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *dy,
                          const float *x, DwLaunch &L) {
    if (sp->k != 3 || sp->stride != 1 || sp->cin * 9 > 32 || sp->ow > SMC_PIX || n == 0)
        return false;
    DwSmallArgs a;
    std::memset(&a, 0, sizeof(a));
    a.dy = dy;
    a.x = x;
    a.N = (int)n;
    a.CO = sp->cout;
    a.CI = sp->cin;
    a.H = sp->h;
    a.W = sp->w;
    a.OH = sp->oh;
    a.OW = sp->ow;
    a.pad = sp->pad;
    // every row start of dY is then 16-byte aligned too (OW, OH*OW multiples of 4)
    a.vec = (a.OW & 3) == 0 && ((uintptr_t)dy & 15) == 0;
    a.R = std::max(1, std::min(SMC_PIX / a.OW, a.OH));
    if ((long long)a.CI * (a.R + 2) * (a.OW + 2) > SMC_XMAX) return false;
    if ((long long)n * std::max((long long)a.CI * a.H * a.W, (long long)a.CO * a.OH * a.OW) >=
        (1ll << 40))
        return false;
    a.tiles_a = (a.OH + a.R - 1) / a.R;
    a.ntiles = a.tiles_a * (int)n;
    a.fd_xplane = make_fastdiv((a.R + 2) * (a.OW + 2));
    a.fd_xw = make_fastdiv(a.OW + 2);
    const int ncb = (a.CO + 31) / 32;
    static int occ = 0;
    if (occ == 0 && (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                         &occ, (const void *)conv_dw_smallc_kernel, SMC_THREADS, 0) != hipSuccess ||
                     occ < 1))
        occ = 1;
    const int nz = std::min(std::max(1, occ * ctx->num_cus / ncb), a.ntiles);
    L.small = true;
    L.gs = a;
    L.kern = (const void *)conv_dw_smallc_kernel;
    L.lds = 0;
    L.grid = dim3(nz, ncb, 1);
    L.threads = SMC_THREADS;
    L.nz = nz;
    L.len = (size_t)a.CO * a.CI * 9;
    return true;
}

static int dw_plan(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *dy,
                   const float *x, DwLaunch &L) {
    if (dw_small_plan(ctx, sp, n, dy, x, L)) return RNN_OK;
    const int K = sp->k;
    if (K != 1 && K != 3) return rnn_fail(ctx, RNN_E_UNSUPPORTED, "conv dW: k must be 1 or 3");
    if (sp->stride != 1 && sp->stride != 2)
        return rnn_fail(ctx, RNN_E_UNSUPPORTED, "conv dW: stride must be 1 or 2");
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
    g.S = sp->stride;
    g.pad = sp->pad;
    g.OWP = (sp->ow + 7) & ~7;
    g.hw = g.H * g.W;
    g.ohw = g.OH * g.OW;
    if ((long long)g.CI * g.hw >= (1ll << 24) || (long long)g.CO * g.ohw >= (1ll << 24))
        return rnn_fail(ctx, RNN_E_UNSUPPORTED, "conv dW: image planes beyond 2^24 elements");
    g.cihw = g.CI * g.hw;
    g.cohw = g.CO * g.ohw;
    // Plan: RNN_DW_PLAN="TR,IMGS,NZ[,NBUF]" overrides (tuning sweeps).
    // Otherwise the tile (TR rows of IMGS images) with the most useful
    // 8-pixel groups -- groups times the fraction of tile rows inside the
    // image -- whose two stage buffers fit in LDS (one workgroup per CU, so
    // staging must overlap compute) with at most 4 DMA rows per channel (the
    // 8-row lane tables cost registers); larger tables, then a single buffer,
    // only when nothing smaller fits.
    int TR = 0, IMGS = 0, NZ = 0, NB = 0;
    size_t lds = 0;
    if (const char *env = getenv("RNN_DW_PLAN")) {
        if (sscanf(env, "%d,%d,%d,%d", &TR, &IMGS, &NZ, &NB) < 3) TR = IMGS = NZ = 0;
        if (NB != 1) NB = 2;
        if (TR > 0 && IMGS > 0) {
            TR = std::min(TR, g.OH);
            lds = dw_geometry(g, K, TR, IMGS, NB);
            if (lds == 0 || lds > 160 * 1024) TR = 0;
        }
    }
    const int ncb = (g.CO + 31) / 32, ncib = (g.CI + 31) / 32;
    auto kernel_of = [&](const DwArgs &a) -> const void * {
        const int mt = std::max(a.mx, a.md);
        if (K == 3 && mt == 0)  // 16-byte staging
            return a.S == 1 ? dw_kernel_ptr<3, 1, 0, 2>() : dw_kernel_ptr<3, 2, 0, 2>();
        if (K == 3)
            return a.S == 1 ? dw_pick<3, 1>(mt, a.nbuf) : dw_pick<3, 2>(mt, a.nbuf);
        return a.S == 1 ? dw_pick<1, 1>(mt, a.nbuf) : dw_pick<1, 2>(mt, a.nbuf);
    };
    auto slabs_of = [&](const void *kern, size_t l, int ntiles) {
        // occupancy per (kernel, LDS bytes), cached: the planner asks for
        // every candidate tile on every call
        static std::mutex mu;
        static std::map<std::pair<const void *, size_t>, int> cache;
        int occ = 0;
        {
            std::lock_guard<std::mutex> lk(mu);
            auto it = cache.find({kern, l});
            if (it != cache.end()) {
                occ = it->second;
            } else {
                if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, dw_threads_of(K), l) !=
                        hipSuccess ||
                    occ < 1)
                    occ = 1;
                cache[{kern, l}] = occ;
            }
        }
        return std::min(std::max(1, occ * ctx->num_cus / (ncb * ncib)), ntiles);
    };
    // 16-byte staging for 3x3 stride-1 pad-1 shapes with whole tiles
    // (RNN_DW_X4=0: the 4-byte staging everywhere)
    const char *x4env = getenv("RNN_DW_X4");
    const bool try4 = K == 3 && !(x4env && x4env[0] == '0');
    bool use4 = false;
    if (TR > 0 && IMGS > 0 && try4 && NB == 2) {
        DwArgs t = g;
        use4 = dw_geometry4(t, TR, IMGS, n) != 0;
    }
    if (TR <= 0 || IMGS <= 0) {
        // The tile with the shortest critical path: every workgroup walks
        // ceil(ntiles / NZ) tiles of ngroups 8-pixel groups plus a fixed
        // per-tile cost (the barrier and the restart of the operand
        // pipeline, about two groups).  The 16-byte staging first, then
        // double-buffered plans; a single buffer only when no
        // double-buffered tile fits.
        double best = 0;
        if (try4)
            for (int tr = 1; tr <= g.OH; tr++)
                for (int im = 1; im <= (tr == g.OH ? 16 : 1); im *= 2) {
                    const size_t l = dw_geometry4(g, tr, im, n);
                    if (l == 0 || l > 160 * 1024) continue;
                    const int ntiles = (g.OH / tr) * (int)(n / im);
                    const int nz = slabs_of(kernel_of(g), l, ntiles);
                    const double cost = (double)((ntiles + nz - 1) / nz) * (g.ngroups + 2);
                    if (best == 0 || cost < best) {
                        best = cost;
                        TR = tr;
                        IMGS = im;
                        NB = 2;
                        use4 = true;
                    }
                }
        for (int nb = 2; nb >= 1 && best == 0; nb--)
            for (int tr = 1; tr <= g.OH; tr++)
                for (int im = 1; im <= (tr == g.OH ? 16 : 1); im *= 2) {
                    const size_t l = dw_geometry(g, K, tr, im, nb);
                    if (l == 0 || l > 160 * 1024) continue;
                    const int ntiles = ((g.OH + tr - 1) / tr) * (int)((n + im - 1) / im);
                    const int nz = slabs_of(kernel_of(g), l, ntiles);
                    const double cost = (double)((ntiles + nz - 1) / nz) * (g.ngroups + 2);
                    if (best == 0 || cost < best) {
                        best = cost;
                        TR = tr;
                        IMGS = im;
                        NB = nb;
                    }
                }
        if (best == 0) return rnn_fail(ctx, RNN_E_UNSUPPORTED, "conv dW: tile exceeds LDS");
    }
    lds = use4 ? dw_geometry4(g, TR, IMGS, n) : dw_geometry(g, K, TR, IMGS, NB);
    if ((long long)IMGS * std::max(g.cihw, g.cohw) * 4 >= 0x7FFFFFF0ll)
        return rnn_fail(ctx, RNN_E_UNSUPPORTED, "conv dW: tile source beyond 2 GiB");
    g.tiles_a = (g.OH + g.TR - 1) / g.TR;
    g.ntiles = g.tiles_a * (int)((n + IMGS - 1) / IMGS);
    const void *kern = kernel_of(g);
    // persistent: as many workgroups as fit on the chip at once
    if (NZ <= 0) NZ = slabs_of(kern, lds, g.ntiles);
    NZ = std::min(NZ, g.ntiles);
    g.nz = NZ;
    L.g = g;
    L.kern = kern;
    L.lds = lds;
    L.grid = dim3(NZ, ncb, ncib);
    L.threads = dw_threads_of(K);
    L.nz = NZ;
    L.len = (size_t)g.CO * g.CI * K * K;
    return RNN_OK;
}

size_t rnn_conv_dw_slab_floats(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n) {
    DwLaunch L;
    if (dw_plan(ctx, sp, n, nullptr, nullptr, L) != RNN_OK) return 0;
    return (size_t)L.nz * L.len;
}

int rnn_conv_dw_slabs(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *dy,
                      const float *x, float *slabs, int *nz) {
    DwLaunch L;
    int rc = dw_plan(ctx, sp, n, dy, x, L);
    if (rc) return rc;
    L.set_part(slabs);
    void *args[] = {L.arg()};
    RNN_HIP(ctx, hipLaunchKernel(L.kern, L.grid, dim3(L.threads), args, L.lds, ctx->stream));
    if (nz) *nz = L.nz;
    return RNN_OK;
}

// dW += over the batch (k = 1 or 3): slabs in `part` (cap floats) or, with
// part null, in the context workspace; then one reduce in slab order.
int rnn_conv_dw(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *dy, const float *x,
                float *dw, float *part, size_t cap) {
    DwLaunch L;
    int rc = dw_plan(ctx, sp, n, dy, x, L);
    if (rc) return rc;
    const size_t need = (size_t)L.nz * L.len;
    float *ws = part;
    if (ws) {
        if (need > cap)
            return rnn_fail(ctx, RNN_E_UNSUPPORTED,
                            "conv dW: %zu bytes of partial slabs exceed the fixed scratch of "
                            "%zu bytes",
                            need * sizeof(float), cap * sizeof(float));
    } else {
        ws = (float *)rnn_workspace(ctx, need * sizeof(float));
        if (!ws) return RNN_E_NOMEM;
    }
    L.set_part(ws);
    void *args[] = {L.arg()};
    RNN_HIP(ctx, hipLaunchKernel(L.kern, L.grid, dim3(L.threads), args, L.lds, ctx->stream));
    hipLaunchKernelGGL(slab_reduce_kernel, dim3((unsigned)rnn_div_up(L.len, 32)), dim3(256), 0,
                       ctx->stream, ws, L.nz, (long long)L.len, dw);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

// ------------------------------------------------------------ grouped dW

// Plans one launch for the weight gradients of `count` 3x3 convolutions of
// one stride (double-buffered tap-kernel plans; the few-input-channel stem
// is not one of them).  Each conv keeps the tile its own plan takes; its
// slab count nz is chosen so that the jobs -- (conv, slab, co block, ci
// block), each walking ceil(ntiles / nz) tiles -- fill the chip's resident
// workgroups with the smallest longest job: starting from one slab per
// conv, the conv with the longest job gets the next slab count that
// shortens it while the jobs still fit.  Sets m[i].nz; the caller then
// allocates nz * cout * cin * 9 floats of slabs per conv and the table
// (L->table_bytes) and calls rnn_conv_dw_group_upload.
int rnn_conv_dw_group_plan(rnn_ctx *ctx, size_t n, DwGroupMember *m, int count,
                           DwGroupLaunch *L) {
    if (!ctx || !m || !L) return RNN_E_NULL;
    if (count <= 0 || count > 255 || n == 0)
        return rnn_fail(ctx, RNN_E_UNSUPPORTED, "grouped dW: 1 to 255 convolutions");
    std::vector<DwLaunch> pl(count);
    int S = -1, mt = 0;
    size_t lds = 0;
    for (int i = 0; i < count; i++) {
        if (m[i].sp.k != 3 || (S >= 0 && (int)m[i].sp.stride != S))
            return rnn_fail(ctx, RNN_E_UNSUPPORTED, "grouped dW: 3x3 convolutions of one stride");
        S = (int)m[i].sp.stride;
        const int rc = dw_plan(ctx, &m[i].sp, n, nullptr, nullptr, pl[i]);
        if (rc) return rc;
        if (pl[i].small || pl[i].g.nbuf != 2)
            return rnn_fail(ctx, RNN_E_UNSUPPORTED, "grouped dW: conv %d has no tap-kernel plan", i);
        const int ncb = (pl[i].g.CO + 31) / 32, ncib = (pl[i].g.CI + 31) / 32;
        if (ncb > 64 || ncib > 64)
            return rnn_fail(ctx, RNN_E_UNSUPPORTED, "grouped dW: more than 2048 channels");
        const int mti = std::max(pl[i].g.mx, pl[i].g.md);  // 0: the 16-byte staging
        if (i > 0 && (mti == 0) != (mt == 0))
            return rnn_fail(ctx, RNN_E_UNSUPPORTED, "grouped dW: one staging for every conv");
        mt = std::max(mt, mti);
        lds = std::max(lds, pl[i].lds);
    }
    const void *kern = dw_group_pick(S, mt);
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, dw_threads<3>(), lds) !=
            hipSuccess ||
        occ < 1)
        occ = 1;
    const long long budget = (long long)occ * ctx->num_cus;
    std::vector<int> nz(count, 1), pairs(count), tiles(count);
    std::vector<long long> w(count);
    long long jobs = 0;
    for (int i = 0; i < count; i++) {
        const DwArgs &g = pl[i].g;
        pairs[i] = ((g.CO + 31) / 32) * ((g.CI + 31) / 32);
        tiles[i] = g.ntiles;
        w[i] = g.ngroups + 2;
        jobs += pairs[i];
    }
    auto cost = [&](int i) { return (long long)((tiles[i] + nz[i] - 1) / nz[i]) * w[i]; };
    for (;;) {
        int worst = 0;
        for (int i = 1; i < count; i++)
            if (cost(i) > cost(worst)) worst = i;
        const int per = (tiles[worst] + nz[worst] - 1) / nz[worst];
        if (per <= 1) break;
        const int next = (tiles[worst] + per - 2) / (per - 1);  // fewest slabs for per-1 tiles
        if (next > 4095 || jobs + (long long)pairs[worst] * (next - nz[worst]) > budget) break;
        jobs += (long long)pairs[worst] * (next - nz[worst]);
        nz[worst] = next;
    }
    L->conv.clear();
    L->jobs.clear();
    for (int i = 0; i < count; i++) {
        DwArgs g = pl[i].g;
        g.nz = nz[i];
        m[i].nz = nz[i];
        const int ncb = (g.CO + 31) / 32, ncib = (g.CI + 31) / 32;
        for (int z = 0; z < nz[i]; z++)
            for (int cb = 0; cb < ncb; cb++)
                for (int ib = 0; ib < ncib; ib++)
                    L->jobs.push_back((uint32_t)i | (uint32_t)z << 8 | (uint32_t)cb << 20 |
                                      (uint32_t)ib << 26);
        std::vector<unsigned char> b(sizeof(DwArgs));
        std::memcpy(b.data(), &g, sizeof(DwArgs));
        L->conv.push_back(b);
    }
    L->kern = kern;
    L->lds = lds;
    L->threads = dw_threads<3>();
    L->njobs = (int)L->jobs.size();
    L->table_bytes = (size_t)count * sizeof(DwArgs) + L->jobs.size() * sizeof(uint32_t);
    L->count = count;
    return RNN_OK;
}

// Writes the operand and slab pointers of every conv into the plan and
// uploads the tables to L->table (device, L->table_bytes, set by the
// caller; synchronous).
int rnn_conv_dw_group_upload(rnn_ctx *ctx, const DwGroupMember *m, DwGroupLaunch *L) {
    if (!ctx || !m || !L || !L->table) return RNN_E_NULL;
    std::vector<unsigned char> host(L->table_bytes);
    for (int i = 0; i < L->count; i++) {
        if (!m[i].dy || !m[i].x || !m[i].slabs)
            return rnn_fail(ctx, RNN_E_NULL, "grouped dW: conv %d has a null operand", i);
        DwArgs g;
        std::memcpy(&g, L->conv[i].data(), sizeof(DwArgs));
        g.dy = m[i].dy;
        g.x = m[i].x;
        g.part = m[i].slabs;
        std::memcpy(host.data() + (size_t)i * sizeof(DwArgs), &g, sizeof(DwArgs));
    }
    std::memcpy(host.data() + (size_t)L->count * sizeof(DwArgs), L->jobs.data(),
                L->jobs.size() * sizeof(uint32_t));
    RNN_HIP(ctx, hipMemcpy(L->table, host.data(), host.size(), hipMemcpyHostToDevice));
    return RNN_OK;
}

// The grouped launch on the context's stream: every conv's slabs written.
int rnn_conv_dw_group_launch(rnn_ctx *ctx, const DwGroupLaunch *L) {
    if (!L->njobs) return RNN_OK;
    const DwArgs *tab = (const DwArgs *)L->table;
    const uint32_t *jobs = (const uint32_t *)((const char *)L->table +
                                              (size_t)L->count * sizeof(DwArgs));
    void *args[] = {(void *)&tab, (void *)&jobs};
    RNN_HIP(ctx, hipLaunchKernel(L->kern, dim3((unsigned)L->njobs), dim3(L->threads), args, L->lds,
                                 ctx->stream));
    return RNN_OK;
}
