// Device helpers shared by the convolution kernels: division by run-time
// constants, the zero-padded LDS staging of source windows, and the tap
// geometry of forward / dX convolution.
#pragma once

#include "rnn_internal.h"

#include <type_traits>
#include <utility>

// Division by a run-time divisor d via one multiply-high: q = umulhi(n, m)
// with m = ceil(2^32 / d) is exact for n * d < 2^32 (all tile indices here
// are below 2^20 and divisors below 2^12).  d == 1 uses m = 0.
struct FastDiv {
    uint32_t d, m;
};

static inline FastDiv make_fastdiv(uint32_t d) {
    FastDiv f;
    f.d = d;
    f.m = d <= 1 ? 0u : (uint32_t)(((1ull << 32) + d - 1) / d);
    return f;
}

__device__ __forceinline__ uint32_t fdiv(uint32_t n, FastDiv f) {
    return f.m ? __umulhi(n, f.m) : n;
}

// A zero-padded window of a [N][C][H][W] tensor staged in LDS as
// [ch][img][ty][tile col].  Tile row ty of image img reads source row
// y0 + ty*rowstep; tile column tx reads source column x0 + tx*colstep and is
// stored at column tx, or de-interleaved by parity ((tx&1)*half + tx/2) so
// that lanes reading every other column read consecutive words.
struct TileGeo {
    int IMGS, TIH, TIW, TIWP, HALF, deint;
    int rowstep, colstep;
    int chs, imgs;  // LDS strides of a channel and of an image
    FastDiv fd_tiw, fd_tih, fd_imgs;
    FastDiv fd_chs, fd_imgstr, fd_tiwp;  // for the LDS-position -> source decode
};

static inline void tilegeo_finish(TileGeo &t) {
    t.fd_tiw = make_fastdiv(t.TIW);
    t.fd_tih = make_fastdiv(t.TIH);
    t.fd_imgs = make_fastdiv(t.IMGS);
    t.fd_chs = make_fastdiv(t.chs);
    t.fd_imgstr = make_fastdiv(t.imgs);
    t.fd_tiwp = make_fastdiv(t.TIWP);
}

// LDS words reserved for a staged region: whole 64-word DMA rows.
static inline size_t dma_region(size_t words) { return (words + 63) & ~(size_t)63; }


// Asynchronously stages a window with buffer_load_dword ... lds: LDS word L of
// [0, nch*t.chs) receives source element (n0 + img, c0 + ch, y0 + ty*rowstep,
// x0 + tx*colstep) of the [N][C][H][W] tensor behind `rs` (whose base is image
// n0), or 0 outside it.  Each wave instruction fills 64 consecutive words, so
// the region must be dma_region()-sized.  Completion: s_waitcnt vmcnt(0) +
// barrier.
__device__ __forceinline__ void dma_tile(__amdgpu_buffer_rsrc_t rs, int N, int C, int H, int W,
                                         int n0, int c0, int nch, int y0, int x0,
                                         const TileGeo &t, float *lds, int wave, int nw,
                                         int lane) {
    const int total = nch * t.chs;
    for (int L0 = wave * 64; L0 < total; L0 += nw * 64) {
        const int L = L0 + lane;
        uint32_t off = DMA_OOB;
        if (L < total) {
            const int ch = (int)fdiv((uint32_t)L, t.fd_chs);
            int rem = L - ch * t.chs;
            const int img = (int)fdiv((uint32_t)rem, t.fd_imgstr);
            rem -= img * t.imgs;
            const int ty = (int)fdiv((uint32_t)rem, t.fd_tiwp), col = rem - ty * t.TIWP;
            const int tx = t.deint ? (col < t.HALF ? 2 * col : 2 * (col - t.HALF) + 1) : col;
            const int n = n0 + img, c = c0 + ch, y = y0 + ty * t.rowstep, x = x0 + tx * t.colstep;
            if (img < t.IMGS && ty < t.TIH && tx < t.TIW && n < N && c < C && y >= 0 && y < H &&
                x >= 0 && x < W)
                off = ((((uint32_t)img * C + c) * H + y) * W + x) * 4u;
        }
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(lds + L0), 4, off, 0, 0, 0);
    }
}

// Asynchronously copies nf contiguous floats (nf a multiple of 64) starting at
// byte offset `src` of `rs` into lds, 16 bytes per lane when nf allows.
__device__ __forceinline__ void dma_copy(__amdgpu_buffer_rsrc_t rs, uint32_t src, float *lds,
                                         int nf, int wave, int nw, int lane) {
    if ((nf & 255) == 0) {
        for (int i = wave * 256; i < nf; i += nw * 256)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(lds + i), 16,
                                                     src + (uint32_t)(i + 4 * lane) * 4u, 0, 0, 0);
    } else {
        for (int i = wave * 64; i < nf; i += nw * 64)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(lds + i), 4,
                                                     src + (uint32_t)(i + lane) * 4u, 0, 0, 0);
    }
}

// Waits for this wave's outstanding DMA, then for the whole workgroup.
__device__ __forceinline__ void dma_wait_barrier() {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
}

__device__ __forceinline__ int tile_col(int tx, int deint, int half) {
    return deint ? (tx & 1) * half + (tx >> 1) : tx;
}

// Stages nch channels starting at c0 of images n0.. into lds.  U loads are
// issued before the first LDS write so U global latencies overlap.
template <int U>
__device__ __forceinline__ void stage_tile(const float *__restrict__ src, int N, int C, int H, int W,
                                           int n0, int c0, int nch, int y0, int x0,
                                           const TileGeo &t, float *lds, int tid, int nthreads) {
    const int total = nch * t.IMGS * t.TIH * t.TIW;
    for (int e0 = tid; e0 < total; e0 += nthreads * U) {
        float v[U];
        int dst[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int e = e0 + u * nthreads;
            v[u] = 0.f;
            dst[u] = -1;
            if (e < total) {
                const int row = (int)fdiv((uint32_t)e, t.fd_tiw), tx = e - row * t.TIW;
                const int q = (int)fdiv((uint32_t)row, t.fd_tih), ty = row - q * t.TIH;
                const int ch = (int)fdiv((uint32_t)q, t.fd_imgs), img = q - ch * t.IMGS;
                const int n = n0 + img, c = c0 + ch, y = y0 + ty * t.rowstep, x = x0 + tx * t.colstep;
                if (n < N && c < C && y >= 0 && y < H && x >= 0 && x < W)
                    v[u] = src[(((long long)n * C + c) * H + y) * W + x];
                dst[u] = ch * t.chs + img * t.imgs + ty * t.TIWP + tile_col(tx, t.deint, t.HALF);
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++)
            if (dst[u] >= 0) lds[dst[u]] = v[u];
    }
}

// Tap geometry of a K x K, stride S, pad P convolution.
//  forward (DX = false): output (a, b) reads source (a*S + kh - P, b*S + kw - P).
//  dX      (DX = true):  output block (a, b) holds dX at (a*S + py, b*S + px)
//      for the S*S parity classes (py, px); tap (kh, kw) feeds class
//      ((kh - P) mod S, (kw - P) mod S) and reads dY at (a + dy, b + dx) with
//      dy = (py + P - kh) / S (exact).  Every dX element gathers its taps
//      once, so the col2im needs no accumulation across workgroups.
template <int K, int S, int P, bool DX>
struct ConvTaps {
    static constexpr int KK = K * K;
    static constexpr int NCLS = DX ? S * S : 1;
    static constexpr int IS = DX ? 1 : S;  // source step per output position
    static constexpr int OS = DX ? S : 1;  // destination step per output position
    __host__ __device__ static constexpr int pmod(int a) { return ((a % S) + S) % S; }
    __host__ __device__ static constexpr int cls(int t) {
        return DX ? pmod(t / K - P) * S + pmod(t % K - P) : 0;
    }
    __host__ __device__ static constexpr int dy(int t) {
        return DX ? (pmod(t / K - P) + P - t / K) / S : t / K - P;
    }
    __host__ __device__ static constexpr int dx(int t) {
        return DX ? (pmod(t % K - P) + P - t % K) / S : t % K - P;
    }
};

// Compile-time loop: f(std::integral_constant<int, I>) for I in [0, N).
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}
