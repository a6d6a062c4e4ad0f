// Internal declarations shared by the HIP sources of librnn.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <functional>
#include <map>
#include <mutex>
#include <vector>

#include "../../include/rnn.h"

// A small table (pointers, lengths) kept on the device for kernels that walk a
// list of tensors.  Uploaded again only when its bytes change, so a caller
// that passes the same list every step issues no copy after the first.
struct RnnDevTable {
    std::vector<char> host;  // bytes of the last upload
    void *dev = nullptr;
    size_t cap = 0;
};

// One attention relidx table on the device: relidx [tq*tk], the inverse
// index (rowptr [nrel+1], positions [tq*tk]) and, for the workgroup kernels,
// the table in lane order; the host copy identifies it.
struct RnnRelTable {
    std::vector<uint32_t> host;
    uint32_t tq = 0, tk = 0, nrel = 0;
    uint32_t *dev = nullptr;
    uint32_t *pinned = nullptr;  // the upload's staging, kept with the table
};

// One deferred parameter-gradient reduction (rnn_ctx_set_defer): partial
// rows left in the context's arena by a backward entry point, summed into
// the gradient at the flush by the same code, in the same order, as the
// entry point's own reduction kernel would have.
enum {
    RNN_DEFER_COLS = 0,    // f64 rows [nrow][len], 16 groups of rows (rnn_colsum_red_block)
    RNN_DEFER_CHUNKS = 1,  // f32 rows [nrow][len] in row order (rnn_chunk_sum)
    RNN_DEFER_ROWS64 = 2,  // f64 rows [nrow][len] in row order (rnn_rows64_sum)
    RNN_DEFER_ATTN = 3,    // attention dtau / drel (rnn_attn_reduce_block): part = dtau
                           // partials, part2 = drel partials, out0 = drel, out1 = dtau,
                           // len = h*nrel + h, split = h*nrel, nrow = n images
    RNN_DEFER_CHUNKS4 = 4, // CHUNKS with len % 4 == 0 and 16-byte aligned rows and out0,
                           // four elements a thread (rnn_chunk_sum4)
};
struct RnnDeferSeg {
    const void *part, *part2;
    float *out0, *out1;  // COLS: columns j < split go to out0[j], the rest to out1[j - split]
    long long len, split;
    int nrow, kind, acc;  // CHUNKS: acc = 0 overwrites out0
};

struct rnn_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    bool own_stream = false;
    int num_cus = 256;
    // Device address of this device's copy of the fixed scratch array of the
    // no-allocation entry points (RNN_NOALLOC_SCRATCH_BYTES, rnn_ctx.hip),
    // looked up by the first such call (rnn_noalloc_scratch).
    float *noalloc_scratch = nullptr;
    // Growing device workspace (split-K partials, packed weights, attention
    // reductions).  Reallocated only when a call needs more; the stream is
    // synchronised first so no in-flight kernel still reads the old block.
    void *ws = nullptr;
    size_t ws_bytes = 0;
    // Staging block of the *_host entry points (host slices copied in and
    // out around a device call); grows like the workspace.
    void *hstage = nullptr;
    size_t hstage_bytes = 0;
    // Attention relative-index tables, each uploaded once and kept until the
    // context ends (a step that switches between geometries never waits).
    std::vector<RnnRelTable> rel_tables;
    size_t rel_last = 0;  // the table the last attention call used
    // Tensor-list tables of the optimizer entry points (slot -> table).
    std::map<int, RnnDevTable> tables;
    // Deferred parameter-gradient reductions: on, the pending segments in
    // call order, and the arena their partials live in until the flush
    // (device blocks kept across flushes; block `dblk`, offset `doff` next).
    bool defer = false;
    std::vector<RnnDeferSeg> dsegs;
    std::vector<std::pair<char *, size_t>> darena;
    size_t dblk = 0, doff = 0;
    std::recursive_mutex mu;
    char err[512] = {0};
};

// Device memory that stays untouched until the next rnn_ctx_flush (deferred
// partials); null (with the error recorded) when it cannot be allocated.
void *rnn_defer_take(rnn_ctx *ctx, size_t bytes);
// Queues a reduction for the flush.
void rnn_defer_push(rnn_ctx *ctx, const RnnDeferSeg &s);

// Block `blk` of a column reduction: columns [16 blk, 16 blk + 16) of part
// [nblk][len] (f64), each summed over the rows in 16 consecutive groups --
// each group in order, 16 loads ahead -- then the group sums in order, and
// added into out0[j] (j < split) or out1[j - split].  256 threads.
__device__ __forceinline__ void rnn_colsum_red_block(int nblk, size_t len, size_t split,
                                                     const double *__restrict__ part,
                                                     float *__restrict__ out0,
                                                     float *__restrict__ out1, unsigned blk) {
    constexpr int COLS = 16, NG = 256 / COLS;
    __shared__ double red[NG][COLS];
    const int jl = threadIdx.x % COLS, q = threadIdx.x / COLS;
    const size_t j = (size_t)blk * COLS + jl, jc = min(j, len - 1);
    const int G = (nblk + NG - 1) / NG, k0 = min(nblk, q * G), k1 = min(nblk, k0 + G);
    double s = 0.0;
    for (int k = k0; k < k1; k += 16) {
        double v[16];
#pragma unroll
        for (int u = 0; u < 16; u++) v[u] = part[(size_t)min(k + u, k1 - 1) * len + jc];
#pragma unroll
        for (int u = 0; u < 16; u++)
            if (k + u < k1) s += v[u];
    }
    red[q][jl] = s;
    __syncthreads();
    if (q != 0 || j >= len) return;
    double t = red[0][jl];
    for (int g = 1; g < NG; g++) t += red[g][jl];
    if (j < split)
        out0[j] += (float)t;
    else
        out1[j - split] += (float)t;
}

// Element e of a chunk reduction: out[e] (+)= sum_z part[z][e] (f32, z in
// order, 8 loads ahead of their adds).
__device__ __forceinline__ void rnn_chunk_sum(const float *part, int nz, long long len, float *out,
                                              int accumulate, long long e) {
    float s = 0.f;
    for (int z0 = 0; z0 < nz; z0 += 8) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = z0 + i < nz ? part[(long long)(z0 + i) * len + e] : 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++)
            if (z0 + i < nz) s = (z0 + i == 0) ? v[i] : s + v[i];
    }
    out[e] = accumulate ? out[e] + s : s;
}

// Elements e .. e + 3 (e % 4 == 0) of a chunk reduction, as rnn_chunk_sum
// computes each of them (the same adds in the same order), with 16-byte
// loads: part's rows and out 16-byte aligned, len % 4 == 0.
__device__ __forceinline__ void rnn_chunk_sum4(const float *part, int nz, long long len,
                                               float *out, int accumulate, long long e) {
    float4 old = make_float4(0.f, 0.f, 0.f, 0.f);
    if (accumulate) old = *(const float4 *)(out + e);
    float4 s = old;
    for (int z0 = 0; z0 < nz; z0 += 8) {
        float4 v[8];
#pragma unroll
        for (int i = 0; i < 8; i++)
            v[i] = z0 + i < nz ? *(const float4 *)(part + (long long)(z0 + i) * len + e)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            if (z0 + i >= nz) continue;
            if (z0 + i == 0) {
                s = v[i];
            } else {
                s.x = s.x + v[i].x;
                s.y = s.y + v[i].y;
                s.z = s.z + v[i].z;
                s.w = s.w + v[i].w;
            }
        }
    }
    if (accumulate) {
        s.x = old.x + s.x;
        s.y = old.y + s.y;
        s.z = old.z + s.z;
        s.w = old.w + s.w;
    }
    *(float4 *)(out + e) = s;
}

// Block `blk` of the attention parameter reduction (32 outputs a block, 256
// threads): drel[e] (e < h*nrel) += the f32 sum of drel_part[i][e] over the
// n (image) rows, dtau[e - h*nrel] += the f64 sum of dtau_part[i][...], each
// over 8 consecutive groups of rows in order, then the group sums in order.
__device__ __forceinline__ void rnn_attn_reduce_block(const double *dtau_part,
                                                      const float *drel_part, int n, int h,
                                                      int nrel, float *dtau, float *drel,
                                                      unsigned blk) {
    constexpr int ATTN_RED_PARTS = 8;
    __shared__ double part[ATTN_RED_PARTS][32];
    const int el = threadIdx.x & 31, j = threadIdx.x >> 5;
    const int e = (int)blk * 32 + el;
    const int per = h * nrel;
    const bool is_rel = e < per, live = e < per + h;
    const long long stride = is_rel ? per : h;
    const int G = (n + ATTN_RED_PARTS - 1) / ATTN_RED_PARTS;
    const int i0 = j * G, i1 = min(n, i0 + G);
    // the value added to, loaded ahead (its latency overlaps the partials')
    float old = 0.f;
    if (j == 0 && live) old = is_rel ? drel[e] : dtau[e - per];
    double s = 0.0;
    if (live && is_rel) {
        float fs = 0.f;
        const float *src = drel_part + e;
        for (int b = i0; b < i1; b += 16) {
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; u++) v[u] = b + u < i1 ? src[(long long)(b + u) * stride] : 0.f;
#pragma unroll
            for (int u = 0; u < 16; u++)
                if (b + u < i1) fs = (b + u == i0) ? v[u] : fs + v[u];
        }
        s = fs;
    } else if (live) {
        const double *src = dtau_part + (e - per);
        for (int b = i0; b < i1; b += 16) {
            double v[16];
#pragma unroll
            for (int u = 0; u < 16; u++) v[u] = b + u < i1 ? src[(long long)(b + u) * stride] : 0.0;
#pragma unroll
            for (int u = 0; u < 16; u++)
                if (b + u < i1) s += v[u];
        }
    }
    part[j][el] = s;
    __syncthreads();
    if (j == 0 && live) {
        if (is_rel) {
            float t = 0.f;
            bool first = true;
            for (int q = 0; q < ATTN_RED_PARTS; q++) {
                if (q * G >= n) break;
                t = first ? (float)part[q][el] : t + (float)part[q][el];
                first = false;
            }
            drel[e] = old + t;
        } else {
            double t = 0.0;
            for (int q = 0; q < ATTN_RED_PARTS; q++) {
                if (q * G >= n) break;
                t += part[q][el];
            }
            dtau[e - per] = old + (float)t;
        }
    }
}

// Element m of an f64 row reduction: out[m] += (float) sum_z part[z][m], z in
// order.
__device__ __forceinline__ void rnn_rows64_sum(const double *part, int nz, long long len,
                                               float *out, long long m) {
    double t = 0.0;
    for (int z = 0; z < nz; z++) t += part[(long long)z * len + m];
    out[m] += (float)t;
}

// Size of the fixed device scratch behind rnn_conv2d_backward_w_noalloc.
#define RNN_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
// The device address of ctx's device's copy of that scratch (looked up once
// per device with hipGetSymbolAddress; no allocation).
int rnn_noalloc_scratch(rnn_ctx *ctx, float **out);
// Runs `enqueue` (the kernels that use the scratch) under the device's
// no-allocation lock.  Outside graph capture, a call on another stream than
// the previous call on the device first waits (hipStreamWaitEvent) for that
// call's kernels, and an event is recorded after its own; under capture the
// caller orders the calls.
int rnn_noalloc_run(rnn_ctx *ctx, const std::function<int()> &enqueue);

// Records a message and returns `code`.
int rnn_fail(rnn_ctx *ctx, int code, const char *fmt, ...);

#define RNN_HIP(ctx, expr)                                                              \
    do {                                                                                \
        hipError_t e_ = (expr);                                                         \
        if (e_ != hipSuccess)                                                           \
            return rnn_fail((ctx), RNN_E_HIP, "%s failed: %s (%s:%d)", #expr,           \
                            hipGetErrorString(e_), __FILE__, __LINE__);                 \
    } while (0)

// Checks the launch status of the kernel just enqueued.
#define RNN_LAUNCHED(ctx)                                                               \
    do {                                                                                \
        hipError_t e_ = hipGetLastError();                                              \
        if (e_ != hipSuccess)                                                           \
            return rnn_fail((ctx), RNN_E_HIP, "kernel launch failed: %s (%s:%d)",       \
                            hipGetErrorString(e_), __FILE__, __LINE__);                 \
    } while (0)

// Returns a device workspace of at least `bytes` (256-byte aligned), or
// nullptr after recording RNN_E_NOMEM / RNN_E_HIP in ctx.
void *rnn_workspace(rnn_ctx *ctx, size_t bytes);

// Device copy of `bytes` bytes at `src` in table `t`: a table whose bytes are
// unchanged since its last upload is reused as it is; otherwise the stream is
// drained (queued kernels may still read the old copy), the copy is made
// synchronously, and the new device address returned in *dev.  An upload is
// refused while the stream is being captured into a graph.
int rnn_dev_table(rnn_ctx *ctx, RnnDevTable &t, const void *src, size_t bytes, void **dev);
void rnn_dev_table_free(RnnDevTable &t);
// Slots of rnn_ctx::tables.
enum { RNN_TABLE_CLIP = 1, RNN_TABLE_EMA = 2 };

// rng.rs (Rng::new, next_u64, next_u32, below, uniform, normal) for host and
// device code: splitmix64-seeded xoshiro256++, 24-bit uniforms, Box-Muller.
// The integer stream is bit-identical to the reference's.  normal() takes
// the host's logf / cosf (the C library the reference's f32::ln / f32::cos
// call); on the device it evaluates log and cos in double and rounds once, so
// its floats are the correctly rounded values, which the host library's
// results equal in all but rare cases (its own error is under one ulp).
__device__ __forceinline__ float rnn_dev_logf(float x) { return (float)log((double)x); }
__device__ __forceinline__ float rnn_dev_cosf(float x) { return (float)cos((double)x); }
__device__ __forceinline__ float rnn_dev_sinf(float x) { return (float)sin((double)x); }
struct RnnRng {
    uint64_t s[4];
    __host__ __device__ explicit RnnRng(uint64_t seed) {
        uint64_t z = seed + 0x9E3779B97F4A7C15ull;
        for (int i = 0; i < 4; i++) {
            z += 0x9E3779B97F4A7C15ull;
            uint64_t x = z;
            x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
            x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
            s[i] = x ^ (x >> 31);
        }
    }
    __host__ __device__ static uint64_t rotl(uint64_t x, int k) {
        return (x << k) | (x >> (64 - k));
    }
    __host__ __device__ uint64_t next() {
        const uint64_t r = rotl(s[0] + s[3], 23) + s[0];
        const uint64_t t = s[1] << 17;
        s[2] ^= s[0];
        s[3] ^= s[1];
        s[1] ^= s[2];
        s[0] ^= s[3];
        s[2] ^= t;
        s[3] = rotl(s[3], 45);
        return r;
    }
    __host__ __device__ uint32_t next_u32() { return (uint32_t)(next() >> 32); }
    __host__ __device__ uint64_t below(uint64_t n) { return next() % n; }
    __host__ __device__ float uniform() { return (float)(next() >> 40) * (1.0f / 16777216.0f); }
    __host__ __device__ float normal() {
        float u1 = uniform();
        if (!(u1 > 1e-7f)) u1 = 1e-7f;
        const float u2 = uniform();
#if defined(__HIP_DEVICE_COMPILE__)
        return sqrtf(-2.0f * rnn_dev_logf(u1)) * rnn_dev_cosf(6.28318530717958647692f * u2);
#else
        return sqrtf(-2.0f * logf(u1)) * cosf(6.28318530717958647692f * u2);
#endif
    }
};

// Bump allocator over one workspace block.
struct WsCarve {
    size_t off = 0;
    size_t take(size_t bytes) {
        size_t o = off;
        off += (bytes + 255) & ~size_t(255);
        return o;
    }
};

static inline size_t rnn_div_up(size_t a, size_t b) { return (a + b - 1) / b; }
static inline size_t rnn_round_up(size_t a, size_t b) { return rnn_div_up(a, b) * b; }

// fp32 MFMA operand / accumulator vectors.
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

typedef __attribute__((address_space(3))) void *lds_ptr_t;

// Buffer resource over [base, base + bytes) with bytes < 2^31: a load at a
// byte offset >= bytes returns 0 (used for zero halos and tile edges).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                             0x00020000);
}
constexpr uint32_t DMA_OOB = 0x7FFFFFF0u;

// Index of the calling wave in its workgroup, as a wave-uniform (scalar)
// value: loops and branches on it stay scalar instead of exec-masked.
__device__ __forceinline__ int wave_index() {
    return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

// v from the lane a DPP pattern names (both 32-bit halves moved).
template <int CTRL>
__device__ __forceinline__ double rnn_dpp_d(double v) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_mov_dpp((int)b, CTRL, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_mov_dpp((int)(b >> 32), CTRL, 0xf, 0xf, false);
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}
// Sum over the 64 lanes of a wave with every lane active, every lane
// receiving it, in a fixed tree: quads by DPP xor 1 and 2, rows of 8 and 16
// by DPP mirrors, then xor 16 and 32 across rows.
__device__ __forceinline__ double rnn_wave_sum_d(double v) {
    v += rnn_dpp_d<0xB1>(v);   // quad_perm [1, 0, 3, 2]
    v += rnn_dpp_d<0x4E>(v);   // quad_perm [2, 3, 0, 1]
    v += rnn_dpp_d<0x141>(v);  // row_half_mirror
    v += rnn_dpp_d<0x140>(v);  // row_mirror
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

// Entry points implemented in the kernel sources, called from the C ABI.
// One batch of the grouped Newton-Schulz GEMMs (rnn_ns_gemm_launch): cnt
// products C_z = op(A_z) op(B_z) of one shape, [M x K] times [K x N].  The
// layout `lay` says how the operands are stored: NS_LAY_NT: A [M][K], B [N][K];
// NS_LAY_TN: A [K][M], B [K][N]; NS_LAY_NN: A [M][K], B [K][N] (leading
// dimensions lda, ldb).  C and the optional epilogue source E share ldc and
// stride_c.  sym: C is symmetric (M = N, and E symmetric too); only tiles on
// or above the diagonal are computed, each stored twice.  The problem's 64 x 64
// tiles are blocks tile0 .. tile0 + cnt * tmn - 1 of the launch, tn tiles along
// N (tmn = tn (tn + 1) / 2 when sym).
enum { NS_LAY_NT = 0, NS_LAY_TN = 1, NS_LAY_NN = 2 };
struct NsGemmProb {
    const float *a, *b;
    float *c;
    const float *e;
    long long stride_a, stride_b, stride_c;
    int M, N, K, lda, ldb, ldc;
    uint32_t tile0, tn, tmn;
    int lay, sym;
};

// One launch over `nprob` problems (device table, sorted by tile0, the first
// at 0) covering `ntiles` tiles: C = alpha E + beta (A op(B)) where E is set,
// else the product.  vec: 1 when every k-contiguous operand row and batch
// stride is a multiple of 4 floats and 16-byte aligned; 2 when moreover
// every operand of every problem meets ns_dma_ok (the direct-to-LDS tile).
int rnn_ns_gemm_launch(rnn_ctx *ctx, const NsGemmProb *probs, int nprob, size_t ntiles, int vec,
                       float alpha, float beta);
// Whether problem p (host copy, device pointers) can take the direct-to-LDS
// tile: every 16-byte operand quad wholly inside or outside its operand,
// 16-byte aligned bases and batch strides, extents below 2^31 bytes.
bool ns_dma_ok(const NsGemmProb &p, size_t count);

// rnn_gemm_launch with explicit leading dimensions: op(A) [m x k] read from
// rows of stride lda (A stored [k][m] with stride lda when at), likewise B
// (ldb) and C (ldc); batch z at a + z*stride_a etc.  No bias.
int rnn_gemm_launch_ld(rnn_ctx *ctx, size_t count, size_t m, size_t n, size_t k, const float *a,
                       size_t lda, size_t stride_a, int at, const float *b, size_t ldb,
                       size_t stride_b, int bt, float *c, size_t ldc, size_t stride_c, int acc);
// The same over a two-level batch in one launch: problem (z1, z2), z1 <
// count1, z2 < count2, takes its operands at a + z1 stride_a + z2 stride_a2
// (likewise B and C).  count1 * count2 <= 65535.
int rnn_gemm_launch_ld2(rnn_ctx *ctx, size_t count1, size_t count2, size_t m, size_t n, size_t k,
                        const float *a, size_t lda, size_t stride_a, size_t stride_a2, int at,
                        const float *b, size_t ldb, size_t stride_b, size_t stride_b2, int bt,
                        float *c, size_t ldc, size_t stride_c, size_t stride_c2, int acc);

int rnn_gemm_launch(rnn_ctx *ctx, size_t count, size_t m, size_t n, size_t k, const float *a,
                    size_t stride_a, int at, const float *b, size_t stride_b, int bt, float *c,
                    size_t stride_c, int acc, const float *bias);
int rnn_colsum_launch(rnn_ctx *ctx, size_t rows, size_t cols, const float *x, float *out);
// outab[j] += sum_r a[r][j] b[r][j] (b set), outa[j] += sum_r a[r][j] (outa
// set): f64 sums in a fixed order (two launches).
// With rs set, a's row r counts as a[r] * rs[r / rpi].
int rnn_colsum_f64(rnn_ctx *ctx, size_t rows, int c, const float *a, const float *b,
                   float *outab, float *outa, const float *rs = nullptr, size_t rpi = 1);
// Specialised forward (dx = 0) / dX (dx = 1) convolution; RNN_E_UNSUPPORTED
// when (k, stride, pad) has no specialisation.  wp: the weights packed by
// rnn_conv_pack for this direction (the kernels then load each stage's
// weights as one contiguous copy), or null.
// The batch statistics of a forward convolution's output, taken in its store
// pass for the BatchNorm that reads it: (sum y, sum y^2) per channel in f64,
// part[channel][P][2] with P = rnn_conv_fast_parts (one partial per tile,
// the workgroup's waves summed in order), as bn_stats_part_kernel lays out
// its per-image-range partials.
struct ConvStats {
    double *part = nullptr;
};
int rnn_conv_fast(rnn_ctx *ctx, int dx, const rnn_conv_spec *sp, size_t n, const float *src,
                  const float *w, const float *wp, float *dst, const ConvStats *stats = nullptr);
// Partials per channel of the store-pass statistics of a forward of (sp, n);
// -1 when the shape has no specialised plan.
int rnn_conv_fast_parts(const rnn_conv_spec *sp, size_t n);

// Packed weights of one direction: [m-block][chunk][quad][tap][lane 64][4]
// with lane L of slab (quad q, tap t) holding rows m = 32*mblk + L%32 and
// source channels c = chunk*CH + (L/32)*CH/2 + 4q + i of W[m*sm + c*sc + t],
// zero beyond CD rows or CS channels.
struct PackGeo {
    int CS, CD, KK, CH, nchunks, nmblk, sm, sc;
    __host__ __device__ size_t floats() const {
        return (size_t)nmblk * nchunks * CH * KK * 32;
    }
    // 256-float slabs: slab r = ((mblk*nchunks + chunk)*CH/8 + q)*KK + t
    __host__ __device__ int slabs() const { return nmblk * nchunks * (CH >> 3) * KK; }
    // word j = 4L + i of slab r
    __device__ float value(const float *w, int r, int j) const {
        const int cq = CH >> 3;
        const int t = r % KK, rq = r / KK;
        const int q = rq % cq, rc = rq / cq;
        const int chunk = rc % nchunks, mblk = rc / nchunks;
        const int i = j & 3, L = j >> 2;
        const int m = mblk * 32 + (L & 31);
        const int c = chunk * CH + (L >> 5) * (CH >> 1) + 4 * q + i;
        return (m < CD && c < CS) ? w[(size_t)m * sm + (size_t)c * sc + t] : 0.0f;
    }
};
// The packing of `sp` in direction dx (RNN_E_UNSUPPORTED: no specialised
// kernel, nothing to pack).
int rnn_conv_pack_geo(const rnn_conv_spec *sp, int dx, PackGeo *pg);
int rnn_conv_pack(rnn_ctx *ctx, const rnn_conv_spec *sp, int dx, const float *w, float *wp);
// Several packs in one launch: segment k packs src + src_off into
// dst + dst_off with blocks [blk0, blk0 + nblk) of the grid (segs on the
// device, in blk0 order).
struct PackSeg {
    PackGeo geo;
    size_t src, dst;
    uint32_t blk0, nblk;
};
int rnn_conv_pack_multi_launch(rnn_ctx *ctx, const PackSeg *segs, int nseg, int nblocks,
                               const float *src, float *dst);
// Forward / dX with optional packed weights (rnn_conv2d_forward /
// rnn_conv2d_backward_x with wp = null).
int rnn_conv2d_forward_wp(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *x,
                          const float *w, const float *wp, float *y);
int rnn_conv2d_backward_x_wp(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *dy,
                             const float *w, const float *wp, float *dx);
// The forward with the batch statistics of y taken in its store pass
// (ConvStats); RNN_E_UNSUPPORTED when the shape has no specialised kernel.
int rnn_conv2d_forward_stats(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *x,
                             const float *w, const float *wp, float *y, double *part);
// dW += over the batch (k = 1 or 3).  The partial slabs go to `part` (room
// for `cap` floats; RNN_E_UNSUPPORTED when the plan needs more) or, with part
// null, to the context workspace.
int rnn_conv_dw(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *dy, const float *x,
                float *dw, float *part = nullptr, size_t cap = 0);
// The same dW left as *nz partial slabs of cout*cin*k*k floats in `slabs`
// (rnn_conv_dw_slab_floats(...) floats, 0 when the shape is unsupported);
// their slab-order sum is added by rnn_grad_finalize_launch.
size_t rnn_conv_dw_slab_floats(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n);
int rnn_conv_dw_slabs(rnn_ctx *ctx, const rnn_conv_spec *sp, size_t n, const float *dy,
                      const float *x, float *slabs, int *nz);

// Grouped weight gradients: several 3x3 convolutions of one stride in one
// launch (conv_dw.hip).  rnn_conv_dw_group_plan sets each member's slab
// count nz and the launch (kernel, LDS, jobs, table bytes); the caller
// allocates each member's nz * cout * cin * 9 floats of slabs and
// table_bytes of device memory in `table`, then rnn_conv_dw_group_upload
// writes the members' pointers there.  Every launch then writes each
// member's slabs (summed in slab order by rnn_grad_finalize_launch).
struct DwGroupMember {
    rnn_conv_spec sp;
    const float *dy = nullptr, *x = nullptr;
    float *slabs = nullptr;
    int nz = 0;
};
struct DwGroupLaunch {
    const void *kern = nullptr;
    size_t lds = 0;
    int threads = 0, njobs = 0, count = 0;
    size_t table_bytes = 0;
    void *table = nullptr;
    std::vector<std::vector<unsigned char>> conv;  // per member: its plan (host)
    std::vector<uint32_t> jobs;                    // conv | z << 8 | cob << 20 | cib << 26
};
int rnn_conv_dw_group_plan(rnn_ctx *ctx, size_t n, DwGroupMember *m, int count,
                           DwGroupLaunch *L);
int rnn_conv_dw_group_upload(rnn_ctx *ctx, const DwGroupMember *m, DwGroupLaunch *L);
int rnn_conv_dw_group_launch(rnn_ctx *ctx, const DwGroupLaunch *L);

// ResNet layer launchers (nn.hip).  One BatchNorm2d layer's device state:
struct RnnBn {
    const double *part = nullptr;  // train: [c][P][2] partial sums of the layer input
    // partials per channel in part: 0 = the launchers' per-image-range split
    // (rnn_bn_stats_launch / the backward's partial pass), else the count a
    // conv's store pass wrote (rnn_conv_fast_parts)
    int P = 0;
    float m = 0.f, mom = 0.1f, eps = 1e-5f;  // m = n*hw (set by the launchers)
    float *mean = nullptr, *invstd = nullptr;  // batch statistics (train forward writes)
    float *rm = nullptr, *rv = nullptr;        // running statistics (train: updated if set)
    const float *gamma = nullptr, *beta = nullptr;
    float *dgamma = nullptr, *dbeta = nullptr;  // backward accumulators (may be null)
};
// f64 elements of BN partial-sum scratch for n images of c channels.
size_t rnn_bn_scratch_doubles(size_t n, size_t c);
// Partial sums (x, x^2) per (channel, image range) into part.
int rnn_bn_stats_launch(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *x, double *part);
// out = [relu](bn(x) [+ skip | + sbn(skip)]); skip_mode 0 / 1 / 2 (1 and 2
// imply relu).  Train mode finalises the statistics from bn.part (and
// sbn->part) and stores mean / invstd / running statistics; eval mode reads
// the running statistics.
int rnn_bn_apply_launch(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *x, RnnBn bn,
                        bool eval, int relu, int skip_mode, const float *skip, const RnnBn *sbn,
                        float *out);
// BN backward with relu_back by `mask` folded in (mask may be null): partial
// sums into `part`, then dx; bn.dgamma / bn.dbeta accumulate.
int rnn_bn_backward_launch(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *dy,
                           const float *mask, const float *x, RnnBn bn, double *part, float *dx);
// The dx pass alone, from partial sums already in `part`.
int rnn_bn_backward_apply_launch(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *dy,
                                 const float *mask, const float *x, RnnBn bn,
                                 const double *part, float *dx);
// A block's starting gradient d = relu_back_(a + add, mask) (or, with gsrc,
// of the GAP backward gsrc / hw), written over a, plus the BN-backward partial
// sums of bn1 (input x1) and optionally bn2 (input x2) over d.
int rnn_resid_bwd_launch(rnn_ctx *ctx, size_t n, size_t c, size_t hw, float *a, const float *add,
                         const float *mask, const float *gsrc, const RnnBn &bn1, const float *x1,
                         double *part1, const RnnBn *bn2, const float *x2, double *part2);
// a += [mask] b.
int rnn_add_launch(rnn_ctx *ctx, size_t len, float *a, const float *b, const float *mask);
// relu_back_ (nn.rs:432-439): d = 0 where y <= 0.
int rnn_relu_back_launch(rnn_ctx *ctx, size_t len, float *d, const float *y);
int rnn_gap_forward_launch(rnn_ctx *ctx, size_t nc, size_t hw, const float *x, float *y);
// dx = dy / hw broadcast over each plane.
int rnn_gap_backward_launch(rnn_ctx *ctx, size_t nc, size_t hw, const float *dy, float *dx);
int rnn_fc_forward_launch(rnn_ctx *ctx, size_t rows, size_t fin, size_t fout, const float *x,
                          const float *w, const float *b, float *y);
// gap (pooled [rows][fin]) then the classifier y = pooled W^T + b in one
// launch, the same bits as the two launches.
int rnn_gap_fc_forward_launch(rnn_ctx *ctx, size_t rows, size_t fin, size_t hw, size_t fout,
                              const float *x, const float *w, const float *b, float *pooled,
                              float *y);
int rnn_fc_backward_launch(rnn_ctx *ctx, size_t rows, size_t fin, size_t fout, const float *dy,
                           const float *x, const float *w, float *dw, float *db, float *dx);
// scal (device, may be null) overrides smooth with scal[3].  With ticket (a
// device word that is 0 between launches) and rowbuf (2*rows floats) set,
// the rows are spread over several blocks and the last one to finish adds
// them; the same values as the one-block form.
int rnn_softmax_ce_launch(rnn_ctx *ctx, size_t rows, size_t nclass, const float *logits,
                          const uint32_t *labels, float smooth, const float *scal, float *dl,
                          float *loss, uint32_t *correct, uint32_t *ticket = nullptr,
                          float *rowbuf = nullptr);
// Nesterov SGD over [0, len), weight decay on [0, ndecay); scal (device, may
// be null) overrides (lr, mom, wd) with scal[0..3].
int rnn_sgd_launch(rnn_ctx *ctx, size_t len, size_t ndecay, float *v, float *g, float *m, float lr,
                   float mom, float wd, const float *scal);
int rnn_set_scalars_launch(rnn_ctx *ctx, float *scal, float a, float b, float c, float d);

// One parameter tensor of a flat (v, g, m) layout for rnn_grad_finalize_launch:
// g[off, off+len) += the slab-order sum of nz slabs (nz may be 0); blk0 is the
// segment's first block (32 elements per block, segments in order).
struct GradSeg {
    long long off, len, blk0;
    const float *slabs;
    int nz, decay;
};
// Over every segment: g += slab sums; with do_sgd, then Param::step with
// (lr, mom, wd) from scal[0..3] (wd only where decay) and g zeroed.
int rnn_grad_finalize_launch(rnn_ctx *ctx, const GradSeg *segs, int nseg, long long nblocks,
                             float *v, float *g, float *m, const float *scal, int do_sgd);
