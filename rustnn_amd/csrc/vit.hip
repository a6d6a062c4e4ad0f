// vit.rs on the device: DropPath, the depthwise branch's per-channel gate,
// the 2x2 token merge, TaxoHead's parent gather and the NCHW <-> token
// layout changes (tok.rs).
//
// Reference: DropPath (vit.rs:25-74), Block's `a += gamma * dw(h)`
// (vit.rs:150-158), token_merge / token_merge_back (vit.rs:612-650),
// TaxoHead::forward / backward (vit.rs:282-312), Tok::from_tensor /
// to_tensor (tok.rs).  All HBM-bound copies and scalings; DropPath's mask is
// drawn on the device from Rng::new(seed) (rng.rs, splitmix64-seeded
// xoshiro256++, 24-bit uniforms), so the step needs no host round trip and
// draws the reference's mask bit for bit.
#include "rnn_internal.h"

#include <algorithm>

#pragma clang fp contract(off)

namespace {

constexpr int NT = 256;

unsigned ew_grid(size_t len) {
    return (unsigned)std::max<size_t>(1, std::min<size_t>(rnn_div_up(len, NT), 16384));
}

// DropPath::forward's mask (vit.rs:44-51): image i keeps its branch with the
// i-th uniform of Rng::new(seed) below 1 - p, scaled by 1 / keep, else 0.
// The generator is sequential: one wave draws all n with the state
// wave-uniform (scalar registers, scalar ALU), and lane i % 64 stores mask[i].
__device__ __forceinline__ void draw_drop_mask(size_t n, float p, uint64_t seed,
                                               float *__restrict__ mask) {
    const int lane = (int)threadIdx.x;
    RnnRng rng(seed);
    const float keep = 1.0f - p;
    for (size_t i = 0; i < n; i++) {
        const float u = rng.uniform();
        if ((int)(i & 63) == lane) mask[i] = u < keep ? 1.0f / keep : 0.0f;
    }
}

__global__ __launch_bounds__(64) void drop_path_mask_kernel(size_t n, float p, uint64_t seed,
                                                            float *__restrict__ mask) {
    draw_drop_mask(n, p, seed, mask);
}

// The masks of up to DP_BATCH DropPath layers in one launch, one wave each
// (the per-layer generators are independent).
constexpr int DP_BATCH = 32;
struct DropMasks {
    uint64_t seed[DP_BATCH];
    float *mask[DP_BATCH];
    float p[DP_BATCH];
    unsigned long long n;
};

__global__ __launch_bounds__(64) void drop_path_masks_kernel(DropMasks a) {
    const int k = (int)blockIdx.x;
    draw_drop_mask((size_t)a.n, a.p[k], a.seed[k], a.mask[k]);
}

// Rows times the mask, skipping the rows whose factor is 1 (the forward's
// scaling, vit.rs:52-57, and DropPath::backward, vit.rs:61-73).
__global__ __launch_bounds__(NT) void drop_path_bwd_kernel(size_t per, float *dy,
                                                           const float *__restrict__ mask) {
    const size_t img = blockIdx.y;
    const float f = mask[img];
    if (f == 1.0f) return;
    float *r = dy + img * per;
    for (size_t i = (size_t)blockIdx.x * NT + threadIdx.x; i < per; i += (size_t)gridDim.x * NT)
        r[i] *= f;
}

// y[r][j] += l[j] x[r][j] (vit.rs:153-158: a += gamma * dw).
__global__ void axpy_cols_kernel(size_t len, int c, float *y, const float *__restrict__ l,
                                 const float *__restrict__ x) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < len;
         i += (size_t)gridDim.x * blockDim.x)
        y[i] += l[i % c] * x[i];
}

// token_merge (vit.rs:612-630): y[n][t2*t2][4c] with the four neighbours
// (0,0), (0,1), (1,0), (1,1) of each 2x2 cell concatenated; back = the
// inverse copy.  One thread per element of y.
__global__ void token_merge_kernel(size_t n, int th, int c, const float *__restrict__ z,
                                   float *__restrict__ y, int back) {
    const int t2 = th / 2;
    const size_t len = n * (size_t)t2 * t2 * 4 * c;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < len;
         e += (size_t)gridDim.x * blockDim.x) {
        const int j = (int)(e % c);
        const size_t r = e / c;
        const int qd = (int)(r % 4);
        const size_t cell = r / 4;
        const int ox = (int)(cell % t2), oy = (int)((cell / t2) % t2);
        const size_t img = cell / ((size_t)t2 * t2);
        const int sy = 2 * oy + (qd >> 1), sx = 2 * ox + (qd & 1);
        const size_t s = (img * th * th + (size_t)sy * th + sx) * c + j;
        if (back)
            const_cast<float *>(z)[s] = y[e];
        else
            y[e] = z[s];
    }
}

// The same gather / scatter four channels a thread (c % 4 == 0, 16-byte
// aligned tensors, fewer than 2^31 quads), with 32-bit index arithmetic.
__global__ void token_merge4_kernel(uint32_t len4, int th, int c4, const float4 *__restrict__ z,
                                    float4 *__restrict__ y, int back) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= len4) return;
    const uint32_t t2 = (uint32_t)th / 2;
    const uint32_t r = i / (uint32_t)c4, j4 = i - r * (uint32_t)c4;
    const uint32_t qd = r & 3, cell = r >> 2;
    const uint32_t rest = cell / t2, ox = cell - rest * t2;
    const uint32_t img = rest / t2, oy = rest - img * t2;
    const uint32_t sy = 2 * oy + (qd >> 1), sx = 2 * ox + (qd & 1);
    const size_t s = ((size_t)img * th * th + (size_t)sy * th + sx) * c4 + j4;
    if (back)
        const_cast<float4 *>(z)[s] = y[i];
    else
        y[i] = z[s];
}

// TaxoHead (vit.rs:282-293): zf[i][j] += zc[i][parent[j]].
__global__ void taxo_fwd_kernel(size_t n, int nf, int nc, const uint32_t *__restrict__ parent,
                                float *zf, const float *__restrict__ zc) {
    const size_t len = n * nf;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < len;
         e += (size_t)gridDim.x * blockDim.x) {
        const size_t i = e / nf;
        const int j = (int)(e - i * nf);
        const uint32_t pj = parent[j];
        zf[e] += pj < (uint32_t)nc ? zc[i * nc + pj] : NAN;
    }
}

// TaxoHead::backward's coarse gradient (vit.rs:296-306): dc = dzc, then
// dc[parent[j]] += dzf[j] for j in order; one thread per row.
__global__ void taxo_bwd_kernel(size_t n, int nf, int nc, const uint32_t *__restrict__ parent,
                                const float *__restrict__ dzf, const float *__restrict__ dzc,
                                float *__restrict__ dc) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float *cr = dc + i * nc;
    for (int k = 0; k < nc; k++) cr[k] = dzc[i * nc + k];
    for (int j = 0; j < nf; j++) {
        const uint32_t pj = parent[j];
        if (pj < (uint32_t)nc) cr[pj] += dzf[i * nf + j];
    }
}

// The same for nc <= TAXO_LDS_NC: the row's accumulators in LDS (the adds in
// j order, as above), its dzf values loaded 16 ahead; 64 rows a block.
constexpr int TAXO_LDS_NC = 128;
__global__ __launch_bounds__(64) void taxo_bwd_lds_kernel(size_t n, int nf, int nc,
                                                          const uint32_t *__restrict__ parent,
                                                          const float *__restrict__ dzf,
                                                          const float *__restrict__ dzc,
                                                          float *__restrict__ dc) {
    extern __shared__ float acc[];  // [64][nc + 1]
    const size_t i = (size_t)blockIdx.x * 64 + threadIdx.x;
    if (i >= n) return;
    float *a = acc + threadIdx.x * (nc + 1);
    for (int k = 0; k < nc; k++) a[k] = dzc[i * nc + k];
    const float *dr = dzf + i * nf;
    for (int j0 = 0; j0 < nf; j0 += 16) {
        float v[16];
        uint32_t pv[16];
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const int j = min(j0 + u, nf - 1);
            v[u] = dr[j];
            pv[u] = parent[j];
        }
#pragma unroll
        for (int u = 0; u < 16; u++)
            if (j0 + u < nf && pv[u] < (uint32_t)nc) a[pv[u]] += v[u];
    }
    float *cr = dc + i * nc;
    for (int k = 0; k < nc; k++) cr[k] = a[k];
}

// [n][c][hw] <-> [n][hw][c] (Tok::from_tensor / to_tensor): 32 x 32 tiles
// through LDS so both sides are read and written along rows.
__global__ __launch_bounds__(NT) void nchw_tok_kernel(int c, int hw, const float *__restrict__ src,
                                                      float *__restrict__ dst, int to_tok) {
    __shared__ float tile[32][33];
    const size_t img = blockIdx.z;
    const int rows = to_tok ? c : hw, cols = to_tok ? hw : c;  // src is [rows][cols]
    const int r0 = blockIdx.y * 32, c0 = blockIdx.x * 32;
    const float *s = src + img * (size_t)c * hw;
    float *d = dst + img * (size_t)c * hw;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
    for (int k = ty; k < 32; k += 8) {
        const int r = r0 + k, cc = c0 + tx;
        if (r < rows && cc < cols) tile[k][tx] = s[(size_t)r * cols + cc];
    }
    __syncthreads();
    for (int k = ty; k < 32; k += 8) {
        const int cc = c0 + k, r = r0 + tx;  // dst is [cols][rows]
        if (cc < cols && r < rows) d[(size_t)cc * rows + r] = tile[tx][k];
    }
}

}  // namespace

extern "C" {

int rnn_drop_path_forward(rnn_ctx *ctx, size_t n, size_t per, float *x, float p, uint64_t seed,
                          float *mask) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (n == 0) return RNN_OK;
    if (!x || !mask) return rnn_fail(ctx, RNN_E_NULL, "drop_path: null operand");
    if (!(p > 0.0f) || !(p < 1.0f) || n > 65535)
        return rnn_fail(ctx, RNN_E_INVALID, "drop_path: p %g (0 < p < 1), n %zu (<= 65535)",
                        (double)p, n);
    drop_path_mask_kernel<<<1, 64, 0, ctx->stream>>>(n, p, seed, mask);
    RNN_LAUNCHED(ctx);
    const unsigned gx = (unsigned)std::max<size_t>(1, std::min<size_t>(rnn_div_up(per, NT), 64));
    drop_path_bwd_kernel<<<dim3(gx, (unsigned)n), NT, 0, ctx->stream>>>(per, x, mask);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_drop_path_masks(rnn_ctx *ctx, size_t count, size_t n, const float *p,
                        const uint64_t *seeds, float *const *masks) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (count == 0 || n == 0) return RNN_OK;
    if (!p || !seeds || !masks) return rnn_fail(ctx, RNN_E_NULL, "drop_path_masks: null operand");
    if (n > 65535) return rnn_fail(ctx, RNN_E_INVALID, "drop_path_masks: n %zu (<= 65535)", n);
    for (size_t k0 = 0; k0 < count; k0 += DP_BATCH) {
        const size_t cnt = std::min<size_t>(DP_BATCH, count - k0);
        DropMasks a{};
        a.n = n;
        for (size_t k = 0; k < cnt; k++) {
            const float pk = p[k0 + k];
            if (!(pk > 0.0f) || !(pk < 1.0f))
                return rnn_fail(ctx, RNN_E_INVALID, "drop_path_masks: p %g (0 < p < 1)",
                                (double)pk);
            if (!masks[k0 + k]) return rnn_fail(ctx, RNN_E_NULL, "drop_path_masks: null mask");
            a.seed[k] = seeds[k0 + k];
            a.mask[k] = masks[k0 + k];
            a.p[k] = pk;
        }
        drop_path_masks_kernel<<<(unsigned)cnt, 64, 0, ctx->stream>>>(a);
        RNN_LAUNCHED(ctx);
    }
    return RNN_OK;
}

int rnn_drop_path_backward(rnn_ctx *ctx, size_t n, size_t per, float *dy, const float *mask) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (n == 0) return RNN_OK;
    if (!dy || !mask) return rnn_fail(ctx, RNN_E_NULL, "drop_path_backward: null operand");
    if (n > 65535) return rnn_fail(ctx, RNN_E_INVALID, "drop_path: n %zu (<= 65535)", n);
    const unsigned gx = (unsigned)std::max<size_t>(1, std::min<size_t>(rnn_div_up(per, NT), 64));
    drop_path_bwd_kernel<<<dim3(gx, (unsigned)n), NT, 0, ctx->stream>>>(per, dy, mask);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_axpy_cols(rnn_ctx *ctx, size_t rows, size_t c, float *y, const float *l, const float *x) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (rows == 0 || c == 0) return RNN_OK;
    if (!y || !l || !x) return rnn_fail(ctx, RNN_E_NULL, "axpy_cols: null operand");
    if (c > 0x7fffffff) return rnn_fail(ctx, RNN_E_INVALID, "axpy_cols: c %zu", c);
    axpy_cols_kernel<<<ew_grid(rows * c), NT, 0, ctx->stream>>>(rows * c, (int)c, y, l, x);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

// The four-channel token merge: c % 4 == 0, aligned tensors, quads in 32 bits.
static bool merge_vec(size_t c, size_t len, const void *a, const void *b) {
    return c % 4 == 0 && len / 4 < ((size_t)1 << 31) &&
           (((uintptr_t)a | (uintptr_t)b) & 15) == 0;
}

int rnn_token_merge(rnn_ctx *ctx, size_t n, size_t th, size_t c, const float *z, float *y) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (n == 0 || c == 0) return RNN_OK;
    if (!z || !y) return rnn_fail(ctx, RNN_E_NULL, "token_merge: null operand");
    if (th < 2 || th % 2 || th > 65536 || c > (1u << 24))
        return rnn_fail(ctx, RNN_E_INVALID, "token_merge: th %zu (even), c %zu", th, c);
    const size_t len = n * th * th * c;
    if (merge_vec(c, len, z, y))
        token_merge4_kernel<<<(unsigned)rnn_div_up(len / 4, (size_t)NT), NT, 0, ctx->stream>>>(
            (uint32_t)(len / 4), (int)th, (int)(c / 4), (const float4 *)z, (float4 *)y, 0);
    else
        token_merge_kernel<<<ew_grid(len), NT, 0, ctx->stream>>>(n, (int)th, (int)c, z, y, 0);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_token_merge_backward(rnn_ctx *ctx, size_t n, size_t th, size_t c, const float *dy,
                             float *dz) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (n == 0 || c == 0) return RNN_OK;
    if (!dy || !dz) return rnn_fail(ctx, RNN_E_NULL, "token_merge_backward: null operand");
    if (th < 2 || th % 2 || th > 65536 || c > (1u << 24))
        return rnn_fail(ctx, RNN_E_INVALID, "token_merge: th %zu (even), c %zu", th, c);
    const size_t len = n * th * th * c;
    if (merge_vec(c, len, dz, dy))
        token_merge4_kernel<<<(unsigned)rnn_div_up(len / 4, (size_t)NT), NT, 0, ctx->stream>>>(
            (uint32_t)(len / 4), (int)th, (int)(c / 4), (const float4 *)dz,
            (float4 *)const_cast<float *>(dy), 1);
    else
        token_merge_kernel<<<ew_grid(len), NT, 0, ctx->stream>>>(n, (int)th, (int)c, dz,
                                                                  const_cast<float *>(dy), 1);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_taxo_head_combine(rnn_ctx *ctx, size_t n, size_t nf, size_t nc, const uint32_t *parent,
                          float *zf, const float *zc) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (n == 0 || nf == 0) return RNN_OK;
    if (!parent || !zf || !zc) return rnn_fail(ctx, RNN_E_NULL, "taxo_head: null operand");
    if (nf > (1u << 24) || nc > (1u << 24))
        return rnn_fail(ctx, RNN_E_INVALID, "taxo_head: nf %zu nc %zu", nf, nc);
    taxo_fwd_kernel<<<ew_grid(n * nf), NT, 0, ctx->stream>>>(n, (int)nf, (int)nc, parent, zf, zc);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_taxo_head_combine_backward(rnn_ctx *ctx, size_t n, size_t nf, size_t nc,
                                   const uint32_t *parent, const float *dzf, const float *dzc,
                                   float *dc) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (n == 0 || nc == 0) return RNN_OK;
    if (!parent || !dzf || !dzc || !dc)
        return rnn_fail(ctx, RNN_E_NULL, "taxo_head_backward: null operand");
    if (nf > (1u << 24) || nc > (1u << 24))
        return rnn_fail(ctx, RNN_E_INVALID, "taxo_head: nf %zu nc %zu", nf, nc);
    if (nc <= (size_t)TAXO_LDS_NC)
        taxo_bwd_lds_kernel<<<(unsigned)rnn_div_up(n, (size_t)64), 64,
                              64 * (nc + 1) * sizeof(float), ctx->stream>>>(
            n, (int)nf, (int)nc, parent, dzf, dzc, dc);
    else
        taxo_bwd_kernel<<<(unsigned)rnn_div_up(n, (size_t)NT), NT, 0, ctx->stream>>>(
            n, (int)nf, (int)nc, parent, dzf, dzc, dc);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_nchw_to_tokens(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *x, float *t) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (n == 0 || c == 0 || hw == 0) return RNN_OK;
    if (!x || !t) return rnn_fail(ctx, RNN_E_NULL, "nchw_to_tokens: null operand");
    if (n > 65535 || c > (1u << 24) || hw > (1u << 24))
        return rnn_fail(ctx, RNN_E_INVALID, "nchw_to_tokens: %zu x %zu x %zu", n, c, hw);
    const dim3 grid((unsigned)rnn_div_up(hw, (size_t)32), (unsigned)rnn_div_up(c, (size_t)32),
                    (unsigned)n);
    nchw_tok_kernel<<<grid, NT, 0, ctx->stream>>>((int)c, (int)hw, x, t, 1);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_tokens_to_nchw(rnn_ctx *ctx, size_t n, size_t c, size_t hw, const float *t, float *x) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (n == 0 || c == 0 || hw == 0) return RNN_OK;
    if (!x || !t) return rnn_fail(ctx, RNN_E_NULL, "tokens_to_nchw: null operand");
    if (n > 65535 || c > (1u << 24) || hw > (1u << 24))
        return rnn_fail(ctx, RNN_E_INVALID, "tokens_to_nchw: %zu x %zu x %zu", n, c, hw);
    const dim3 grid((unsigned)rnn_div_up(c, (size_t)32), (unsigned)rnn_div_up(hw, (size_t)32),
                    (unsigned)n);
    nchw_tok_kernel<<<grid, NT, 0, ctx->stream>>>((int)c, (int)hw, t, x, 0);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

}  // extern "C"
