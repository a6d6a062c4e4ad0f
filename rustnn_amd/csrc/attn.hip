// Batched small attention (attn.rs Core) on gfx950: one workgroup per
// (image, head), all operands resident in LDS, 32x32 fp32 MFMA tiles and
// wave-wide reductions for the row softmax.
//
// Reference: Core::forward (attn.rs:148-223) runs per image (rayon) and per
// head: gather Q/K/V rows, S = QK^T (gemm_small), x = tau*S + rel[idx] with the
// diagonal masked, row softmax, O = PV.  Core::backward (attn.rs:226-343):
// dV = P^T dO, dP = dO V^T, dS = P o (dP - rowdot), recomputed raw S for dtau,
// drel scatter by rel index, dQ = tau*dS K, dK = tau*dS^T Q.
//
// Here dtau and drel are reduced without atomics: each workgroup writes its
// (image, head) partial -- drel through an inverse index (for every bias slot,
// the positions that map to it, in ascending order) -- and a second kernel
// adds the partials over images in image order.
#include "rnn_internal.h"

#include <algorithm>
#include <cstring>

namespace {

constexpr int MAXT = 64;   // tq, tk limit (padded to 32 or 64)
constexpr int MAXDH = 64;  // head-dim limit

struct AttnArgs {
    const float *q, *kv, *tau, *rel, *p, *dout;
    float *pout, *o, *dq, *dkv;
    float *dtau_part, *drel_part;  // [n][h], [n][h][nrel]
    const uint32_t *relidx;        // [tq*tk]
    const uint32_t *rowptr;        // [nrel+1] inverse index (drel gather)
    const uint32_t *pos;           // [tq*tk]
    long long qstride, qoff, kvstride, koff, voff;
    int n, h, dh, tq, tk, nrel, mask;
    int TQ, TK, DHP, DHK;  // padded sizes (tiles of 32; even K for MFMA)
};

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// acc += A * B for one 32x32 tile with A(m, k) = LA[m*sam + k*sak] and
// B(k, n) = LB[k*sbk + n*sbn], k in [0, K) with K even.  Odd row strides keep
// every b32 LDS read conflict-free.
__device__ __forceinline__ void tile_mma(f32x16 &acc, const float *LA, int sam, int sak,
                                         const float *LB, int sbk, int sbn, int K, int lane) {
    const int l32 = lane & 31, h = lane >> 5;
    const float *pa = LA + l32 * sam + h * sak;
    const float *pb = LB + h * sbk + l32 * sbn;
    for (int k0 = 0; k0 < K; k0 += 2) {
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(pa[k0 * sak], pb[k0 * sbk], acc, 0, 0, 0);
    }
}

__device__ __forceinline__ void zero16(f32x16 &a) {
#pragma unroll
    for (int v = 0; v < 16; v++) a[v] = 0.f;
}

// Loads rows [0, rows) x cols [0, cols) of a strided matrix into LDS
// (row stride ld), zero-padding up to prow x pcol.
__device__ __forceinline__ void load_rows(float *dst, int ld, const float *src, long long sstride,
                                          int rows, int cols, int prow, int pcol, int tid,
                                          int nthreads) {
    for (int idx = tid; idx < prow * pcol; idx += nthreads) {
        int r = idx / pcol, c = idx - r * pcol;
        dst[r * ld + c] = (r < rows && c < cols) ? src[r * sstride + c] : 0.f;
    }
}

__global__ __launch_bounds__(256) void attn_fwd_kernel(AttnArgs g) {
    extern __shared__ float smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_index(), nthreads = blockDim.x;
    const int img = blockIdx.x / g.h, hd = blockIdx.x % g.h;
    const int DS = g.DHP + 1, PS = g.TK + 1;
    float *Qs = smem, *Ks = Qs + g.TQ * DS, *Vs = Ks + g.TK * DS, *Ps = Vs + g.TK * DS;

    const float *qsrc = g.q + (long long)img * g.tq * g.qstride + g.qoff + (long long)hd * g.dh;
    const float *ksrc = g.kv + (long long)img * g.tk * g.kvstride + g.koff + (long long)hd * g.dh;
    const float *vsrc = g.kv + (long long)img * g.tk * g.kvstride + g.voff + (long long)hd * g.dh;
    load_rows(Qs, DS, qsrc, g.qstride, g.tq, g.dh, g.TQ, g.DHP, tid, nthreads);
    load_rows(Ks, DS, ksrc, g.kvstride, g.tk, g.dh, g.TK, g.DHP, tid, nthreads);
    load_rows(Vs, DS, vsrc, g.kvstride, g.tk, g.dh, g.TK, g.DHP, tid, nthreads);
    __syncthreads();

    const float t = g.tau[hd];
    const float *rb = g.rel + (long long)hd * g.nrel;
    const int l32 = lane & 31, lh = lane >> 5;
    // S = Q K^T, epilogue x = tau*S + rel[idx], diagonal -> -inf (attn.rs:187-198)
    const int stm = g.TQ / 32, stn = g.TK / 32;
    if (wave < stm * stn) {
        const int mt = wave / stn, nt = wave % stn;
        f32x16 acc;
        zero16(acc);
        tile_mma(acc, Qs + mt * 32 * DS, DS, 1, Ks + nt * 32 * DS, 1, DS, g.DHK, lane);
#pragma unroll
        for (int v = 0; v < 16; v++) {
            int qi = mt * 32 + 8 * (v >> 2) + 4 * lh + (v & 3), kj = nt * 32 + l32;
            float x = -INFINITY;
            if (qi < g.tq && kj < g.tk) {
                x = t * acc[v] + rb[g.relidx[qi * g.tk + kj]];
                if (g.mask && kj == qi) x = -INFINITY;
            }
            Ps[qi * PS + kj] = x;
        }
    }
    __syncthreads();
    // Row softmax: exp(x - max) (-inf -> 0), sum, times 1/sum (attn.rs:199-210).
    float *pg = g.pout + ((long long)img * g.h + hd) * g.tq * g.tk;
    for (int qi = wave; qi < g.TQ; qi += nthreads >> 6) {
        float *row = Ps + qi * PS;
        if (qi >= g.tq) {
            for (int kj = lane; kj < g.TK; kj += 64) row[kj] = 0.f;
            continue;
        }
        float x0 = lane < g.tk ? row[lane] : -INFINITY;
        float mx = wave_max(x0);
        float e0 = (x0 == -INFINITY) ? 0.f : expf(x0 - mx);
        float sum = wave_sum(e0);
        float inv = 1.0f / sum;
        float p0 = e0 * inv;
        if (lane < g.TK) row[lane] = lane < g.tk ? p0 : 0.f;
        if (lane < g.tk) pg[(long long)qi * g.tk + lane] = p0;
    }
    __syncthreads();
    // O = P V (attn.rs:213-220), written at column hd*dh of o[n][tq][h*dh].
    const int otm = g.TQ / 32, otn = g.DHP / 32;
    if (wave < otm * otn) {
        const int mt = wave / otn, nt = wave % otn;
        f32x16 acc;
        zero16(acc);
        tile_mma(acc, Ps + mt * 32 * PS, PS, 1, Vs + nt * 32, DS, 1, g.TK, lane);
        const int c = g.h * g.dh;
        float *od = g.o + (long long)img * g.tq * c + (long long)hd * g.dh;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            int qi = mt * 32 + 8 * (v >> 2) + 4 * lh + (v & 3), d = nt * 32 + l32;
            if (qi < g.tq && d < g.dh) od[(long long)qi * c + d] = acc[v];
        }
    }
}

__global__ __launch_bounds__(256) void attn_bwd_kernel(AttnArgs g) {
    extern __shared__ float smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_index(), nthreads = blockDim.x;
    const int nwaves = nthreads >> 6;
    const int img = blockIdx.x / g.h, hd = blockIdx.x % g.h;
    const int DS = g.DHP + 1, PS = g.TK + 1;
    float *Qs = smem, *Ks = Qs + g.TQ * DS, *Vs = Ks + g.TK * DS, *Os = Vs + g.TK * DS;
    float *Ps = Os + g.TQ * DS, *Ss = Ps + g.TQ * PS, *red = Ss + g.TQ * PS;
    const int l32 = lane & 31, lh = lane >> 5;
    const int c = g.h * g.dh;

    const float *qsrc = g.q + (long long)img * g.tq * g.qstride + g.qoff + (long long)hd * g.dh;
    const float *ksrc = g.kv + (long long)img * g.tk * g.kvstride + g.koff + (long long)hd * g.dh;
    const float *vsrc = g.kv + (long long)img * g.tk * g.kvstride + g.voff + (long long)hd * g.dh;
    const float *dosrc = g.dout + (long long)img * g.tq * c + (long long)hd * g.dh;
    const float *psrc = g.p + ((long long)img * g.h + hd) * g.tq * g.tk;
    load_rows(Qs, DS, qsrc, g.qstride, g.tq, g.dh, g.TQ, g.DHP, tid, nthreads);
    load_rows(Ks, DS, ksrc, g.kvstride, g.tk, g.dh, g.TK, g.DHP, tid, nthreads);
    load_rows(Vs, DS, vsrc, g.kvstride, g.tk, g.dh, g.TK, g.DHP, tid, nthreads);
    load_rows(Os, DS, dosrc, c, g.tq, g.dh, g.TQ, g.DHP, tid, nthreads);
    load_rows(Ps, PS, psrc, g.tk, g.tq, g.tk, g.TQ, g.TK, tid, nthreads);
    __syncthreads();

    float *dqi = g.dq + (long long)img * g.tq * g.qstride + g.qoff + (long long)hd * g.dh;
    float *dki = g.dkv + (long long)img * g.tk * g.kvstride + g.koff + (long long)hd * g.dh;
    float *dvi = g.dkv + (long long)img * g.tk * g.kvstride + g.voff + (long long)hd * g.dh;

    // dV = P^T dO -> dkv at voff (attn.rs:270-274)
    {
        const int tm = g.TK / 32, tn = g.DHP / 32;
        if (wave < tm * tn) {
            const int mt = wave / tn, nt = wave % tn;
            f32x16 acc;
            zero16(acc);
            tile_mma(acc, Ps + mt * 32, 1, PS, Os + nt * 32, DS, 1, g.TQ, lane);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                int kj = mt * 32 + 8 * (v >> 2) + 4 * lh + (v & 3), d = nt * 32 + l32;
                if (kj < g.tk && d < g.dh) dvi[(long long)kj * g.kvstride + d] += acc[v];
            }
        }
    }
    // dP = dO V^T into Ss (attn.rs:276-279)
    {
        const int tm = g.TQ / 32, tn = g.TK / 32;
        if (wave < tm * tn) {
            const int mt = wave / tn, nt = wave % tn;
            f32x16 acc;
            zero16(acc);
            tile_mma(acc, Os + mt * 32 * DS, DS, 1, Vs + nt * 32 * DS, 1, DS, g.DHK, lane);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                int qi = mt * 32 + 8 * (v >> 2) + 4 * lh + (v & 3), kj = nt * 32 + l32;
                Ss[qi * PS + kj] = acc[v];
            }
        }
    }
    __syncthreads();
    // dS = P o (dP - <dP, P>) per row (attn.rs:280-290)
    for (int qi = wave; qi < g.TQ; qi += nwaves) {
        float *sr = Ss + qi * PS;
        const float *pr = Ps + qi * PS;
        if (qi >= g.tq) {
            for (int kj = lane; kj < g.TK; kj += 64) sr[kj] = 0.f;
            continue;
        }
        float dp = lane < g.tk ? sr[lane] : 0.f, pp = lane < g.tk ? pr[lane] : 0.f;
        float dot = wave_sum(dp * pp);
        if (lane < g.TK) sr[lane] = lane < g.tk ? pp * (dp - dot) : 0.f;
    }
    __syncthreads();
    // dtau partial: sum of dS o raw QK^T (attn.rs:292-308)
    {
        const int tm = g.TQ / 32, tn = g.TK / 32;
        float part = 0.f;
        if (wave < tm * tn) {
            const int mt = wave / tn, nt = wave % tn;
            f32x16 acc;
            zero16(acc);
            tile_mma(acc, Qs + mt * 32 * DS, DS, 1, Ks + nt * 32 * DS, 1, DS, g.DHK, lane);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                int qi = mt * 32 + 8 * (v >> 2) + 4 * lh + (v & 3), kj = nt * 32 + l32;
                part += Ss[qi * PS + kj] * acc[v];  // padded entries of dS are 0
            }
        }
        part = wave_sum(part);
        if (lane == 0) red[wave] = part;
    }
    // drel partial: gather by inverse index in ascending position (attn.rs:309-315)
    float *drp = g.drel_part + ((long long)img * g.h + hd) * g.nrel;
    for (int r = tid; r < g.nrel; r += nthreads) {
        float s = 0.f;
        for (uint32_t e = g.rowptr[r]; e < g.rowptr[r + 1]; e++) {
            uint32_t ps = g.pos[e];
            s += Ss[(ps / g.tk) * PS + ps % g.tk];
        }
        drp[r] = s;
    }
    __syncthreads();
    if (tid == 0) {
        float s = 0.f;
        for (int w = 0; w < nwaves; w++) s += red[w];
        g.dtau_part[(long long)img * g.h + hd] = s;
    }
    // dS *= tau (attn.rs:316)
    const float t = g.tau[hd];
    for (int idx = tid; idx < g.TQ * g.TK; idx += nthreads) {
        int qi = idx / g.TK, kj = idx - qi * g.TK;
        Ss[qi * PS + kj] *= t;
    }
    __syncthreads();
    // dQ = dS K -> dq at qoff (attn.rs:319-323)
    {
        const int tm = g.TQ / 32, tn = g.DHP / 32;
        if (wave < tm * tn) {
            const int mt = wave / tn, nt = wave % tn;
            f32x16 acc;
            zero16(acc);
            tile_mma(acc, Ss + mt * 32 * PS, PS, 1, Ks + nt * 32, DS, 1, g.TK, lane);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                int qi = mt * 32 + 8 * (v >> 2) + 4 * lh + (v & 3), d = nt * 32 + l32;
                if (qi < g.tq && d < g.dh) dqi[(long long)qi * g.qstride + d] += acc[v];
            }
        }
    }
    // dK = dS^T Q -> dkv at koff (attn.rs:324-327)
    {
        const int tm = g.TK / 32, tn = g.DHP / 32;
        if (wave < tm * tn) {
            const int mt = wave / tn, nt = wave % tn;
            f32x16 acc;
            zero16(acc);
            tile_mma(acc, Ss + mt * 32, 1, PS, Qs + nt * 32, DS, 1, g.TQ, lane);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                int kj = mt * 32 + 8 * (v >> 2) + 4 * lh + (v & 3), d = nt * 32 + l32;
                if (kj < g.tk && d < g.dh) dki[(long long)kj * g.kvstride + d] += acc[v];
            }
        }
    }
}

// dtau[h] += sum_img part[img][h]; drel[h*nrel + r] += sum_img part[img][h][r]
// (image order, attn.rs:333-342).  A block takes 32 elements; thread (j, e)
// sums images [j*G, j*G + G) of element e with the loads issued ahead of the
// in-order adds, then the 8 partials are added in j order (fixed order:
// bit-reproducible).
constexpr int ATTN_RED_PARTS = 8;
__global__ __launch_bounds__(256) void attn_reduce_kernel(const float *dtau_part,
                                                          const float *drel_part, int n, int h,
                                                          int nrel, float *dtau, float *drel) {
    __shared__ float part[ATTN_RED_PARTS][32];
    const int el = threadIdx.x & 31, j = threadIdx.x >> 5;
    const int e = blockIdx.x * 32 + el;
    const int per = h * nrel;
    const bool is_rel = e < per, live = e < per + h;
    const float *src = is_rel ? drel_part + e : dtau_part + (e - per);
    const long long stride = is_rel ? per : h;
    const int G = (n + ATTN_RED_PARTS - 1) / ATTN_RED_PARTS;
    const int i0 = j * G, i1 = min(n, i0 + G);
    float s = 0.f;
    if (live) {
        for (int b = i0; b < i1; b += 16) {
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; u++) v[u] = b + u < i1 ? src[(long long)(b + u) * stride] : 0.f;
#pragma unroll
            for (int u = 0; u < 16; u++)
                if (b + u < i1) s = (b + u == i0) ? v[u] : s + v[u];
        }
    }
    part[j][el] = s;
    __syncthreads();
    if (j == 0 && live) {
        float t = 0.f;
        bool first = true;
        for (int q = 0; q < ATTN_RED_PARTS; q++) {
            if (q * G >= n) break;
            t = first ? part[q][el] : t + part[q][el];
            first = false;
        }
        if (is_rel)
            drel[e] += t;
        else
            dtau[e - per] += t;
    }
}

__global__ void rel_index_kernel(int th, int tw, int mh, int mw, uint32_t *idx) {
    long long total = (long long)th * tw * mh * mw;
    long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= total) return;
    int mx = (int)(e % mw);
    long long r = e / mw;
    int my = (int)(r % mh);
    r /= mh;
    int qx = (int)(r % tw), qy = (int)(r / tw);
    int sx, scale, oy, ox;
    if (mh == th) {
        sx = 2 * tw - 1;
        scale = 1;
        oy = th - 1;
        ox = tw - 1;
    } else {
        sx = 2 * (tw - 1) + mw;
        scale = 2;
        oy = mh - 1;
        ox = mw - 1;
    }
    int dy = scale * qy - my + oy, dx = scale * qx - mx + ox;
    idx[e] = (uint32_t)(dy * sx + dx);
}

int check_desc(rnn_ctx *ctx, const rnn_attn_desc *d) {
    if (!d) return rnn_fail(ctx, RNN_E_NULL, "attn: desc is null");
    if (!d->relidx) return rnn_fail(ctx, RNN_E_NULL, "attn: relidx is null");
    if (!d->h || !d->dh || !d->tq || !d->tk || !d->nrel)
        return rnn_fail(ctx, RNN_E_INVALID, "attn: zero dimension");
    if (d->tq > MAXT || d->tk > MAXT || d->dh > MAXDH)
        return rnn_fail(ctx, RNN_E_UNSUPPORTED,
                        "attn: tq=%u tk=%u dh=%u beyond the LDS-resident kernel (64/64/64)", d->tq,
                        d->tk, d->dh);
    for (size_t i = 0; i < (size_t)d->tq * d->tk; i++)
        if (d->relidx[i] >= d->nrel) return rnn_fail(ctx, RNN_E_INVALID, "attn: relidx >= nrel");
    return RNN_OK;
}

// Uploads relidx and its inverse index (CSR over bias slots) when the table
// differs from the last one.
int upload_rel(rnn_ctx *ctx, const rnn_attn_desc *d) {
    size_t cnt = (size_t)d->tq * d->tk;
    if (ctx->rel_dev && ctx->rel_nrel == d->nrel && ctx->rel_host.size() == cnt &&
        std::memcmp(ctx->rel_host.data(), d->relidx, cnt * 4) == 0)
        return RNN_OK;
    size_t need = cnt + (d->nrel + 1) + cnt;
    // The previous upload (and kernels reading it) must be done before reuse.
    RNN_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (need > ctx->rel_cap) {
        if (ctx->rel_dev) (void)hipFree(ctx->rel_dev);
        ctx->rel_dev = nullptr;
        RNN_HIP(ctx, hipMalloc(&ctx->rel_dev, need * 4));
        ctx->rel_cap = need;
    }
    if (need > ctx->rel_pinned_cap) {
        if (ctx->rel_pinned) (void)hipHostFree(ctx->rel_pinned);
        ctx->rel_pinned = nullptr;
        RNN_HIP(ctx, hipHostMalloc((void **)&ctx->rel_pinned, need * 4, hipHostMallocDefault));
        ctx->rel_pinned_cap = need;
    }
    uint32_t *h = ctx->rel_pinned;
    std::memcpy(h, d->relidx, cnt * 4);
    uint32_t *rowptr = h + cnt, *pos = rowptr + d->nrel + 1;
    std::vector<uint32_t> count(d->nrel + 1, 0);
    for (size_t i = 0; i < cnt; i++) count[d->relidx[i] + 1]++;
    for (uint32_t r = 0; r < d->nrel; r++) count[r + 1] += count[r];
    for (uint32_t r = 0; r <= d->nrel; r++) rowptr[r] = count[r];
    for (size_t i = 0; i < cnt; i++) pos[count[d->relidx[i]]++] = (uint32_t)i;
    RNN_HIP(ctx, hipMemcpyAsync(ctx->rel_dev, h, need * 4, hipMemcpyHostToDevice, ctx->stream));
    ctx->rel_host.assign(d->relidx, d->relidx + cnt);
    ctx->rel_nrel = d->nrel;
    return RNN_OK;
}

void fill_args(AttnArgs &g, rnn_ctx *ctx, const rnn_attn_desc *d, size_t n) {
    std::memset(&g, 0, sizeof(g));
    g.qstride = (long long)d->qstride;
    g.qoff = (long long)d->qoff;
    g.kvstride = (long long)d->kvstride;
    g.koff = (long long)d->koff;
    g.voff = (long long)d->voff;
    g.n = (int)n;
    g.h = d->h;
    g.dh = d->dh;
    g.tq = d->tq;
    g.tk = d->tk;
    g.nrel = d->nrel;
    g.mask = d->mask_diag ? 1 : 0;
    g.TQ = (int)rnn_round_up(d->tq, 32);
    g.TK = (int)rnn_round_up(d->tk, 32);
    g.DHP = (int)rnn_round_up(d->dh, 32);
    g.DHK = (int)rnn_round_up(d->dh, 2);
    size_t cnt = (size_t)d->tq * d->tk;
    g.relidx = ctx->rel_dev;
    g.rowptr = ctx->rel_dev + cnt;
    g.pos = ctx->rel_dev + cnt + d->nrel + 1;
}

bool lds_attr_done = false;
void set_lds_limits() {
    if (lds_attr_done) return;
    lds_attr_done = true;
    (void)hipFuncSetAttribute((const void *)attn_fwd_kernel,
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    (void)hipFuncSetAttribute((const void *)attn_bwd_kernel,
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
}

}  // namespace

extern "C" {

int rnn_attn_forward(rnn_ctx *ctx, const rnn_attn_desc *d, size_t n, const float *q,
                     const float *kv, const float *tau, const float *rel, float *p, float *o) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    int rc = check_desc(ctx, d);
    if (rc) return rc;
    if (n == 0) return RNN_OK;
    if (!q || !kv || !tau || !rel || !p || !o)
        return rnn_fail(ctx, RNN_E_NULL, "attn_forward: null operand");
    if (n * d->h > 0x7fffffffu) return rnn_fail(ctx, RNN_E_UNSUPPORTED, "attn: too many problems");
    set_lds_limits();
    rc = upload_rel(ctx, d);
    if (rc) return rc;
    AttnArgs g;
    fill_args(g, ctx, d, n);
    g.q = q;
    g.kv = kv;
    g.tau = tau;
    g.rel = rel;
    g.pout = p;
    g.o = o;
    size_t lds = ((size_t)g.TQ * (g.DHP + 1) + 2 * (size_t)g.TK * (g.DHP + 1) +
                  (size_t)g.TQ * (g.TK + 1)) * 4;
    hipLaunchKernelGGL(attn_fwd_kernel, dim3((unsigned)(n * d->h)), dim3(256), lds, ctx->stream, g);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_attn_backward(rnn_ctx *ctx, const rnn_attn_desc *d, size_t n, const float *q,
                      const float *kv, const float *tau, const float *p, const float *dout,
                      float *dq, float *dkv, float *dtau, float *drel) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    int rc = check_desc(ctx, d);
    if (rc) return rc;
    if (n == 0) return RNN_OK;
    if (!q || !kv || !tau || !p || !dout || !dq || !dkv || !dtau || !drel)
        return rnn_fail(ctx, RNN_E_NULL, "attn_backward: null operand");
    if (n * d->h > 0x7fffffffu) return rnn_fail(ctx, RNN_E_UNSUPPORTED, "attn: too many problems");
    set_lds_limits();
    rc = upload_rel(ctx, d);
    if (rc) return rc;
    AttnArgs g;
    fill_args(g, ctx, d, n);
    size_t parts = n * d->h + n * d->h * (size_t)d->nrel;
    float *ws = (float *)rnn_workspace(ctx, parts * sizeof(float));
    if (!ws) return RNN_E_NOMEM;
    g.q = q;
    g.kv = kv;
    g.tau = tau;
    g.p = p;
    g.dout = dout;
    g.dq = dq;
    g.dkv = dkv;
    g.dtau_part = ws;
    g.drel_part = ws + n * d->h;
    size_t lds = ((size_t)2 * g.TQ * (g.DHP + 1) + 2 * (size_t)g.TK * (g.DHP + 1) +
                  2 * (size_t)g.TQ * (g.TK + 1) + 8) * 4;
    hipLaunchKernelGGL(attn_bwd_kernel, dim3((unsigned)(n * d->h)), dim3(256), lds, ctx->stream, g);
    RNN_LAUNCHED(ctx);
    int tot = (int)(d->h * d->nrel + d->h);
    hipLaunchKernelGGL(attn_reduce_kernel, dim3((unsigned)rnn_div_up(tot, 32)), dim3(256), 0,
                       ctx->stream, (const float *)g.dtau_part, (const float *)g.drel_part, (int)n,
                       (int)d->h, (int)d->nrel, dtau, drel);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_dbg_rel_index(rnn_ctx *ctx, uint32_t th, uint32_t tw, uint32_t mh, uint32_t mw,
                      uint32_t *idx) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (!idx) return RNN_E_NULL;
    if (!th || !tw || !mh || !mw) return rnn_fail(ctx, RNN_E_INVALID, "rel_index: zero grid");
    long long total = (long long)th * tw * mh * mw;
    hipLaunchKernelGGL(rel_index_kernel, dim3((unsigned)rnn_div_up(total, 256)), dim3(256), 0,
                       ctx->stream, (int)th, (int)tw, (int)mh, (int)mw, idx);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

}  // extern "C"
