// Batched small attention (attn.rs Core) on gfx950.
//
// Reference: Core::forward (attn.rs:148-223) runs per image (rayon) and per
// head: gather Q/K/V rows, S = QK^T (gemm_small), x = tau*S + rel[idx] with the
// diagonal masked, row softmax, O = PV.  Core::backward (attn.rs:226-343):
// dV = P^T dO, dP = dO V^T, dS = P o (dP - rowdot), recomputed raw S for dtau,
// drel scatter by rel index, dQ = tau*dS K, dK = tau*dS^T Q.
//
// tq, tk <= 64 and dh <= 64 (every Core of the reference's models but the
// rustvit's cross-attention over 256 memory tokens): one workgroup per
// (image, head) of up to four waves; wave w owns queries [16w, 16w + 16) and
// every product runs on 16x16x4 fp32 MFMA tiles.  K and V (and, in the
// backward, Q and dO) are staged once per workgroup in LDS and shared by the
// waves, so HBM sees each tensor once.
//
// Score tiles are computed transposed (S^T = K Q^T): lane l of wave w then
// holds query 16w + l%16 and, in register v of key tile t, key 16t + 4(l/16)
// + v.  A query's row spans the four lanes l%16 + 16g: max and sum take two
// cross-lane steps, and P's registers are, step for step, the A operand of the
// products over keys (O = P V, dS K) -- step (t, v) pairs key 16t + 4(l/16) +
// v for A and B alike, which the B operands read as 4 consecutive floats of a
// transposed LDS copy.
//
// dtau uses the identity sum dS o (Q K^T) = sum_q Q[q] . (dS K)[q]: the
// product dS K is the one dQ needs anyway, so the reference's recomputed QK^T
// is not needed; the partial sums are f64 (the terms cancel to about 1% of
// their size).  dtau and drel are reduced without atomics: each workgroup
// writes its (image, head) partial -- drel through an inverse index (for
// every bias slot, the positions that map to it, in ascending order) -- and a
// second kernel adds the partials over images in image order.
#include "rnn_internal.h"

#include <algorithm>
#include <cstring>
#include <mutex>

namespace {

constexpr int MAXT = 64;   // tq, tk limit of the workgroup kernels
constexpr int MAXDH = 64;  // head-dim limit
constexpr int TS = 68;     // LDS row stride of the [64]-wide transposed tiles
constexpr int LT = 4096;   // u32 entries of the lane-order relidx table

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct AttnArgs {
    const float *q, *kv, *tau, *rel, *p, *dout;
    float *pout, *o, *dq, *dkv;
    double *dtau_part;          // [n][h]
    float *drel_part;           // [n][h][nrel]
    const uint32_t *rowptr;     // [nrel+1] inverse index (drel gather)
    const uint32_t *pos;        // [tq*tk] LDS offsets key*TS + q in the dS^T tile, by slot
    const uint4 *lidx;          // [4 w][4 t][64 lanes] relidx of (query, keys) in lane order
    long long qstride, qoff, kvstride, koff, voff;
    int n, h, dh, tq, tk, nrel, mask;
    const u32x4 *blob;  // the drel index blob: rowptr u32 [nrel+1], positions u16 [tq*tk]
    int blob_chunks;    // its 16-byte chunks, 0: gather through rowptr / pos in HBM
};

__device__ __forceinline__ f32x4 mfma16(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// v from the lane a DPP pattern names (both 32-bit halves moved).
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_mov_dpp((int)b, CTRL, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_mov_dpp((int)(b >> 32), CTRL, 0xf, 0xf, false);
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}
// Sum over the 64 lanes, every lane receiving it (a fixed tree: quads by
// DPP xor 1 and 2, rows of 8 and 16 by DPP mirrors, then xor 16 and 32).
__device__ __forceinline__ double wave_sum_d(double v) {
    v += dpp_d<0xB1>(v);   // quad_perm [1, 0, 3, 2]
    v += dpp_d<0x4E>(v);   // quad_perm [2, 3, 0, 1]
    v += dpp_d<0x141>(v);  // row_half_mirror
    v += dpp_d<0x140>(v);  // row_mirror
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

__device__ __forceinline__ float keep(float v, bool c) {
    return __uint_as_float(__float_as_uint(v) & (c ? 0xffffffffu : 0u));
}

// Four consecutive floats of row `row` (clamped into [0, nrows)) at column
// c0: one float4 load when VEC, else four loads from columns clamped below
// dh.  Nothing is masked here -- an operation on a loaded value waits for the
// load, and a branch around one splits the loads into blocks waited on in
// turn -- so callers zero what lies past (nrows, dh) with mask4 where they
// use the values.
template <bool VEC>
__device__ __forceinline__ float4 load4(const float *base, long long stride, int row, int nrows,
                                        int c0, int dh) {
    const float *p = base + (long long)min(row, nrows - 1) * stride;
    if constexpr (VEC) return *reinterpret_cast<const float4 *>(p + c0);
    float4 r;
    r.x = p[min(c0, dh - 1)];
    r.y = p[min(c0 + 1, dh - 1)];
    r.z = p[min(c0 + 2, dh - 1)];
    r.w = p[min(c0 + 3, dh - 1)];
    return r;
}
// v with every column past dh, or all of it when !row_ok, set to 0.
__device__ __forceinline__ float4 mask4(float4 v, bool row_ok, int c0, int dh) {
    return make_float4(keep(v.x, row_ok && c0 < dh), keep(v.y, row_ok && c0 + 1 < dh),
                       keep(v.z, row_ok && c0 + 2 < dh), keep(v.w, row_ok && c0 + 3 < dh));
}

// Rows [0, 64) x columns [0, DHP) of a strided [rows][dh] matrix, staged
// into LDS by the 256 threads of a workgroup in two halves: load() issues the
// thread's DHP/16 float4 loads together, store() zeroes what lies past
// (nrows, dh) and puts them in LDS transposed (dst[c][r], stride TS) or as
// rows (dst[r][c], stride DHP + 4).  Several tiles' loads are issued before
// any store, so their latencies overlap.
template <int DHP>
struct Tile {
    static constexpr int G = DHP / 4, CPT = 64 * G / 256;  // float4 chunks per thread
    float4 v[CPT];
    template <bool VEC>
    __device__ __forceinline__ void load(const float *src, long long stride, int nrows, int dh,
                                         int tid) {
#pragma unroll
        for (int j = 0; j < CPT; j++) {
            const int i = tid + 256 * j, r = i / G, c = (i % G) * 4;
            v[j] = load4<VEC>(src, stride, r, nrows, c, dh);
        }
    }
    template <bool TRANS>
    __device__ __forceinline__ void store(float *dst, int nrows, int dh, int tid) const {
#pragma unroll
        for (int j = 0; j < CPT; j++) {
            const int i = tid + 256 * j, r = i / G, c = (i % G) * 4;
            const float4 x = mask4(v[j], r < nrows, c, dh);
            if constexpr (TRANS) {
                dst[(c + 0) * TS + r] = x.x;
                dst[(c + 1) * TS + r] = x.y;
                dst[(c + 2) * TS + r] = x.z;
                dst[(c + 3) * TS + r] = x.w;
            } else {
                *reinterpret_cast<float4 *>(dst + r * (DHP + 4) + c) = x;
            }
        }
    }
};

__device__ __forceinline__ float4 lds4(const float *p) { return *reinterpret_cast<const float4 *>(p); }

// Core::forward (attn.rs:148-223) for one (image, head): DHP (16, 32, 64) is
// dh padded, NT = ceil(tk / 16) key tiles, one wave per 16 queries.
//   * K rows and V^T staged in LDS, the head's bias slots too; each lane's Q
//     slice (query 16w + l%16, head dims [g DHP/4, (g+1) DHP/4), g = l/16)
//     and its 4 NT relidx entries straight from HBM; V is loaded last and
//     stored to LDS after the softmax, so its latency overlaps the scores;
//   * S^T = K Q^T, x = tau*S + rel[relidx], the diagonal -inf when masked,
//     -inf past tk; softmax per query: max, exp(x - max) (-inf -> 0), times
//     1/sum (attn.rs:199-210);
//   * P rows to HBM (4 consecutive keys per lane and tile), O = P V.
template <int DHP, int NT, bool VEC>
__global__ __launch_bounds__(256) void attn_fwd_kernel(AttnArgs g) {
    constexpr int KSL = DHP / 4;  // head dims per lane slice
    extern __shared__ float smem[];
    float *Kl = smem;                    // [64][DHP + 4]
    float *Vt = Kl + 64 * (DHP + 4);     // [DHP][TS]
    float *rels = Vt + DHP * TS;         // [nrel]
    const int tid = threadIdx.x, lane = tid & 63, w = wave_index(), nth = blockDim.x;
    const int l16 = lane & 15, grp = lane >> 4;
    const int img = blockIdx.x / g.h, hd = blockIdx.x % g.h;
    const int tq = g.tq, tk = g.tk, dh = g.dh;
    const float *qb = g.q + (long long)img * tq * g.qstride + g.qoff + (long long)hd * dh;
    const float *kb = g.kv + (long long)img * tk * g.kvstride + g.koff + (long long)hd * dh;
    const float *vb = g.kv + (long long)img * tk * g.kvstride + g.voff + (long long)hd * dh;
    const int qi = 16 * w + l16;
    const float tau = g.tau[hd];  // (issued before the barrier, not waited for at it)

    // this lane's operands first (the load counter is in order), then the
    // staged tiles
    float4 qraw[KSL / 4];
#pragma unroll
    for (int i = 0; i < KSL; i += 4) qraw[i / 4] = load4<VEC>(qb, g.qstride, qi, tq, grp * KSL + i, dh);
    uint4 ri[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) ri[t] = g.lidx[(w * 4 + t) * 64 + lane];
    Tile<DHP> kt, vt;
    kt.template load<VEC>(kb, g.kvstride, tk, dh, tid);
    const float *relh = g.rel + (long long)hd * g.nrel;
    const float rel0 = relh[min(tid, g.nrel - 1)];
    // V last: only O = P V needs it, so its latency overlaps the scores
    vt.template load<VEC>(vb, g.kvstride, tk, dh, tid);
    kt.template store<false>(Kl, tk, dh, tid);
    if (tid < g.nrel) rels[tid] = rel0;
    for (int e = tid + nth; e < g.nrel; e += nth) rels[e] = relh[e];
    __syncthreads();

    float qs[KSL];
#pragma unroll
    for (int i = 0; i < KSL; i += 4) {
        const float4 t4 = mask4(qraw[i / 4], qi < tq, grp * KSL + i, dh);
        qs[i] = t4.x;
        qs[i + 1] = t4.y;
        qs[i + 2] = t4.z;
        qs[i + 3] = t4.w;
    }

    f32x4 st[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        st[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        const float *kr = Kl + (16 * t + l16) * (DHP + 4) + grp * KSL;
#pragma unroll
        for (int s = 0; s < KSL; s += 4) {
            const float4 a = lds4(kr + s);
            st[t] = mfma16(a.x, qs[s], st[t]);
            st[t] = mfma16(a.y, qs[s + 1], st[t]);
            st[t] = mfma16(a.z, qs[s + 2], st[t]);
            st[t] = mfma16(a.w, qs[s + 3], st[t]);
        }
    }
    float x[NT][4];
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const uint32_t idx[4] = {ri[t].x, ri[t].y, ri[t].z, ri[t].w};
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int kj = 16 * t + 4 * grp + v;
            const bool live = kj < tk && !(g.mask && kj == qi);
            const float xv = tau * st[t][v] + rels[idx[v]];
            x[t][v] = __uint_as_float(live ? __float_as_uint(xv) : 0xff800000u);  // -inf
            mx = fmaxf(mx, x[t][v]);
        }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    float sum = 0.f;
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const float e = x[t][v] == -INFINITY ? 0.f : __expf(x[t][v] - mx);
            x[t][v] = e;
            sum += e;
        }
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    const float inv = 1.0f / sum;
    const bool qlive = qi < tq;
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int v = 0; v < 4; v++) x[t][v] = qlive ? x[t][v] * inv : 0.f;

    if (qlive) {
        float *pr = g.pout + (((long long)img * g.h + hd) * tq + qi) * tk;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const int k0 = 16 * t + 4 * grp;
            if constexpr (VEC) {
                if (k0 < tk)
                    *reinterpret_cast<float4 *>(pr + k0) =
                        make_float4(x[t][0], x[t][1], x[t][2], x[t][3]);
            } else {
#pragma unroll
                for (int v = 0; v < 4; v++)
                    if (k0 + v < tk) pr[k0 + v] = x[t][v];
            }
        }
    }
    vt.template store<true>(Vt, tk, dh, tid);
    __syncthreads();
    // O = P V: A = P (this lane's registers), B = V^T rows from LDS
    const int c = g.h * dh;
    float *od = g.o + (long long)img * tq * c + (long long)hd * dh;
#pragma unroll
    for (int dt = 0; dt < DHP / 16; dt++) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        const float *vr = Vt + (16 * dt + l16) * TS + 4 * grp;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const float4 b = lds4(vr + 16 * t);
            acc = mfma16(x[t][0], b.x, acc);
            acc = mfma16(x[t][1], b.y, acc);
            acc = mfma16(x[t][2], b.z, acc);
            acc = mfma16(x[t][3], b.w, acc);
        }
        const int d = 16 * dt + l16;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int q = 16 * w + 4 * grp + v;
            if (q < tq && d < dh) od[(long long)q * c + d] = acc[v];
        }
    }
}

// Core::forward for tq <= 64 and tk = 16 NT keys above 64 (the rustvit's
// cross-attention over 256 memory tokens), one workgroup per (image, head),
// as attn_fwd_kernel with float4 accesses: K rows staged in LDS [tk][DHP+4];
// V loaded into registers while the scores run and stored transposed
// ([DHP][tk+4]) over the K rows once every wave is done with them; the
// relidx entries of the lane's query and keys read from the composed path's
// [tq][tk] table.  Two workgroups fit a CU.
template <int DHP, int NT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void
attn_fwd_long_kernel(AttnArgs g, const uint32_t *__restrict__ relidx) {
    constexpr int KSL = DHP / 4, TK = 16 * NT, KS = DHP + 4, VS = TK + 4;
    constexpr int AW = TK * KS > DHP * VS ? TK * KS : DHP * VS;
    constexpr int G = DHP / 4, CPT = TK * G / 256;  // float4 chunks of K (or V) per thread
    extern __shared__ float smem[];
    float *A = smem;          // K rows [TK][KS], then V^T [DHP][VS]
    float *rels = smem + AW;  // [nrel]
    const int tid = threadIdx.x, lane = tid & 63, w = wave_index();
    const int l16 = lane & 15, grp = lane >> 4;
    const int img = blockIdx.x / g.h, hd = blockIdx.x % g.h;
    const int tq = g.tq, dh = g.dh;
    const float *qb = g.q + (long long)img * tq * g.qstride + g.qoff + (long long)hd * dh;
    const float *kb = g.kv + (long long)img * TK * g.kvstride + g.koff + (long long)hd * dh;
    const float *vb = g.kv + (long long)img * TK * g.kvstride + g.voff + (long long)hd * dh;
    const int qi = 16 * w + l16;
    const float tau = g.tau[hd];
    float4 qraw[KSL / 4];
#pragma unroll
    for (int i = 0; i < KSL; i += 4)
        qraw[i / 4] = load4<true>(qb, g.qstride, qi, tq, grp * KSL + i, dh);
    const uint32_t *rq = relidx + (long long)min(qi, tq - 1) * TK + 4 * grp;
    uint4 ri[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) ri[t] = *reinterpret_cast<const uint4 *>(rq + 16 * t);
    float4 kv4[CPT];
#pragma unroll
    for (int j = 0; j < CPT; j++) {
        const int i = tid + 256 * j, r = i / G, c = (i % G) * 4;
        kv4[j] = load4<true>(kb, g.kvstride, r, TK, c, dh);
    }
    const float *relh = g.rel + (long long)hd * g.nrel;
    const float rel0 = relh[min(tid, g.nrel - 1)];
#pragma unroll
    for (int j = 0; j < CPT; j++) {
        const int i = tid + 256 * j, r = i / G, c = (i % G) * 4;
        *reinterpret_cast<float4 *>(A + r * KS + c) = kv4[j];
    }
    // V next: only O = P V needs it, so its latency overlaps the scores
#pragma unroll
    for (int j = 0; j < CPT; j++) {
        const int i = tid + 256 * j, r = i / G, c = (i % G) * 4;
        kv4[j] = load4<true>(vb, g.kvstride, r, TK, c, dh);
    }
    if (tid < g.nrel) rels[tid] = rel0;
    for (int e = tid + 256; e < g.nrel; e += 256) rels[e] = relh[e];
    __syncthreads();

    float qs[KSL];
#pragma unroll
    for (int i = 0; i < KSL; i += 4) {
        const float4 t4 = mask4(qraw[i / 4], qi < tq, grp * KSL + i, dh);
        qs[i] = t4.x;
        qs[i + 1] = t4.y;
        qs[i + 2] = t4.z;
        qs[i + 3] = t4.w;
    }
    f32x4 st[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        st[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        const float *kr = A + (16 * t + l16) * KS + grp * KSL;
#pragma unroll
        for (int s = 0; s < KSL; s += 4) {
            const float4 a = lds4(kr + s);
            st[t] = mfma16(a.x, qs[s], st[t]);
            st[t] = mfma16(a.y, qs[s + 1], st[t]);
            st[t] = mfma16(a.z, qs[s + 2], st[t]);
            st[t] = mfma16(a.w, qs[s + 3], st[t]);
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const uint32_t idx[4] = {ri[t].x, ri[t].y, ri[t].z, ri[t].w};
#pragma unroll
        for (int v = 0; v < 4; v++) {
            st[t][v] = tau * st[t][v] + rels[idx[v]];
            mx = fmaxf(mx, st[t][v]);
        }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    float sum = 0.f;
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const float e = __expf(st[t][v] - mx);
            st[t][v] = e;
            sum += e;
        }
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    const float inv = 1.0f / sum;
    const bool qlive = qi < tq;
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int v = 0; v < 4; v++) st[t][v] = qlive ? st[t][v] * inv : 0.f;
    if (qlive) {
        float *pr = g.pout + (((long long)img * g.h + hd) * tq + qi) * TK + 4 * grp;
#pragma unroll
        for (int t = 0; t < NT; t++)
            *reinterpret_cast<float4 *>(pr + 16 * t) =
                make_float4(st[t][0], st[t][1], st[t][2], st[t][3]);
    }
    __syncthreads();  // every wave is done with the K rows
#pragma unroll
    for (int j = 0; j < CPT; j++) {
        const int i = tid + 256 * j, r = i / G, c = (i % G) * 4;
        A[(c + 0) * VS + r] = kv4[j].x;
        A[(c + 1) * VS + r] = kv4[j].y;
        A[(c + 2) * VS + r] = kv4[j].z;
        A[(c + 3) * VS + r] = kv4[j].w;
    }
    __syncthreads();
    const int c = g.h * dh;
    float *od = g.o + (long long)img * tq * c + (long long)hd * dh;
#pragma unroll
    for (int dt = 0; dt < DHP / 16; dt++) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        const float *vr = A + (16 * dt + l16) * VS + 4 * grp;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const float4 b = lds4(vr + 16 * t);
            acc = mfma16(st[t][0], b.x, acc);
            acc = mfma16(st[t][1], b.y, acc);
            acc = mfma16(st[t][2], b.z, acc);
            acc = mfma16(st[t][3], b.w, acc);
        }
        const int d = 16 * dt + l16;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int q = 16 * w + 4 * grp + v;
            if (q < tq) od[(long long)q * c + d] = acc[v];
        }
    }
}

template <int DHP, int NT>
constexpr size_t bwd_long_words() {
    return (size_t)(16 * NT) * (DHP + 4) > (size_t)DHP * (16 * NT + 4)
               ? std::max<size_t>((size_t)(16 * NT) * (DHP + 4), (size_t)MAXT * 16 * NT)
               : std::max<size_t>((size_t)DHP * (16 * NT + 4), (size_t)MAXT * 16 * NT);
}

template <int DHP, int NT>
constexpr size_t fwd_long_words() {
    return (size_t)((16 * NT) * (DHP + 4) > DHP * (16 * NT + 4) ? (16 * NT) * (DHP + 4)
                                                               : DHP * (16 * NT + 4));
}

// dst[r][d] = old[v] + scale * val[v] (ACC) or scale * val[v] for the 4
// rows r = r0 + v (column d), where in range; old holds the values loaded
// earlier (old4).
__device__ __forceinline__ void old4(float (&old)[4], const float *dst, long long stride, int r0,
                                     int nrows, int d, int dh) {
    const int dc = min(d, dh - 1);
#pragma unroll
    for (int v = 0; v < 4; v++) old[v] = dst[(long long)min(r0 + v, nrows - 1) * stride + dc];
}
template <bool ACC>
__device__ __forceinline__ void store4(float *dst, long long stride, int r0, int nrows, int d,
                                       int dh, const float (&old)[4], const f32x4 &val,
                                       float scale) {
#pragma unroll
    for (int v = 0; v < 4; v++)
        if (r0 + v < nrows && d < dh)
            dst[(long long)(r0 + v) * stride + d] = ACC ? old[v] + scale * val[v] : scale * val[v];
}

// u32 chunks of 16 bytes of the drel index blob a thread carries in
// registers from the start of the backward to the LDS it is copied to.
constexpr int BLOB_CHUNKS = 6;

// Core::backward (attn.rs:226-343) for one (image, head), same limits.
// ACC: dQ, dK, dV accumulate (the reference's scatter_add); else they are
// overwritten, which is what SelfAttn::backward's zeroed buffers yield
// (attn.rs:418-438) without reading them.
//
// Loads in two groups, each thread's in issue order (the load counter
// retires in order, so a wait for the first group leaves the second in
// flight):
//   1. phase 1's operands: P (query 16w + l%16, keys 16t + 4(l/16) + v) into
//      registers; dO, V and K tiles, staged as dO^T, V rows, K^T;
//   2. Q (staged as Q^T after phase 1), the old dQ, dK, dV (ACC) and the
//      drel index blob (rowptr u32, positions u16), carried in registers
//      into the LDS of V and K^T once phase 1 is done with them.
// Phase 1 (wave w, queries [16w, 16w + 16)): dP^T = V dO^T, the row dot
// <dP, P>, dS = P o (dP - dot); P^T and dS^T to LDS; dSK = dS K.  After the
// second barrier: dQ = tau dSK and dtau += Q . dSK; phase 2 (wave w, keys
// [16w, 16w + 16)): dV = P^T dO and dK = tau dS^T Q over the query tiles;
// then the drel partial of the (image, head) through the inverse index.  QT
// / NT: query / key tiles; the waves cover max(QT, NT).
template <int DHP, int NT, bool VEC, bool ACC>
__global__ __launch_bounds__(256) void attn_bwd_kernel(AttnArgs g) {
    constexpr int KSL = DHP / 4, NDT = DHP / 16;
    extern __shared__ float smem[];
    float *Vr = smem;                // [64][DHP + 4]
    float *Kt = Vr + 64 * (DHP + 4); // [DHP][TS]
    float *Qt = Kt + DHP * TS;       // [DHP][TS]
    float *Ot = Qt + DHP * TS;       // [DHP][TS] dO^T
    float *Pt = Ot + DHP * TS;       // [64][TS] P^T  [key][q]
    float *St = Pt + 64 * TS;        // [64][TS] dS^T [key][q]
    double *dred = reinterpret_cast<double *>(St + 64 * TS);  // [4], 8-byte aligned
    const int tid = threadIdx.x, lane = tid & 63, w = wave_index(), nth = blockDim.x;
    const int l16 = lane & 15, grp = lane >> 4;
    const int img = blockIdx.x / g.h, hd = blockIdx.x % g.h;
    const int tq = g.tq, tk = g.tk, dh = g.dh, c = g.h * dh;
    const int QT = (tq + 15) >> 4;
    const float *qb = g.q + (long long)img * tq * g.qstride + g.qoff + (long long)hd * dh;
    const float *kb = g.kv + (long long)img * tk * g.kvstride + g.koff + (long long)hd * dh;
    const float *vb = g.kv + (long long)img * tk * g.kvstride + g.voff + (long long)hd * dh;
    const float *ob = g.dout + (long long)img * tq * c + (long long)hd * dh;
    float *dqi = g.dq + (long long)img * tq * g.qstride + g.qoff + (long long)hd * dh;
    float *dki = g.dkv + (long long)img * tk * g.kvstride + g.koff + (long long)hd * dh;
    float *dvi = g.dkv + (long long)img * tk * g.kvstride + g.voff + (long long)hd * dh;
    const int qi = 16 * w + l16, r0 = 16 * w + 4 * grp;
    const bool qwave = w < QT, qlive = qi < tq, kwave = 16 * w < tk;
    const float tau = g.tau[hd];

    // (every load unconditional, from clamped addresses: a branch would
    // split them into blocks the compiler waits between)
    float pv[NT][4];
    {
        const float *pr = g.p + (((long long)img * g.h + hd) * tq + min(qi, tq - 1)) * tk;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const int k0 = 16 * t + 4 * grp;
            if constexpr (VEC) {
                const float4 p4 = *reinterpret_cast<const float4 *>(pr + min(k0, tk - 4));
                pv[t][0] = p4.x;
                pv[t][1] = p4.y;
                pv[t][2] = p4.z;
                pv[t][3] = p4.w;
            } else {
#pragma unroll
                for (int v = 0; v < 4; v++) pv[t][v] = pr[min(k0 + v, tk - 1)];
            }
        }
    }
    Tile<DHP> ot, vt, kt, qt;
    ot.template load<VEC>(ob, c, tq, dh, tid);
    vt.template load<VEC>(vb, g.kvstride, tk, dh, tid);
    kt.template load<VEC>(kb, g.kvstride, tk, dh, tid);
    qt.template load<VEC>(qb, g.qstride, tq, dh, tid);
    float oq[NDT][4], ok[NDT][4], ov[NDT][4];
    if constexpr (ACC) {
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            old4(oq[dt], dqi, g.qstride, r0, tq, 16 * dt + l16, dh);
            old4(ok[dt], dki, g.kvstride, r0, tk, 16 * dt + l16, dh);
            old4(ov[dt], dvi, g.kvstride, r0, tk, 16 * dt + l16, dh);
        }
    }
    // (a native vector type: a HIP uint4 array is copied through scratch)
    u32x4 blob[BLOB_CHUNKS];
    {
        const int last = max(g.blob_chunks, 1) - 1;  // the blob holds one chunk at least
#pragma unroll
        for (int j = 0; j < BLOB_CHUNKS; j++) blob[j] = g.blob[min(tid + j * nth, last)];
    }
    ot.template store<true>(Ot, tq, dh, tid);
    vt.template store<false>(Vr, tk, dh, tid);
    kt.template store<true>(Kt, tk, dh, tid);
    __syncthreads();

    f32x4 dsk[NDT];
    if (qwave) {
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int v = 0; v < 4; v++)
                pv[t][v] = keep(pv[t][v], qlive && 16 * t + 4 * grp + v < tk);
        // this lane's dO slice (query qi, head dims [grp KSL, (grp+1) KSL))
        float os[KSL];
#pragma unroll
        for (int s = 0; s < KSL; s++) os[s] = Ot[(grp * KSL + s) * TS + qi];
        // dP^T = V dO^T (attn.rs:272-278): the score-tile layout of P
        f32x4 dp[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) {
            dp[t] = f32x4{0.f, 0.f, 0.f, 0.f};
            const float *vr = Vr + (16 * t + l16) * (DHP + 4) + grp * KSL;
#pragma unroll
            for (int s = 0; s < KSL; s += 4) {
                const float4 a = lds4(vr + s);
                dp[t] = mfma16(a.x, os[s], dp[t]);
                dp[t] = mfma16(a.y, os[s + 1], dp[t]);
                dp[t] = mfma16(a.z, os[s + 2], dp[t]);
                dp[t] = mfma16(a.w, os[s + 3], dp[t]);
            }
        }
        // dS = P o (dP - <dP, P>) (attn.rs:280-290)
        float dot = 0.f;
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int v = 0; v < 4; v++) dot += dp[t][v] * pv[t][v];
        dot += __shfl_xor(dot, 16, 64);
        dot += __shfl_xor(dot, 32, 64);
        float ds[NT][4];
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                ds[t][v] = pv[t][v] * (dp[t][v] - dot);  // 0 where P is 0
                const int kj = 16 * t + 4 * grp + v;
                Pt[kj * TS + qi] = pv[t][v];
                St[kj * TS + qi] = ds[t][v];
            }
        // dSK = dS K (attn.rs:316-323, before the tau scaling)
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            dsk[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
            const float *kr = Kt + (16 * dt + l16) * TS + 4 * grp;
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const float4 b = lds4(kr + 16 * t);
                dsk[dt] = mfma16(ds[t][0], b.x, dsk[dt]);
                dsk[dt] = mfma16(ds[t][1], b.y, dsk[dt]);
                dsk[dt] = mfma16(ds[t][2], b.z, dsk[dt]);
                dsk[dt] = mfma16(ds[t][3], b.w, dsk[dt]);
            }
        }
    }
    // (waves past the query tiles write no P^T / dS^T columns: phase 2 reads
    // only the columns of the first QT tiles)
    qt.template store<true>(Qt, tq, dh, tid);
    __syncthreads();

    double tpart = 0.0;
    if (qwave) {
        // dQ = tau dSK (attn.rs:316-323); dtau += Q . dSK
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            const int d = 16 * dt + l16;
            const float4 q4 = lds4(Qt + d * TS + r0);
            tpart += (double)(dsk[dt][0] * q4.x) + (double)(dsk[dt][1] * q4.y) +
                     (double)(dsk[dt][2] * q4.z) + (double)(dsk[dt][3] * q4.w);
            store4<ACC>(dqi, g.qstride, r0, tq, d, dh, oq[dt], dsk[dt], tau);
        }
    }
    tpart = wave_sum_d(tpart);
    if (lane == 0) dred[w] = tpart;

    // V and K^T are dead: the drel index blob goes where they were
    uint32_t *lblob = reinterpret_cast<uint32_t *>(smem);
    if (g.blob_chunks) {
#pragma unroll
        for (int j = 0; j < BLOB_CHUNKS; j++) {
            const int ch = tid + j * nth;
            if (ch < g.blob_chunks) reinterpret_cast<u32x4 *>(lblob)[ch] = blob[j];
        }
    }
    // phase 2: keys [16w, 16w + 16); k runs over queries q = 16ta + 4grp + v
    // (per query tile: P^T and dS^T read once, 2 NDT accumulators)
    if (kwave) {
        const int kr0 = 16 * w + l16;
        f32x4 av[NDT], ak[NDT];
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            av[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
            ak[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int ta = 0; ta < 4; ta++) {
            if (ta >= QT) break;
            const int q0 = 16 * ta + 4 * grp;
            const float4 pa = lds4(Pt + kr0 * TS + q0);
            const float4 sa = lds4(St + kr0 * TS + q0);
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
                const int d = 16 * dt + l16;
                const float4 ob4 = lds4(Ot + d * TS + q0);
                const float4 qb4 = lds4(Qt + d * TS + q0);
                av[dt] = mfma16(pa.x, ob4.x, av[dt]);
                ak[dt] = mfma16(sa.x, qb4.x, ak[dt]);
                av[dt] = mfma16(pa.y, ob4.y, av[dt]);
                ak[dt] = mfma16(sa.y, qb4.y, ak[dt]);
                av[dt] = mfma16(pa.z, ob4.z, av[dt]);
                ak[dt] = mfma16(sa.z, qb4.z, ak[dt]);
                av[dt] = mfma16(pa.w, ob4.w, av[dt]);
                ak[dt] = mfma16(sa.w, qb4.w, ak[dt]);
            }
        }
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            const int d = 16 * dt + l16;
            store4<ACC>(dvi, g.kvstride, r0, tk, d, dh, ov[dt], av[dt], 1.0f);
            store4<ACC>(dki, g.kvstride, r0, tk, d, dh, ok[dt], ak[dt], tau);
        }
    }
    __syncthreads();  // the blob in LDS, the dtau shares in dred
    // drel partial: gather by inverse index in ascending position (attn.rs:309-315)
    float *drp = g.drel_part + ((long long)img * g.h + hd) * g.nrel;
    if (g.blob_chunks) {
        const uint16_t *lpos = reinterpret_cast<const uint16_t *>(lblob + g.nrel + 1);
        for (int r = tid; r < g.nrel; r += nth) {
            float sacc = 0.f;
            const uint32_t e0 = lblob[r], e1 = lblob[r + 1];
            // 8 positions, then 8 values, read ahead of the in-order adds
            for (uint32_t e = e0; e < e1; e += 8) {
                uint32_t off[8];
                float val[8];
#pragma unroll
                for (int u = 0; u < 8; u++) off[u] = lpos[min(e + u, e1 - 1)];
#pragma unroll
                for (int u = 0; u < 8; u++) val[u] = St[off[u]];
#pragma unroll
                for (int u = 0; u < 8; u++)
                    if (e + u < e1) sacc += val[u];
            }
            drp[r] = sacc;
        }
    } else {
        for (int r = tid; r < g.nrel; r += nth) {
            float sacc = 0.f;
            const uint32_t e0 = g.rowptr[r], e1 = g.rowptr[r + 1];
            for (uint32_t e = e0; e < e1; e += 8) {
                uint32_t off[8];
#pragma unroll
                for (int u = 0; u < 8; u++) off[u] = e + u < e1 ? g.pos[e + u] : 0u;
#pragma unroll
                for (int u = 0; u < 8; u++)
                    if (e + u < e1) sacc += St[off[u]];
            }
            drp[r] = sacc;
        }
    }
    if (tid == 0) {
        double s = 0.0;
        for (int i = 0; i < (int)(blockDim.x >> 6); i++) s += dred[i];
        g.dtau_part[(long long)img * g.h + hd] = s;
    }
}

// Core::backward's query half for tq <= 64 and tk = 16 NT keys above 64
// (the rustvit's cross-attention), one workgroup per (image, head), wave w
// on queries [16w, 16w + 16) as in attn_bwd_kernel's phase 1: dP^T = V dO^T
// with V's rows in LDS; dS = P o (dP - <dP, P>), with tau dS written to s2
// ([tq][tk] per (image, head)) for the key half (attn_bwd_long_k_kernel);
// then dSK = dS K with K^T in LDS over V's rows (K held in registers
// meanwhile); dQ = tau dSK, set or added (ACC); the (image, head) shares of
// dtau (sum Q . dSK, f64) and of drel (dS staged in LDS [tq][tk] over K^T and
// gathered through the inverse index, each slot's positions in ascending
// order) into g.dtau_part / g.drel_part.
template <int DHP, int NT, bool ACC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void
attn_bwd_long_q_kernel(AttnArgs g, float *__restrict__ s2) {
    constexpr int KSL = DHP / 4, NDT = DHP / 16, TK = 16 * NT, KS = DHP + 4, VS = TK + 4;
    constexpr int AW0 = TK * KS > DHP * VS ? TK * KS : DHP * VS;
    constexpr int AW = AW0 > MAXT * TK ? AW0 : MAXT * TK;  // also dS [64][tk]
    constexpr int G = DHP / 4, CPT = TK * G / 256;
    static_assert(AW % 2 == 0, "8-byte aligned reduction slots");
    extern __shared__ float smem[];
    float *A = smem;                                         // V rows, then K^T
    double *dred = reinterpret_cast<double *>(smem + AW);    // [4]
    const int tid = threadIdx.x, lane = tid & 63, w = wave_index();
    const int l16 = lane & 15, grp = lane >> 4;
    const int img = blockIdx.x / g.h, hd = blockIdx.x % g.h;
    const int tq = g.tq, dh = g.dh, c = g.h * dh;
    const float *qb = g.q + (long long)img * tq * g.qstride + g.qoff + (long long)hd * dh;
    const float *kb = g.kv + (long long)img * TK * g.kvstride + g.koff + (long long)hd * dh;
    const float *vb = g.kv + (long long)img * TK * g.kvstride + g.voff + (long long)hd * dh;
    const float *ob = g.dout + (long long)img * tq * c + (long long)hd * dh;
    float *dqi = g.dq + (long long)img * tq * g.qstride + g.qoff + (long long)hd * dh;
    const int qi = 16 * w + l16, r0 = 16 * w + 4 * grp;
    const bool qlive = qi < tq;
    const float tau = g.tau[hd];
    const long long prow = ((long long)img * g.h + hd) * tq;

    float4 pv4[NT];
    {
        const float *pr = g.p + (prow + min(qi, tq - 1)) * TK + 4 * grp;
#pragma unroll
        for (int t = 0; t < NT; t++) pv4[t] = *reinterpret_cast<const float4 *>(pr + 16 * t);
    }
    float4 oraw[KSL / 4];
#pragma unroll
    for (int i = 0; i < KSL; i += 4) oraw[i / 4] = load4<true>(ob, c, qi, tq, grp * KSL + i, dh);
    float4 kv4[CPT];
#pragma unroll
    for (int j = 0; j < CPT; j++) {
        const int i = tid + 256 * j, r = i / G, cc = (i % G) * 4;
        kv4[j] = load4<true>(vb, g.kvstride, r, TK, cc, dh);
    }
#pragma unroll
    for (int j = 0; j < CPT; j++) {
        const int i = tid + 256 * j, r = i / G, cc = (i % G) * 4;
        *reinterpret_cast<float4 *>(A + r * KS + cc) = kv4[j];
    }
    __syncthreads();

    float os[KSL];
#pragma unroll
    for (int i = 0; i < KSL; i += 4) {
        const float4 t4 = mask4(oraw[i / 4], qlive, grp * KSL + i, dh);
        os[i] = t4.x;
        os[i + 1] = t4.y;
        os[i + 2] = t4.z;
        os[i + 3] = t4.w;
    }
    // dP^T = V dO^T (attn.rs:272-278): the score-tile layout of P
    f32x4 dp[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        dp[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        const float *vr = A + (16 * t + l16) * KS + grp * KSL;
#pragma unroll
        for (int s = 0; s < KSL; s += 4) {
            const float4 a = lds4(vr + s);
            dp[t] = mfma16(a.x, os[s], dp[t]);
            dp[t] = mfma16(a.y, os[s + 1], dp[t]);
            dp[t] = mfma16(a.z, os[s + 2], dp[t]);
            dp[t] = mfma16(a.w, os[s + 3], dp[t]);
        }
    }
    // K next, once dO's slice is dead (the registers are scarce): only dS K
    // needs it, so its latency overlaps dS and its stores
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < CPT; j++) {
        const int i = tid + 256 * j, r = i / G, cc = (i % G) * 4;
        kv4[j] = load4<true>(kb, g.kvstride, r, TK, cc, dh);
    }
    // dS = P o (dP - <dP, P>) (attn.rs:280-290)
    float pv[NT][4];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        pv[t][0] = keep(pv4[t].x, qlive);
        pv[t][1] = keep(pv4[t].y, qlive);
        pv[t][2] = keep(pv4[t].z, qlive);
        pv[t][3] = keep(pv4[t].w, qlive);
    }
    float dot = 0.f;
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int v = 0; v < 4; v++) dot += dp[t][v] * pv[t][v];
    dot += __shfl_xor(dot, 16, 64);
    dot += __shfl_xor(dot, 32, 64);
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int v = 0; v < 4; v++) dp[t][v] = pv[t][v] * (dp[t][v] - dot);  // dS; 0 where P is 0
    if (qlive) {
        float *d2 = s2 + (prow + qi) * TK + 4 * grp;
#pragma unroll
        for (int t = 0; t < NT; t++)
            *reinterpret_cast<float4 *>(d2 + 16 * t) =
                make_float4(dp[t][0] * tau, dp[t][1] * tau, dp[t][2] * tau, dp[t][3] * tau);
    }
    __syncthreads();  // every wave is done with V's rows
#pragma unroll
    for (int j = 0; j < CPT; j++) {
        const int i = tid + 256 * j, r = i / G, cc = (i % G) * 4;
        A[(cc + 0) * VS + r] = kv4[j].x;
        A[(cc + 1) * VS + r] = kv4[j].y;
        A[(cc + 2) * VS + r] = kv4[j].z;
        A[(cc + 3) * VS + r] = kv4[j].w;
    }
    // Q (for dtau) and the old dQ: loaded late, the registers are scarce
    float oq[NDT][4], qv[NDT][4];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) {
        if constexpr (ACC) old4(oq[dt], dqi, g.qstride, r0, tq, 16 * dt + l16, dh);
#pragma unroll
        for (int v = 0; v < 4; v++)
            qv[dt][v] = qb[(long long)min(r0 + v, tq - 1) * g.qstride + 16 * dt + l16];
    }
    __syncthreads();
    // dSK = dS K (attn.rs:316-323, before the tau scaling); dQ = tau dSK;
    // dtau += Q . dSK
    double tpart = 0.0;
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) {
        f32x4 dsk = {0.f, 0.f, 0.f, 0.f};
        const float *kr = A + (16 * dt + l16) * VS + 4 * grp;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const float4 b = lds4(kr + 16 * t);
            dsk = mfma16(dp[t][0], b.x, dsk);
            dsk = mfma16(dp[t][1], b.y, dsk);
            dsk = mfma16(dp[t][2], b.z, dsk);
            dsk = mfma16(dp[t][3], b.w, dsk);
        }
        tpart += (double)(dsk[0] * qv[dt][0]) + (double)(dsk[1] * qv[dt][1]) +
                 (double)(dsk[2] * qv[dt][2]) + (double)(dsk[3] * qv[dt][3]);
        store4<ACC>(dqi, g.qstride, r0, tq, 16 * dt + l16, dh, oq[dt], dsk, tau);
    }
    tpart = wave_sum_d(tpart);
    if (lane == 0) dred[w] = tpart;
    __syncthreads();  // every wave is done with K^T; the dtau shares are in dred
    if (tid == 0)
        g.dtau_part[(long long)img * g.h + hd] = ((dred[0] + dred[1]) + dred[2]) + dred[3];
    // dS in LDS as [tq][tk] (position q*tk + k, as the inverse index numbers
    // them), then drel's share of every bias slot (attn.rs:309-315)
    if (qlive) {
#pragma unroll
        for (int t = 0; t < NT; t++)
            *reinterpret_cast<float4 *>(A + qi * TK + 16 * t + 4 * grp) =
                make_float4(dp[t][0], dp[t][1], dp[t][2], dp[t][3]);
    }
    __syncthreads();
    float *drp = g.drel_part + ((long long)img * g.h + hd) * g.nrel;
    for (int r = tid; r < g.nrel; r += 256) {
        const uint32_t e0 = g.rowptr[r], e1 = g.rowptr[r + 1];
        float sacc = 0.f;
        for (uint32_t e = e0; e < e1; e += 8) {
            uint32_t off[8];
#pragma unroll
            for (int u = 0; u < 8; u++) off[u] = g.pos[min(e + u, e1 - 1)];
            float val[8];
#pragma unroll
            for (int u = 0; u < 8; u++) val[u] = A[off[u]];
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (e + u < e1) sacc += val[u];
        }
        drp[r] = sacc;
    }
}

// Core::backward's key half for the same shapes: dV = P^T dO and
// dK = (tau dS)^T Q over the (image, head)'s queries, set or added (ACC);
// wave w on keys [TK/4 w, TK/4 (w + 1)), 16 at a time, as attn_bwd_kernel's
// phase 2: dO^T and Q^T staged in LDS, the A operands (P and tau dS for the
// lane's key and four queries) read from HBM.
template <int DHP, int NT, bool ACC>
__global__ __launch_bounds__(256) void attn_bwd_long_k_kernel(AttnArgs g,
                                                              const float *__restrict__ s2) {
    constexpr int NDT = DHP / 16, TK = 16 * NT, KPW = NT / 4;  // key tiles a wave
    extern __shared__ float smem[];
    float *Qt = smem;            // [DHP][TS]
    float *Ot = Qt + DHP * TS;   // [DHP][TS] dO^T
    const int tid = threadIdx.x, lane = tid & 63, w = wave_index();
    const int l16 = lane & 15, grp = lane >> 4;
    const int img = blockIdx.x / g.h, hd = blockIdx.x % g.h;
    const int tq = g.tq, dh = g.dh, c = g.h * dh;
    const int QT = (tq + 15) >> 4;
    const float *qb = g.q + (long long)img * tq * g.qstride + g.qoff + (long long)hd * dh;
    const float *ob = g.dout + (long long)img * tq * c + (long long)hd * dh;
    float *dki = g.dkv + (long long)img * TK * g.kvstride + g.koff + (long long)hd * dh;
    float *dvi = g.dkv + (long long)img * TK * g.kvstride + g.voff + (long long)hd * dh;
    const long long prow = ((long long)img * g.h + hd) * tq;
    const float *pb = g.p + prow * TK, *sb = s2 + prow * TK;
    Tile<DHP> ot, qt;
    ot.template load<true>(ob, c, tq, dh, tid);
    qt.template load<true>(qb, g.qstride, tq, dh, tid);
    ot.template store<true>(Ot, tq, dh, tid);
    qt.template store<true>(Qt, tq, dh, tid);
    __syncthreads();
#pragma unroll 1
    for (int kt = 0; kt < KPW; kt++) {
        const int k0 = 16 * (KPW * w + kt), kr = k0 + l16, r0 = k0 + 4 * grp;
        float ov[NDT][4], ok[NDT][4];
        if constexpr (ACC) {
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
                old4(ov[dt], dvi, g.kvstride, r0, TK, 16 * dt + l16, dh);
                old4(ok[dt], dki, g.kvstride, r0, TK, 16 * dt + l16, dh);
            }
        }
        // the lane's key, queries 16 ta + 4 grp + v (rows past tq read row
        // tq - 1 and are zeroed)
        float pa[4][4], sa[4][4];
#pragma unroll
        for (int ta = 0; ta < 4; ta++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int q = 16 * ta + 4 * grp + v;
                const long long o = (long long)min(q, tq - 1) * TK + kr;
                pa[ta][v] = pb[o];
                sa[ta][v] = sb[o];
            }
        f32x4 av[NDT], ak[NDT];
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            av[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
            ak[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int ta = 0; ta < 4; ta++) {
            if (ta >= QT) break;
            const int q0 = 16 * ta + 4 * grp;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                pa[ta][v] = keep(pa[ta][v], q0 + v < tq);
                sa[ta][v] = keep(sa[ta][v], q0 + v < tq);
            }
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
                const int d = 16 * dt + l16;
                const float4 ob4 = lds4(Ot + d * TS + q0);
                const float4 qb4 = lds4(Qt + d * TS + q0);
                av[dt] = mfma16(pa[ta][0], ob4.x, av[dt]);
                ak[dt] = mfma16(sa[ta][0], qb4.x, ak[dt]);
                av[dt] = mfma16(pa[ta][1], ob4.y, av[dt]);
                ak[dt] = mfma16(sa[ta][1], qb4.y, ak[dt]);
                av[dt] = mfma16(pa[ta][2], ob4.z, av[dt]);
                ak[dt] = mfma16(sa[ta][2], qb4.z, ak[dt]);
                av[dt] = mfma16(pa[ta][3], ob4.w, av[dt]);
                ak[dt] = mfma16(sa[ta][3], qb4.w, ak[dt]);
            }
        }
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            const int d = 16 * dt + l16;
            store4<ACC>(dvi, g.kvstride, r0, TK, d, dh, ov[dt], av[dt], 1.0f);
            store4<ACC>(dki, g.kvstride, r0, TK, d, dh, ok[dt], ak[dt], 1.0f);
        }
    }
}

// dtau[h] += sum_img part[img][h]; drel[h*nrel + r] += sum_img part[img][h][r]
// (image order, attn.rs:333-342).  A block takes 32 elements; thread (j, e)
// sums images [j*G, j*G + G) of element e with the loads issued ahead of the
// in-order adds, then the 8 partials are added in j order (fixed order:
// bit-reproducible).  The dtau partials are f64 and summed in f64.
__global__ __launch_bounds__(256) void attn_reduce_kernel(const double *dtau_part,
                                                          const float *drel_part, int n, int h,
                                                          int nrel, float *dtau, float *drel) {
    rnn_attn_reduce_block(dtau_part, drel_part, n, h, nrel, dtau, drel, blockIdx.x);
}

// Columns [off, off + width) of `rows` rows of stride `stride` set to 0:
// one wave per row (4 per block).
__global__ __launch_bounds__(256) void attn_zero_cols_kernel(float *x, long long rows,
                                                             long long stride, long long off,
                                                             int width) {
    const long long r = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    float *row = x + r * stride + off;
    for (int j = threadIdx.x & 63; j < width; j += 64) row[j] = 0.f;
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

// tq or tk above 64: the composed path (batched GEMMs + row kernels).

// ---------------------------------------------------------------------------
// The composed path for tq or tk above 64 (the rustvit's cross-attention:
// tq 64, tk 256, dh 64, nrel 900).  The reference's own structure: per head, a
// batched GEMM over the images (strided Q/K/V through leading dimensions) for
// S = QK^T, a row kernel for the biased, masked softmax (P kept, as the
// backward reads it), a batched GEMM for O = PV; the backward likewise.

// Softmax of the rows of P in place (attn.rs:190-212): x = tau S + rel[idx],
// the diagonal -inf when masked; max, exp(x - max) (-inf -> 0), sum, times
// 1/sum.  One wave per row (image, head, query).
// NV > 0: the row (tk <= 64 NV) held in registers, read and written once.
template <int NV>
__global__ __launch_bounds__(256) void attn_softmax_rows_kernel(
    float *p, const float *__restrict__ tau, const float *__restrict__ rel,
    const uint32_t *__restrict__ relidx, long long rows, int h, int tq, int tk, int nrel,
    int mask) {
    if constexpr (NV > 0) {
        const long long r = (long long)blockIdx.x * 4 + wave_index();
        if (r >= rows) return;
        const int lane = threadIdx.x & 63;
        const int qi = (int)(r % tq), hd = (int)((r / tq) % h);
        float *row = p + r * tk;
        const float t = tau[hd];
        const float *rh = rel + (long long)hd * nrel;
        const uint32_t *ix = relidx + (long long)qi * tk;
        float raw[NV], xv[NV];
        uint32_t id[NV];
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int k = min(lane + 64 * i, tk - 1);
            raw[i] = row[k];
            id[i] = ix[k];
        }
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int k = lane + 64 * i;
            const float x = (k >= tk || (mask && k == qi)) ? -INFINITY : t * raw[i] + rh[id[i]];
            xv[i] = x;
            mx = fmaxf(mx, x);
        }
        for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const float e = xv[i] == -INFINITY ? 0.f : expf(xv[i] - mx);
            xv[i] = e;
            sum += e;
        }
        for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o, 64);
        const float inv = 1.0f / sum;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int k = lane + 64 * i;
            if (k < tk) row[k] = xv[i] * inv;
        }
        return;
    }
    const long long r = (long long)blockIdx.x * 4 + wave_index();
    if (r >= rows) return;
    const int lane = threadIdx.x & 63;
    const int qi = (int)(r % tq), hd = (int)((r / tq) % h);
    float *row = p + r * tk;
    const float t = tau[hd];
    const float *rh = rel + (long long)hd * nrel;
    const uint32_t *ix = relidx + (long long)qi * tk;
    float mx = -INFINITY;
    for (int k = lane; k < tk; k += 64) {
        const float x = (mask && k == qi) ? -INFINITY : t * row[k] + rh[ix[k]];
        row[k] = x;
        mx = fmaxf(mx, x);
    }
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    float sum = 0.f;
    for (int k = lane; k < tk; k += 64) {
        const float x = row[k];
        const float e = x == -INFINITY ? 0.f : expf(x - mx);
        row[k] = e;
        sum += e;
    }
    for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o, 64);
    const float inv = 1.0f / sum;
    for (int k = lane; k < tk; k += 64) row[k] *= inv;
}

// Backward rows (attn.rs:280-330): s1 holds dP, s2 the recomputed raw S.
// dS = P o (dP - <dP, P>) goes to s1 (for drel), tau dS to s2 (for dQ, dK);
// part[row] = sum dS o S_raw (the dtau share of the row, summed in f64: dtau
// is a sum whose terms cancel to about 1% of their size).
__global__ __launch_bounds__(256) void attn_dsoft_rows_kernel(
    const float *__restrict__ p, float *s1, float *s2, const float *__restrict__ tau,
    double *__restrict__ part, long long rows, int h, int tq, int tk) {
    const long long r = (long long)blockIdx.x * 4 + wave_index();
    if (r >= rows) return;
    const int lane = threadIdx.x & 63;
    const int hd = (int)((r / tq) % h);
    const float *pr = p + r * tk;
    float *dp = s1 + r * tk, *sr = s2 + r * tk;
    float dot = 0.f;
    for (int k = lane; k < tk; k += 64) dot += dp[k] * pr[k];
    for (int o = 32; o >= 1; o >>= 1) dot += __shfl_xor(dot, o, 64);
    const float t = tau[hd];
    double dt = 0.0;
    for (int k = lane; k < tk; k += 64) {
        const float ds = pr[k] * (dp[k] - dot);
        dt += (double)(ds * sr[k]);
        dp[k] = ds;
        sr[k] = ds * t;
    }
    dt = wave_sum_d(dt);
    if (lane == 0) part[r] = dt;
}

// dtau[hd] += sum over (image, query) rows of head hd of part (block hd;
// strided per thread, then a fixed tree).
__global__ __launch_bounds__(256) void attn_head_sum_kernel(const double *__restrict__ part,
                                                            long long n, int h, int tq,
                                                            float *dtau) {
    __shared__ double red[4];
    const int hd = blockIdx.x;
    const long long per = n * tq;
    double s = 0.0;
    for (long long i = threadIdx.x; i < per; i += 256) {
        const long long img = i / tq, q = i - img * tq;
        s += part[(img * h + hd) * tq + q];
    }
    s = wave_sum_d(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) dtau[hd] += (float)((red[0] + red[1]) + (red[2] + red[3]));
}

// drel partials: part[chunk][hd*nrel + slot] = sum over the images of the
// chunk (in order) and the positions of the slot (the inverse index,
// ascending) of dS.  One thread per (chunk, head, slot); 8 loads ahead.
__global__ __launch_bounds__(256) void attn_drel_part_kernel(
    const float *__restrict__ ds, const uint32_t *__restrict__ rowptr,
    const uint32_t *__restrict__ pos, long long n, long long ipc, int h, int nrel,
    long long cnt, float *__restrict__ part) {
    const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
    const long long per = (long long)h * nrel;
    if (e >= per) return;
    const int hd = (int)(e / nrel), slot = (int)(e - (long long)hd * nrel);
    const uint32_t p0 = rowptr[slot], p1 = rowptr[slot + 1];
    const long long i0 = (long long)blockIdx.y * ipc, i1 = min(n, i0 + ipc);
    float s = 0.f;
    for (long long img = i0; img < i1; img++) {
        const float *base = ds + (img * h + hd) * cnt;
        uint32_t i = p0;
        for (; i + 8 <= p1; i += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = base[pos[i + u]];
#pragma unroll
            for (int u = 0; u < 8; u++) s += v[u];
        }
        for (; i < p1; i++) s += base[pos[i]];
    }
    part[(long long)blockIdx.y * per + e] = s;
}

// drel[e] += sum over chunks of part[chunk][e], in chunk order (16 loads
// ahead of their adds).
__global__ __launch_bounds__(256) void attn_drel_sum_kernel(const float *__restrict__ part,
                                                            int nchunk, long long per,
                                                            float *drel) {
    const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
    if (e >= per) return;
    float s = 0.f;
    for (int k0 = 0; k0 < nchunk; k0 += 16) {
        float v[16];
#pragma unroll
        for (int u = 0; u < 16; u++) v[u] = part[(long long)min(k0 + u, nchunk - 1) * per + e];
#pragma unroll
        for (int u = 0; u < 16; u++)
            if (k0 + u < nchunk) s += v[u];
    }
    drel[e] += s;
}


// tq or tk above 64: the composed path (batched GEMMs + row kernels).
bool large_desc(const rnn_attn_desc *d) { return d->tq > MAXT || d->tk > MAXT; }

int check_desc(rnn_ctx *ctx, const rnn_attn_desc *d) {
    if (!d) return rnn_fail(ctx, RNN_E_NULL, "attn: desc is null");
    if (!d->relidx) return rnn_fail(ctx, RNN_E_NULL, "attn: relidx is null");
    if (!d->h || !d->dh || !d->tq || !d->tk || !d->nrel)
        return rnn_fail(ctx, RNN_E_INVALID, "attn: zero dimension");
    if (d->dh > MAXDH && !large_desc(d))
        return rnn_fail(ctx, RNN_E_UNSUPPORTED,
                        "attn: dh=%u beyond the workgroup kernels (64) at tq=%u tk=%u", d->dh,
                        d->tq, d->tk);
    if ((size_t)d->tq * d->tk > ((size_t)1 << 26) || d->tk > (1u << 20))
        return rnn_fail(ctx, RNN_E_UNSUPPORTED, "attn: tq=%u tk=%u too large", d->tq, d->tk);
    return RNN_OK;
}

// u32 offset of the lane-order table in a table's device block (16-byte
// aligned): after relidx, rowptr and pos; then the drel index blob (rowptr
// u32, positions u16) that the backward copies into LDS.
size_t lane_table_off(size_t cnt, size_t nrel) { return rnn_round_up(cnt + (nrel + 1) + cnt, 4); }
size_t blob_off(size_t cnt, size_t nrel) { return lane_table_off(cnt, nrel) + LT; }
size_t blob_bytes(size_t cnt, size_t nrel) { return rnn_round_up(4 * (nrel + 1) + 2 * cnt, 16); }

// The device copy of the relidx table of `d`: found by content among the
// tables this context has uploaded (the last one used first), else checked
// (every slot below nrel), completed on the host with its inverse index --
// for every bias slot the positions that map to it, ascending, as offsets
// into the backward's dS^T tile (key * TS + q) or, on the composed path, into
// the [tq][tk] score matrix -- and, for the workgroup kernels, the table in
// lane order, then uploaded once.  The copy runs on the context's stream from
// a pinned buffer kept with the table, so no call waits for the device and
// every table a step uses stays resident (a graph can replay them).
int rel_table(rnn_ctx *ctx, const rnn_attn_desc *d, const RnnRelTable **out) {
    const size_t cnt = (size_t)d->tq * d->tk;
    auto same = [&](const RnnRelTable &t) {
        return t.tq == d->tq && t.tk == d->tk && t.nrel == d->nrel &&
               std::memcmp(t.host.data(), d->relidx, cnt * 4) == 0;
    };
    auto &tabs = ctx->rel_tables;
    if (ctx->rel_last < tabs.size() && same(tabs[ctx->rel_last])) {
        *out = &tabs[ctx->rel_last];
        return RNN_OK;
    }
    for (size_t i = 0; i < tabs.size(); i++)
        if (same(tabs[i])) {
            ctx->rel_last = i;
            *out = &tabs[i];
            return RNN_OK;
        }
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    RNN_HIP(ctx, hipStreamIsCapturing(ctx->stream, &cs));
    if (cs != hipStreamCaptureStatusNone)
        return rnn_fail(ctx, RNN_E_INVALID,
                        "attn: a new relidx table during graph capture (call once before "
                        "capturing)");
    for (size_t i = 0; i < cnt; i++)
        if (d->relidx[i] >= d->nrel) return rnn_fail(ctx, RNN_E_INVALID, "attn: relidx >= nrel");
    const bool large = large_desc(d);
    const size_t lane_off = lane_table_off(cnt, d->nrel);
    const size_t need = large ? cnt + (d->nrel + 1) + cnt
                              : blob_off(cnt, d->nrel) + blob_bytes(cnt, d->nrel) / 4;
    RnnRelTable t;
    t.tq = d->tq;
    t.tk = d->tk;
    t.nrel = d->nrel;
    t.host.assign(d->relidx, d->relidx + cnt);
    RNN_HIP(ctx, hipHostMalloc((void **)&t.pinned, need * 4, hipHostMallocDefault));
    hipError_t e = hipMalloc((void **)&t.dev, need * 4);
    if (e != hipSuccess) {
        (void)hipHostFree(t.pinned);
        return rnn_fail(ctx, RNN_E_NOMEM, "attn: relidx table hipMalloc: %s", hipGetErrorString(e));
    }
    uint32_t *h = t.pinned;
    std::memset(h, 0, need * 4);
    std::memcpy(h, d->relidx, cnt * 4);
    uint32_t *rowptr = h + cnt, *pos = rowptr + d->nrel + 1;
    std::vector<uint32_t> count(d->nrel + 1, 0);
    for (size_t i = 0; i < cnt; i++) count[d->relidx[i] + 1]++;
    for (uint32_t r = 0; r < d->nrel; r++) count[r + 1] += count[r];
    for (uint32_t r = 0; r <= d->nrel; r++) rowptr[r] = count[r];
    for (size_t i = 0; i < cnt; i++) {
        const uint32_t q = (uint32_t)(i / d->tk), k = (uint32_t)(i % d->tk);
        pos[count[d->relidx[i]]++] = large ? (uint32_t)i : k * TS + q;
    }
    if (!large) {
        // entry ((w*4 + t)*64 + lane)*4 + v: query 16w + lane%16, key
        // 16t + 4(lane/16) + v, both clamped into the table (a valid slot)
        uint32_t *lt = h + lane_off;
        for (int w = 0; w < 4; w++)
            for (int tt = 0; tt < 4; tt++)
                for (int l = 0; l < 64; l++)
                    for (int v = 0; v < 4; v++) {
                        const int q = std::min(16 * w + (l & 15), (int)d->tq - 1);
                        const int k = std::min(16 * tt + 4 * (l >> 4) + v, (int)d->tk - 1);
                        lt[((w * 4 + tt) * 64 + l) * 4 + v] = d->relidx[(size_t)q * d->tk + k];
                    }
        // the blob: rowptr, then the positions as u16 (below 64 * TS)
        uint32_t *bl = h + blob_off(cnt, d->nrel);
        std::memcpy(bl, rowptr, (d->nrel + 1) * 4);
        uint16_t *p16 = reinterpret_cast<uint16_t *>(bl + d->nrel + 1);
        for (size_t i = 0; i < cnt; i++) p16[i] = (uint16_t)pos[i];
    }
    e = hipMemcpyAsync(t.dev, h, need * 4, hipMemcpyHostToDevice, ctx->stream);
    if (e != hipSuccess) {
        (void)hipFree(t.dev);
        (void)hipHostFree(t.pinned);
        return rnn_fail(ctx, RNN_E_HIP, "attn: relidx upload: %s", hipGetErrorString(e));
    }
    tabs.push_back(std::move(t));
    ctx->rel_last = tabs.size() - 1;
    *out = &tabs.back();
    return RNN_OK;
}

void fill_args(AttnArgs &g, const RnnRelTable &tab, const rnn_attn_desc *d, size_t n) {
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
    const size_t cnt = (size_t)d->tq * d->tk;
    g.rowptr = tab.dev + cnt;
    g.pos = tab.dev + cnt + d->nrel + 1;
    g.lidx = reinterpret_cast<const uint4 *>(tab.dev + lane_table_off(cnt, d->nrel));
    g.blob = reinterpret_cast<const u32x4 *>(tab.dev + blob_off(cnt, d->nrel));
}

int dhp_of(uint32_t dh) { return dh <= 16 ? 16 : dh <= 32 ? 32 : 64; }

inline bool al16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// float4 accesses need dh == DHP (no column padding) and 16-byte aligned row
// starts for every image and head.
int use_vec(const AttnArgs &g) {
    return g.dh == dhp_of(g.dh) && g.qstride % 4 == 0 && g.qoff % 4 == 0 && al16(g.q) &&
           g.kvstride % 4 == 0 && g.koff % 4 == 0 && g.voff % 4 == 0 && al16(g.kv) &&
           (g.dout == nullptr || al16(g.dout));
}

size_t fwd_lds(int dhp, size_t nrel) { return ((size_t)64 * (dhp + 4) + dhp * TS + nrel) * 4; }
size_t bwd_lds(int dhp) {
    return ((size_t)64 * (dhp + 4) + 3 * dhp * TS + 2 * 64 * TS) * 4 + 4 * sizeof(double);
}

template <int DHP, bool VEC>
const void *fwd_kernel_nt(int nt) {
    switch (nt) {
        case 1: return (const void *)attn_fwd_kernel<DHP, 1, VEC>;
        case 2: return (const void *)attn_fwd_kernel<DHP, 2, VEC>;
        case 3: return (const void *)attn_fwd_kernel<DHP, 3, VEC>;
        default: return (const void *)attn_fwd_kernel<DHP, 4, VEC>;
    }
}
template <int DHP, bool VEC, bool ACC>
const void *bwd_kernel_nt(int nt) {
    switch (nt) {
        case 1: return (const void *)attn_bwd_kernel<DHP, 1, VEC, ACC>;
        case 2: return (const void *)attn_bwd_kernel<DHP, 2, VEC, ACC>;
        case 3: return (const void *)attn_bwd_kernel<DHP, 3, VEC, ACC>;
        default: return (const void *)attn_bwd_kernel<DHP, 4, VEC, ACC>;
    }
}
template <bool VEC>
const void *fwd_kernel_v(int dhp, int nt) {
    return dhp == 16 ? fwd_kernel_nt<16, VEC>(nt) : dhp == 32 ? fwd_kernel_nt<32, VEC>(nt)
                                                              : fwd_kernel_nt<64, VEC>(nt);
}
template <bool VEC, bool ACC>
const void *bwd_kernel_v(int dhp, int nt) {
    return dhp == 16   ? bwd_kernel_nt<16, VEC, ACC>(nt)
           : dhp == 32 ? bwd_kernel_nt<32, VEC, ACC>(nt)
                       : bwd_kernel_nt<64, VEC, ACC>(nt);
}
// VEC: float4 accesses (dh == DHP, every row start 16-byte aligned, tk % 4
// == 0 and P 16-byte aligned); else scalar accesses throughout.
const void *fwd_kernel(int dhp, int nt, bool vec) {
    return vec ? fwd_kernel_v<true>(dhp, nt) : fwd_kernel_v<false>(dhp, nt);
}
const void *bwd_kernel(int dhp, int nt, bool vec, bool acc) {
    return vec ? (acc ? bwd_kernel_v<true, true>(dhp, nt) : bwd_kernel_v<true, false>(dhp, nt))
               : (acc ? bwd_kernel_v<false, true>(dhp, nt) : bwd_kernel_v<false, false>(dhp, nt));
}

// Above 64 KiB of dynamic LDS a kernel needs the attribute raised, once.
std::once_flag lds_attr_once;
void set_lds_limits() {
    std::call_once(lds_attr_once, [] {
        for (int dhp : {16, 32, 64})
            for (int nt = 1; nt <= 4; nt++)
                for (const void *k :
                     {fwd_kernel(dhp, nt, false), fwd_kernel(dhp, nt, true),
                      bwd_kernel(dhp, nt, false, false), bwd_kernel(dhp, nt, false, true),
                      bwd_kernel(dhp, nt, true, false), bwd_kernel(dhp, nt, true, true)})
                    // a refusal leaves the default limit, which the launch reports
                    if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                            160 * 1024) != hipSuccess)
                        (void)hipGetLastError();
    });
}


// The fused kernel for a long key axis (attn_fwd_long_kernel), or null:
// tq <= 64, tk 128 or 256, dh 32 or 64 with float4 accesses, no diagonal
// mask, the bias slots in LDS beside the tiles (RNN_ATTN_LONG=0: never).
const void *fwd_long_kernel(const rnn_attn_desc *d, bool vec, size_t *lds) {
    static const bool on = !(getenv("RNN_ATTN_LONG") && getenv("RNN_ATTN_LONG")[0] == '0');
    if (!on || !vec || d->mask_diag || d->tq > MAXT || (d->tk != 128 && d->tk != 256) ||
        (d->dh != 32 && d->dh != 64))
        return nullptr;
    const void *k;
    size_t words;
    if (d->dh == 64) {
        k = d->tk == 256 ? (const void *)attn_fwd_long_kernel<64, 16>
                         : (const void *)attn_fwd_long_kernel<64, 8>;
        words = d->tk == 256 ? fwd_long_words<64, 16>() : fwd_long_words<64, 8>();
    } else {
        k = d->tk == 256 ? (const void *)attn_fwd_long_kernel<32, 16>
                         : (const void *)attn_fwd_long_kernel<32, 8>;
        words = d->tk == 256 ? fwd_long_words<32, 16>() : fwd_long_words<32, 8>();
    }
    *lds = (words + d->nrel) * 4;
    if (*lds > 160 * 1024) return nullptr;
    static std::once_flag once;
    std::call_once(once, [] {
        for (const void *f : {(const void *)attn_fwd_long_kernel<64, 16>,
                              (const void *)attn_fwd_long_kernel<64, 8>,
                              (const void *)attn_fwd_long_kernel<32, 16>,
                              (const void *)attn_fwd_long_kernel<32, 8>})
            if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) !=
                hipSuccess)
                (void)hipGetLastError();
    });
    return k;
}

// The fused backward for a long key axis under the forward's conditions:
// the query half (acc_q: dQ added) and the key half (acc_kv: dK, dV added)
// with their LDS bytes, or nulls.
struct LongBwd {
    const void *qk = nullptr, *kk = nullptr;
    size_t qlds = 0, klds = 0;
};
LongBwd bwd_long_kernels(const rnn_attn_desc *d, bool vec, bool acc_q, bool acc_kv) {
    static const bool on = !(getenv("RNN_ATTN_LONG") && getenv("RNN_ATTN_LONG")[0] == '0');
    LongBwd r;
    if (!on || !vec || d->mask_diag || d->tq > MAXT || (d->tk != 128 && d->tk != 256) ||
        (d->dh != 32 && d->dh != 64))
        return r;
    size_t words;
#define RNN_LONG_PAIR(DH_, NT_)                                                                 \
    r.qk = acc_q ? (const void *)attn_bwd_long_q_kernel<DH_, NT_, true>                         \
                 : (const void *)attn_bwd_long_q_kernel<DH_, NT_, false>;                       \
    r.kk = acc_kv ? (const void *)attn_bwd_long_k_kernel<DH_, NT_, true>                        \
                  : (const void *)attn_bwd_long_k_kernel<DH_, NT_, false>;                      \
    words = bwd_long_words<DH_, NT_>();                                                         \
    r.klds = (size_t)2 * DH_ * TS * 4;
    if (d->dh == 64 && d->tk == 256) {
        RNN_LONG_PAIR(64, 16)
    } else if (d->dh == 64) {
        RNN_LONG_PAIR(64, 8)
    } else if (d->tk == 256) {
        RNN_LONG_PAIR(32, 16)
    } else {
        RNN_LONG_PAIR(32, 8)
    }
#undef RNN_LONG_PAIR
    r.qlds = words * 4 + 4 * sizeof(double);
    if (r.qlds > 160 * 1024) return LongBwd{};
    static std::once_flag once;
    std::call_once(once, [] {
        for (const void *f : {(const void *)attn_bwd_long_q_kernel<64, 16, true>,
                              (const void *)attn_bwd_long_q_kernel<64, 16, false>,
                              (const void *)attn_bwd_long_q_kernel<64, 8, true>,
                              (const void *)attn_bwd_long_q_kernel<64, 8, false>,
                              (const void *)attn_bwd_long_q_kernel<32, 16, true>,
                              (const void *)attn_bwd_long_q_kernel<32, 16, false>,
                              (const void *)attn_bwd_long_q_kernel<32, 8, true>,
                              (const void *)attn_bwd_long_q_kernel<32, 8, false>})
            if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) !=
                hipSuccess)
                (void)hipGetLastError();
    });
    return r;
}

// Core::forward on the composed path (see attn_softmax_rows_kernel).
int attn_forward_large(rnn_ctx *ctx, const RnnRelTable &tab, const rnn_attn_desc *d, size_t n,
                       const float *q, const float *kv, const float *tau, const float *rel,
                       float *p, float *o) {
    const size_t tq = d->tq, tk = d->tk, dh = d->dh, h = d->h, c = h * dh;
    // S = Q K^T for every (image, head) in one launch
    int rc = rnn_gemm_launch_ld2(ctx, n, h, tq, tk, dh, q + d->qoff, d->qstride, tq * d->qstride,
                                 dh, 0, kv + d->koff, d->kvstride, tk * d->kvstride, dh, 1, p, tk,
                                 h * tq * tk, tq * tk, 0);
    if (rc) return rc;
    const long long rows = (long long)n * h * tq;
    {
        const unsigned grid = (unsigned)rnn_div_up((size_t)rows, 4);
        const int m = d->mask_diag ? 1 : 0;
        auto sm = [&](auto kern) {
            kern<<<grid, 256, 0, ctx->stream>>>(p, tau, rel, tab.dev, rows, (int)h, (int)tq,
                                                (int)tk, (int)d->nrel, m);
        };
        switch (rnn_div_up(tk, (size_t)64)) {
            case 1: sm(attn_softmax_rows_kernel<1>); break;
            case 2: sm(attn_softmax_rows_kernel<2>); break;
            case 3: sm(attn_softmax_rows_kernel<3>); break;
            case 4: sm(attn_softmax_rows_kernel<4>); break;
            case 5: sm(attn_softmax_rows_kernel<5>); break;
            case 6: sm(attn_softmax_rows_kernel<6>); break;
            case 7: sm(attn_softmax_rows_kernel<7>); break;
            case 8: sm(attn_softmax_rows_kernel<8>); break;
            default: sm(attn_softmax_rows_kernel<0>); break;
        }
    }
    RNN_LAUNCHED(ctx);
    // O = P V
    return rnn_gemm_launch_ld2(ctx, n, h, tq, dh, tk, p, tk, h * tq * tk, tq * tk, 0,
                               kv + d->voff, d->kvstride, tk * d->kvstride, dh, 0, o, c, tq * c,
                               dh, 0);
}

// Core::backward on the composed path: dV = P^T dO, dP = dO V^T, the raw S
// recomputed, the row kernel (dS, tau dS, dtau shares), dtau and drel, then
// dQ = (tau dS) K and dK = (tau dS)^T Q; dtau and drel accumulate, dq and
// dkv too unless flags overwrite them.
int attn_backward_large(rnn_ctx *ctx, const RnnRelTable &tab, const rnn_attn_desc *d, size_t n,
                        const float *q, const float *kv, const float *tau, const float *p, const float *dout,
                        float *dq, float *dkv, float *dtau, float *drel, uint32_t flags) {
    const int acc_q = (flags & RNN_ATTN_SET_DQ) ? 0 : 1, acc_kv = (flags & RNN_ATTN_SET_DKV) ? 0 : 1;
    const size_t tq = d->tq, tk = d->tk, dh = d->dh, h = d->h, c = h * dh;
    const size_t cnt = tq * tk, mat = n * h * cnt;
    const long long rows = (long long)n * h * tq;
    const size_t per = h * d->nrel;
    AttnArgs g;
    fill_args(g, tab, d, n);
    g.q = q;
    g.kv = kv;
    g.tau = tau;
    g.p = p;
    g.dout = dout;
    g.dq = dq;
    g.dkv = dkv;
    const LongBwd lb = bwd_long_kernels(d, use_vec(g) && tk % 4 == 0 && al16(p), acc_q != 0,
                                        acc_kv != 0);
    if (lb.qk) {
        // two fused launches, then the dtau / drel partials summed over the
        // images in image order (deferred with the context's other
        // parameter-gradient reductions when it defers them)
        const size_t tau_bytes = rnn_round_up(n * h * sizeof(double), 256);
        const size_t part_bytes = tau_bytes + n * per * sizeof(float);
        WsCarve cv;
        const size_t o_s2 = cv.take(mat * 4), o_pw = ctx->defer ? 0 : cv.take(part_bytes);
        char *ws = (char *)rnn_workspace(ctx, cv.off);
        if (!ws) return RNN_E_NOMEM;
        float *s2 = (float *)(ws + o_s2);
        char *pw = ctx->defer ? (char *)rnn_defer_take(ctx, part_bytes) : ws + o_pw;
        if (!pw) return RNN_E_NOMEM;
        g.dtau_part = (double *)pw;
        g.drel_part = (float *)(pw + tau_bytes);
        void *qargs[] = {&g, &s2};
        RNN_HIP(ctx, hipLaunchKernel(lb.qk, dim3((unsigned)(n * h)), dim3(256), qargs, lb.qlds,
                                     ctx->stream));
        void *kargs[] = {&g, &s2};
        RNN_HIP(ctx, hipLaunchKernel(lb.kk, dim3((unsigned)(n * h)), dim3(256), kargs, lb.klds,
                                     ctx->stream));
        const int tot = (int)(per + h);
        if (ctx->defer) {
            RnnDeferSeg sg{};
            sg.part = g.dtau_part;
            sg.part2 = g.drel_part;
            sg.out0 = drel;
            sg.out1 = dtau;
            sg.len = tot;
            sg.split = (long long)per;
            sg.nrow = (int)n;
            sg.kind = RNN_DEFER_ATTN;
            rnn_defer_push(ctx, sg);
            return RNN_OK;
        }
        hipLaunchKernelGGL(attn_reduce_kernel, dim3((unsigned)rnn_div_up(tot, 32)), dim3(256), 0,
                           ctx->stream, (const double *)g.dtau_part, (const float *)g.drel_part,
                           (int)n, (int)h, (int)d->nrel, dtau, drel);
        RNN_LAUNCHED(ctx);
        return RNN_OK;
    }
    // drel partials over chunks of ipc images: enough chunks to fill the
    // chip (16 chunks left it latency-bound: 61 us a call at the rustvit's
    // cross-attention shape)
    const size_t ipc = rnn_div_up(n, (size_t)64), nchunk = rnn_div_up(n, ipc);
    WsCarve cv;
    const size_t o1 = cv.take(mat * 4), o2 = cv.take(mat * 4), o3 = cv.take((size_t)rows * 8);
    const size_t o4 = cv.take(nchunk * per * 4);
    char *ws = (char *)rnn_workspace(ctx, cv.off);
    if (!ws) return RNN_E_NOMEM;
    float *s1 = (float *)(ws + o1), *s2 = (float *)(ws + o2);
    double *part = (double *)(ws + o3);
    float *rpart = (float *)(ws + o4);
    // each GEMM over every (image, head) in one launch
    // dV += P^T dO (attn.rs:262-270)
    int rc = rnn_gemm_launch_ld2(ctx, n, h, tk, dh, tq, p, tk, h * cnt, cnt, 1, dout, c, tq * c,
                                 dh, 0, dkv + d->voff, d->kvstride, tk * d->kvstride, dh, acc_kv);
    if (rc) return rc;
    // dP = dO V^T (attn.rs:272-278)
    rc = rnn_gemm_launch_ld2(ctx, n, h, tq, tk, dh, dout, c, tq * c, dh, 0, kv + d->voff,
                             d->kvstride, tk * d->kvstride, dh, 1, s1, tk, h * cnt, cnt, 0);
    if (rc) return rc;
    // the raw scores again (attn.rs:292-300)
    rc = rnn_gemm_launch_ld2(ctx, n, h, tq, tk, dh, q + d->qoff, d->qstride, tq * d->qstride, dh,
                             0, kv + d->koff, d->kvstride, tk * d->kvstride, dh, 1, s2, tk,
                             h * cnt, cnt, 0);
    if (rc) return rc;
    attn_dsoft_rows_kernel<<<(unsigned)rnn_div_up((size_t)rows, 4), 256, 0, ctx->stream>>>(
        p, s1, s2, tau, part, rows, (int)h, (int)tq, (int)tk);
    RNN_LAUNCHED(ctx);
    attn_head_sum_kernel<<<(unsigned)h, 256, 0, ctx->stream>>>(part, (long long)n, (int)h,
                                                              (int)tq, dtau);
    RNN_LAUNCHED(ctx);
    attn_drel_part_kernel<<<dim3((unsigned)rnn_div_up(per, (size_t)256), (unsigned)nchunk), 256,
                            0, ctx->stream>>>(s1, tab.dev + cnt,
                                              tab.dev + cnt + d->nrel + 1, (long long)n,
                                              (long long)ipc, (int)h, (int)d->nrel,
                                              (long long)cnt, rpart);
    RNN_LAUNCHED(ctx);
    attn_drel_sum_kernel<<<(unsigned)rnn_div_up(per, (size_t)256), 256, 0, ctx->stream>>>(
        rpart, (int)nchunk, (long long)per, drel);
    RNN_LAUNCHED(ctx);
    // dQ += (tau dS) K (attn.rs:317-322)
    rc = rnn_gemm_launch_ld2(ctx, n, h, tq, dh, tk, s2, tk, h * cnt, cnt, 0, kv + d->koff,
                             d->kvstride, tk * d->kvstride, dh, 0, dq + d->qoff, d->qstride,
                             tq * d->qstride, dh, acc_q);
    if (rc) return rc;
    // dK += (tau dS)^T Q (attn.rs:324-330)
    return rnn_gemm_launch_ld2(ctx, n, h, tk, dh, tq, s2, tk, h * cnt, cnt, 1, q + d->qoff,
                               d->qstride, tq * d->qstride, dh, 0, dkv + d->koff, d->kvstride,
                               tk * d->kvstride, dh, acc_kv);
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
    const RnnRelTable *tab = nullptr;
    rc = rel_table(ctx, d, &tab);
    if (rc) return rc;
    AttnArgs g;
    fill_args(g, *tab, d, n);
    g.q = q;
    g.kv = kv;
    g.tau = tau;
    g.rel = rel;
    g.pout = p;
    g.o = o;
    const bool vec = use_vec(g) && d->tk % 4 == 0 && al16(p);
    if (large_desc(d)) {
        size_t llds = 0;
        if (const void *k = fwd_long_kernel(d, vec, &llds)) {
            const uint32_t *relidx = tab->dev;
            void *largs[] = {&g, &relidx};
            RNN_HIP(ctx, hipLaunchKernel(k, dim3((unsigned)(n * d->h)), dim3(256), largs, llds,
                                         ctx->stream));
            return RNN_OK;
        }
        return attn_forward_large(ctx, *tab, d, n, q, kv, tau, rel, p, o);
    }
    set_lds_limits();
    const int dhp = dhp_of(d->dh), nt = (int)(d->tk + 15) / 16;
    const size_t lds = fwd_lds(dhp, d->nrel);
    if (lds > 160 * 1024)
        return rnn_fail(ctx, RNN_E_UNSUPPORTED, "attn: nrel %u bias slots exceed LDS", d->nrel);
    void *args[] = {&g};
    RNN_HIP(ctx, hipLaunchKernel(fwd_kernel(dhp, nt, vec), dim3((unsigned)(n * d->h)), dim3(256),
                                 args, lds, ctx->stream));
    return RNN_OK;
}

int rnn_attn_backward(rnn_ctx *ctx, const rnn_attn_desc *d, size_t n, const float *q,
                      const float *kv, const float *tau, const float *p, const float *dout,
                      float *dq, float *dkv, float *dtau, float *drel) {
    return rnn_attn_backward_ex(ctx, d, n, q, kv, tau, p, dout, dq, dkv, dtau, drel, 0);
}

int rnn_attn_backward_ex(rnn_ctx *ctx, const rnn_attn_desc *d, size_t n, const float *q,
                         const float *kv, const float *tau, const float *p, const float *dout,
                         float *dq, float *dkv, float *dtau, float *drel, uint32_t flags) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    int rc = check_desc(ctx, d);
    if (rc) return rc;
    if (flags & ~(uint32_t)(RNN_ATTN_SET_DQ | RNN_ATTN_SET_DKV))
        return rnn_fail(ctx, RNN_E_INVALID, "attn_backward: unknown flags 0x%x", flags);
    if (n == 0) return RNN_OK;
    if (!q || !kv || !tau || !p || !dout || !dq || !dkv || !dtau || !drel)
        return rnn_fail(ctx, RNN_E_NULL, "attn_backward: null operand");
    if (n * d->h > 0x7fffffffu) return rnn_fail(ctx, RNN_E_UNSUPPORTED, "attn: too many problems");
    const RnnRelTable *tab = nullptr;
    rc = rel_table(ctx, d, &tab);
    if (rc) return rc;
    if (large_desc(d))
        return attn_backward_large(ctx, *tab, d, n, q, kv, tau, p, dout, dq, dkv, dtau, drel,
                                   flags);
    set_lds_limits();
    // The workgroup kernels overwrite both or accumulate into both; with one
    // flag only, the overwritten operand's columns are cleared first.
    const bool set_q = flags & RNN_ATTN_SET_DQ, set_kv = flags & RNN_ATTN_SET_DKV;
    const bool acc = !(set_q && set_kv);
    if (acc && set_q) {
        hipLaunchKernelGGL(attn_zero_cols_kernel, dim3((unsigned)rnn_div_up(n * d->tq, (size_t)4)),
                           dim3(256), 0, ctx->stream, dq, (long long)(n * d->tq),
                           (long long)d->qstride, (long long)d->qoff, (int)(d->h * d->dh));
        RNN_LAUNCHED(ctx);
    }
    if (acc && set_kv)
        for (size_t off : {(size_t)d->koff, (size_t)d->voff}) {
            hipLaunchKernelGGL(attn_zero_cols_kernel,
                               dim3((unsigned)rnn_div_up(n * d->tk, (size_t)4)), dim3(256), 0,
                               ctx->stream, dkv, (long long)(n * d->tk), (long long)d->kvstride,
                               (long long)off, (int)(d->h * d->dh));
            RNN_LAUNCHED(ctx);
        }
    AttnArgs g;
    fill_args(g, *tab, d, n);
    const size_t tau_bytes = rnn_round_up(n * d->h * sizeof(double), 256);
    const size_t ws_bytes = tau_bytes + n * d->h * (size_t)d->nrel * sizeof(float);
    // the dtau / drel partials wait in the deferral arena when the context
    // defers parameter-gradient reductions
    char *ws = (char *)(ctx->defer ? rnn_defer_take(ctx, ws_bytes) : rnn_workspace(ctx, ws_bytes));
    if (!ws) return RNN_E_NOMEM;
    g.q = q;
    g.kv = kv;
    g.tau = tau;
    g.p = p;
    g.dout = dout;
    g.dq = dq;
    g.dkv = dkv;
    g.dtau_part = (double *)ws;
    g.drel_part = (float *)(ws + tau_bytes);
    const bool vec = use_vec(g) && d->tk % 4 == 0 && al16(p);
    const int dhp = dhp_of(d->dh), nt = (int)(d->tk + 15) / 16;
    const int nth = 256;  // four waves: the staging splits every tile over 256 threads
    // the drel index blob rides in registers into the LDS of V and K^T when
    // it fits both
    const size_t bb = blob_bytes((size_t)d->tq * d->tk, d->nrel);
    const size_t region = ((size_t)64 * (dhp + 4) + (size_t)dhp * TS) * 4;
    g.blob_chunks = (bb <= region && bb / 16 <= (size_t)BLOB_CHUNKS * nth) ? (int)(bb / 16) : 0;
    void *args[] = {&g};
    RNN_HIP(ctx, hipLaunchKernel(bwd_kernel(dhp, nt, vec, acc), dim3((unsigned)(n * d->h)),
                                 dim3(nth), args, bwd_lds(dhp), ctx->stream));
    int tot = (int)(d->h * d->nrel + d->h);
    if (ctx->defer) {
        RnnDeferSeg sg{};
        sg.part = g.dtau_part;
        sg.part2 = g.drel_part;
        sg.out0 = drel;
        sg.out1 = dtau;
        sg.len = tot;
        sg.split = (long long)(d->h * d->nrel);
        sg.nrow = (int)n;
        sg.kind = RNN_DEFER_ATTN;
        rnn_defer_push(ctx, sg);
        return RNN_OK;
    }
    hipLaunchKernelGGL(attn_reduce_kernel, dim3((unsigned)rnn_div_up(tot, 32)), dim3(256), 0,
                       ctx->stream, (const double *)g.dtau_part, (const float *)g.drel_part, (int)n,
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
