// Batched small attention (attn.rs Core) on gfx950: one workgroup of two
// waves per (image, head), each wave 32 query rows; the operands live in
// registers (contiguous half-row loads in the k order the MFMA A and B
// layouts share), the score tiles are computed transposed (S^T = K Q^T) so
// that a query row spans lanes l and l^32 only, and 32x32 fp32 MFMA tiles
// do every product.
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
    double *dtau_part;             // [n][h]
    float *drel_part;              // [n][h][nrel]
    const uint32_t *relidx;        // [tq*tk]
    const uint32_t *rowptr;        // [nrel+1] inverse index (drel gather)
    const uint32_t *pos;           // [tq*tk] LDS offsets (row*LS + col), by bias slot
    const uint32_t *rperm;         // [64][2][32] relidx in lane order (see key_of)
    long long qstride, qoff, kvstride, koff, voff;
    int n, h, dh, tq, tk, nrel, mask;
    int DHP;  // dh padded to 32 or 64
};

// Row reductions over the 32 lanes of a wave half (the 32 columns a 32x32
// MFMA tile spreads over lanes): xor offsets below 32 stay inside the half.
__device__ __forceinline__ float half_max(float v) {
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float half_sum(float v) {
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ void zero16(f32x16 &a) {
#pragma unroll
    for (int v = 0; v < 16; v++) a[v] = 0.f;
}

// MFMA operands of a product over the head dimension (S = Q K^T, dP = dO V^T):
// step s of lane half hh takes k = hh*HALF + s, for A and B alike, so a lane
// holds HALF consecutive columns of one row -- a contiguous half-row.
//
// Loads are unconditional, from clamped (in-range) addresses.  Rows past the
// matrix need no zeroing: they only reach score entries that are masked or
// products with a zero P.  Columns past dh are summed over, so they are
// zeroed (VEC = false only; VEC means dh == DHP with aligned rows, read as
// float4).  A guarded load -- or a select the compiler may turn back into one
// -- becomes a branch of its own, and the loads can no longer be issued
// together.
__device__ __forceinline__ float keep(float v, bool c) {
    return __uint_as_float(__float_as_uint(v) & (c ? 0xffffffffu : 0u));
}

template <int HALF, bool VEC>
__device__ __forceinline__ void load_half(float (&r)[HALF], const float *base, long long stride,
                                          int row, int nrows, int c0, int dh) {
    const float *p = base + (long long)min(row, nrows - 1) * stride;
    if constexpr (VEC) {
#pragma unroll
        for (int i = 0; i < HALF; i += 4) {
            const float4 t = *reinterpret_cast<const float4 *>(p + c0 + i);
            r[i] = t.x;
            r[i + 1] = t.y;
            r[i + 2] = t.z;
            r[i + 3] = t.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < HALF; i++) r[i] = keep(p[min(c0 + i, dh - 1)], c0 + i < dh);
    }
}

template <int HALF>
__device__ __forceinline__ void mma_half(f32x16 &acc, const float (&a)[HALF],
                                         const float (&b)[HALF]) {
#pragma unroll
    for (int s = 0; s < HALF; s++) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], b[s], acc, 0, 0, 0);
}

// Rows [0, 64) x cols [0, DHP) of a strided matrix into LDS (row stride XS),
// zero past (nrows, dh); 4-float groups with float4 loads when `vec`.
template <int DHP>
__device__ __forceinline__ void stage_rows(float *dst, int XS, const float *src, long long stride,
                                           int nrows, int dh, bool vec, int tid, int nthreads) {
    constexpr int G = DHP / 4;  // 4-float groups per row (a power of two)
    for (int idx = tid; idx < 64 * G; idx += nthreads) {
        const int r = idx / G, c = (idx % G) * 4;
        float t[4] = {0.f, 0.f, 0.f, 0.f};
        if (r < nrows) {
            const float *p = src + (long long)r * stride + c;
            if (vec && c + 4 <= dh) {
                const float4 v = *reinterpret_cast<const float4 *>(p);
                t[0] = v.x;
                t[1] = v.y;
                t[2] = v.z;
                t[3] = v.w;
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) t[i] = c + i < dh ? p[i] : 0.f;
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) dst[r * XS + c + i] = t[i];
    }
}

constexpr int LS = 65;  // LDS row stride of the 64 x 64 P / dS tiles

// Transposed score tiles: S^T = K Q^T with A = K (key rows) and B = Q (query
// rows), so in the accumulator layout lane l holds query qi = 32w + l%32 and
// register v of key tile nt holds key kj = 32nt + 8(v/4) + 4(l/32) + v%4.  A
// query row is then split over two lanes only (l and l ^ 32): row max and
// sum take one cross-lane step.  And those registers are, step for step, the
// A operand of a product over keys (O = P V, dQ = dS K): MFMA step s = 16nt
// + v pairs key kj(s, half) for both operands.
__device__ __forceinline__ int key_of(int nt, int v, int hh) {
    return 32 * nt + 8 * (v >> 2) + 4 * hh + (v & 3);
}

// dst[r][d] += acc[v] for the 16 rows r = r0 + 8(v/4) + 4hh + v%4 of an
// accumulator tile (column d): the 16 old values are loaded together (clamped
// addresses), then added and stored where in range.
__device__ __forceinline__ void accumulate16(float *dst, long long stride, int r0, int nrows, int d,
                                             int dh, int hh, const f32x16 &acc) {
    float old[16];
    const int dc = min(d, dh - 1);
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const int r = min(r0 + 8 * (v >> 2) + 4 * hh + (v & 3), nrows - 1);
        old[v] = dst[(long long)r * stride + dc];
    }
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const int r = r0 + 8 * (v >> 2) + 4 * hh + (v & 3);
        if (r < nrows && d < dh) dst[(long long)r * stride + d] = old[v] + acc[v];
    }
}

// Core::forward (attn.rs:148-223) for one (image, head), tq, tk <= 64,
// dh <= DHP (32 or 64).  Two waves; wave w owns queries [32w, 32w + 32):
//   * S^T from half-row operands (K, Q straight from HBM into registers);
//   * x = tau*S + rel[relidx] (the head's bias slots and the index table
//     staged in LDS), diagonal -> -inf when masked, -inf outside (tq, tk);
//   * softmax per query: exp(x - max) (-inf -> 0), times 1/sum (attn.rs:
//     199-210), max and sum in-lane plus one exchange with lane ^ 32;
//   * O = P V with P from the registers and V rows from HBM.
template <int DHP, bool VEC>
__global__ __launch_bounds__(128) void attn_fwd_kernel(AttnArgs g) {
    constexpr int HALF = DHP / 2, NDT = DHP / 32;
    extern __shared__ float smem[];
    float *Pw = smem + wave_index() * 32 * LS;  // [32][LS] P rows of this wave
    uint32_t *rp = reinterpret_cast<uint32_t *>(smem + 64 * LS);  // [64][2][32] lane-order relidx
    float *rels = smem + 64 * LS + 4096;        // [nrel] bias slots of the head
    const int tid = threadIdx.x, lane = tid & 63, w = wave_index();
    const int l32 = lane & 31, hh = lane >> 5;
    const int img = blockIdx.x / g.h, hd = blockIdx.x % g.h;
    const int tq = g.tq, tk = g.tk, dh = g.dh;
    const float *qb = g.q + (long long)img * tq * g.qstride + g.qoff + (long long)hd * dh;
    const float *kb = g.kv + (long long)img * tk * g.kvstride + g.koff + (long long)hd * dh;
    const float *vb = g.kv + (long long)img * tk * g.kvstride + g.voff + (long long)hd * dh;
    const int qi = 32 * w + l32;

    // Operands of S^T first (the load counter is in order: what is needed
    // first is issued first), then the tables, then V.
    float qb_[HALF], ka[2][HALF];
    load_half<HALF, VEC>(qb_, qb, g.qstride, qi, tq, hh * HALF, dh);
#pragma unroll
    for (int nt = 0; nt < 2; nt++)
        load_half<HALF, VEC>(ka[nt], kb, g.kvstride, 32 * nt + l32, tk, hh * HALF, dh);
    {  // relidx in lane order: 16 KB, coalesced 16-byte loads
        const uint4 *src = reinterpret_cast<const uint4 *>(g.rperm);
        uint4 t4[8];
#pragma unroll
        for (int i = 0; i < 8; i++) t4[i] = src[tid + 128 * i];
#pragma unroll
        for (int i = 0; i < 8; i++) reinterpret_cast<uint4 *>(rp)[tid + 128 * i] = t4[i];
    }
    for (int e = tid; e < g.nrel; e += blockDim.x) rels[e] = g.rel[(long long)hd * g.nrel + e];
    f32x16 st[2];
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        zero16(st[nt]);
        mma_half<HALF>(st[nt], ka[nt], qb_);
    }
    // V rows as the B operand of O = P V (step s = 16nt + v).
    float vv[NDT][32];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++)
#pragma unroll
        for (int s2 = 0; s2 < 32; s2++) {
            const int kj = key_of(s2 >> 4, s2 & 15, hh), d = 32 * dt + l32;
            // rows past tk meet P = 0; columns past dh are not stored
            vv[dt][s2] = vb[(long long)min(kj, tk - 1) * g.kvstride + min(d, dh - 1)];
        }
    __syncthreads();
    const float t = g.tau[hd];
    float x[2][16];
    // bias reads first, all of them (the table holds valid slots everywhere)
    {
        const uint4 *mine = reinterpret_cast<const uint4 *>(rp + (qi * 2 + hh) * 32);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint4 r4 = mine[i];
            x[i >> 2][(i & 3) * 4 + 0] = rels[r4.x];
            x[i >> 2][(i & 3) * 4 + 1] = rels[r4.y];
            x[i >> 2][(i & 3) * 4 + 2] = rels[r4.z];
            x[i >> 2][(i & 3) * 4 + 3] = rels[r4.w];
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int nt = 0; nt < 2; nt++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int kj = key_of(nt, v, hh);
            const bool live = qi < tq && kj < tk && !(g.mask && kj == qi);
            const float xv = t * st[nt][v] + x[nt][v];
            x[nt][v] = __uint_as_float(live ? __float_as_uint(xv) : 0xff800000u);  // -inf
            mx = fmaxf(mx, x[nt][v]);
        }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    float sum = 0.f;
#pragma unroll
    for (int nt = 0; nt < 2; nt++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const float e = x[nt][v] == -INFINITY ? 0.f : __expf(x[nt][v] - mx);
            x[nt][v] = e;
            sum += e;
        }
    sum += __shfl_xor(sum, 32, 64);
    const float inv = 1.0f / sum;
#pragma unroll
    for (int nt = 0; nt < 2; nt++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const float p = qi < tq ? x[nt][v] * inv : 0.f;
            x[nt][v] = p;
            Pw[l32 * LS + key_of(nt, v, hh)] = p;
        }
    // P rows to HBM through LDS: one coalesced row per store instruction.
    float *pg = g.pout + ((long long)img * g.h + hd) * tq * tk;
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes done
    __builtin_amdgcn_wave_barrier();
    const int rows = min(32, tq - 32 * w);
    if (lane < tk) {
        float pr[32];
#pragma unroll
        for (int r = 0; r < 32; r++) pr[r] = Pw[r * LS + lane];
#pragma unroll
        for (int r = 0; r < 32; r++)
            if (r < rows) pg[(long long)(32 * w + r) * tk + lane] = pr[r];
    }
    const int c = g.h * dh;
    float *od = g.o + (long long)img * tq * c + (long long)hd * dh;
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) {
        f32x16 acc;
        zero16(acc);
#pragma unroll
        for (int s2 = 0; s2 < 32; s2++)
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(x[s2 >> 4][s2 & 15], vv[dt][s2], acc, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int q = 32 * w + 8 * (v >> 2) + 4 * hh + (v & 3), d = 32 * dt + l32;
            if (q < tq && d < dh) od[(long long)q * c + d] = acc[v];
        }
    }
}

// Core::backward (attn.rs:226-343) for one (image, head), same limits and
// waves.  Phase 1 in registers, lane = query (as the forward): dP^T = V dO^T,
// the recomputed raw S^T = K Q^T, P from HBM, the row dot <dP, P> (in-lane
// plus one exchange), dS = P o (dP - dot), the dtau partial sum(dS o S).
// dQ = tau*dS K takes dS straight from the registers and K rows from HBM.
// P and dS go to LDS for the drel partial (inverse index, ascending
// positions) and for dK = tau*dS^T Q and dV = P^T dO (key rows, Q and dO rows
// from HBM).  dQ, dK, dV accumulate into HBM.
template <int DHP, bool VEC>
__global__ __launch_bounds__(128) void attn_bwd_kernel(AttnArgs g) {
    constexpr int HALF = DHP / 2, NDT = DHP / 32;
    extern __shared__ float smem[];
    float *Pl = smem, *Sl = Pl + 64 * LS;
    double *dred = (double *)(Sl + 64 * LS);  // 8-byte aligned: 2 * 64 * LS floats before it
    const int tid = threadIdx.x, lane = tid & 63, w = wave_index(), nthreads = blockDim.x;
    const int l32 = lane & 31, hh = lane >> 5;
    const int img = blockIdx.x / g.h, hd = blockIdx.x % g.h;
    const int tq = g.tq, tk = g.tk, dh = g.dh, c = g.h * dh;
    const float *qb = g.q + (long long)img * tq * g.qstride + g.qoff + (long long)hd * dh;
    const float *kb = g.kv + (long long)img * tk * g.kvstride + g.koff + (long long)hd * dh;
    const float *vb = g.kv + (long long)img * tk * g.kvstride + g.voff + (long long)hd * dh;
    const float *ob = g.dout + (long long)img * tq * c + (long long)hd * dh;
    const float *pb = g.p + ((long long)img * g.h + hd) * tq * tk;
    const int qi = 32 * w + l32;

    // P of this wave's rows into LDS with coalesced row loads (0 outside).
#pragma unroll 8
    for (int r = 0; r < 32; r++) {
        const int q = 32 * w + r;
        const float t0 = pb[(long long)min(q, tq - 1) * tk + min(lane, tk - 1)];
        Pl[q * LS + lane] = keep(t0, q < tq && lane < tk);
    }
    float qv[HALF], ov[HALF];
    load_half<HALF, VEC>(qv, qb, g.qstride, qi, tq, hh * HALF, dh);
    load_half<HALF, VEC>(ov, ob, c, qi, tq, hh * HALF, dh);
    f32x16 dp[2], sr[2];
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        float ka[HALF], va[HALF];
        load_half<HALF, VEC>(ka, kb, g.kvstride, 32 * nt + l32, tk, hh * HALF, dh);
        load_half<HALF, VEC>(va, vb, g.kvstride, 32 * nt + l32, tk, hh * HALF, dh);
        zero16(dp[nt]);
        zero16(sr[nt]);
        mma_half<HALF>(dp[nt], va, ov);
        mma_half<HALF>(sr[nt], ka, qv);
    }
    // K rows as the B operand of dQ = dS K (step s = 16nt + v).
    float kk[NDT][32];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++)
#pragma unroll
        for (int s2 = 0; s2 < 32; s2++) {
            const int kj = key_of(s2 >> 4, s2 & 15, hh), d = 32 * dt + l32;
            // rows past tk meet dS = 0; columns past dh are not stored
            kk[dt][s2] = kb[(long long)min(kj, tk - 1) * g.kvstride + min(d, dh - 1)];
        }
    // P in the accumulator layout, from this wave's LDS rows.
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    float pv[2][16];
#pragma unroll
    for (int nt = 0; nt < 2; nt++)
#pragma unroll
        for (int v = 0; v < 16; v++) pv[nt][v] = Pl[qi * LS + key_of(nt, v, hh)];
    // dS = P o (dP - <dP, P>) (attn.rs:280-290); dtau partial (attn.rs:292-308)
    float dot = 0.f;
#pragma unroll
    for (int nt = 0; nt < 2; nt++)
#pragma unroll
        for (int v = 0; v < 16; v++) dot += dp[nt][v] * pv[nt][v];
    dot += __shfl_xor(dot, 32, 64);
    float tpart = 0.f;
    const float t = g.tau[hd];
    float ds[2][16];
#pragma unroll
    for (int nt = 0; nt < 2; nt++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int kj = key_of(nt, v, hh);
            const float d0 = pv[nt][v] * (dp[nt][v] - dot);  // 0 outside (tq, tk): P is 0
            tpart += d0 * sr[nt][v];
            Sl[qi * LS + kj] = d0;
            ds[nt][v] = d0 * t;  // attn.rs:316: dS *= tau
        }
    // dtau is a sum whose terms cancel to about 1% of their size: the lane
    // partials are added in f64 from here on
    const double tsum = wave_sum_d((double)tpart);
    if (lane == 0) dred[w] = tsum;
    // dQ = tau*dS K (attn.rs:319-323): queries of this lane, from registers
    float *dqi = g.dq + (long long)img * tq * g.qstride + g.qoff + (long long)hd * dh;
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) {
        f32x16 acc;
        zero16(acc);
#pragma unroll
        for (int s2 = 0; s2 < 32; s2++)
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(ds[s2 >> 4][s2 & 15], kk[dt][s2], acc, 0, 0, 0);
        accumulate16(dqi, g.qstride, 32 * w, tq, 32 * dt + l32, dh, hh, acc);
    }
    __syncthreads();
    // drel partial: gather by inverse index in ascending position (attn.rs:309-315)
    float *drp = g.drel_part + ((long long)img * g.h + hd) * g.nrel;
    for (int r = tid; r < g.nrel; r += nthreads) {
        float sacc = 0.f;
        const uint32_t e0 = g.rowptr[r], e1 = g.rowptr[r + 1];
        for (uint32_t e = e0; e < e1; e += 8) {
            uint32_t off[8];
#pragma unroll
            for (int u = 0; u < 8; u++) off[u] = e + u < e1 ? g.pos[e + u] : 0u;
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (e + u < e1) sacc += Sl[off[u]];
        }
        drp[r] = sacc;
    }
    if (tid == 0) g.dtau_part[(long long)img * g.h + hd] = dred[0] + dred[1];
    // dK = tau*dS^T Q and dV = P^T dO (attn.rs:270-274, 324-327): key rows
    // [32w, 32w + 32), A from LDS (transposed reads), Q / dO rows from HBM.
    float *dki = g.dkv + (long long)img * tk * g.kvstride + g.koff + (long long)hd * dh;
    float *dvi = g.dkv + (long long)img * tk * g.kvstride + g.voff + (long long)hd * dh;
    const int kr = 32 * w + l32;
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) {
        f32x16 ak, av;
        zero16(ak);
        zero16(av);
        for (int s0 = 0; s0 < 32; s0 += 16) {
            float qv2[16], ov2[16];
#pragma unroll
            for (int u = 0; u < 16; u++) {
                const int q = key_of((s0 + u) >> 4, (s0 + u) & 15, hh), d = 32 * dt + l32;
                // rows past tq meet dS = P = 0; columns past dh are not stored
                const int qc = min(q, tq - 1), dc = min(d, dh - 1);
                qv2[u] = qb[(long long)qc * g.qstride + dc];
                ov2[u] = ob[(long long)qc * c + dc];
            }
#pragma unroll
            for (int u = 0; u < 16; u++) {
                const int q = key_of((s0 + u) >> 4, (s0 + u) & 15, hh);
                ak = __builtin_amdgcn_mfma_f32_32x32x2f32(t * Sl[q * LS + kr], qv2[u], ak, 0, 0, 0);
                av = __builtin_amdgcn_mfma_f32_32x32x2f32(Pl[q * LS + kr], ov2[u], av, 0, 0, 0);
            }
        }
        accumulate16(dki, g.kvstride, 32 * w, tk, 32 * dt + l32, dh, hh, ak);
        accumulate16(dvi, g.kvstride, 32 * w, tk, 32 * dt + l32, dh, hh, av);
    }
}

// dtau[h] += sum_img part[img][h]; drel[h*nrel + r] += sum_img part[img][h][r]
// (image order, attn.rs:333-342).  A block takes 32 elements; thread (j, e)
// sums images [j*G, j*G + G) of element e with the loads issued ahead of the
// in-order adds, then the 8 partials are added in j order (fixed order:
// bit-reproducible).  The dtau partials are f64 and summed in f64.
constexpr int ATTN_RED_PARTS = 8;
__global__ __launch_bounds__(256) void attn_reduce_kernel(const double *dtau_part,
                                                          const float *drel_part, int n, int h,
                                                          int nrel, float *dtau, float *drel) {
    __shared__ double part[ATTN_RED_PARTS][32];
    const int el = threadIdx.x & 31, j = threadIdx.x >> 5;
    const int e = blockIdx.x * 32 + el;
    const int per = h * nrel;
    const bool is_rel = e < per, live = e < per + h;
    const long long stride = is_rel ? per : h;
    const int G = (n + ATTN_RED_PARTS - 1) / ATTN_RED_PARTS;
    const int i0 = j * G, i1 = min(n, i0 + G);
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
        for (int b = i0; b < i1; b++) s += src[(long long)b * stride];
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
            drel[e] += t;
        } else {
            double t = 0.0;
            for (int q = 0; q < ATTN_RED_PARTS; q++) {
                if (q * G >= n) break;
                t += part[q][el];
            }
            dtau[e - per] += (float)t;
        }
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

// tq or tk above 64: the composed path (batched GEMMs + row kernels).
bool large_desc(const rnn_attn_desc *d) { return d->tq > MAXT || d->tk > MAXT; }

int check_desc(rnn_ctx *ctx, const rnn_attn_desc *d) {
    if (!d) return rnn_fail(ctx, RNN_E_NULL, "attn: desc is null");
    if (!d->relidx) return rnn_fail(ctx, RNN_E_NULL, "attn: relidx is null");
    if (!d->h || !d->dh || !d->tq || !d->tk || !d->nrel)
        return rnn_fail(ctx, RNN_E_INVALID, "attn: zero dimension");
    if (d->dh > MAXDH && !large_desc(d))
        return rnn_fail(ctx, RNN_E_UNSUPPORTED,
                        "attn: dh=%u beyond the register-resident kernel (64) at tq=%u tk=%u",
                        d->dh, d->tq, d->tk);
    if ((size_t)d->tq * d->tk > ((size_t)1 << 26) || d->tk > (1u << 20))
        return rnn_fail(ctx, RNN_E_UNSUPPORTED, "attn: tq=%u tk=%u too large", d->tq, d->tk);
    // The table last uploaded was validated already.
    const size_t cnt = (size_t)d->tq * d->tk;
    if (ctx->rel_dev && ctx->rel_nrel == d->nrel && ctx->rel_host.size() == cnt &&
        std::memcmp(ctx->rel_host.data(), d->relidx, cnt * 4) == 0)
        return RNN_OK;
    for (size_t i = 0; i < cnt; i++)
        if (d->relidx[i] >= d->nrel) return rnn_fail(ctx, RNN_E_INVALID, "attn: relidx >= nrel");
    return RNN_OK;
}

// The lane-order table's place in the uploaded block: after relidx, rowptr
// and pos, rounded up to 16 bytes.
uint32_t *rperm_of(uint32_t *base, size_t cnt, size_t nrel) {
    return base + rnn_round_up(cnt + (nrel + 1) + cnt, 4);
}

// Uploads relidx, its inverse index (CSR over bias slots) and the lane-order
// table when the table differs from the last one.
int upload_rel(rnn_ctx *ctx, const rnn_attn_desc *d) {
    size_t cnt = (size_t)d->tq * d->tk;
    if (ctx->rel_dev && ctx->rel_nrel == d->nrel && ctx->rel_host.size() == cnt &&
        ctx->rel_tk == d->tk && std::memcmp(ctx->rel_host.data(), d->relidx, cnt * 4) == 0)
        return RNN_OK;
    const bool large = large_desc(d);
    // + the lane-order table (16-byte aligned) of the register-resident kernels
    size_t need = cnt + (d->nrel + 1) + cnt + (large ? 0 : 4096 + 4);
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
    // positions: offsets into the kernels' LDS [tq][LS] score tiles, or, on
    // the composed path, flat offsets q*tk + k into a [tq][tk] score matrix
    for (size_t i = 0; i < cnt; i++)
        pos[count[d->relidx[i]]++] =
            large ? (uint32_t)i : (uint32_t)((i / d->tk) * LS + i % d->tk);
    // relidx in the forward's lane order: entry (qi*2 + half)*32 + 16nt + v is
    // the slot of query qi, key key_of(nt, v, half); clamped into the table,
    // so every entry is a valid slot.
    if (!large) {
        uint32_t *rperm = rperm_of(h, cnt, d->nrel);
        for (int q = 0; q < 64; q++)
            for (int hf = 0; hf < 2; hf++)
                for (int nt = 0; nt < 2; nt++)
                    for (int v = 0; v < 16; v++) {
                        const int kj = 32 * nt + 8 * (v >> 2) + 4 * hf + (v & 3);
                        const int qc = std::min(q, (int)d->tq - 1);
                        const int kc = std::min(kj, (int)d->tk - 1);
                        rperm[(q * 2 + hf) * 32 + 16 * nt + v] =
                            d->relidx[(size_t)qc * d->tk + kc];
                    }
    }
    RNN_HIP(ctx, hipMemcpyAsync(ctx->rel_dev, h, need * 4, hipMemcpyHostToDevice, ctx->stream));
    ctx->rel_host.assign(d->relidx, d->relidx + cnt);
    ctx->rel_nrel = d->nrel;
    ctx->rel_tk = d->tk;
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
    g.DHP = d->dh <= 32 ? 32 : 64;
    size_t cnt = (size_t)d->tq * d->tk;
    g.relidx = ctx->rel_dev;
    g.rowptr = ctx->rel_dev + cnt;
    g.pos = ctx->rel_dev + cnt + d->nrel + 1;
    g.rperm = rperm_of(ctx->rel_dev, cnt, d->nrel);
}

inline bool al16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// float4 row loads need 16-byte aligned row starts for every image and head.
// VEC kernels: dh == DHP (no column padding) and float4-aligned rows.
bool use_vec(const AttnArgs &g) {
    return g.dh == g.DHP && g.qstride % 4 == 0 && g.qoff % 4 == 0 && al16(g.q) &&
           g.kvstride % 4 == 0 && g.koff % 4 == 0 && g.voff % 4 == 0 && al16(g.kv) &&
           (g.dout == nullptr || al16(g.dout));
}

// ---------------------------------------------------------------------------
// The composed path for tq or tk above 64 (the rustvit's cross-attention:
// tq 64, tk 256, dh 64, nrel 900).  The reference's own structure: per head, a
// batched GEMM over the images (strided Q/K/V through leading dimensions) for
// S = QK^T, a row kernel for the biased, masked softmax (P kept, as the
// backward reads it), a batched GEMM for O = PV; the backward likewise.

// Softmax of the rows of P in place (attn.rs:190-212): x = tau S + rel[idx],
// the diagonal -inf when masked; max, exp(x - max) (-inf -> 0), sum, times
// 1/sum.  One wave per row (image, head, query).
__global__ __launch_bounds__(256) void attn_softmax_rows_kernel(
    float *p, const float *__restrict__ tau, const float *__restrict__ rel,
    const uint32_t *__restrict__ relidx, long long rows, int h, int tq, int tk, int nrel,
    int mask) {
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

// drel[e] += sum over chunks of part[chunk][e], in chunk order.
__global__ __launch_bounds__(256) void attn_drel_sum_kernel(const float *__restrict__ part,
                                                            int nchunk, long long per,
                                                            float *drel) {
    const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
    if (e >= per) return;
    float s = 0.f;
    for (int k = 0; k < nchunk; k++) s += part[(long long)k * per + e];
    drel[e] += s;
}

size_t bwd_lds() { return (size_t)2 * 64 * LS * 4 + 2 * sizeof(double); }
size_t fwd_lds(size_t nrel) { return ((size_t)64 * LS + 4096 + nrel) * 4; }

bool lds_attr_done = false;
void set_lds_limits() {
    if (lds_attr_done) return;
    lds_attr_done = true;
    const void *ks[] = {(const void *)attn_bwd_kernel<32, false>,
                        (const void *)attn_bwd_kernel<32, true>,
                        (const void *)attn_bwd_kernel<64, false>,
                        (const void *)attn_bwd_kernel<64, true>,
                        (const void *)attn_fwd_kernel<32, false>,
                        (const void *)attn_fwd_kernel<32, true>,
                        (const void *)attn_fwd_kernel<64, false>,
                        (const void *)attn_fwd_kernel<64, true>};
    // a refusal here leaves the default limit, which the launch then reports
    for (const void *k : ks)
        if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) !=
            hipSuccess)
            (void)hipGetLastError();
}

// Core::forward on the composed path (see attn_softmax_rows_kernel).
int attn_forward_large(rnn_ctx *ctx, const rnn_attn_desc *d, size_t n, const float *q,
                       const float *kv, const float *tau, const float *rel, float *p, float *o) {
    const size_t tq = d->tq, tk = d->tk, dh = d->dh, h = d->h, c = h * dh;
    for (size_t hd = 0; hd < h; hd++) {
        int rc = rnn_gemm_launch_ld(ctx, n, tq, tk, dh, q + d->qoff + hd * dh, d->qstride,
                                    tq * d->qstride, 0, kv + d->koff + hd * dh, d->kvstride,
                                    tk * d->kvstride, 1, p + hd * tq * tk, tk, h * tq * tk, 0);
        if (rc) return rc;
    }
    const long long rows = (long long)n * h * tq;
    attn_softmax_rows_kernel<<<(unsigned)rnn_div_up((size_t)rows, 4), 256, 0, ctx->stream>>>(
        p, tau, rel, ctx->rel_dev, rows, (int)h, (int)tq, (int)tk, (int)d->nrel,
        d->mask_diag ? 1 : 0);
    RNN_LAUNCHED(ctx);
    for (size_t hd = 0; hd < h; hd++) {
        int rc = rnn_gemm_launch_ld(ctx, n, tq, dh, tk, p + hd * tq * tk, tk, h * tq * tk, 0,
                                    kv + d->voff + hd * dh, d->kvstride, tk * d->kvstride, 0,
                                    o + hd * dh, c, tq * c, 0);
        if (rc) return rc;
    }
    return RNN_OK;
}

// Core::backward on the composed path: dV = P^T dO, dP = dO V^T, the raw S
// recomputed, the row kernel (dS, tau dS, dtau shares), dtau and drel, then
// dQ = (tau dS) K and dK = (tau dS)^T Q; dq, dkv, dtau, drel accumulate.
int attn_backward_large(rnn_ctx *ctx, const rnn_attn_desc *d, size_t n, const float *q,
                        const float *kv, const float *tau, const float *p, const float *dout,
                        float *dq, float *dkv, float *dtau, float *drel) {
    const size_t tq = d->tq, tk = d->tk, dh = d->dh, h = d->h, c = h * dh;
    const size_t cnt = tq * tk, mat = n * h * cnt;
    const long long rows = (long long)n * h * tq;
    const size_t per = h * d->nrel;
    const size_t ipc = rnn_div_up(n, (size_t)16), nchunk = rnn_div_up(n, ipc);
    WsCarve cv;
    const size_t o1 = cv.take(mat * 4), o2 = cv.take(mat * 4), o3 = cv.take((size_t)rows * 8);
    const size_t o4 = cv.take(nchunk * per * 4);
    char *ws = (char *)rnn_workspace(ctx, cv.off);
    if (!ws) return RNN_E_NOMEM;
    float *s1 = (float *)(ws + o1), *s2 = (float *)(ws + o2);
    double *part = (double *)(ws + o3);
    float *rpart = (float *)(ws + o4);
    for (size_t hd = 0; hd < h; hd++) {
        // dV += P^T dO (attn.rs:262-270)
        int rc = rnn_gemm_launch_ld(ctx, n, tk, dh, tq, p + hd * cnt, tk, h * cnt, 1,
                                    dout + hd * dh, c, tq * c, 0, dkv + d->voff + hd * dh,
                                    d->kvstride, tk * d->kvstride, 1);
        if (rc) return rc;
        // dP = dO V^T (attn.rs:272-278)
        rc = rnn_gemm_launch_ld(ctx, n, tq, tk, dh, dout + hd * dh, c, tq * c, 0,
                                kv + d->voff + hd * dh, d->kvstride, tk * d->kvstride, 1,
                                s1 + hd * cnt, tk, h * cnt, 0);
        if (rc) return rc;
        // the raw scores again (attn.rs:292-300)
        rc = rnn_gemm_launch_ld(ctx, n, tq, tk, dh, q + d->qoff + hd * dh, d->qstride,
                                tq * d->qstride, 0, kv + d->koff + hd * dh, d->kvstride,
                                tk * d->kvstride, 1, s2 + hd * cnt, tk, h * cnt, 0);
        if (rc) return rc;
    }
    attn_dsoft_rows_kernel<<<(unsigned)rnn_div_up((size_t)rows, 4), 256, 0, ctx->stream>>>(
        p, s1, s2, tau, part, rows, (int)h, (int)tq, (int)tk);
    RNN_LAUNCHED(ctx);
    attn_head_sum_kernel<<<(unsigned)h, 256, 0, ctx->stream>>>(part, (long long)n, (int)h,
                                                              (int)tq, dtau);
    RNN_LAUNCHED(ctx);
    attn_drel_part_kernel<<<dim3((unsigned)rnn_div_up(per, (size_t)256), (unsigned)nchunk), 256,
                            0, ctx->stream>>>(s1, ctx->rel_dev + cnt,
                                              ctx->rel_dev + cnt + d->nrel + 1, (long long)n,
                                              (long long)ipc, (int)h, (int)d->nrel,
                                              (long long)cnt, rpart);
    RNN_LAUNCHED(ctx);
    attn_drel_sum_kernel<<<(unsigned)rnn_div_up(per, (size_t)256), 256, 0, ctx->stream>>>(
        rpart, (int)nchunk, (long long)per, drel);
    RNN_LAUNCHED(ctx);
    for (size_t hd = 0; hd < h; hd++) {
        // dQ += (tau dS) K (attn.rs:317-322)
        int rc = rnn_gemm_launch_ld(ctx, n, tq, dh, tk, s2 + hd * cnt, tk, h * cnt, 0,
                                    kv + d->koff + hd * dh, d->kvstride, tk * d->kvstride, 0,
                                    dq + d->qoff + hd * dh, d->qstride, tq * d->qstride, 1);
        if (rc) return rc;
        // dK += (tau dS)^T Q (attn.rs:324-330)
        rc = rnn_gemm_launch_ld(ctx, n, tk, dh, tq, s2 + hd * cnt, tk, h * cnt, 1,
                                q + d->qoff + hd * dh, d->qstride, tq * d->qstride, 0,
                                dkv + d->koff + hd * dh, d->kvstride, tk * d->kvstride, 1);
        if (rc) return rc;
    }
    return RNN_OK;
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
    rc = upload_rel(ctx, d);
    if (rc) return rc;
    if (large_desc(d)) return attn_forward_large(ctx, d, n, q, kv, tau, rel, p, o);
    set_lds_limits();
    AttnArgs g;
    fill_args(g, ctx, d, n);
    g.q = q;
    g.kv = kv;
    g.tau = tau;
    g.rel = rel;
    g.pout = p;
    g.o = o;
    const dim3 grid((unsigned)(n * d->h));
    const size_t lds = fwd_lds(d->nrel);
    if (lds > 160 * 1024)
        return rnn_fail(ctx, RNN_E_UNSUPPORTED, "attn: nrel %u bias slots exceed LDS", d->nrel);
    const bool vec = use_vec(g);
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(128), lds, ctx->stream, g); };
    if (g.DHP == 32)
        vec ? go(attn_fwd_kernel<32, true>) : go(attn_fwd_kernel<32, false>);
    else
        vec ? go(attn_fwd_kernel<64, true>) : go(attn_fwd_kernel<64, false>);
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
    rc = upload_rel(ctx, d);
    if (rc) return rc;
    if (large_desc(d))
        return attn_backward_large(ctx, d, n, q, kv, tau, p, dout, dq, dkv, dtau, drel);
    set_lds_limits();
    AttnArgs g;
    fill_args(g, ctx, d, n);
    const size_t tau_bytes = rnn_round_up(n * d->h * sizeof(double), 256);
    char *ws = (char *)rnn_workspace(ctx, tau_bytes + n * d->h * (size_t)d->nrel * sizeof(float));
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
    const dim3 grid((unsigned)(n * d->h));
    const bool vec = use_vec(g);
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, dim3(128), bwd_lds(), ctx->stream, g);
    };
    if (g.DHP == 32)
        vec ? go(attn_bwd_kernel<32, true>) : go(attn_bwd_kernel<32, false>);
    else
        vec ? go(attn_bwd_kernel<64, true>) : go(attn_bwd_kernel<64, false>);
    RNN_LAUNCHED(ctx);
    int tot = (int)(d->h * d->nrel + d->h);
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
