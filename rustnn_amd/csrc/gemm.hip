// Dense fp32 GEMM on gfx950 MFMA: matmul / gemm_small (batched) / matmul_dw
// (split-K) / Linear, plus the PackedA / PackedB debug exports.
//
// Reference: gemm.rs (6x16 AVX2 micro-kernel over KC=256 packed panels,
// parallel over 6-row C panels), linear.rs.  Here one workgroup owns a
// BM x BN tile of C; its 4 compute waves each own a (BM/2) x (BN/2) sub-tile
// made of 32x32 v_mfma_f32_32x32x2f32 accumulators.  The k order inside a
// block of 8 is permuted identically for A and B (step s of group g, lane
// half h  <->  k = 8g + 4h + s), so a k-contiguous operand gives a lane the
// values of 4 MFMA steps with one ds_read_b128.  Two ways to stage operands:
//   * gemm_dma_kernel (every operand whose 16-byte quads are whole): 4 more
//     waves DMA the slabs from HBM straight into a multi-stage LDS ring;
//   * gemm_kernel (any shape and alignment): the 4 waves load a slab into
//     registers and store it k-contiguous (16 k values + 4 pad floats a row)
//     into a double-buffered LDS tile.
#include "rnn_internal.h"

#include <algorithm>
#include <cstdlib>

namespace {

constexpr int BK = 16;
constexpr int LDK = BK + 4;  // padded row: conflict-free b128 reads/writes

struct GemmArgs {
    const float *a, *b;
    float *c;
    const float *bias;     // per output column, may be null
    long long stride_a, stride_b, stride_c;  // per z1 (z1 = z % zc1)
    // A second batch level: problem z covers z1 = z % zc1 and z2 = z / zc1,
    // operands at base + z1 * stride + z2 * stride2 (zc1 = the count and
    // stride2 = 0 for a plain batch).
    int zc1;
    long long stride_a2, stride_b2, stride_c2;
    int M, N;
    int kchunk, ktotal;    // problem z covers k = min(kchunk, ktotal - z*kchunk)
    int lda, ldb, ldc;
    int acc;               // C += result
    // Row sums of op(A) over this problem's k (gemm_dma_kernel with RS):
    // added into rsum_out[m] (one problem), or stored as f64 partials
    // rsum_part[z * M + m] (split-K problems, reduced in z order).
    float *rsum_out;
    double *rsum_part;
    // Residual epilogue (one problem, no acc): res[row][col] += (C l[col]) m
    // with m = res_mask[row >> res_shift] (no mask: 1), res laid out as C --
    // LayerScale, DropPath and add_ of a residual branch (vit.rs:155-176) in
    // residual_add_scaled's rounding order.
    float *res;
    const float *res_l, *res_mask;
    int res_shift;
};

// The residual branch fed by a GEMM's output (GemmArgs::res).
struct GemmRes {
    float *out;
    const float *l, *mask;
    int shift;
};

__device__ __forceinline__ float res_term(const GemmArgs &g, int row, int col, float val) {
    float t = val * g.res_l[col];
    if (g.res_mask) t = t * g.res_mask[row >> g.res_shift];
    return t;
}

__device__ __forceinline__ long long zoff(const GemmArgs &g, long long z, long long s1,
                                          long long s2) {
    const unsigned zu = (unsigned)z, c1 = (unsigned)g.zc1;  // z < 65536
    return (long long)(zu % c1) * s1 + (long long)(zu / c1) * s2;
}

// 4 consecutive elements starting at p[0], p[step], ... with bounds
// (count valid), zero elsewhere.
__device__ __forceinline__ float4 load4(const float *p, long long step, int valid, bool vec) {
    float4 r = make_float4(0.f, 0.f, 0.f, 0.f);
    if (vec && step == 1 && valid >= 4) return *reinterpret_cast<const float4 *>(p);
    if (valid > 0) r.x = p[0];
    if (valid > 1) r.y = p[step];
    if (valid > 2) r.z = p[2 * step];
    if (valid > 3) r.w = p[3 * step];
    return r;
}

// Loads the BMxBK slab of an operand as k-quads.  TRANS=false: operand stored
// [rows][k] (row-major, ld = row length); TRANS=true: stored [k][rows].
template <int BM, bool TRANS, bool VEC>
struct Slab {
    static constexpr int Q = BM * 4 / 256;  // quads per thread
    float4 r[Q];
    __device__ __forceinline__ void load(const float *base, int ld, int row0, int rows, int k0,
                                         int kz, int tid) {
#pragma unroll
        for (int j = 0; j < Q; j++) {
            int idx = tid + 256 * j;
            int m, kq;
            if (!TRANS) {
                kq = idx & 3;
                m = idx >> 2;
            } else {
                m = idx % BM;
                kq = idx / BM;
            }
            int row = row0 + m, k = k0 + 4 * kq;
            int valid = (row < rows) ? min(4, kz - k) : 0;
            if (!TRANS)
                r[j] = load4(base + (long long)row * ld + k, 1, valid, VEC);
            else
                r[j] = load4(base + (long long)k * ld + row, ld, valid, false);
        }
    }
    __device__ __forceinline__ void store(float *lds, int tid) const {
#pragma unroll
        for (int j = 0; j < Q; j++) {
            int idx = tid + 256 * j;
            int m, kq;
            if (!TRANS) {
                kq = idx & 3;
                m = idx >> 2;
            } else {
                m = idx % BM;
                kq = idx / BM;
            }
            *reinterpret_cast<float4 *>(lds + m * LDK + 4 * kq) = r[j];
        }
    }
};

// The MFMA main loop of one BM x BN tile of C = op(A) op(B) over kz values of
// k, rows m0.. of op(A) and columns n0.. of op(B); leaves the tile in acc.
template <int BM, int BN, bool AT, bool BT, bool VEC>
struct GemmTile {
    static constexpr int WTM = BM / 2, WTN = BN / 2, TM = WTM / 32, TN = WTN / 32;
    f32x16 acc[TM][TN];

    __device__ __forceinline__ void run(const float *A, int lda, int M, const float *B, int ldb,
                                        int N, int kz, int m0, int n0, float (*As)[BM * LDK],
                                        float (*Bs)[BN * LDK]) {
        const int tid = threadIdx.x, lane = tid & 63, wave = wave_index();
        const int wm = wave >> 1, wn = wave & 1;
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int v = 0; v < 16; v++) acc[i][j][v] = 0.f;

        Slab<BM, AT, VEC> sa;
        Slab<BN, !BT, VEC> sb;  // B^T stored [n][k] is the "rows = n" layout
        const int nk = (kz + BK - 1) / BK;
        if (nk > 0) {
            sa.load(A, lda, m0, M, 0, kz, tid);
            sb.load(B, ldb, n0, N, 0, kz, tid);
            sa.store(As[0], tid);
            sb.store(Bs[0], tid);
        }
        __syncthreads();
        const int lr = lane & 31, lh = lane >> 5;
        for (int it = 0; it < nk; it++) {
            const int buf = it & 1;
            if (it + 1 < nk) {
                sa.load(A, lda, m0, M, (it + 1) * BK, kz, tid);
                sb.load(B, ldb, n0, N, (it + 1) * BK, kz, tid);
            }
#pragma unroll
            for (int gk = 0; gk < 2; gk++) {
                float4 af[TM], bf[TN];
#pragma unroll
                for (int i = 0; i < TM; i++)
                    af[i] = *reinterpret_cast<const float4 *>(
                        &As[buf][(wm * WTM + i * 32 + lr) * LDK + 8 * gk + 4 * lh]);
#pragma unroll
                for (int j = 0; j < TN; j++)
                    bf[j] = *reinterpret_cast<const float4 *>(
                        &Bs[buf][(wn * WTN + j * 32 + lr) * LDK + 8 * gk + 4 * lh]);
#pragma unroll
                for (int s = 0; s < 4; s++)
#pragma unroll
                    for (int i = 0; i < TM; i++)
#pragma unroll
                        for (int j = 0; j < TN; j++)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][s], bf[j][s],
                                                                             acc[i][j], 0, 0, 0);
            }
            if (it + 1 < nk) {
                sa.store(As[buf ^ 1], tid);
                sb.store(Bs[buf ^ 1], tid);
            }
            __syncthreads();
        }
    }

    // Element v of accumulator (i, j) of this lane sits at tile row
    // wm*WTM + 32i + 8(v/4) + 4(lane/32) + v%4, column wn*WTN + 32j + lane%32
    // (the 32x32 MFMA accumulator layout).
    template <typename F>
    __device__ __forceinline__ void each(F f) const {
        const int lane = threadIdx.x & 63, wave = wave_index();
        const int wm = wave >> 1, wn = wave & 1, lr = lane & 31, lh = lane >> 5;
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int v = 0; v < 16; v++)
                    f(wm * WTM + i * 32 + 8 * (v >> 2) + 4 * lh + (v & 3), wn * WTN + j * 32 + lr,
                      acc[i][j][v]);
    }
};

// ---------------------------------------------------------------------------
// Direct-to-LDS variant.  Operand slabs go from HBM straight into an NS-stage
// LDS ring by buffer_load_dwordx4 ... lds (16 bytes per lane, no registers,
// no LDS writes by the waves); stage it + NS - 1 is in flight while stage it
// is multiplied.  Each operand keeps the layout it has in memory:
//   * k-contiguous (A [m][k], B^T [n][k]): [row][BK] with the 16-byte quad q
//     of row r at position q ^ kswz(r), so the ds_read_b128 of 8 (or 16)
//     consecutive rows at one quad hit distinct banks;
//   * row-contiguous (A^T [k][m], B [k][n]): [BK][rows] as stored, read one
//     float per MFMA step (32 consecutive floats per half-wave).
// k order inside a stage matches the register-staged kernel: step s of
// group g, lane half h <-> k = 8g + 4h + s.  Eligible when every 16-byte quad
// is either wholly inside the operand or wholly outside (rows and k multiples
// of 4 where they run along a quad, 16-byte aligned bases): a quad outside
// the k range reads zero through an out-of-range offset; rows beyond M / N
// only feed C rows / columns that are never stored.

// s_waitcnt with vmcnt <= N, other counters not waited on (vmcnt bits 3:0 and
// 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Quad position swizzle of a k-contiguous row: conflict-free b128 reads for
// both 8-lane (32-bank) and 16-lane (64-bank) LDS read phases.
template <int BK>
__device__ __forceinline__ int kswz(int r) {
    if constexpr (BK == 32)
        return (r ^ (r >> 3)) & 7;
    else
        return ((r >> 1) ^ (r >> 2)) & 3;
}

template <int R, int BK, bool KMAJOR>
struct DmaOperand {
    static constexpr int WORDS = R * BK;             // LDS floats per stage
    static constexpr int PER = WORDS / 4 / 256;      // dwordx4 DMAs per thread
    static_assert(WORDS % 1024 == 0, "whole DMA rows");

    // Issues this thread's DMAs of rows r0.. (KMAJOR) or columns r0.. of
    // k values k0 .. k0 + BK (of kz) into lds.
    __device__ __forceinline__ static void issue(__amdgpu_buffer_rsrc_t rs, int ld, int rows,
                                                 int r0, int k0, int kz, float *lds, int wave,
                                                 int lane) {
#pragma unroll
        for (int u = 0; u < PER; u++) {
            const int c0 = (u * 4 + wave) * 64;  // first quad of this wave instruction
            const int j = c0 + lane;
            uint32_t off;
            if (KMAJOR) {
                constexpr int QPR = BK / 4;
                const int r = j / QPR, q = (j % QPR) ^ kswz<BK>(r);
                const int row = r0 + r, k = k0 + 4 * q;
                off = (row < rows && k < kz) ? (uint32_t)(row * ld + k) * 4u : DMA_OOB;
            } else {
                constexpr int QPR = R / 4;
                const int kr = j / QPR, col = r0 + (j % QPR) * 4, k = k0 + kr;
                off = (k < kz && col < rows) ? (uint32_t)(k * ld + col) * 4u : DMA_OOB;
            }
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(lds + 4 * c0), 16, off, 0, 0,
                                                     0);
        }
    }

    // The operand values of MFMA steps 0..3 of group g for tile row (or
    // column) `row` and lane half h.
    __device__ __forceinline__ static f32x4 frag(const float *lds, int row, int g, int h) {
        if (KMAJOR) {
            const int q = (2 * g + h) ^ kswz<BK>(row);
            return *reinterpret_cast<const f32x4 *>(lds + row * BK + 4 * q);
        } else {
            const float *p = lds + (8 * g + 4 * h) * R + row;
            f32x4 v;
            v[0] = p[0];
            v[1] = p[R];
            v[2] = p[2 * R];
            v[3] = p[3 * R];
            return v;
        }
    }
};

// One BM x BN tile of C = op(A) op(B) over kz values of k by 8 waves.
// Waves 0..3 multiply (a 2 x 2 grid of (BM/2) x (BN/2) sub-tiles); waves
// 4..7 only issue the DMAs, a whole stage at a time, so the compute waves
// never wait on the memory pipeline.  One barrier per stage: when it
// completes, stage it has landed (each producer waited for its own DMAs) and
// every compute wave is done with stage it - 1, whose buffer the producers
// then refill with stage it + NS - 1.  A wave with a single 32 x 32 block
// alternates two accumulators so that consecutive MFMAs are independent.
template <int BM, int BN, int BK, int NS, bool AT, bool BT>
struct DmaTile {
    using OA = DmaOperand<BM, BK, !AT>;
    using OB = DmaOperand<BN, BK, BT>;
    static constexpr int STAGE = OA::WORDS + OB::WORDS;
    static constexpr size_t LDS_BYTES = (size_t)NS * STAGE * 4;
    static constexpr int WTM = BM / 2, WTN = BN / 2, TM = WTM / 32, TN = WTN / 32;
    static constexpr int NACC = TM * TN == 1 ? 2 : 1;
    f32x16 acc[TM][TN][NACC];
    // With rsum, the f64 sums of the A values this lane multiplies: row
    // wm*WTM + 32i + lr at k = 8g + 4lh + s, stage by stage in k order.
    double rs[TM];

    // Producer waves return false once their last DMA is issued; compute
    // waves return true with the tile in acc.  A, B: this problem's operands
    // (extents below 2^31 bytes, checked by the host).
    __device__ __forceinline__ bool run(const float *A, int lda, int M, const float *B, int ldb,
                                        int N, int kz, int m0, int n0, bool rsum, float *lds) {
        const int lane = threadIdx.x & 63, wave = wave_index();
        const int nk = (kz + BK - 1) / BK;
        if (wave >= 4) {
            const int pw = wave - 4;
            const uint32_t abytes = (uint32_t)((AT ? (long long)kz * lda : (long long)M * lda) * 4);
            const uint32_t bbytes = (uint32_t)((BT ? (long long)N * ldb : (long long)kz * ldb) * 4);
            const __amdgpu_buffer_rsrc_t ra = make_rsrc(A, abytes), rb = make_rsrc(B, bbytes);
            auto issue = [&](int st) {
                float *buf = lds + (st % NS) * STAGE;
                OA::issue(ra, lda, M, m0, st * BK, kz, buf, pw, lane);
                OB::issue(rb, ldb, N, n0, st * BK, kz, buf + OA::WORDS, pw, lane);
            };
#pragma unroll
            for (int st = 0; st < NS - 1; st++)
                if (st < nk) issue(st);
            for (int it = 0; it < nk; it++) {
                if (it + NS - 2 < nk)
                    wait_vmcnt<(NS - 2) * (OA::PER + OB::PER)>();
                else
                    wait_vmcnt<0>();
                // a bare barrier: __syncthreads()'s release fence would also
                // wait for the DMAs of the later stages still in flight
                asm volatile("" ::: "memory");
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
                if (it + NS - 1 < nk) issue(it + NS - 1);
            }
            return false;
        }
        const int wm = wave >> 1, wn = wave & 1, lr = lane & 31, lh = lane >> 5;
#pragma unroll
        for (int i = 0; i < TM; i++) rs[i] = 0.0;
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int a = 0; a < NACC; a++)
#pragma unroll
                    for (int v = 0; v < 16; v++) acc[i][j][a][v] = 0.f;
        for (int it = 0; it < nk; it++) {
            __syncthreads();
            const float *As = lds + (it % NS) * STAGE, *Bs = As + OA::WORDS;
            f32x4 af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) af[i] = OA::frag(As, wm * WTM + i * 32 + lr, 0, lh);
#pragma unroll
            for (int j = 0; j < TN; j++) bf[j] = OB::frag(Bs, wn * WTN + j * 32 + lr, 0, lh);
#pragma unroll
            for (int gk = 0; gk < BK / 8; gk++) {
                f32x4 an[TM], bn[TN];
                if (gk + 1 < BK / 8) {
#pragma unroll
                    for (int i = 0; i < TM; i++)
                        an[i] = OA::frag(As, wm * WTM + i * 32 + lr, gk + 1, lh);
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        bn[j] = OB::frag(Bs, wn * WTN + j * 32 + lr, gk + 1, lh);
                }
                // keep the next group's reads ahead of this group's MFMAs
                __builtin_amdgcn_sched_barrier(0);
                if (rsum) {
#pragma unroll
                    for (int i = 0; i < TM; i++)
#pragma unroll
                        for (int s = 0; s < 4; s++) rs[i] += (double)af[i][s];
                }
#pragma unroll
                for (int s = 0; s < 4; s++)
#pragma unroll
                    for (int i = 0; i < TM; i++)
#pragma unroll
                        for (int j = 0; j < TN; j++)
                            acc[i][j][s % NACC] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                                af[i][s], bf[j][s], acc[i][j][s % NACC], 0, 0, 0);
                if (gk + 1 < BK / 8) {
#pragma unroll
                    for (int i = 0; i < TM; i++) af[i] = an[i];
#pragma unroll
                    for (int j = 0; j < TN; j++) bf[j] = bn[j];
                }
            }
        }
        return true;
    }

    // f(r, c, v) for each element of the tile this compute lane holds (tile
    // row r = wm*WTM + 32i + 8(v/4) + 4(lane/32) + v%4, column wn*WTN + 32j +
    // lane%32: the 32x32 MFMA accumulator layout).
    template <typename F>
    __device__ __forceinline__ void each(F f) const {
        const int lane = threadIdx.x & 63, wave = wave_index();
        const int wm = wave >> 1, wn = wave & 1, lr = lane & 31, lh = lane >> 5;
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    float val = acc[i][j][0][v];
                    if (NACC == 2) val += acc[i][j][NACC - 1][v];
                    f(wm * WTM + i * 32 + 8 * (v >> 2) + 4 * lh + (v & 3), wn * WTN + j * 32 + lr,
                      val);
                }
    }
};

template <int BM, int BN, int BK, int NS, bool AT, bool BT, bool RS>
__global__ __launch_bounds__(512) void gemm_dma_kernel(GemmArgs g) {
    extern __shared__ float lds[];
    using Tile = DmaTile<BM, BN, BK, NS, AT, BT>;
    const long long z = blockIdx.z;
    const int kz = min(g.kchunk, g.ktotal - (int)z * g.kchunk);
    // XCD-aware tile order, as in gemm_kernel
    const int gx = gridDim.x, T = gx * gridDim.y;
    const int L = blockIdx.y * gx + blockIdx.x;
    const int per = T >> 3, rem = T & 7, xcd = L & 7, loc = L >> 3;
    const int tl = xcd < rem ? xcd * (per + 1) + loc : rem * (per + 1) + (xcd - rem) * per + loc;
    const int m0 = (tl / gx) * BM, n0 = (tl % gx) * BN;
    // RS: the compute waves of the first column tile also sum A's values
    const int lane = threadIdx.x & 63, wave = wave_index(), lr = lane & 31, lh = lane >> 5;
    const bool rsum = RS && n0 == 0 && (wave & 1) == 0;
    Tile t;
    if (!t.run(g.a + zoff(g, z, g.stride_a, g.stride_a2), g.lda, g.M,
               g.b + zoff(g, z, g.stride_b, g.stride_b2), g.ldb, g.N, kz, m0, n0,
               rsum, lds))
        return;
    if (rsum) {
#pragma unroll
        for (int i = 0; i < Tile::TM; i++) {
            // the two lane halves' sums, added in half order on both halves
            const double o = __shfl_xor(t.rs[i], 32, 64);
            const double s = lh == 0 ? t.rs[i] + o : o + t.rs[i];
            const int row = m0 + (wave >> 1) * Tile::WTM + i * 32 + lr;
            if (lh == 0 && row < g.M) {
                if (g.rsum_part)
                    g.rsum_part[z * g.M + row] = s;
                else
                    g.rsum_out[row] += (float)s;
            }
        }
    }
    float *Cp = g.c + zoff(g, z, g.stride_c, g.stride_c2);
    // The epilogue.  Every value a store needs -- the bias and the residual's
    // LayerScale factor (one per tile column of the lane), the old C (acc)
    // or the residual's old value and mask (res) -- is loaded before the
    // stores, eight elements at a time, so the loads are in flight together
    // instead of each waiting behind the stores before it (eight: the
    // registers keep three 64 x 64 workgroups a CU).  Element (i, j, v):
    // tile row wm*WTM + 32i + 8(v/4) + 4(lane/32) + v%4, column
    // wn*WTN + 32j + lane%32 (the 32x32 MFMA accumulator layout).
    const bool acc = g.acc != 0, res = g.res != nullptr, bias = g.bias != nullptr;
    const int wm = wave >> 1, wn = wave & 1;
    if (!acc && !res) {
        // (the plain store, written this way, measured faster than the
        // loop below with the bias preloaded: 5.84 vs 5.92 ms rustvit step)
        t.each([&](int r, int c, float val) {
            const int row = m0 + r, col = n0 + c;
            if (row < g.M && col < g.N) {
                if (bias) val += g.bias[col];
                Cp[(long long)row * g.ldc + col] = val;
            }
        });
        return;
    }
#pragma unroll
    for (int j = 0; j < Tile::TN; j++) {
        const int col = n0 + wn * Tile::WTN + j * 32 + lr, colc = min(col, g.N - 1);
        const float bj = bias ? g.bias[colc] : 0.f, lj = res ? g.res_l[colc] : 0.f;
#pragma unroll
        for (int i = 0; i < Tile::TM; i++)
#pragma unroll
            for (int h = 0; h < 16; h += 8) {
                float old[8], mv[8];
                if (acc || res) {
#pragma unroll
                    for (int u = 0; u < 8; u++) {
                        const int v = h + u;
                        const int row = m0 + wm * Tile::WTM + i * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
                        const long long o = (long long)min(row, g.M - 1) * g.ldc + colc;
                        old[u] = acc ? Cp[o] : g.res[o];
                        mv[u] = (res && g.res_mask) ? g.res_mask[min(row, g.M - 1) >> g.res_shift]
                                                    : 1.0f;
                    }
                }
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const int v = h + u;
                    const int row = m0 + wm * Tile::WTM + i * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
                    if (row < g.M && col < g.N) {
                        float val = t.acc[i][j][0][v];
                        if constexpr (Tile::NACC == 2) val += t.acc[i][j][1][v];
                        if (bias) val += bj;
                        const long long o = (long long)row * g.ldc + col;
                        Cp[o] = acc ? old[u] + val : val;
                        if (res) {
                            float tr = val * lj;
                            if (g.res_mask) tr = tr * mv[u];
                            g.res[o] = old[u] + tr;
                        }
                    }
                }
            }
    }
}

template <int BM, int BN, bool AT, bool BT, bool VEC>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs g) {
    __shared__ float As[2][BM * LDK];
    __shared__ float Bs[2][BN * LDK];
    const long long z = blockIdx.z;
    const float *A = g.a + zoff(g, z, g.stride_a, g.stride_a2);
    const float *B = g.b + zoff(g, z, g.stride_b, g.stride_b2);
    float *Cp = g.c + zoff(g, z, g.stride_c, g.stride_c2);
    const int kz = min(g.kchunk, g.ktotal - (int)z * g.kchunk);
    // XCD-aware tile order: workgroup L of a problem runs on XCD L % 8, so
    // XCD x takes the x-th contiguous run of tiles (row-major over (m, n)):
    // the tiles that share an A panel meet in one L2 (16384x768x256: 86 ->
    // 89 TFLOP/s)
    const int gx = gridDim.x, T = gx * gridDim.y;
    const int L = blockIdx.y * gx + blockIdx.x;
    const int per = T >> 3, rem = T & 7, xcd = L & 7, loc = L >> 3;
    const int tl = xcd < rem ? xcd * (per + 1) + loc : rem * (per + 1) + (xcd - rem) * per + loc;
    const int m0 = (tl / gx) * BM, n0 = (tl % gx) * BN;
    GemmTile<BM, BN, AT, BT, VEC> t;
    t.run(A, g.lda, g.M, B, g.ldb, g.N, kz, m0, n0, As, Bs);
    t.each([&](int r, int c, float val) {
        const int row = m0 + r, col = n0 + c;
        if (row < g.M && col < g.N) {
            if (g.bias) val += g.bias[col];
            float *cp = Cp + (long long)row * g.ldc + col;
            if (g.acc) val = *cp + val;
            *cp = val;
            if (g.res) {
                float *rp = g.res + (long long)row * g.ldc + col;
                *rp = *rp + res_term(g, row, col, val);
            }
        }
    });
}

// One 64 x 64 tile of a grouped Newton-Schulz problem with operand layout
// (AT, BT); stores C = alpha E + beta (A op(B)) when E is set, else the
// product, and for a symmetric problem the mirrored tile too.
template <bool AT, bool BT, bool VEC>
__device__ __forceinline__ void ns_tile(const NsGemmProb &p, uint32_t z, int ti, int tj,
                                        float alpha, float beta, float (*As)[64 * LDK],
                                        float (*Bs)[64 * LDK]) {
#pragma clang fp contract(off)
    const int m0 = ti * 64, n0 = tj * 64;
    GemmTile<64, 64, AT, BT, VEC> t;
    t.run(p.a + z * p.stride_a, p.lda, p.M, p.b + z * p.stride_b, p.ldb, p.N, p.K, m0, n0, As,
          Bs);
    float *Cp = p.c + z * p.stride_c;
    const float *Ep = p.e ? p.e + z * p.stride_c : nullptr;
    const bool mirror = p.sym && ti != tj;
    t.each([&](int rr, int cc, float val) {
        const int row = m0 + rr, col = n0 + cc;
        if (row < p.M && col < p.N) {
            const long long o = (long long)row * p.ldc + col;
            const float v = Ep ? alpha * Ep[o] + beta * val : val;
            Cp[o] = v;
            if (mirror) Cp[(long long)col * p.ldc + row] = v;
        }
    });
}

// Grouped GEMMs of the Newton-Schulz iteration: problem p (found from the
// block index) is a batch of cnt same-shape products; a symmetric problem
// (C = C^T, M = N) computes the tiles on and above the diagonal only.
template <bool VEC>
__global__ __launch_bounds__(256) void ns_gemm_kernel(const NsGemmProb *__restrict__ probs,
                                                      int nprob, float alpha, float beta) {
    __shared__ float As[2][64 * LDK];
    __shared__ float Bs[2][64 * LDK];
    int lo = 0, hi = nprob - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (probs[mid].tile0 <= blockIdx.x)
            lo = mid;
        else
            hi = mid - 1;
    }
    const NsGemmProb p = probs[lo];
    const uint32_t local = blockIdx.x - p.tile0;
    const uint32_t z = local / p.tmn;
    uint32_t r = local - z * p.tmn;
    int ti, tj;
    if (p.sym) {
        // row ti of the upper triangle holds tn - ti tiles
        ti = 0;
        while (r >= p.tn - (uint32_t)ti) r -= p.tn - (uint32_t)ti++;
        tj = ti + (int)r;
    } else {
        ti = (int)(r / p.tn);
        tj = (int)(r % p.tn);
    }
    if (p.lay == NS_LAY_NT)
        ns_tile<false, true, VEC>(p, z, ti, tj, alpha, beta, As, Bs);
    else if (p.lay == NS_LAY_TN)
        ns_tile<true, false, VEC>(p, z, ti, tj, alpha, beta, As, Bs);
    else
        ns_tile<false, false, VEC>(p, z, ti, tj, alpha, beta, As, Bs);
}

// ns_gemm_kernel on the direct-to-LDS tile (every operand of every problem
// of the launch with whole 16-byte quads): 8 waves, 64 x 64 tiles.
template <bool AT, bool BT>
__device__ __forceinline__ void ns_tile_dma(const NsGemmProb &p, uint32_t z, int ti, int tj,
                                            float alpha, float beta, float *lds) {
#pragma clang fp contract(off)
    using Tile = DmaTile<64, 64, 32, 3, AT, BT>;
    const int m0 = ti * 64, n0 = tj * 64;
    Tile t;
    if (!t.run(p.a + z * p.stride_a, p.lda, p.M, p.b + z * p.stride_b, p.ldb, p.N, p.K, m0, n0,
               false, lds))
        return;
    float *Cp = p.c + z * p.stride_c;
    const float *Ep = p.e ? p.e + z * p.stride_c : nullptr;
    const bool mirror = p.sym && ti != tj;
    t.each([&](int rr, int cc, float val) {
        const int row = m0 + rr, col = n0 + cc;
        if (row < p.M && col < p.N) {
            const long long o = (long long)row * p.ldc + col;
            const float v = Ep ? alpha * Ep[o] + beta * val : val;
            Cp[o] = v;
            if (mirror) Cp[(long long)col * p.ldc + row] = v;
        }
    });
}

constexpr size_t NS_DMA_LDS = DmaTile<64, 64, 32, 3, false, false>::LDS_BYTES;

__global__ __launch_bounds__(512) void ns_gemm_dma_kernel(const NsGemmProb *__restrict__ probs,
                                                          int nprob, float alpha, float beta) {
    extern __shared__ float lds[];
    int lo = 0, hi = nprob - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (probs[mid].tile0 <= blockIdx.x)
            lo = mid;
        else
            hi = mid - 1;
    }
    const NsGemmProb p = probs[lo];
    const uint32_t local = blockIdx.x - p.tile0;
    const uint32_t z = local / p.tmn;
    uint32_t r = local - z * p.tmn;
    int ti, tj;
    if (p.sym) {
        ti = 0;
        while (r >= p.tn - (uint32_t)ti) r -= p.tn - (uint32_t)ti++;
        tj = ti + (int)r;
    } else {
        ti = (int)(r / p.tn);
        tj = (int)(r % p.tn);
    }
    if (p.lay == NS_LAY_NT)
        ns_tile_dma<false, true>(p, z, ti, tj, alpha, beta, lds);
    else if (p.lay == NS_LAY_TN)
        ns_tile_dma<true, false>(p, z, ti, tj, alpha, beta, lds);
    else
        ns_tile_dma<false, false>(p, z, ti, tj, alpha, beta, lds);
}

__global__ void fill_kernel(float *p, long long n, float v) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long st = (long long)gridDim.x * blockDim.x;
    for (; i < n; i += st) p[i] = v;
}

// out[e] (+)= sum_z part[z*len + e], z in order (deterministic split-K
// reduce).  Loads go out 8 at a time ahead of the in-order adds.
__global__ void splitk_reduce_kernel(const float *part, int nz, long long len, float *out,
                                     int accumulate, const double *rpart, int rlen, float *rout) {
    long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= len) {
        // the split-K row sums of op(A): rout[m] += sum_z rpart[z][m], z in order
        const long long m = e - len;
        if (!rpart || m >= rlen) return;
        rnn_rows64_sum(rpart, nz, rlen, rout, m);
        return;
    }
    rnn_chunk_sum(part, nz, len, out, accumulate, e);
}

// PackedA::pack / pack_t layout (gemm.rs:54-113): element e of block q =
// panel i, position p*MR + r -> A[i*MR + r][q*KC + p].
__global__ void pack_a_kernel(const float *a, long long m, long long k, int transposed, float *out,
                              long long mpad, long long total) {
    const int MR = 6, KC = 256;
    long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= total) return;
    long long q = e / (KC * mpad), rem = e % (KC * mpad);
    long long kc = min((long long)KC, k - q * KC);
    if (rem >= kc * mpad) return;  // never written by the reference
    long long i = rem / (kc * MR), w = rem % (kc * MR), p = w / MR, r = w % MR;
    long long row = i * MR + r, col = q * KC + p;
    float v = 0.f;
    if (row < m) v = transposed ? a[col * m + row] : a[row * k + col];
    out[e] = v;
}

// PackedB::pack / pack_t layout (gemm.rs:340-400): panel j, position p*NR + t
// -> B[q*KC + p][j*NR + t].
__global__ void pack_b_kernel(const float *b, long long n, long long k, int transposed, float *out,
                              long long npad, long long total) {
    const int NR = 16, KC = 256;
    long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= total) return;
    long long q = e / (KC * npad), rem = e % (KC * npad);
    long long kc = min((long long)KC, k - q * KC);
    if (rem >= kc * npad) return;
    long long j = rem / (kc * NR), w = rem % (kc * NR), p = w / NR, t = w % NR;
    long long col = j * NR + t, row = q * KC + p;
    float v = 0.f;
    if (col < n) v = transposed ? b[col * k + row] : b[row * n + col];
    out[e] = v;
}

template <int BM, int BN, bool AT, bool BT>
int launch_t(rnn_ctx *ctx, const GemmArgs &g, int count, bool vec) {
    dim3 grid((g.N + BN - 1) / BN, (g.M + BM - 1) / BM, count);
    if (vec)
        hipLaunchKernelGGL((gemm_kernel<BM, BN, AT, BT, true>), grid, dim3(256), 0, ctx->stream, g);
    else
        hipLaunchKernelGGL((gemm_kernel<BM, BN, AT, BT, false>), grid, dim3(256), 0, ctx->stream, g);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

template <int BM, int BN, int BK, int NS, bool AT, bool BT, bool RS>
int launch_dma_t(rnn_ctx *ctx, const GemmArgs &g, int count) {
    constexpr size_t lds = DmaTile<BM, BN, BK, NS, AT, BT>::LDS_BYTES;
    static bool attr = false;
    if (!attr) {
        attr = true;
        (void)hipFuncSetAttribute((const void *)gemm_dma_kernel<BM, BN, BK, NS, AT, BT, RS>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    }
    dim3 grid((g.N + BN - 1) / BN, (g.M + BM - 1) / BM, count);
    hipLaunchKernelGGL((gemm_dma_kernel<BM, BN, BK, NS, AT, BT, RS>), grid, dim3(512), lds,
                       ctx->stream, g);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

// The row sums of op(A) ride along only in the weight-gradient layout (A^T B).
template <int BM, int BN, int BK, int NS>
int launch_dma_bm(rnn_ctx *ctx, const GemmArgs &g, int count, bool at, bool bt) {
    if (g.rsum_out || g.rsum_part) {
        if (!at || bt) return rnn_fail(ctx, RNN_E_INVALID, "gemm: row sums need the A^T B layout");
        return launch_dma_t<BM, BN, BK, NS, true, false, true>(ctx, g, count);
    }
    if (!at && !bt) return launch_dma_t<BM, BN, BK, NS, false, false, false>(ctx, g, count);
    if (!at && bt) return launch_dma_t<BM, BN, BK, NS, false, true, false>(ctx, g, count);
    if (at && !bt) return launch_dma_t<BM, BN, BK, NS, true, false, false>(ctx, g, count);
    return launch_dma_t<BM, BN, BK, NS, true, true, false>(ctx, g, count);
}

template <int BM, int BN>
int launch_bm(rnn_ctx *ctx, const GemmArgs &g, int count, bool at, bool bt, bool vec) {
    if (!at && !bt) return launch_t<BM, BN, false, false>(ctx, g, count, vec);
    if (!at && bt) return launch_t<BM, BN, false, true>(ctx, g, count, vec);
    if (at && !bt) return launch_t<BM, BN, true, false>(ctx, g, count, vec);
    return launch_t<BM, BN, true, true>(ctx, g, count, vec);
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

// Whether every operand quad of the direct-to-LDS kernel is wholly inside or
// wholly outside its operand, and every problem's operand spans under 2^31
// bytes (buffer offsets).
static bool dma_ok(size_t count, size_t m, size_t n, size_t kchunk, size_t ktotal, const float *a,
                   size_t stride_a, int lda, int at, const float *b, size_t stride_b, int ldb,
                   int bt) {
    const size_t lim = 0x7FFF0000u / 4;
    const size_t kz = std::min(kchunk, ktotal);
    auto aligned = [](const void *p, size_t stride, int ld) {
        return ((uintptr_t)p & 15) == 0 && stride % 4 == 0 && ld % 4 == 0;
    };
    if (!aligned(a, stride_a, lda) || !aligned(b, stride_b, ldb)) return false;
    // quads run along k for k-contiguous operands, along m / n otherwise
    if ((!at || bt) && (kchunk % 4 || ktotal % 4)) return false;
    if (at && m % 4) return false;
    if (!bt && n % 4) return false;
    const size_t ea = at ? kz * (size_t)lda : m * (size_t)lda;
    const size_t eb = bt ? n * (size_t)ldb : kz * (size_t)ldb;
    return ea < lim && eb < lim;
}

// Enqueues `count` GEMMs C_z = op(A_z) op(B_z) (+C_z) (+bias) with problem z
// covering k = min(kchunk, ktotal - z*kchunk) (kchunk = k for plain batches).
bool ns_dma_ok(const NsGemmProb &p, size_t count) {
    const int at = p.lay == NS_LAY_TN, bt = p.lay == NS_LAY_NT;
    return dma_ok(count, (size_t)p.M, (size_t)p.N, (size_t)p.K, (size_t)p.K, p.a,
                  (size_t)p.stride_a, p.lda, at, p.b, (size_t)p.stride_b, p.ldb, bt);
}

static bool dma_enabled() {
    static const bool on = getenv("RNN_GEMM_NODMA") == nullptr;
    return on;
}

// Whether C += A^T B (A [k x m], B [k x n]) takes the direct-to-LDS kernel,
// which can then also sum A's columns (the row sums of A^T).
static bool dw_rowsum_ok(size_t m, size_t n, size_t k, const float *a, const float *b) {
    return dma_enabled() && dma_ok(1, m, n, k, k, a, 0, (int)m, 1, b, 0, (int)n, 0);
}

// rs_out / rs_part: the row sums of op(A) (A^T B layout and the direct-to-LDS
// kernel only; the caller checks dw_rowsum_ok).
static int gemm_enqueue(rnn_ctx *ctx, size_t count, size_t m, size_t n, size_t kchunk,
                        size_t ktotal, const float *a, size_t stride_a, int lda, int at,
                        const float *b, size_t stride_b, int ldb, int bt, float *c,
                        size_t stride_c, int ldc, int acc, const float *bias,
                        float *rs_out = nullptr, double *rs_part = nullptr, size_t zc1 = 0,
                        size_t stride_a2 = 0, size_t stride_b2 = 0, size_t stride_c2 = 0,
                        const GemmRes *res = nullptr) {
    if (m > INT32_MAX || n > INT32_MAX || ktotal > INT32_MAX || count > 65535)
        return rnn_fail(ctx, RNN_E_UNSUPPORTED, "gemm: dimension beyond 32-bit tile indexing");
    GemmArgs g;
    g.a = a;
    g.b = b;
    g.c = c;
    g.bias = bias;
    g.stride_a = (long long)stride_a;
    g.stride_b = (long long)stride_b;
    g.stride_c = (long long)stride_c;
    g.M = (int)m;
    g.N = (int)n;
    g.kchunk = (int)kchunk;
    g.ktotal = (int)ktotal;
    g.lda = lda;
    g.ldb = ldb;
    g.ldc = ldc;
    g.acc = acc;
    g.rsum_out = rs_out;
    g.rsum_part = rs_part;
    g.res = res ? res->out : nullptr;
    g.res_l = res ? res->l : nullptr;
    g.res_mask = res ? res->mask : nullptr;
    g.res_shift = res ? res->shift : 0;
    g.zc1 = (int)(zc1 ? zc1 : count);
    g.stride_a2 = (long long)stride_a2;
    g.stride_b2 = (long long)stride_b2;
    g.stride_c2 = (long long)stride_c2;
    // float4 loads along k need 16-byte aligned rows of the k-contiguous operands.
    bool vec = true;
    if (!at) vec = vec && aligned16(a) && (lda % 4 == 0) && (stride_a % 4 == 0) &&
                   (stride_a2 % 4 == 0);
    if (bt) vec = vec && aligned16(b) && (ldb % 4 == 0) && (stride_b % 4 == 0) &&
                  (stride_b2 % 4 == 0);
    size_t tiles128 = rnn_div_up(m, 128) * rnn_div_up(n, 128) * count;
    if (dma_enabled() && stride_a2 % 4 == 0 && stride_b2 % 4 == 0 &&
        dma_ok(count, m, n, kchunk, ktotal, a, stride_a, lda, at, b, stride_b, ldb, bt)) {
        // 128 x 128 tiles only from four tiles per CU: below that the 64 x 64
        // grid's extra workgroups hide more latency than the larger tile's
        // operand reuse saves (measured on MI355X: 8192x768x256 99 vs 79
        // TFLOP/s, 4096^3 124 vs 136)
        if (m >= 128 && n >= 128 && tiles128 >= 4 * (size_t)ctx->num_cus)
            return launch_dma_bm<128, 128, 16, 4>(ctx, g, (int)count, at, bt);
        return launch_dma_bm<64, 64, 32, 3>(ctx, g, (int)count, at, bt);
    }
    if (rs_out || rs_part) return rnn_fail(ctx, RNN_E_INVALID, "gemm: row sums need the DMA path");
    const bool big = m >= 128 && n >= 128 && tiles128 >= (size_t)ctx->num_cus;
    if (big) return launch_bm<128, 128>(ctx, g, (int)count, at, bt, vec);
    return launch_bm<64, 64>(ctx, g, (int)count, at, bt, vec);
}

int rnn_gemm_launch(rnn_ctx *ctx, size_t count, size_t m, size_t n, size_t k, const float *a,
                    size_t stride_a, int at, const float *b, size_t stride_b, int bt, float *c,
                    size_t stride_c, int acc, const float *bias) {
    int lda = at ? (int)m : (int)k, ldb = bt ? (int)k : (int)n;
    return gemm_enqueue(ctx, count, m, n, k, k * count, a, stride_a, lda, at, b, stride_b, ldb, bt,
                        c, stride_c, (int)n, acc, bias);
}

int rnn_ns_gemm_launch(rnn_ctx *ctx, const NsGemmProb *probs, int nprob, size_t ntiles, int vec,
                       float alpha, float beta) {
    if (ntiles == 0) return RNN_OK;
    if (ntiles > 0x7fffffffu) return rnn_fail(ctx, RNN_E_UNSUPPORTED, "ns_gemm: too many tiles");
    const dim3 grid((unsigned)ntiles);
    if (vec == 2) {
        static bool attr = false;
        if (!attr) {
            attr = true;
            (void)hipFuncSetAttribute((const void *)ns_gemm_dma_kernel,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)NS_DMA_LDS);
        }
        hipLaunchKernelGGL(ns_gemm_dma_kernel, grid, dim3(512), NS_DMA_LDS, ctx->stream, probs,
                           nprob, alpha, beta);
    } else if (vec)
        hipLaunchKernelGGL(ns_gemm_kernel<true>, grid, dim3(256), 0, ctx->stream, probs, nprob,
                           alpha, beta);
    else
        hipLaunchKernelGGL(ns_gemm_kernel<false>, grid, dim3(256), 0, ctx->stream, probs, nprob,
                           alpha, beta);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_gemm_launch_ld(rnn_ctx *ctx, size_t count, size_t m, size_t n, size_t k, const float *a,
                       size_t lda, size_t stride_a, int at, const float *b, size_t ldb,
                       size_t stride_b, int bt, float *c, size_t ldc, size_t stride_c, int acc) {
    if (lda > INT32_MAX || ldb > INT32_MAX || ldc > INT32_MAX)
        return rnn_fail(ctx, RNN_E_UNSUPPORTED, "gemm: leading dimension beyond 32 bits");
    return gemm_enqueue(ctx, count, m, n, k, k * count, a, stride_a, (int)lda, at, b, stride_b,
                        (int)ldb, bt, c, stride_c, (int)ldc, acc, nullptr);
}

int rnn_gemm_launch_ld2(rnn_ctx *ctx, size_t count1, size_t count2, size_t m, size_t n, size_t k,
                        const float *a, size_t lda, size_t stride_a, size_t stride_a2, int at,
                        const float *b, size_t ldb, size_t stride_b, size_t stride_b2, int bt,
                        float *c, size_t ldc, size_t stride_c, size_t stride_c2, int acc) {
    if (lda > INT32_MAX || ldb > INT32_MAX || ldc > INT32_MAX)
        return rnn_fail(ctx, RNN_E_UNSUPPORTED, "gemm: leading dimension beyond 32 bits");
    const size_t count = count1 * count2;
    if (count == 0) return RNN_OK;
    return gemm_enqueue(ctx, count, m, n, k, k * count, a, stride_a, (int)lda, at, b, stride_b,
                        (int)ldb, bt, c, stride_c, (int)ldc, acc, nullptr, nullptr, nullptr,
                        count1, stride_a2, stride_b2, stride_c2);
}

static int fill(rnn_ctx *ctx, float *p, size_t len, float v) {
    if (!len) return RNN_OK;
    int blocks = (int)std::min<size_t>(rnn_div_up(len, 256), 4096);
    hipLaunchKernelGGL(fill_kernel, dim3(blocks), dim3(256), 0, ctx->stream, p, (long long)len, v);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_colsum_launch(rnn_ctx *ctx, size_t rows, size_t cols, const float *x, float *out) {
    // out[c] += sum_r x[r][c] (f64, fixed order)
    if (cols > (size_t)INT32_MAX) return rnn_fail(ctx, RNN_E_UNSUPPORTED, "colsum: too many columns");
    return rnn_colsum_f64(ctx, rows, (int)cols, x, nullptr, nullptr, out);
}

// C = op(A) op(B) (+ C) with K split into nz chunks (multiples of 16) when
// the C tiles alone cannot fill the chip; the chunk partials are added into C
// in chunk order (deterministic).  Returns -1 when splitting does not pay.
static int gemm_splitk(rnn_ctx *ctx, size_t m, size_t n, size_t k, const float *a, int at,
                       const float *b, int bt, float *c, int acc, float *rsum = nullptr,
                       bool deferrable = false) {
    const size_t tiles = rnn_div_up(m, 64) * rnn_div_up(n, 64);
    if (tiles >= (size_t)ctx->num_cus || k < 1024) return -1;
    // about three workgroups per CU, each over at least 512 values of k
    // (measured on the qkv / linear dW shapes: 768x256x16384 0.37 -> 0.47)
    size_t nz = std::min(rnn_div_up(3 * (size_t)ctx->num_cus, tiles), k / 512);
    nz = std::min<size_t>(nz, 64);
    if (nz <= 1) return -1;
    const size_t kchunk = rnn_round_up(rnn_div_up(k, nz), 16);
    nz = rnn_div_up(k, kchunk);
    // a parameter gradient's partials wait in the deferral arena when the
    // context defers (the flush adds them into C, and into rsum)
    const bool defer = deferrable && ctx->defer;
    const size_t pbytes = rnn_round_up(nz * m * n * sizeof(float), 256);
    const size_t bytes = pbytes + (rsum ? nz * m * sizeof(double) : 0);
    float *part = (float *)(defer ? rnn_defer_take(ctx, bytes) : rnn_workspace(ctx, bytes));
    if (!part) return RNN_E_NOMEM;
    double *rpart = rsum ? (double *)((char *)part + pbytes) : nullptr;
    // chunk z of A: rows z*kchunk of [k x m] (at) or columns z*kchunk of [m x k]
    const size_t sa = at ? kchunk * m : kchunk, sb = bt ? kchunk : kchunk * n;
    const int lda = at ? (int)m : (int)k, ldb = bt ? (int)k : (int)n;
    int rc = gemm_enqueue(ctx, nz, m, n, kchunk, k, a, sa, lda, at, b, sb, ldb, bt, part, m * n,
                          (int)n, 0, nullptr, nullptr, rpart);
    if (rc) return rc;
    if (defer) {
        RnnDeferSeg sg{};
        sg.part = part;
        sg.out0 = c;
        sg.len = (long long)(m * n);
        sg.nrow = (int)nz;
        // part is 256-byte aligned, so its rows are 16-byte aligned when len is
        // a multiple of 4
        sg.kind = (m * n) % 4 == 0 && (uintptr_t)c % 16 == 0 ? RNN_DEFER_CHUNKS4
                                                            : RNN_DEFER_CHUNKS;
        sg.acc = acc;
        rnn_defer_push(ctx, sg);
        if (rsum) {
            RnnDeferSeg sr{};
            sr.part = rpart;
            sr.out0 = rsum;
            sr.len = (long long)m;
            sr.nrow = (int)nz;
            sr.kind = RNN_DEFER_ROWS64;
            rnn_defer_push(ctx, sr);
        }
        return RNN_OK;
    }
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(rnn_div_up(m * n + (rsum ? m : 0), 256)),
                       dim3(256), 0, ctx->stream, part, (int)nz, (long long)(m * n), c, acc,
                       (const double *)rpart, (int)m, rsum);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

extern "C" {

int rnn_matmul(rnn_ctx *ctx, size_t m, size_t n, size_t k, const float *a, int at, const float *b,
               int bt, float *c, int acc) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (m == 0 || n == 0) return RNN_OK;  // gemm.rs:446-448
    if (!c) return rnn_fail(ctx, RNN_E_NULL, "matmul: c is null");
    if (k == 0) return acc ? RNN_OK : fill(ctx, c, m * n, 0.f);  // gemm.rs:449-454
    if (!a || !b) return rnn_fail(ctx, RNN_E_NULL, "matmul: a or b is null");
    const int rc = gemm_splitk(ctx, m, n, k, a, at, b, bt, c, acc);
    if (rc != -1) return rc;
    return rnn_gemm_launch(ctx, 1, m, n, k, a, 0, at, b, 0, bt, c, 0, acc, nullptr);
}

int rnn_gemm_small_batched(rnn_ctx *ctx, size_t count, size_t m, size_t n, size_t k,
                           const float *a, size_t stride_a, int at, const float *b,
                           size_t stride_b, int bt, float *c, size_t stride_c, int acc) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (count == 0 || m == 0 || n == 0 || k == 0) return RNN_OK;  // k == 0: C untouched
    if (!a || !b || !c) return rnn_fail(ctx, RNN_E_NULL, "gemm_small: null operand");
    for (size_t z0 = 0; z0 < count; z0 += 65535) {
        size_t cnt = std::min<size_t>(65535, count - z0);
        int rc = rnn_gemm_launch(ctx, cnt, m, n, k, a + z0 * stride_a, stride_a, at,
                                 b + z0 * stride_b, stride_b, bt, c + z0 * stride_c, stride_c,
                                 acc, nullptr);
        if (rc) return rc;
    }
    return RNN_OK;
}

int rnn_matmul_dw(rnn_ctx *ctx, size_t m, size_t n, size_t k, const float *a, const float *b,
                  float *c) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (m == 0 || n == 0 || k == 0) return RNN_OK;  // gemm.rs:556-558
    if (!a || !b || !c) return rnn_fail(ctx, RNN_E_NULL, "matmul_dw: null operand");
    // C += A^T B: split K when the C tiles cannot fill the chip (chunk
    // partials added into C in chunk order), else one accumulating GEMM.
    const int rc = gemm_splitk(ctx, m, n, k, a, 1, b, 0, c, 1);
    if (rc != -1) return rc;
    return gemm_enqueue(ctx, 1, m, n, k, k, a, 0, (int)m, 1, b, 0, (int)n, 0, c, 0, (int)n, 1,
                        nullptr);
}

int rnn_linear_forward(rnn_ctx *ctx, size_t rows, size_t fin, size_t fout, const float *x,
                       const float *w, const float *b, float *y) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (rows == 0 || fout == 0) return RNN_OK;
    if (!x || !w || !y) return rnn_fail(ctx, RNN_E_NULL, "linear_forward: null operand");
    if (fin == 0) {
        int rc = fill(ctx, y, rows * fout, 0.f);
        if (rc || !b) return rc;
        return rnn_gemm_launch(ctx, 1, rows, fout, 0, x, 0, 0, w, 0, 1, y, 0, 1, b);
    }
    // y = x W^T (+ b fused in the epilogue)
    return rnn_gemm_launch(ctx, 1, rows, fout, fin, x, 0, 0, w, 0, 1, y, 0, 0, b);
}

int rnn_linear_forward_residual(rnn_ctx *ctx, size_t rows, size_t fin, size_t fout,
                                const float *x, const float *w, const float *b, float *y,
                                const float *l, const float *mask, size_t rpi, float *out) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (rows == 0 || fout == 0) return RNN_OK;
    if (!x || !w || !y || !l || !out)
        return rnn_fail(ctx, RNN_E_NULL, "linear_forward_residual: null operand");
    if (out == y || out == x) return rnn_fail(ctx, RNN_E_INVALID, "linear_forward_residual: aliased out");
    if (mask && (rpi == 0 || rows % rpi))
        return rnn_fail(ctx, RNN_E_INVALID, "linear_forward_residual: %zu rows per image of %zu",
                        rpi, rows);
    // the fused epilogue takes a power-of-two image size; else two passes
    const bool pow2 = !mask || (rpi & (rpi - 1)) == 0;
    if (fin == 0 || !pow2) {
        int rc = rnn_linear_forward(ctx, rows, fin, fout, x, w, b, y);
        if (!rc) rc = rnn_residual_add_scaled(ctx, rows, fout, out, y, l, mask, rpi, out);
        return rc;
    }
    int shift = 0;
    while (mask && ((size_t)1 << shift) < rpi) shift++;
    const GemmRes gr{out, l, mask, shift};
    return gemm_enqueue(ctx, 1, rows, fout, fin, fin, x, 0, (int)fin, 0, w, 0, (int)fin, 1, y, 0,
                        (int)fout, 0, b, nullptr, nullptr, 0, 0, 0, 0, &gr);
}

int rnn_linear_backward(rnn_ctx *ctx, size_t rows, size_t fin, size_t fout, const float *dy,
                        const float *x, const float *w, float *dw, float *db, float *dx) {
    return rnn_linear_backward_ex(ctx, rows, fin, fout, dy, x, w, dw, db, dx, 0);
}

int rnn_linear_backward_ex(rnn_ctx *ctx, size_t rows, size_t fin, size_t fout, const float *dy,
                           const float *x, const float *w, float *dw, float *db, float *dx,
                           uint32_t flags) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (!dy || !x || !w || !dw || !dx)
        return rnn_fail(ctx, RNN_E_NULL, "linear_backward: null operand");
    if (flags & ~RNN_LINEAR_ACC_DX)
        return rnn_fail(ctx, RNN_E_INVALID, "linear_backward: flags 0x%x", flags);
    // dW[fout, fin] += dY^T X (linear.rs:69); db += the column sums of dY
    // (linear.rs:70-89), summed in f64 by the dW GEMM itself when it takes
    // the direct-to-LDS kernel, else by the column-sum kernels
    int rc;
    if (db && rows && fout && fin && dw_rowsum_ok(fout, fin, rows, dy, x)) {
        rc = gemm_splitk(ctx, fout, fin, rows, dy, 1, x, 0, dw, 1, db, true);
        if (rc == -1)
            rc = gemm_enqueue(ctx, 1, fout, fin, rows, rows, dy, 0, (int)fout, 1, x, 0, (int)fin,
                              0, dw, 0, (int)fin, 1, nullptr, db, nullptr);
        if (rc) return rc;
    } else {
        rc = rows && fout && fin ? gemm_splitk(ctx, fout, fin, rows, dy, 1, x, 0, dw, 1, nullptr, true)
                                 : RNN_OK;
        if (rc == -1) rc = rnn_matmul_dw(ctx, fout, fin, rows, dy, x, dw);
        if (rc) return rc;
        if (db && rows && fout) {
            rc = rnn_colsum_launch(ctx, rows, fout, dy, db);
            if (rc) return rc;
        }
    }
    // dX[rows, fin] = dY W (linear.rs:91-94), or dX += dY W
    return rnn_matmul(ctx, rows, fin, fout, dy, 0, w, 0, dx, (flags & RNN_LINEAR_ACC_DX) ? 1 : 0);
}

int rnn_dbg_pack_a(rnn_ctx *ctx, const float *a, size_t m, size_t k, int transposed, float *out) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (m == 0 || k == 0) return RNN_OK;
    if (!a || !out) return RNN_E_NULL;
    size_t mpad = rnn_div_up(m, 6) * 6, total = rnn_div_up(k, 256) * 256 * mpad;
    hipLaunchKernelGGL(pack_a_kernel, dim3(rnn_div_up(total, 256)), dim3(256), 0, ctx->stream, a,
                       (long long)m, (long long)k, transposed, out, (long long)mpad,
                       (long long)total);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_dbg_pack_b(rnn_ctx *ctx, const float *b, size_t n, size_t k, int transposed, float *out) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (n == 0 || k == 0) return RNN_OK;
    if (!b || !out) return RNN_E_NULL;
    size_t npad = rnn_div_up(n, 16) * 16, total = rnn_div_up(k, 256) * 256 * npad;
    hipLaunchKernelGGL(pack_b_kernel, dim3(rnn_div_up(total, 256)), dim3(256), 0, ctx->stream, b,
                       (long long)n, (long long)k, transposed, out, (long long)npad,
                       (long long)total);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

}  // extern "C"
