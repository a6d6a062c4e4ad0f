/*
 * orc_gemm.c -- restatement of the reference GEMM core (gemm.rs).  Test
 * infrastructure only (see orc.h).
 *
 * Summation order kept from the reference: every C element is one FMA chain
 * over a K block of at most KC=256 (AVX2 path, gemm.rs:139-149) starting from
 * zero, and successive K blocks are added into C with a separate add
 * (gemm.rs:150-161, accumulate = q > 0 || acc).
 */
#include <stdlib.h>
#include <string.h>
#ifdef __AVX2__
#include <immintrin.h>
#endif
#ifdef _OPENMP
#include <omp.h>
#endif

#include "orc.h"

#define MR ORC_MR
#define NR ORC_NR
#define KC ORC_KC
/* gemm.rs:15 -- only decides serial vs parallel packing; no effect on values. */
#define PAR_MIN (1u << 18)

static int g_threads = 1;
#ifdef __AVX2__
static int g_simd = 1;
#else
static int g_simd = 0;
#endif

int orc_set_threads(int t) {
    int old = g_threads;
    g_threads = t < 1 ? 1 : t;
    return old;
}
int orc_get_threads(void) { return g_threads; }
int orc_set_simd(int on) {
    int old = g_simd;
#ifdef __AVX2__
    g_simd = on ? 1 : 0;
#else
    (void)on;
#endif
    return old;
}

static inline size_t div_ceil(size_t a, size_t b) { return (a + b - 1) / b; }
static inline size_t min_sz(size_t a, size_t b) { return a < b ? a : b; }

/* PackedA::prepare (gemm.rs:36-45): block q at q*KC*mpad. */
size_t orc_packed_a_len(size_t m, size_t k) { return div_ceil(k, KC) * KC * div_ceil(m, MR) * MR; }
size_t orc_packed_b_len(size_t n, size_t k) { return div_ceil(k, KC) * KC * div_ceil(n, NR) * NR; }

/* PackedA::pack / pack_t (gemm.rs:54-113).  Panel i of block q sits at
 * q*KC*mpad + i*kc*MR and holds panel[p*MR + r] = A[i*MR + r, q*KC + p]
 * (0 for rows >= m). */
void orc_pack_a(const float *a, size_t m, size_t k, int transposed, float *out) {
    size_t mpan = div_ceil(m, MR), mpad = mpan * MR, nb = div_ceil(k, KC);
    for (size_t q = 0; q < nb; q++) {
        size_t pc = q * KC, kc = min_sz(KC, k - pc);
        float *dst = out + q * KC * mpad;
#pragma omp parallel for num_threads(g_threads) if (m * kc >= PAR_MIN && g_threads > 1)
        for (size_t i = 0; i < mpan; i++) {
            float *panel = dst + i * kc * MR;
            if (!transposed) {
                for (size_t r = 0; r < MR; r++) {
                    size_t row = i * MR + r;
                    if (row >= m) {
                        for (size_t p = 0; p < kc; p++) panel[p * MR + r] = 0.0f;
                        continue;
                    }
                    const float *src = a + row * k + pc;
                    for (size_t p = 0; p < kc; p++) panel[p * MR + r] = src[p];
                }
            } else {
                for (size_t p = 0; p < kc; p++) {
                    const float *src = a + (pc + p) * m;
                    for (size_t r = 0; r < MR; r++) {
                        size_t row = i * MR + r;
                        panel[p * MR + r] = row < m ? src[row] : 0.0f;
                    }
                }
            }
        }
    }
}

#ifdef __AVX2__
/* transpose8x8 (gemm.rs:238-269). */
__attribute__((target("avx2"))) static void transpose8x8(const float *src, size_t lds, float *dst,
                                                         size_t ldd) {
    __m256 r0 = _mm256_loadu_ps(src + 0 * lds), r1 = _mm256_loadu_ps(src + 1 * lds);
    __m256 r2 = _mm256_loadu_ps(src + 2 * lds), r3 = _mm256_loadu_ps(src + 3 * lds);
    __m256 r4 = _mm256_loadu_ps(src + 4 * lds), r5 = _mm256_loadu_ps(src + 5 * lds);
    __m256 r6 = _mm256_loadu_ps(src + 6 * lds), r7 = _mm256_loadu_ps(src + 7 * lds);
    __m256 t0 = _mm256_unpacklo_ps(r0, r1), t1 = _mm256_unpackhi_ps(r0, r1);
    __m256 t2 = _mm256_unpacklo_ps(r2, r3), t3 = _mm256_unpackhi_ps(r2, r3);
    __m256 t4 = _mm256_unpacklo_ps(r4, r5), t5 = _mm256_unpackhi_ps(r4, r5);
    __m256 t6 = _mm256_unpacklo_ps(r6, r7), t7 = _mm256_unpackhi_ps(r6, r7);
    __m256 u0 = _mm256_shuffle_ps(t0, t2, 0x44), u1 = _mm256_shuffle_ps(t0, t2, 0xEE);
    __m256 u2 = _mm256_shuffle_ps(t1, t3, 0x44), u3 = _mm256_shuffle_ps(t1, t3, 0xEE);
    __m256 u4 = _mm256_shuffle_ps(t4, t6, 0x44), u5 = _mm256_shuffle_ps(t4, t6, 0xEE);
    __m256 u6 = _mm256_shuffle_ps(t5, t7, 0x44), u7 = _mm256_shuffle_ps(t5, t7, 0xEE);
    _mm256_storeu_ps(dst + 0 * ldd, _mm256_permute2f128_ps(u0, u4, 0x20));
    _mm256_storeu_ps(dst + 1 * ldd, _mm256_permute2f128_ps(u1, u5, 0x20));
    _mm256_storeu_ps(dst + 2 * ldd, _mm256_permute2f128_ps(u2, u6, 0x20));
    _mm256_storeu_ps(dst + 3 * ldd, _mm256_permute2f128_ps(u3, u7, 0x20));
    _mm256_storeu_ps(dst + 4 * ldd, _mm256_permute2f128_ps(u0, u4, 0x31));
    _mm256_storeu_ps(dst + 5 * ldd, _mm256_permute2f128_ps(u1, u5, 0x31));
    _mm256_storeu_ps(dst + 6 * ldd, _mm256_permute2f128_ps(u2, u6, 0x31));
    _mm256_storeu_ps(dst + 7 * ldd, _mm256_permute2f128_ps(u3, u7, 0x31));
}
#endif

/* transpose_to_panel (gemm.rs:277-304). */
void orc_transpose_to_panel(const float *src, size_t lds, size_t kc, float *bp) {
    size_t p = 0;
#ifdef __AVX2__
    if (g_simd) {
        size_t n8 = kc & ~(size_t)7;
        for (; p < n8; p += 8) {
            transpose8x8(src + p, lds, bp + p * NR, NR);
            transpose8x8(src + 8 * lds + p, lds, bp + p * NR + 8, NR);
        }
    }
#endif
    for (; p < kc; p++)
        for (size_t t = 0; t < NR; t++) bp[p * NR + t] = src[t * lds + p];
}

/* PackedB::pack / pack_t (gemm.rs:340-400).  Panel j of block q holds
 * panel[p*NR + t] = B[q*KC + p, j*NR + t] (0 for columns >= n). */
void orc_pack_b(const float *b, size_t n, size_t k, int transposed, float *out) {
    size_t npan = div_ceil(n, NR), npad = npan * NR, nb = div_ceil(k, KC);
    for (size_t q = 0; q < nb; q++) {
        size_t pc = q * KC, kc = min_sz(KC, k - pc);
        float *dst = out + q * KC * npad;
#pragma omp parallel for num_threads(g_threads) if (n * kc >= PAR_MIN && g_threads > 1)
        for (size_t j = 0; j < npan; j++) {
            float *panel = dst + j * kc * NR;
            size_t nr = min_sz(NR, n - j * NR);
            if (!transposed) {
                for (size_t p = 0; p < kc; p++) {
                    const float *src = b + (pc + p) * n + j * NR;
                    float *d = panel + p * NR;
                    memcpy(d, src, nr * sizeof(float));
                    for (size_t t = nr; t < NR; t++) d[t] = 0.0f;
                }
            } else if (nr == NR) {
                orc_transpose_to_panel(b + (j * NR) * k + pc, k, kc, panel);
            } else {
                for (size_t p = 0; p < kc; p++)
                    for (size_t t = 0; t < NR; t++)
                        panel[p * NR + t] = t < nr ? b[(j * NR + t) * k + pc + p] : 0.0f;
            }
        }
    }
}

#ifdef __AVX2__
/* micro_avx2 (gemm.rs:122-179): 12 ymm accumulators, FMA chain from zero. */
__attribute__((target("avx2,fma"))) static void micro_avx2(size_t kc, const float *ap,
                                                           const float *bp, float *c, size_t ldc,
                                                           size_t mr, size_t nr, int accumulate) {
    __m256 c0[MR], c1[MR];
    for (int i = 0; i < MR; i++) {
        c0[i] = _mm256_setzero_ps();
        c1[i] = _mm256_setzero_ps();
    }
    const float *apk = ap, *bpk = bp;
    for (size_t p = 0; p < kc; p++) {
        __m256 b0 = _mm256_loadu_ps(bpk);
        __m256 b1 = _mm256_loadu_ps(bpk + 8);
        for (int i = 0; i < MR; i++) {
            __m256 a = _mm256_broadcast_ss(apk + i);
            c0[i] = _mm256_fmadd_ps(a, b0, c0[i]);
            c1[i] = _mm256_fmadd_ps(a, b1, c1[i]);
        }
        apk += MR;
        bpk += NR;
    }
    if (mr == MR && nr == NR) {
        for (int i = 0; i < MR; i++) {
            float *d = c + i * ldc;
            if (accumulate) {
                _mm256_storeu_ps(d, _mm256_add_ps(_mm256_loadu_ps(d), c0[i]));
                _mm256_storeu_ps(d + 8, _mm256_add_ps(_mm256_loadu_ps(d + 8), c1[i]));
            } else {
                _mm256_storeu_ps(d, c0[i]);
                _mm256_storeu_ps(d + 8, c1[i]);
            }
        }
    } else {
        float tmp[MR * NR];
        for (int i = 0; i < MR; i++) {
            _mm256_storeu_ps(tmp + i * NR, c0[i]);
            _mm256_storeu_ps(tmp + i * NR + 8, c1[i]);
        }
        for (size_t i = 0; i < mr; i++) {
            float *row = c + i * ldc;
            if (accumulate)
                for (size_t j = 0; j < nr; j++) row[j] += tmp[i * NR + j];
            else
                memcpy(row, tmp + i * NR, nr * sizeof(float));
        }
    }
}
#endif

/* micro_scalar (gemm.rs:181-214): unfused mul + add. */
static void micro_scalar(size_t kc, const float *ap, const float *bp, float *c, size_t ldc,
                         size_t mr, size_t nr, int accumulate) {
    float acc[MR][NR];
    memset(acc, 0, sizeof(acc));
    for (size_t p = 0; p < kc; p++) {
        const float *bv = bp + p * NR, *av = ap + p * MR;
        for (int i = 0; i < MR; i++) {
            float a = av[i];
            for (int j = 0; j < NR; j++) acc[i][j] += a * bv[j];
        }
    }
    for (size_t i = 0; i < mr; i++) {
        float *row = c + i * ldc;
        if (accumulate)
            for (size_t j = 0; j < nr; j++) row[j] += acc[i][j];
        else
            memcpy(row, acc[i], nr * sizeof(float));
    }
}

/* micro_kernel (gemm.rs:218-236). */
void orc_micro_kernel(size_t kc, const float *ap, const float *bp, float *c, size_t ldc,
                      size_t mr, size_t nr, int accumulate) {
#ifdef __AVX2__
    if (g_simd) {
        micro_avx2(kc, ap, bp, c, ldc, mr, nr, accumulate);
        return;
    }
#endif
    micro_scalar(kc, ap, bp, c, ldc, mr, nr, accumulate);
}

/* Panel accessors (gemm.rs:116-119, 403-406). */
static inline const float *panel_a(const float *d, size_t mpad, size_t q, size_t i, size_t kc) {
    return d + q * KC * mpad + i * kc * MR;
}
static inline const float *panel_b(const float *d, size_t npad, size_t q, size_t j, size_t kc) {
    return d + q * KC * npad + j * kc * NR;
}

/* Shared body of matmul / gemm_small: j outer, q inner per 6-row panel i
 * (gemm.rs:471-490, 526-544). */
static void gemm_panel_row(size_t i, size_t m, size_t n, size_t k, const float *ap, size_t mpad,
                           const float *bp, size_t npad, float *c, int acc) {
    size_t npan = div_ceil(n, NR), nb = div_ceil(k, KC);
    size_t mr = min_sz(MR, m - i * MR);
    for (size_t j = 0; j < npan; j++) {
        size_t nr = min_sz(NR, n - j * NR);
        for (size_t q = 0; q < nb; q++) {
            size_t kc = min_sz(KC, k - q * KC);
            orc_micro_kernel(kc, panel_a(ap, mpad, q, i, kc), panel_b(bp, npad, q, j, kc),
                             c + i * MR * n + j * NR, n, mr, nr, q > 0 || acc);
        }
    }
}

/* matmul (gemm.rs:434-493). */
void orc_matmul(size_t m, size_t n, size_t k, const float *a, int at, const float *b, int bt,
                float *c, int acc) {
    if (m == 0 || n == 0) return;
    if (k == 0) {
        if (!acc) memset(c, 0, m * n * sizeof(float));
        return;
    }
    float *ap = (float *)calloc(orc_packed_a_len(m, k), sizeof(float));
    float *bp = (float *)calloc(orc_packed_b_len(n, k), sizeof(float));
    orc_pack_a(a, m, k, at, ap);
    orc_pack_b(b, n, k, bt, bp);
    size_t mpad = div_ceil(m, MR) * MR, npad = div_ceil(n, NR) * NR, mpan = div_ceil(m, MR);
#pragma omp parallel for num_threads(g_threads) schedule(dynamic, 1) if (g_threads > 1)
    for (size_t i = 0; i < mpan; i++) gemm_panel_row(i, m, n, k, ap, mpad, bp, npad, c, acc);
    free(ap);
    free(bp);
}

/* gemm_small (gemm.rs:500-545): no early return, so k == 0 leaves C as is. */
void orc_gemm_small(size_t m, size_t n, size_t k, const float *a, int at, const float *b, int bt,
                    float *c, int acc) {
    size_t la = orc_packed_a_len(m, k), lb = orc_packed_b_len(n, k);
    float *ap = (float *)calloc(la ? la : 1, sizeof(float));
    float *bp = (float *)calloc(lb ? lb : 1, sizeof(float));
    orc_pack_a(a, m, k, at, ap);
    orc_pack_b(b, n, k, bt, bp);
    size_t mpad = div_ceil(m, MR) * MR, npad = div_ceil(n, NR) * NR, mpan = div_ceil(m, MR);
    for (size_t i = 0; i < mpan; i++) gemm_panel_row(i, m, n, k, ap, mpad, bp, npad, c, acc);
    free(ap);
    free(bp);
}

/*
 * Leaf ranges of a rayon fold over `len` items.  With one worker rayon's
 * adaptive splitter splits an indexed producer once, at len/2, so the fold
 * produces two accumulators that the reduce then adds (left + right).  With
 * more workers the split is dynamic; here it is T contiguous ranges ("parity
 * unpinned": no reference test pins a multi-thread order).  Returns the
 * number of leaves written to lo[]/hi[] (at most max_leaves).
 */
size_t orc_fold_leaves(size_t len, int threads, size_t *lo, size_t *hi, size_t max_leaves) {
    if (len == 0) return 0;
    size_t nl;
    if (threads <= 1) {
        if (len >= 2 && max_leaves >= 2) {
            lo[0] = 0;
            hi[0] = len / 2;
            lo[1] = len / 2;
            hi[1] = len;
            return 2;
        }
        lo[0] = 0;
        hi[0] = len;
        return 1;
    }
    nl = (size_t)threads;
    if (nl > len) nl = len;
    if (nl > max_leaves) nl = max_leaves;
    for (size_t t = 0; t < nl; t++) {
        lo[t] = len * t / nl;
        hi[t] = len * (t + 1) / nl;
    }
    return nl;
}

/* matmul_dw (gemm.rs:555-598). */
void orc_matmul_dw(size_t m, size_t n, size_t k, const float *a, const float *b, float *c) {
    if (m == 0 || n == 0 || k == 0) return;
    int flip = n < m;
    size_t mm = flip ? n : m, nn = flip ? m : n;
    const float *aa = flip ? b : a, *bb = flip ? a : b;
    size_t rows = min_sz(KC, k);
    if (rows < 1) rows = 1;
    size_t nchunk = div_ceil(k, rows);
    size_t lo[256], hi[256];
    size_t nl = orc_fold_leaves(nchunk, g_threads, lo, hi, 256);
    float *accs = (float *)calloc(nl * mm * nn, sizeof(float));
#pragma omp parallel for num_threads(g_threads) schedule(static, 1) if (g_threads > 1)
    for (size_t l = 0; l < nl; l++) {
        float *acc = accs + l * mm * nn;
        for (size_t ch = lo[l]; ch < hi[l]; ch++) {
            size_t r0 = ch * rows, kk = min_sz(rows, k - r0);
            orc_gemm_small(mm, nn, kk, aa + r0 * mm, 1, bb + r0 * nn, 0, acc, 1);
        }
    }
    /* reduce: identity 0 + first leaf, then left-to-right adds */
    float *red = (float *)calloc(mm * nn, sizeof(float));
    for (size_t l = 0; l < nl; l++)
        for (size_t e = 0; e < mm * nn; e++) red[e] += accs[l * mm * nn + e];
    if (flip) {
        for (size_t i = 0; i < m; i++)
            for (size_t j = 0; j < n; j++) c[i * n + j] += red[j * m + i];
    } else {
        for (size_t e = 0; e < m * n; e++) c[e] += red[e];
    }
    free(red);
    free(accs);
}
