// loss.rs on the device: the soft targets (taxonomy / uniform smoothing with
// the mixup blend of train.rs), soft-target cross-entropy, the distillation
// KL and the hint MSE.
//
// Reference: taxo_target / uniform_target (loss.rs:11-34), ce_soft
// (loss.rs:39-83), kl_distill (loss.rs:87-130), hint_mse (loss.rs:133-151),
// targets (train.rs:121-155).  Each runs rayon over rows.
//
// The rows are few (a batch) and short (100 or 20 classes, or a 384-wide
// feature): one wave per row, the elementwise arithmetic in the reference's
// operation order with contraction off, the sums over classes lane-strided
// then a shuffle tree (the reference sums them sequentially), expf / logf on
// the device.  The per-row losses go to the workspace and one thread adds
// them in row order (ce_soft and kl_distill collect and sum in order;
// hint_mse's rayon sum has no fixed order).  Scalars land in device memory,
// so nothing waits on the host.
#include "rnn_internal.h"

#include <algorithm>
#include <cmath>
#include <cstring>

#pragma clang fp contract(off)

namespace {

constexpr int NT = 256;

__device__ __forceinline__ float wsum(float v) {
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wmax(float v) {
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// ce_soft per row, one wave per row: dz overwritten with scale (softmax - t)
// / n; part[i] = the row's loss, hit[i] = argmax == hard[i] (the first
// maximum, as `v > mx`: ties go to the lower class).  Sums over classes are
// lane-strided, then a shuffle tree.
__global__ __launch_bounds__(NT) void ce_soft_kernel(size_t n, int nc,
                                                     const float *__restrict__ logits,
                                                     const float *__restrict__ target,
                                                     const uint32_t *__restrict__ hard,
                                                     float scale, float *__restrict__ dz,
                                                     float *__restrict__ part,
                                                     uint32_t *__restrict__ hit) {
    const size_t i = (size_t)blockIdx.x * (NT / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (i >= n) return;
    const float *z = logits + i * nc, *t = target + i * nc;
    float *d = dz + i * nc;
    const float inv = 1.0f / (float)n;
    float mx = -INFINITY;
    int arg = nc;
    for (int j = lane; j < nc; j += 64)
        if (z[j] > mx) {
            mx = z[j];
            arg = j;
        }
    for (int o = 32; o >= 1; o >>= 1) {
        const float om = __shfl_xor(mx, o, 64);
        const int oa = __shfl_xor(arg, o, 64);
        if (om > mx || (om == mx && oa < arg)) {
            mx = om;
            arg = oa;
        }
    }
    float sum = 0.0f;
    for (int j = lane; j < nc; j += 64) {
        const float e = expf(z[j] - mx);
        d[j] = e;
        sum += e;
    }
    sum = wsum(sum);
    const float lse = mx + logf(sum);
    float l = 0.0f;
    for (int j = lane; j < nc; j += 64) {
        l += t[j] * (lse - z[j]);
        d[j] = (d[j] / sum - t[j]) * inv * scale;
    }
    l = wsum(l);
    if (lane == 0) {
        part[i] = l;
        if (hit) hit[i] = (uint32_t)arg == hard[i] ? 1u : 0u;
    }
}

// kl_distill per row (loss.rs:114-126), one wave per row: dz += temp (ps -
// pt) / n * scale; part[i] = temp^2 KL(pt || ps), ps / pt the softmaxes of
// z / temp (max, sum of exp((z - max) / temp), times the inverse).
__global__ __launch_bounds__(NT) void kl_distill_kernel(size_t n, int nc,
                                                        const float *__restrict__ student,
                                                        const float *__restrict__ teacher,
                                                        float temp, float scale,
                                                        float *__restrict__ dz,
                                                        float *__restrict__ part) {
    const size_t i = (size_t)blockIdx.x * (NT / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (i >= n) return;
    const float *zs = student + i * nc, *zt = teacher + i * nc;
    float *d = dz + i * nc;
    const float inv = 1.0f / (float)n, it = 1.0f / temp;
    float ms = -INFINITY, mt = -INFINITY;
    for (int j = lane; j < nc; j += 64) {
        ms = fmaxf(ms, zs[j]);
        mt = fmaxf(mt, zt[j]);
    }
    ms = wmax(ms);
    mt = wmax(mt);
    float ss = 0.0f, st = 0.0f;
    for (int j = lane; j < nc; j += 64) {
        ss += expf((zs[j] - ms) * it);
        st += expf((zt[j] - mt) * it);
    }
    const float iss = 1.0f / wsum(ss), ist = 1.0f / wsum(st);
    float l = 0.0f;
    for (int j = lane; j < nc; j += 64) {
        const float ps = expf((zs[j] - ms) * it) * iss;
        const float pt = expf((zt[j] - mt) * it) * ist;
        if (pt > 1e-9f) l += pt * (logf(fmaxf(pt, 1e-9f)) - logf(fmaxf(ps, 1e-9f)));
        d[j] += temp * (ps - pt) * inv * scale;
    }
    l = wsum(l);
    if (lane == 0) part[i] = l * temp * temp;
}

// hint_mse per row (loss.rs:139-150), one wave per row: dz += 2 e / (n c) *
// scale; part[i] = sum e^2.
template <bool SET>
__global__ __launch_bounds__(NT) void hint_mse_kernel(size_t n, int c, const float *__restrict__ pred,
                                                      const float *__restrict__ target,
                                                      float scale, float *__restrict__ dz,
                                                      float *__restrict__ part) {
    const size_t i = (size_t)blockIdx.x * (NT / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (i >= n) return;
    const float inv = 1.0f / (float)(n * c);
    const float *p = pred + i * c, *t = target + i * c;
    float *d = dz + i * c;
    float s = 0.0f;
    for (int j = lane; j < c; j += 64) {
        const float e = p[j] - t[j];
        s += e * e;
        // SET: dz starts at zero (build_loss's fresh g.h1 / g.h2), written
        if constexpr (SET)
            d[j] = 2.0f * e * inv * scale;
        else
            d[j] += 2.0f * e * inv * scale;
    }
    s = wsum(s);
    if (lane == 0) part[i] = s;
}

// out = (sum of part in row order) * mul1 * mul2; hits summed likewise.
__global__ void rows_total_kernel(size_t n, const float *__restrict__ part, float mul1, float mul2,
                                  float *__restrict__ out, const uint32_t *__restrict__ hit,
                                  uint32_t *__restrict__ correct) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    // in row order, 16 loads ahead of their adds
    float s = 0.0f;
    uint32_t h = 0;
    for (size_t i0 = 0; i0 < n; i0 += 16) {
        float v[16];
        uint32_t u16[16];
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const size_t i = min(i0 + u, n - 1);
            v[u] = part[i];
            u16[u] = hit ? hit[i] : 0u;
        }
#pragma unroll
        for (int u = 0; u < 16; u++)
            if (i0 + u < n) {
                s += v[u];
                h += u16[u];
            }
    }
    if (out) *out = s * mul1 * mul2;
    if (correct) *correct = h;
}

// uniform_target (loss.rs:30-34), value at class j for label y of k classes.
__device__ __forceinline__ float uniform_at(int y, int j, int k, float eps) {
    const float v = eps / (float)k;
    return j == y ? v + (1.0f - eps) : v;
}

// taxo_target (loss.rs:11-28), value at class j.
__device__ __forceinline__ float taxo_at(int y, int j, int nf, const uint32_t *parent, float eps,
                                         float sib) {
    const uint32_t py = parent[y];
    int k = 0;
    for (int c = 0; c < nf; c++) k += parent[c] == py;
    if (j == y) return 1.0f - eps;
    if (k > 1 && parent[j] == py) return eps * sib / (float)(k - 1);
    return nf > k ? eps * (1.0f - sib) / (float)(nf - k) : 0.0f;
}

// targets (train.rs:121-155): tf[i][j] = lam a_j + (1 - lam) b_j with a, b the
// The dominant label of a mixed image (Trainer::make_batch, train.rs:313-320):
// its own label when lam >= 0.5, else its partner's.  A partner index out of
// range gives 0xffffffff, which no hit count matches.
__global__ void dominant_kernel(size_t n, const uint32_t *__restrict__ labels,
                                const uint32_t *__restrict__ perm, const float *__restrict__ lam,
                                uint32_t *__restrict__ dom) {
    const size_t i = (size_t)blockIdx.x * NT + threadIdx.x;
    if (i >= n) return;
    const size_t pi = perm[i];
    dom[i] = lam[i] >= 0.5f ? labels[i] : (pi < n ? labels[pi] : 0xffffffffu);
}

// fine targets of labels[i] and labels[perm[i]] (taxonomy or uniform); tc the
// same over the coarse labels with uniform smoothing.
__global__ void targets_kernel(size_t n, int nf, int nc, const uint32_t *__restrict__ labels,
                               const uint32_t *__restrict__ coarse,
                               const uint32_t *__restrict__ perm, const float *__restrict__ lam,
                               const uint32_t *__restrict__ parent, int taxo, float eps,
                               float sib, float *__restrict__ tf, float *__restrict__ tc) {
    const size_t per = (size_t)nf + (tc ? nc : 0);
    const size_t len = n * per;
    for (size_t e = (size_t)blockIdx.x * NT + threadIdx.x; e < len;
         e += (size_t)gridDim.x * NT) {
        const size_t i = e / per;
        const int j = (int)(e - i * per);
        const size_t pi = perm ? perm[i] : i;
        const float l = lam ? lam[i] : 1.0f;
        // an index out of range (a panic in the reference) gives NaN targets
        // instead of an out-of-bounds read
        if (j < nf) {
            float v = NAN;
            if (pi < n) {
                const uint32_t ya = labels[i], yb = labels[pi];
                if (ya < (uint32_t)nf && yb < (uint32_t)nf) {
                    const float a = taxo ? taxo_at((int)ya, j, nf, parent, eps, sib)
                                         : uniform_at((int)ya, j, nf, eps);
                    const float b = taxo ? taxo_at((int)yb, j, nf, parent, eps, sib)
                                         : uniform_at((int)yb, j, nf, eps);
                    v = l * a + (1.0f - l) * b;
                }
            }
            tf[i * nf + j] = v;
        } else {
            const int jc = j - nf;
            float v = NAN;
            if (pi < n) {
                const uint32_t ca = coarse[i], cb = coarse[pi];
                if (ca < (uint32_t)nc && cb < (uint32_t)nc)
                    v = l * uniform_at((int)ca, jc, nc, eps) +
                        (1.0f - l) * uniform_at((int)cb, jc, nc, eps);
            }
            tc[i * nc + jc] = v;
        }
    }
}

bool rows_ok(rnn_ctx *ctx, size_t n, size_t c, const char *what) {
    if (n > 0x7fffffffull || c == 0 || c > (1u << 24)) {
        rnn_fail(ctx, RNN_E_INVALID, "%s: %zu rows of %zu", what, n, c);
        return false;
    }
    return true;
}

}  // namespace

extern "C" {

int rnn_soft_targets(rnn_ctx *ctx, size_t n, size_t nf, size_t nc, const uint32_t *labels,
                     const uint32_t *coarse, const uint32_t *perm, const float *lam,
                     const uint32_t *parent, int taxo, float eps, float sib, float *tf,
                     float *tc) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (n == 0) return RNN_OK;
    if (!labels || !tf || (taxo && !parent) || (tc && !coarse))
        return rnn_fail(ctx, RNN_E_NULL, "soft_targets: null operand");
    if (!rows_ok(ctx, n, nf, "soft_targets") || (tc && !rows_ok(ctx, n, nc, "soft_targets")))
        return RNN_E_INVALID;
    const size_t len = n * (nf + (tc ? nc : 0));
    const unsigned grid = (unsigned)std::min<size_t>(rnn_div_up(len, NT), 4096);
    targets_kernel<<<grid, NT, 0, ctx->stream>>>(n, (int)nf, (int)nc, labels, coarse, perm, lam,
                                                 parent, taxo, eps, sib, tf, tc);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_mix_dominant(rnn_ctx *ctx, size_t n, const uint32_t *labels, const uint32_t *perm,
                     const float *lam, uint32_t *dom) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (n == 0) return RNN_OK;
    if (!labels || !perm || !lam || !dom)
        return rnn_fail(ctx, RNN_E_NULL, "mix_dominant: null operand");
    dominant_kernel<<<(unsigned)rnn_div_up(n, NT), NT, 0, ctx->stream>>>(n, labels, perm, lam,
                                                                           dom);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_ce_soft(rnn_ctx *ctx, size_t n, size_t nclass, const float *logits, const float *target,
                const uint32_t *hard, float scale, float *dz, float *loss, uint32_t *correct) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (n == 0) return RNN_OK;
    if (!logits || !target || !dz || (correct && !hard))
        return rnn_fail(ctx, RNN_E_NULL, "ce_soft: null operand");
    if (!rows_ok(ctx, n, nclass, "ce_soft")) return RNN_E_INVALID;
    WsCarve cv;
    const size_t o_part = cv.take(n * sizeof(float)), o_hit = cv.take(n * sizeof(uint32_t));
    char *ws = (char *)rnn_workspace(ctx, cv.off);
    if (!ws) return RNN_E_NOMEM;
    float *part = (float *)(ws + o_part);
    uint32_t *hit = correct ? (uint32_t *)(ws + o_hit) : nullptr;
    ce_soft_kernel<<<(unsigned)rnn_div_up(n, (size_t)(NT / 64)), NT, 0, ctx->stream>>>(
        n, (int)nclass, logits, target, hard, scale, dz, part, hit);
    RNN_LAUNCHED(ctx);
    if (loss || correct) {
        rows_total_kernel<<<1, 64, 0, ctx->stream>>>(n, part, 1.0f / (float)n, 1.0f, loss, hit,
                                                     correct);
        RNN_LAUNCHED(ctx);
    }
    return RNN_OK;
}

int rnn_kl_distill(rnn_ctx *ctx, size_t n, size_t nclass, const float *student,
                   const float *teacher, float temp, float scale, float *dz, float *loss) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (n == 0) return RNN_OK;
    if (!student || !teacher || !dz) return rnn_fail(ctx, RNN_E_NULL, "kl_distill: null operand");
    if (!rows_ok(ctx, n, nclass, "kl_distill")) return RNN_E_INVALID;
    float *part = (float *)rnn_workspace(ctx, n * sizeof(float));
    if (!part) return RNN_E_NOMEM;
    kl_distill_kernel<<<(unsigned)rnn_div_up(n, (size_t)(NT / 64)), NT, 0, ctx->stream>>>(
        n, (int)nclass, student, teacher, temp, scale, dz, part);
    RNN_LAUNCHED(ctx);
    if (loss) {
        rows_total_kernel<<<1, 64, 0, ctx->stream>>>(n, part, 1.0f / (float)n, 1.0f, loss, nullptr,
                                                     nullptr);
        RNN_LAUNCHED(ctx);
    }
    return RNN_OK;
}

int rnn_hint_mse(rnn_ctx *ctx, size_t n, size_t c, const float *pred, const float *target,
                 float scale, float *dz, float *loss) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (n == 0) return RNN_OK;
    if (!pred || !target || !dz) return rnn_fail(ctx, RNN_E_NULL, "hint_mse: null operand");
    if (!rows_ok(ctx, n, c, "hint_mse")) return RNN_E_INVALID;
    float *part = (float *)rnn_workspace(ctx, n * sizeof(float));
    if (!part) return RNN_E_NOMEM;
    hint_mse_kernel<false><<<(unsigned)rnn_div_up(n, (size_t)(NT / 64)), NT, 0, ctx->stream>>>(
        n, (int)c, pred, target, scale, dz, part);
    RNN_LAUNCHED(ctx);
    if (loss) {
        rows_total_kernel<<<1, 64, 0, ctx->stream>>>(n, part, 1.0f / (float)(n * c), scale, loss,
                                                     nullptr, nullptr);
        RNN_LAUNCHED(ctx);
    }
    return RNN_OK;
}

}  // extern "C"

namespace {

// build_loss's totals (train.rs:70-118) in one launch: lane k of the one
// wave sums the row partials of term k in row order as rows_total_kernel
// does (16 loads ahead of the adds), then lane 0 adds the terms in the
// reference's order and grouping, in f32:
// total = ce (+ cw lc) (+ (w1 l1 + w2 l2)) (+ alpha (k1 + k2)) (+ (h1 + h2)).
struct LossTerms {
    const float *part[8];  // ce, lc, l1, l2, k1, k2, h1, h2 row partials (null: absent)
    float mul1[8], mul2[8];
    const uint32_t *hit;   // ce's row hits
    float cw, w1, w2, alpha;
};

__global__ void loss_totals_kernel(size_t n, LossTerms t, float *__restrict__ total,
                                   float *__restrict__ ce, uint32_t *__restrict__ correct) {
    __shared__ float term[8];
    __shared__ uint32_t hits;
    const int k = threadIdx.x;
    if (k < 8) {
        float s = 0.0f;
        uint32_t h = 0;
        const float *part = t.part[k];
        const uint32_t *hit = k == 0 ? t.hit : nullptr;
        if (part) {
            for (size_t i0 = 0; i0 < n; i0 += 16) {
                float v[16];
                uint32_t u16[16];
#pragma unroll
                for (int u = 0; u < 16; u++) {
                    const size_t i = min(i0 + u, n - 1);
                    v[u] = part[i];
                    u16[u] = hit ? hit[i] : 0u;
                }
#pragma unroll
                for (int u = 0; u < 16; u++)
                    if (i0 + u < n) {
                        s += v[u];
                        h += u16[u];
                    }
            }
        }
        term[k] = s * t.mul1[k] * t.mul2[k];
        if (k == 0) hits = h;
    }
    __syncthreads();
    if (k != 0) return;
    float tot = term[0];
    if (t.part[1]) tot += t.cw * term[1];
    if (t.part[2]) tot += t.w1 * term[2] + t.w2 * term[3];
    if (t.part[4]) tot += t.alpha * (term[4] + term[5]);
    if (t.part[6]) tot += term[6] + term[7];
    if (total) *total = tot;
    if (ce) *ce = term[0];
    if (correct) *correct = hits;
}

__global__ void fill_zero_kernel(float *__restrict__ x, size_t len) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < len;
         i += (size_t)gridDim.x * blockDim.x)
        x[i] = 0.0f;
}

}  // namespace

extern "C" {

int rnn_build_loss(rnn_ctx *ctx, size_t n, size_t nf, size_t nc, size_t d4, const float *tf,
                   const float *tc, const uint32_t *hard, const uint32_t *hardc,
                   const rnn_loss_cfg *cfg, const rnn_loss_io *io, float *total, float *ce,
                   uint32_t *correct) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (!cfg || !io) return rnn_fail(ctx, RNN_E_NULL, "build_loss: null cfg or io");
    if (n == 0) return RNN_OK;
    const bool coarse = cfg->coarse_w > 0.0f && cfg->taxo;
    const bool exits = io->e1 != nullptr;
    if (!io->logits || !io->dlogits || !tf || !hard)
        return rnn_fail(ctx, RNN_E_NULL, "build_loss: null logits / targets");
    if (nc && !io->dcoarse) return rnn_fail(ctx, RNN_E_NULL, "build_loss: null dcoarse");
    if (coarse && (!io->coarse || !tc || !hardc))
        return rnn_fail(ctx, RNN_E_NULL, "build_loss: null coarse operand");
    if (exits && (!io->e2 || !io->de1 || !io->de2 || !io->h1 || !io->h2 || !io->feat ||
                  !io->dh1 || !io->dh2))
        return rnn_fail(ctx, RNN_E_NULL, "build_loss: null exit operand");
    if (!rows_ok(ctx, n, nf, "build_loss") || (nc && !rows_ok(ctx, n, nc, "build_loss")) ||
        (exits && !rows_ok(ctx, n, d4, "build_loss")))
        return RNN_E_INVALID;
    WsCarve cv;
    size_t o_part[8];
    for (int k = 0; k < 8; k++) o_part[k] = cv.take(n * sizeof(float));
    const size_t o_hit = cv.take(n * sizeof(uint32_t));
    char *ws = (char *)rnn_workspace(ctx, cv.off);
    if (!ws) return RNN_E_NOMEM;
    LossTerms t;
    std::memset(&t, 0, sizeof(t));
    float *part[8];
    for (int k = 0; k < 8; k++) {
        part[k] = (float *)(ws + o_part[k]);
        t.mul1[k] = 1.0f / (float)n;
        t.mul2[k] = 1.0f;
    }
    uint32_t *hit = (uint32_t *)(ws + o_hit);
    t.hit = hit;
    t.cw = cfg->coarse_w;
    t.w1 = cfg->exit_w1;
    t.w2 = cfg->exit_w2;
    t.alpha = cfg->alpha;
    const unsigned rows = (unsigned)rnn_div_up(n, (size_t)(NT / 64));
    auto zero = [&](float *x, size_t len) {
        fill_zero_kernel<<<(unsigned)std::min<size_t>(rnn_div_up(len, 256), 1024), 256, 0,
                           ctx->stream>>>(x, len);
    };
    // loss::ce_soft(&out.logits, tf, hard, nf, 1.0, &mut g.logits)
    ce_soft_kernel<<<rows, NT, 0, ctx->stream>>>(n, (int)nf, io->logits, tf, hard, 1.0f,
                                                 io->dlogits, part[0], hit);
    t.part[0] = part[0];
    if (coarse) {
        ce_soft_kernel<<<rows, NT, 0, ctx->stream>>>(n, (int)nc, io->coarse, tc, hardc,
                                                     cfg->coarse_w, io->dcoarse, part[1], nullptr);
        t.part[1] = part[1];
    } else if (nc) {
        zero(io->dcoarse, n * nc);
    }
    if (exits) {
        ce_soft_kernel<<<rows, NT, 0, ctx->stream>>>(n, (int)nf, io->e1, tf, hard, cfg->exit_w1,
                                                     io->de1, part[2], nullptr);
        ce_soft_kernel<<<rows, NT, 0, ctx->stream>>>(n, (int)nf, io->e2, tf, hard, cfg->exit_w2,
                                                     io->de2, part[3], nullptr);
        t.part[2] = part[2];
        t.part[3] = part[3];
        if (cfg->alpha > 0.0f) {
            kl_distill_kernel<<<rows, NT, 0, ctx->stream>>>(n, (int)nf, io->e1, io->logits,
                                                            cfg->temp, cfg->alpha, io->de1,
                                                            part[4]);
            kl_distill_kernel<<<rows, NT, 0, ctx->stream>>>(n, (int)nf, io->e2, io->logits,
                                                            cfg->temp, cfg->alpha, io->de2,
                                                            part[5]);
            t.part[4] = part[4];
            t.part[5] = part[5];
        }
        if (cfg->beta > 0.0f) {
            hint_mse_kernel<true><<<rows, NT, 0, ctx->stream>>>(n, (int)d4, io->h1, io->feat,
                                                                cfg->beta, io->dh1, part[6]);
            hint_mse_kernel<true><<<rows, NT, 0, ctx->stream>>>(n, (int)d4, io->h2, io->feat,
                                                                cfg->beta, io->dh2, part[7]);
            t.part[6] = part[6];
            t.part[7] = part[7];
            t.mul1[6] = t.mul1[7] = 1.0f / (float)(n * d4);
            t.mul2[6] = t.mul2[7] = cfg->beta;
        } else {
            zero(io->dh1, n * d4);
            zero(io->dh2, n * d4);
        }
    }
    loss_totals_kernel<<<1, 64, 0, ctx->stream>>>(n, t, total, ce, correct);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

}  // extern "C"
