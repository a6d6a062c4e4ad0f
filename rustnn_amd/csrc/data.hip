// data.rs on the device: CIFAR-100 batch assembly (crop, flip, normalise,
// random erasing) from the raw u8 images held in HBM, the evaluation batch,
// and the mixup / cutmix blend of mix_batch.
//
// Reference: make_batch_train (data.rs:384-416), crop_offset /
// crop_flip_normalize / normalize_row / random_erase (data.rs:316-382),
// make_batch_eval (data.rs:494-512), mix_batch / cutmix / mixup / beta_like
// (data.rs:418-492).  Every image of a training batch has its own generator,
// Rng::new(seed ^ b * 0x9E3779B97F4A7C15), so one workgroup per image draws
// exactly the reference's numbers (one thread runs the generator; the pixels
// are spread over the workgroup), including RandAugment (data.rs:102-314)
// on an LDS copy of the image.
#include "rnn_internal.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#pragma clang fp contract(off)

namespace {

constexpr int IMG = 32, CH = 3, PIX = CH * IMG * IMG, NT = 256;
constexpr int MAX_ERASE = 32;  // erase side limit (the rectangle is at most 32 x 32)
constexpr int MAX_RA = 16;     // RandAugment operations per image

__device__ __forceinline__ float mean_of(int c) {
    return c == 0 ? 0.5071f : (c == 1 ? 0.4865f : 0.4409f);
}
__device__ __forceinline__ float std_of(int c) {
    return c == 0 ? 0.2673f : (c == 1 ? 0.2564f : 0.2762f);
}

// norm (data.rs:96-98).
__device__ __forceinline__ float norm_px(uint8_t v, int c) {
    return ((float)v / 255.0f - mean_of(c)) / std_of(c);
}

// crop_flip_normalize (data.rs:331-362) of one image into dst, spread over
// the workgroup: out-of-image pixels take -mean/std (the zero of the scale).
__device__ void crop_flip_normalize(const uint8_t *src, float *dst, int dy, int dx, bool flip) {
    for (int e = threadIdx.x; e < PIX; e += NT) {
        const int c = e / (IMG * IMG), y = (e / IMG) % IMG, x = e % IMG;
        const float border = -mean_of(c) / std_of(c);
        const int sy = y + dy;
        const int sx = (flip ? IMG - 1 - x : x) + dx;
        dst[e] = (sy >= 0 && sy < IMG && sx >= 0 && sx < IMG)
                     ? norm_px(src[c * IMG * IMG + sy * IMG + sx], c)
                     : border;
    }
}

// ---- RandAugment (data.rs:102-314) on the workgroup's LDS copy of one image.
__device__ __forceinline__ uint8_t px(const uint8_t *im, int c, int y, int x) {
    if (y < 0 || x < 0 || y >= IMG || x >= IMG) return 128;
    return im[c * IMG * IMG + y * IMG + x];
}

// v.clamp(0, 255) as u8 (a NaN goes to 0, as Rust's saturating cast).
__device__ __forceinline__ uint8_t sat_u8(float v) {
    if (!(v > 0.0f)) return 0;
    return (uint8_t)fminf(v, 255.0f);
}

// affine (data.rs:114-135): inverse mapping with bilinear interpolation,
// outside pixels 128.  im is rewritten from the copy src.
__device__ void affine(uint8_t *im, const uint8_t *src, float a, float b, float tx, float c_,
                       float d, float ty) {
    const float cy = (float)IMG / 2.0f - 0.5f, cx = (float)IMG / 2.0f - 0.5f;
    for (int e = threadIdx.x; e < PIX; e += NT) {
        const int ch = e / (IMG * IMG), y = (e / IMG) % IMG, x = e % IMG;
        const float fy = (float)y - cy, fx = (float)x - cx;
        const float sx = a * fx + b * fy + tx + cx;
        const float sy = c_ * fx + d * fy + ty + cy;
        const float x0f = floorf(sx), y0f = floorf(sy);
        const float wx = sx - x0f, wy = sy - y0f;
        const int x0 = (int)x0f, y0 = (int)y0f;
        const float v = (float)px(src, ch, y0, x0) * (1.0f - wx) * (1.0f - wy) +
                        (float)px(src, ch, y0, x0 + 1) * wx * (1.0f - wy) +
                        (float)px(src, ch, y0 + 1, x0) * (1.0f - wx) * wy +
                        (float)px(src, ch, y0 + 1, x0 + 1) * wx * wy;
        im[e] = sat_u8(v);
    }
}

// blend (data.rs:137-142) of im toward `other` by f.
__device__ void blend(uint8_t *im, const uint8_t *other, float f) {
    for (int e = threadIdx.x; e < PIX; e += NT)
        im[e] = sat_u8((float)other[e] + f * ((float)im[e] - (float)other[e]));
}

// grayscale (data.rs:144-158) into g (all three planes).
__device__ void grayscale(const uint8_t *im, uint8_t *g) {
    for (int p = threadIdx.x; p < IMG * IMG; p += NT) {
        const float v = 0.299f * (float)im[p] + 0.587f * (float)im[IMG * IMG + p] +
                        0.114f * (float)im[2 * IMG * IMG + p];
        const uint8_t u = sat_u8(v);
        for (int c = 0; c < CH; c++) g[c * IMG * IMG + p] = u;
    }
}

// apply_op (data.rs:255-278) for operation op with magnitude v and the sign
// already drawn.  work is the image; src, tmp scratch images; hist / red
// scratch words; every thread of the workgroup calls it.
__device__ void apply_op(uint8_t *work, uint8_t *src, uint8_t *tmp, uint32_t *hist, int op,
                         float v, float sign) {
    const float f = 1.0f + sign * 0.9f * v;
    const int tid = threadIdx.x;
    if (op <= 4) {
        for (int e = tid; e < PIX; e += NT) src[e] = work[e];
        __syncthreads();
        if (op == 0) affine(work, src, 1.0f, sign * 0.3f * v, 0.0f, 0.0f, 1.0f, 0.0f);
        else if (op == 1) affine(work, src, 1.0f, 0.0f, 0.0f, sign * 0.3f * v, 1.0f, 0.0f);
        else if (op == 2) affine(work, src, 1.0f, 0.0f, sign * 10.0f * v, 0.0f, 1.0f, 0.0f);
        else if (op == 3) affine(work, src, 1.0f, 0.0f, 0.0f, 0.0f, 1.0f, sign * 10.0f * v);
        else {
            const float t = sign * 30.0f * v * 3.14159265358979323846f / 180.0f;
            const float ct = rnn_dev_cosf(t), st = rnn_dev_sinf(t);
            affine(work, src, ct, -st, 0.0f, st, ct, 0.0f);
        }
    } else if (op == 5) {  // posterize
        const unsigned bits = 8u - (unsigned)(4.0f * v);
        const uint8_t mask = (uint8_t)~((1u << (8 - bits)) - 1u);
        for (int e = tid; e < PIX; e += NT) work[e] &= mask;
    } else if (op == 6) {  // solarize
        const uint8_t th = sat_u8(255.0f * (1.0f - v));
        for (int e = tid; e < PIX; e += NT)
            if (work[e] >= th) work[e] = (uint8_t)(255 - work[e]);
    } else if (op == 7) {  // autocontrast: per channel min / max
        if (tid < 2 * CH) hist[tid] = tid < CH ? 255u : 0u;
        __syncthreads();
        for (int e = tid; e < PIX; e += NT) {
            const int c = e / (IMG * IMG);
            atomicMin(&hist[c], (uint32_t)work[e]);
            atomicMax(&hist[CH + c], (uint32_t)work[e]);
        }
        __syncthreads();
        for (int e = tid; e < PIX; e += NT) {
            const int c = e / (IMG * IMG);
            const uint32_t lo = hist[c], hi = hist[CH + c];
            if (hi > lo) {
                const float k = 255.0f / (float)(hi - lo);
                work[e] = sat_u8((float)(work[e] - lo) * k);
            }
        }
    } else if (op == 8) {  // equalize: per channel histogram, cdf, lowest non-zero
        for (int e = tid; e < CH * 256; e += NT) hist[e] = 0;
        __syncthreads();
        for (int e = tid; e < PIX; e += NT) atomicAdd(&hist[(e / (IMG * IMG)) * 256 + work[e]], 1u);
        __syncthreads();
        if (tid < CH) {
            uint32_t *h = hist + tid * 256, acc = 0, lo = 0;
            for (int i = 0; i < 256; i++) h[i] = acc += h[i];  // cdf in place
            for (int i = 0; i < 256; i++)
                if (h[i] > 0) {
                    lo = h[i];
                    break;
                }
            hist[CH * 256 + tid] = lo;
        }
        __syncthreads();
        for (int e = tid; e < PIX; e += NT) {
            const int c = e / (IMG * IMG);
            const uint32_t lo = hist[CH * 256 + c];
            uint32_t den = IMG * IMG > lo ? IMG * IMG - lo : 0;
            den = den < 1 ? 1 : den;
            work[e] = (uint8_t)(((hist[c * 256 + work[e]] - lo) * 255u) / den);
        }
    } else if (op == 9) {  // brightness: blend with black
        for (int e = tid; e < PIX; e += NT) tmp[e] = 0;
        __syncthreads();
        blend(work, tmp, f);
    } else if (op == 10) {  // saturation: blend with the grayscale image
        grayscale(work, tmp);
        __syncthreads();
        blend(work, tmp, f);
    } else if (op == 11) {  // contrast: blend with the grayscale mean
        if (tid == 0) hist[0] = 0;
        grayscale(work, tmp);
        __syncthreads();
        for (int p = tid; p < IMG * IMG; p += NT) atomicAdd(&hist[0], (uint32_t)tmp[p]);
        __syncthreads();
        const uint8_t mean = (uint8_t)(hist[0] / (IMG * IMG));
        for (int e = tid; e < PIX; e += NT) tmp[e] = mean;
        __syncthreads();
        blend(work, tmp, f);
    } else {  // sharpness: blend with the 3x3 blur of the interior (data.rs:226-253)
        for (int e = tid; e < PIX; e += NT) src[e] = work[e];
        __syncthreads();
        for (int e = tid; e < PIX; e += NT) {
            const int c = e / (IMG * IMG), y = (e / IMG) % IMG, x = e % IMG;
            uint8_t val = src[e];
            if (y >= 1 && y < IMG - 1 && x >= 1 && x < IMG - 1) {
                float sm = 0.0f;
                for (int dy = 0; dy < 3; dy++)
                    for (int dx = 0; dx < 3; dx++) {
                        const float w = (dy == 1 && dx == 1) ? 5.0f : 1.0f / 8.0f * 3.0f;
                        sm += w * (float)px(src, c, y + dy - 1, x + dx - 1);
                    }
                val = sat_u8(sm / 8.0f);
            }
            tmp[e] = val;
        }
        __syncthreads();
        blend(work, tmp, f);
    }
    __syncthreads();
}

// make_batch_train for batch slot b = blockIdx.x (data.rs:396-415): the
// image's generator gives the crop offsets, the flip, and the random
// erasing's decision, centre and noise (in the reference's draw order).  An
// index past the dataset gives a NaN image and label 0xffffffff (the
// reference would panic).
__global__ __launch_bounds__(NT) void cifar_train_kernel(
    const uint8_t *__restrict__ images, const uint8_t *__restrict__ fine,
    const uint8_t *__restrict__ coarse, size_t nimg, const uint32_t *__restrict__ idx, int pad,
    float ra_mag, int ra_n, float erase, int erase_side, uint64_t seed, float *__restrict__ out,
    uint32_t *__restrict__ labels, uint32_t *__restrict__ coarse_out) {
    __shared__ int prm[7];  // dy, dx, flip, erase?, y0, y1, x0 (x1 in x1s)
    __shared__ int x1s;
    __shared__ float noise[CH * MAX_ERASE * MAX_ERASE];
    __shared__ uint8_t work[PIX], src[PIX], tmp[PIX];
    __shared__ uint32_t hist[CH * 256 + CH];
    __shared__ int ops[MAX_RA];
    __shared__ float opv[MAX_RA], ops_sign[MAX_RA];
    const int b = blockIdx.x;
    const uint32_t i = idx[b];
    float *dst = out + (size_t)b * PIX;
    if (i >= nimg) {
        for (int e = threadIdx.x; e < PIX; e += NT) dst[e] = NAN;
        if (threadIdx.x == 0) {
            labels[b] = 0xffffffffu;
            coarse_out[b] = 0xffffffffu;
        }
        return;
    }
    for (int e = threadIdx.x; e < PIX; e += NT) work[e] = images[(size_t)i * PIX + e];
    if (threadIdx.x == 0) {
        labels[b] = fine[i];
        coarse_out[b] = coarse[i];
        RnnRng rng(seed ^ ((uint64_t)b * 0x9E3779B97F4A7C15ull));
        // randaugment's draws (data.rs:303-314, 255-257): the op, the
        // magnitude around ra_mag, then apply_op's sign
        for (int k = 0; k < (ra_mag > 0.0f ? ra_n : 0); k++) {
            ops[k] = (int)rng.below(13);
            opv[k] = fminf(fmaxf(ra_mag * (1.0f + 0.5f * rng.normal()), 0.0f), 1.0f);
            ops_sign[k] = (rng.next_u32() & 1u) == 1u ? 1.0f : -1.0f;
        }
        int dy = 0, dx = 0;
        if (pad > 0) {  // crop_offset (data.rs:316-325)
            dy = (int)rng.below(2 * (uint64_t)pad + 1) - pad;
            dx = (int)rng.below(2 * (uint64_t)pad + 1) - pad;
        }
        const int flip = (rng.next_u32() & 1u) == 1u;
        int er = 0, y0 = 0, y1 = 0, x0 = 0, x1 = 0;
        if (erase > 0.0f && !(rng.uniform() >= erase)) {  // random_erase (data.rs:364-382)
            const int cy = (int)rng.below(IMG), cx = (int)rng.below(IMG);
            const int h = erase_side / 2;
            y0 = max(cy - h, 0);
            y1 = min(cy + h, IMG);
            x0 = max(cx - h, 0);
            x1 = min(cx + h, IMG);
            er = 1;
            int k = 0;
            for (int c = 0; c < CH; c++)
                for (int y = y0; y < y1; y++)
                    for (int x = x0; x < x1; x++) noise[k++] = rng.normal();
        }
        prm[0] = dy;
        prm[1] = dx;
        prm[2] = flip;
        prm[3] = er;
        prm[4] = y0;
        prm[5] = y1;
        prm[6] = x0;
        x1s = x1;
    }
    __syncthreads();
    for (int k = 0; k < (ra_mag > 0.0f ? ra_n : 0); k++)
        apply_op(work, src, tmp, hist, ops[k], opv[k], ops_sign[k]);
    crop_flip_normalize(work, dst, prm[0], prm[1], prm[2] != 0);
    if (prm[3]) {
        const int y0 = prm[4], y1 = prm[5], x0 = prm[6], x1 = x1s;
        const int hh = y1 - y0, ww = x1 - x0;
        __syncthreads();  // the crop's writes to dst before the rectangle's
        for (int k = threadIdx.x; k < CH * hh * ww; k += NT) {
            const int c = k / (hh * ww), y = y0 + (k / ww) % hh, x = x0 + k % ww;
            dst[c * IMG * IMG + y * IMG + x] = noise[k];
        }
    }
}

// make_batch_eval (data.rs:494-512): images start .. start + bs normalised,
// mirrored when flip (test-time augmentation).
__global__ __launch_bounds__(NT) void cifar_eval_kernel(const uint8_t *__restrict__ images,
                                                        const uint8_t *__restrict__ fine,
                                                        size_t start, int flip,
                                                        float *__restrict__ out,
                                                        uint32_t *__restrict__ labels) {
    const size_t b = blockIdx.x;
    crop_flip_normalize(images + (start + b) * PIX, out + b * PIX, 0, 0, flip != 0);
    if (threadIdx.x == 0 && labels) labels[b] = fine[start + b];
}

// mixup (data.rs:456-467): out[b] = l x[b] + (1 - l) x[perm[b]]; cutmix
// (data.rs:434-454): out[b] = x[b] with the rectangle [y0, y1) x [x0, x1) of
// every channel taken from x[perm[b]].  out must not alias x.
__global__ void mix_kernel(const float *__restrict__ x, float *__restrict__ out, size_t bs,
                           const uint32_t *__restrict__ perm, int cut, float l, int y0, int y1,
                           int x0, int x1) {
    const size_t len = bs * PIX;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < len;
         e += (size_t)gridDim.x * blockDim.x) {
        const size_t b = e / PIX;
        const int o = (int)(e - b * PIX);
        if (perm[b] >= bs) {  // not a permutation of the batch: no out-of-range read
            out[e] = NAN;
            continue;
        }
        const size_t p = (size_t)perm[b] * PIX + o;
        if (cut) {
            const int y = (o / IMG) % IMG, xx = o % IMG;
            out[e] = (y >= y0 && y < y1 && xx >= x0 && xx < x1) ? x[p] : x[e];
        } else {
            out[e] = l * x[e] + (1.0f - l) * x[p];
        }
    }
}

// beta_like (data.rs:418-429).
float beta_like(float a, RnnRng &rng) {
    const float u = rng.uniform();
    if (a >= 1.0f) return u;
    if (u < 0.5f) return powf(2.0f * u, 1.0f / a) * 0.5f;
    return 1.0f - powf(2.0f * (1.0f - u), 1.0f / a) * 0.5f;
}

}  // namespace

extern "C" {

int rnn_cifar_batch_train(rnn_ctx *ctx, const uint8_t *images, const uint8_t *fine,
                          const uint8_t *coarse, size_t nimg, const uint32_t *idx, size_t bs,
                          size_t pad, float ra_mag, size_t ra_n, float erase, size_t erase_side,
                          uint64_t seed, float *out, uint32_t *labels, uint32_t *coarse_out) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (bs == 0) return RNN_OK;
    if (!images || !fine || !coarse || !idx || !out || !labels || !coarse_out)
        return rnn_fail(ctx, RNN_E_NULL, "cifar_batch_train: null operand");
    if (pad > IMG || erase_side > MAX_ERASE || bs > 0x7fffffff || ra_n > (size_t)MAX_RA)
        return rnn_fail(ctx, RNN_E_INVALID,
                        "cifar_batch_train: pad %zu, erase side %zu, bs %zu, ra_n %zu (<= %d)",
                        pad, erase_side, bs, ra_n, MAX_RA);
    cifar_train_kernel<<<(unsigned)bs, NT, 0, ctx->stream>>>(
        images, fine, coarse, nimg, idx, (int)pad, ra_mag, (int)ra_n, erase, (int)erase_side, seed,
        out, labels, coarse_out);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

int rnn_cifar_batch_eval(rnn_ctx *ctx, const uint8_t *images, const uint8_t *fine, size_t nimg,
                         size_t start, size_t bs, int flip, float *out, uint32_t *labels) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (bs == 0) return RNN_OK;
    if (!images || !out || (labels && !fine))
        return rnn_fail(ctx, RNN_E_NULL, "cifar_batch_eval: null operand");
    if (start > nimg || bs > nimg - start || bs > 0x7fffffff)
        return rnn_fail(ctx, RNN_E_INVALID, "cifar_batch_eval: images %zu..%zu of %zu", start,
                        start + bs, nimg);
    cifar_eval_kernel<<<(unsigned)bs, NT, 0, ctx->stream>>>(images, fine, start, flip, out,
                                                            labels);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

uint64_t rnn_fnv1a_bytes(uint64_t hash, const uint8_t *bytes, size_t n) {
    // FNV-1a 64 (ckpt.rs:84-97, train.rs:476-483)
    for (size_t i = 0; i < n; i++) {
        hash ^= bytes[i];
        hash *= 0x00000100000001B3ull;
    }
    return hash;
}

uint64_t rnn_fnv1a_f32(uint64_t hash, const float *values, size_t n) {
    // fnv_f32 (train.rs:478-484): each value's bits as 4 little-endian bytes
    for (size_t i = 0; i < n; i++) {
        uint32_t b;
        std::memcpy(&b, values + i, 4);
        for (int k = 0; k < 4; k++) {
            hash ^= (b >> (8 * k)) & 0xffu;
            hash *= 0x00000100000001B3ull;
        }
    }
    return hash;
}

int rnn_rng_seed(uint64_t seed, uint64_t *state) {
    if (!state) return RNN_E_NULL;
    RnnRng r(seed);
    for (int k = 0; k < 4; k++) state[k] = r.s[k];
    return RNN_OK;
}

uint64_t rnn_rng_next_u64(uint64_t *state) {
    if (!state) return 0;
    RnnRng r(0);
    for (int k = 0; k < 4; k++) r.s[k] = state[k];
    const uint64_t v = r.next();
    for (int k = 0; k < 4; k++) state[k] = r.s[k];
    return v;
}

int rnn_rng_normal_vec(uint64_t *state, size_t n, float scale, float *out) {
    if (!state || (n && !out)) return RNN_E_NULL;
    // rand_vec (rng.rs:70-72) times scale: Param::kaiming (nn.rs:95-100)
    // passes scale = sqrt(2 / fan_in) as f32, rand_vec passes 1.
    RnnRng r(0);
    for (int k = 0; k < 4; k++) r.s[k] = state[k];
    for (size_t i = 0; i < n; i++) out[i] = r.normal() * scale;
    for (int k = 0; k < 4; k++) state[k] = r.s[k];
    return RNN_OK;
}

int rnn_rng_trunc_normal(uint64_t *state, size_t n, float std_, float *out) {
    if (!state || (n && !out)) return RNN_E_NULL;
    // Param::trunc_normal (nn.rs:77-89): up to 8 redraws while |z| > 2, then
    // clamp to [-2, 2] and scale.
    RnnRng r(0);
    for (int k = 0; k < 4; k++) r.s[k] = state[k];
    for (size_t i = 0; i < n; i++) {
        float z = r.normal();
        for (int tries = 0; fabsf(z) > 2.0f && tries < 8; tries++) z = r.normal();
        out[i] = fminf(fmaxf(z, -2.0f), 2.0f) * std_;
    }
    for (int k = 0; k < 4; k++) state[k] = r.s[k];
    return RNN_OK;
}

int rnn_mix_plan(uint64_t *rng_state, size_t bs, float alpha_mix, float alpha_cut, float sw,
                 uint32_t *perm, float *lam, int *cut, float *l, int *rect) {
    if (!rng_state || !perm || !lam || !cut || !l || !rect) return RNN_E_NULL;
    // mix_batch (data.rs:469-492) on the host, from the caller's generator
    RnnRng rng(0);
    for (int k = 0; k < 4; k++) rng.s[k] = rng_state[k];
    std::vector<size_t> p(bs);
    for (size_t i = 0; i < bs; i++) p[i] = i;
    for (size_t i = bs; i-- > 1;) std::swap(p[i], p[(size_t)rng.below(i + 1)]);  // shuffle
    for (size_t i = 0; i < bs; i++) {
        perm[i] = (uint32_t)p[i];
        lam[i] = 1.0f;
    }
    *cut = 0;
    *l = 1.0f;
    rect[0] = rect[1] = rect[2] = rect[3] = 0;
    if (alpha_mix > 0.0f || alpha_cut > 0.0f) {
        const int c = alpha_cut > 0.0f && (alpha_mix <= 0.0f || rng.uniform() < sw);
        const float lv = beta_like(c ? alpha_cut : alpha_mix, rng);
        *cut = c;
        *l = lv;
        if (c) {  // cutmix's rectangle and the area left (data.rs:434-442)
            const float r = sqrtf(1.0f - lv);
            const size_t side = std::min<size_t>((size_t)((float)IMG * r), IMG);
            const size_t cy = (size_t)rng.below(IMG), cx = (size_t)rng.below(IMG);
            const size_t y0 = cy >= side / 2 ? cy - side / 2 : 0, y1 = std::min<size_t>(cy + side / 2, IMG);
            const size_t x0 = cx >= side / 2 ? cx - side / 2 : 0, x1 = std::min<size_t>(cx + side / 2, IMG);
            const float area = (float)((y1 - y0) * (x1 - x0)) / (float)(IMG * IMG);
            rect[0] = (int)y0;
            rect[1] = (int)y1;
            rect[2] = (int)x0;
            rect[3] = (int)x1;
            for (size_t i = 0; i < bs; i++) lam[i] = 1.0f - area;
        } else {
            for (size_t i = 0; i < bs; i++) lam[i] = lv;
        }
    }
    for (int k = 0; k < 4; k++) rng_state[k] = rng.s[k];
    return RNN_OK;
}

int rnn_mix_apply(rnn_ctx *ctx, const float *x, float *out, size_t bs, const uint32_t *perm,
                  int cut, float l, const int *rect) {
    if (!ctx) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (bs == 0) return RNN_OK;
    if (!x || !out || !perm || (cut && !rect))
        return rnn_fail(ctx, RNN_E_NULL, "mix_apply: null operand");
    if (x == out) return rnn_fail(ctx, RNN_E_INVALID, "mix_apply: out must not alias x");
    const int y0 = cut ? rect[0] : 0, y1 = cut ? rect[1] : 0;
    const int x0 = cut ? rect[2] : 0, x1 = cut ? rect[3] : 0;
    const size_t len = bs * PIX;
    const unsigned grid = (unsigned)std::min<size_t>(rnn_div_up(len, NT), 16384);
    mix_kernel<<<grid, NT, 0, ctx->stream>>>(x, out, bs, perm, cut, l, y0, y1, x0, x1);
    RNN_LAUNCHED(ctx);
    return RNN_OK;
}

}  // extern "C"
