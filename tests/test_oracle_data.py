"""Pins of the oracle's data.rs restatement (oracle/orc_data.c) and the host
side of rustnn_amd/data.py.

The reference's own data tests (data.rs:514-622) restated: no shift is pure
normalisation, the flip mirrors columns, a full-image shift leaves only the
border, beta_like stays in [0, 1], mix off is the identity with lam = 1 and
a permutation, mix on gives lam in [0, 1] and finite pixels.  The training
batch is pinned to a numpy statement of crop / flip / normalise driven by the
oracle Rng (itself pinned to a big-int xoshiro256++); the binary reader to
records written here."""
import numpy as np
import pytest

MEAN = np.array([0.5071, 0.4865, 0.4409], np.float32)
STD = np.array([0.2673, 0.2564, 0.2762], np.float32)


def ramp():
    """rampa (data.rs:521-523): every pixel codes its position."""
    return (np.arange(3 * 32 * 32) % 251).astype(np.uint8)


def norm_np(v, c):
    return ((np.float32(v) / np.float32(255.0) - MEAN[c]) / STD[c]).astype(np.float32)


def test_no_shift_is_normalisation(orc):
    src = ramp()
    dst = orc.crop_flip_normalize(src, 0, 0, False).reshape(3, 1024)
    for c in range(3):
        assert np.array_equal(dst[c], norm_np(src.reshape(3, 1024)[c], c))


def test_flip_mirrors_columns(orc):
    src = ramp()
    a = orc.crop_flip_normalize(src, 0, 0, False).reshape(3, 32, 32)
    b = orc.crop_flip_normalize(src, 0, 0, True).reshape(3, 32, 32)
    assert np.array_equal(b, a[:, :, ::-1])
    assert not np.array_equal(a, b)


def test_full_shift_leaves_border(orc):
    dst = orc.crop_flip_normalize(ramp(), 32, 0, False).reshape(3, 1024)
    for c in range(3):
        assert (dst[c] == np.float32(-MEAN[c] / STD[c])).all()


def test_train_batch_matches_numpy_crop(orc):
    rng = np.random.default_rng(0)
    n, bs, seed = 40, 12, 0xC0FFEE
    images = rng.integers(0, 256, (n, 3, 32, 32), dtype=np.uint8)
    fine = rng.integers(0, 100, n).astype(np.uint8)
    coarse = (fine // 5).astype(np.uint8)
    idx = rng.integers(0, n, bs).astype(np.uint32)
    x, lab, co = orc.cifar_batch_train(images, fine, coarse, idx, 4, 0.0, 8, seed)
    assert np.array_equal(lab, fine[idx]) and np.array_equal(co, coarse[idx])
    for b in range(bs):
        r = orc.Rng(seed ^ ((b * 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF))
        dy, dx = r.below(9) - 4, r.below(9) - 4
        flip = r.next_u64() >> 32 & 1
        img = images[idx[b]]
        want = np.empty((3, 32, 32), np.float32)
        for c in range(3):
            want[c] = -MEAN[c] / STD[c]
            for y in range(32):
                sy = y + dy
                if not 0 <= sy < 32:
                    continue
                for xx in range(32):
                    sx = (31 - xx if flip else xx) + dx
                    if 0 <= sx < 32:
                        want[c, y, xx] = norm_np(img[c, sy, sx], c)
        assert np.array_equal(x[b], want), b


def test_random_erase_rectangle(orc):
    images = np.full((1, 3, 32, 32), 128, np.uint8)
    x, _, _ = orc.cifar_batch_train(images, np.zeros(1, np.uint8), np.zeros(1, np.uint8),
                                    np.zeros(1, np.uint32), 0, 1.0, 8, 5)
    base = orc.crop_flip_normalize(images[0].ravel(), 0, 0, False).reshape(3, 32, 32)
    changed = (x[0] != base).any(0)
    ys, xs = np.nonzero(changed)
    assert 1 <= ys.max() - ys.min() + 1 <= 8 and 1 <= xs.max() - xs.min() + 1 <= 8


def test_mix_off_is_identity(orc):
    x = (np.arange(4 * 3072, dtype=np.float32) * 0.001).reshape(4, 3072)
    x0 = x.copy()
    perm, lam = orc.mix_batch(x, 0.0, 0.0, 0.5, orc.Rng(2))
    assert np.array_equal(x, x0) and (lam == 1.0).all()
    assert sorted(perm.tolist()) == [0, 1, 2, 3]


def test_mix_on_gives_valid_lambda(orc):
    r = orc.Rng(17)
    for m, c in ((0.8, 0.0), (0.0, 1.0), (0.8, 1.0)):
        x = ((np.arange(8 * 3072) % 97) * 0.01).astype(np.float32).reshape(8, 3072)
        perm, lam = orc.mix_batch(x, m, c, 0.5, r)
        assert ((lam >= 0) & (lam <= 1)).all() and np.isfinite(x).all()


def test_binary_reader_and_taxonomy(tmp_path):
    pytest.importorskip("torch")
    from rustnn_amd import data
    rng = np.random.default_rng(1)
    n = 7
    fine = rng.integers(0, 100, n).astype(np.uint8)
    fine[:] = np.array([0, 5, 99, 5, 17, 0, 42])
    coarse = (fine // 5).astype(np.uint8)
    pix = rng.integers(0, 256, (n, 3072), dtype=np.uint8)
    rec = np.concatenate([coarse[:, None], fine[:, None], pix], 1)
    path = tmp_path / "train.bin"
    rec.tofile(path)
    raw = np.fromfile(path, np.uint8).reshape(-1, 3074)
    assert np.array_equal(raw[:, 2:], pix) and np.array_equal(raw[:, 1], fine)
    with pytest.raises(ValueError):
        bad = tmp_path / "bad.bin"
        rec.ravel()[:-1].tofile(bad)
        data.Dataset.from_bin(str(bad))


# ---- RandAugment (data.rs:102-314): each operation pinned by a closed form
# or an independent routine, so a wrong sign, axis or weight fails.
def _img(seed=5):
    return np.random.default_rng(seed).integers(0, 256, (3, 32, 32), dtype=np.uint8)


@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_ra_translate_is_an_integer_shift(orc, sign):
    im = _img()
    s = int(sign * 5)  # v = 0.5 -> 5 pixels; output(x) = input(x + s), border 128
    want_x = np.full_like(im, 128)
    want_y = np.full_like(im, 128)
    if s > 0:
        want_x[:, :, :32 - s] = im[:, :, s:]
        want_y[:, :32 - s, :] = im[:, s:, :]
    else:
        want_x[:, :, -s:] = im[:, :, :32 + s]
        want_y[:, -s:, :] = im[:, :32 + s, :]
    assert np.array_equal(orc.ra_op(im, 2, 0.5, sign), want_x)
    assert np.array_equal(orc.ra_op(im, 3, 0.5, sign), want_y)


@pytest.mark.parametrize("op", [0, 1, 2, 3, 4, 9, 10, 11, 12])
def test_ra_zero_magnitude_is_identity(orc, op):
    im = _img()
    # f = 1 for the blends; identity maps for the affine ops.  Saturation and
    # contrast blend with factor 1 exactly; the blends truncate other + 1*(im -
    # other), which is im for integers.
    assert np.array_equal(orc.ra_op(im, op, 0.0, 1.0), im)


def test_ra_rotation_matches_scipy_bilinear(orc):
    from scipy import ndimage
    im = _img()
    t = 30.0 * np.pi / 180.0  # v = 1, sign + : output(y, x) samples R(t) (x, y)
    c, s = np.cos(t), np.sin(t)
    got = orc.ra_op(im, 4, 1.0, 1.0).astype(np.int32)
    ctr = 15.5
    # scipy maps output (row, col) -> input matrix @ (row, col) + offset
    mat = np.array([[c, s], [-s, c]])
    off = np.array([ctr, ctr]) - mat @ np.array([ctr, ctr])
    for ch in range(3):
        want = ndimage.affine_transform(im[ch].astype(np.float64), mat, off, order=1,
                                        mode="constant", cval=128.0)
        # inside, both are bilinear; the reference truncates
        inner = np.zeros((32, 32), bool)
        inner[6:26, 6:26] = True
        assert np.abs(got[ch][inner] - np.floor(want[inner] + 1e-3)).max() <= 1


def test_ra_posterize_solarize(orc):
    im = _img()
    assert np.array_equal(orc.ra_op(im, 5, 1.0, 1.0), im & 0xF0)   # 4 bits kept
    assert np.array_equal(orc.ra_op(im, 5, 0.0, 1.0), im)          # 8 bits
    assert np.array_equal(orc.ra_op(im, 6, 1.0, 1.0), 255 - im)    # threshold 0
    th = int(255 * 0.5)
    assert np.array_equal(orc.ra_op(im, 6, 0.5, 1.0), np.where(im >= th, 255 - im, im))


def test_ra_autocontrast_and_equalize(orc):
    rng = np.random.default_rng(6)
    im = rng.integers(60, 140, (3, 32, 32), dtype=np.uint8)
    ac = orc.ra_op(im, 7, 0.3, 1.0).astype(np.int64)
    for ch in range(3):
        lo, hi = int(im[ch].min()), int(im[ch].max())
        assert ac[ch].min() == 0 and ac[ch].max() == 255
        assert np.array_equal(ac[ch], ((im[ch].astype(np.float32) - lo) *
                                       np.float32(255.0 / (hi - lo))).astype(np.int64))
    eq = orc.ra_op(im, 8, 0.3, 1.0).astype(np.int64)
    for ch in range(3):
        # textbook histogram equalisation: (cdf(p) - cdf_min) * 255 // (N - cdf_min)
        hist = np.bincount(im[ch].ravel(), minlength=256)
        cdf = np.cumsum(hist)
        cmin = cdf[cdf > 0][0]
        want = (cdf[im[ch]] - cmin) * 255 // (1024 - cmin)
        assert np.array_equal(eq[ch], want)
        assert eq[ch].max() == 255
    flat = np.full((3, 32, 32), 77, np.uint8)  # one level: autocontrast keeps it
    assert np.array_equal(orc.ra_op(flat, 7, 0.3, 1.0), flat)


def test_ra_brightness_contrast_sharpness_closed_forms(orc):
    im = _img()
    f = np.float32(1.0 + 0.9 * 0.5)
    assert np.array_equal(orc.ra_op(im, 9, 0.5, 1.0),
                          np.clip(f * im.astype(np.float32), 0, 255).astype(np.uint8))
    flat = np.full((3, 32, 32), 90, np.uint8)
    # a constant image: the 3x3 blur (5 + 8 * 3/8) / 8 = 1 and the grayscale
    # mean leave it fixed, so sharpness and contrast return it for any factor
    assert np.array_equal(orc.ra_op(flat, 12, 1.0, -1.0), flat)
    gray = np.repeat(np.random.default_rng(7).integers(0, 256, (1, 32, 32), dtype=np.uint8),
                     3, 0)
    # contrast toward the mean of a gray image: mean m, out = m + f (p - m)
    m = int(np.floor((0.299 * gray[0] + 0.587 * gray[0] + 0.114 * gray[0]).astype(np.float32)
                     ).astype(np.uint32).sum() // 1024)
    got = orc.ra_op(gray, 11, 0.5, -1.0).astype(np.float64)
    fm = 1.0 - 0.9 * 0.5
    want = m + fm * (gray.astype(np.float64) - m)
    assert np.abs(got - np.clip(want, 0, 255)).max() <= 1.0
    # sharpness with sign -: blend toward the blur, border rows unchanged
    sh = orc.ra_op(im, 12, 1.0, -1.0)
    assert np.array_equal(sh[:, 0, :], im[:, 0, :]) and np.array_equal(sh[:, :, 31], im[:, :, 31])


def test_randaugment_draw_order(orc):
    """ra_n draws of (op, magnitude, sign) from the generator, then nothing
    for ra_mag = 0; the result equals applying ra_op with the same draws."""
    im = _img()
    r1 = orc.Rng(99)
    out = orc.randaugment(im.ravel(), 0.6, 3, r1)
    r2 = orc.Rng(99)
    want = im.copy()
    for _ in range(3):
        op = r2.below(13)
        v = min(max(np.float32(0.6) * (np.float32(1.0) + np.float32(0.5) * np.float32(r2.normal())),
                    0.0), 1.0)
        sign = 1.0 if ((r2.next_u64() >> 32) & 1) == 1 else -1.0  # next_u32, rng.rs:39-41
        want = orc.ra_op(want, op, v, sign)
    assert np.array_equal(out.reshape(im.shape), want)
    assert r1.next_u64() == r2.next_u64()  # the generator advanced alike
    r3 = orc.Rng(99)
    assert np.array_equal(orc.randaugment(im.ravel(), 0.0, 3, r3), im.ravel())
    assert r3.next_u64() == orc.Rng(99).next_u64()
