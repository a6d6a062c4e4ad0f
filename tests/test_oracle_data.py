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
