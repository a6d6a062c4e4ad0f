"""Pins of the oracle's vit.rs pieces (oracle/orc_vit.c): DropPath against
the reference's definition over the oracle Rng (itself pinned to a Python
big-int xoshiro256++ in test_oracle_rng), the token merge against a numpy
reshape / transpose statement, TaxoHead's combine against numpy indexing."""
import numpy as np


def test_drop_path_mask(orc):
    n, per, p, seed = 300, 7, 0.25, 0xABCDEF ^ 3
    x = np.random.default_rng(0).standard_normal(n * per).astype(np.float32)
    y, mask = orc.drop_path(x, n, p, seed)
    rng = orc.Rng(seed)
    keep = np.float32(1.0) - np.float32(p)
    want = np.array([np.float32(1.0) / keep if rng.uniform() < keep else 0.0 for _ in range(n)],
                    np.float32)
    assert np.array_equal(mask, want)
    assert np.array_equal(y.reshape(n, per), x.reshape(n, per) * mask[:, None])
    assert 0.6 < (mask > 0).mean() < 0.9  # about keep = 0.75 of the images kept


def test_token_merge_reshape(orc):
    n, th, c = 3, 6, 5
    z = np.arange(n * th * th * c, dtype=np.float32)
    y = orc.token_merge(z, n, th, c)
    # [n, th/2, 2, th/2, 2, c] -> [n, th/2, th/2, 2 (dy), 2 (dx), c]
    want = z.reshape(n, th // 2, 2, th // 2, 2, c).transpose(0, 1, 3, 2, 4, 5).reshape(-1)
    assert np.array_equal(y, want)


def test_taxo_combine(orc):
    rng = np.random.default_rng(1)
    n, nf, nc = 5, 100, 20
    parent = rng.permutation(np.arange(nf) // 5).astype(np.uint32)
    zf = rng.standard_normal((n, nf)).astype(np.float32)
    zc = rng.standard_normal((n, nc)).astype(np.float32)
    assert np.array_equal(orc.taxo_combine(zf, zc, parent), zf + zc[:, parent])
    dzf = rng.standard_normal((n, nf)).astype(np.float32)
    dzc = rng.standard_normal((n, nc)).astype(np.float32)
    dc = orc.taxo_combine_backward(dzf, dzc, parent)
    want = dzc.astype(np.float64).copy()
    for j in range(nf):
        want[:, parent[j]] += dzf[:, j]
    assert np.allclose(dc, want, rtol=1e-6, atol=1e-6)
