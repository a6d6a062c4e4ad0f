"""Pins the oracle's GEMM core (gemm.rs) on the CPU: packing layouts against
their closed-form definitions (bit-exact), matmul / gemm_small / matmul_dw
against an f64 triple loop and integer-exact inputs, the reference's
gemmcheck shapes and edge cases."""
import numpy as np
import pytest

from conftest import TOL, rel_frob

MR, NR, KC = 6, 16, 256


def pack_a_def(a, m, k, tr):
    """Closed form of PackedA (gemm.rs:21-120), zeros where never written."""
    A = a.reshape(k, m).T if tr else a.reshape(m, k)
    mpad = -(-m // MR) * MR
    nb = -(-k // KC)
    out = np.zeros(nb * KC * mpad, np.float32)
    for q in range(nb):
        kc = min(KC, k - q * KC)
        for i in range(mpad // MR):
            base = q * KC * mpad + i * kc * MR
            for p in range(kc):
                for r in range(MR):
                    row = i * MR + r
                    out[base + p * MR + r] = A[row, q * KC + p] if row < m else 0.0
    return out


def pack_b_def(b, n, k, tr):
    """Closed form of PackedB (gemm.rs:306-407)."""
    B = b.reshape(n, k).T if tr else b.reshape(k, n)
    npad = -(-n // NR) * NR
    nb = -(-k // KC)
    out = np.zeros(nb * KC * npad, np.float32)
    for q in range(nb):
        kc = min(KC, k - q * KC)
        for j in range(npad // NR):
            base = q * KC * npad + j * kc * NR
            for p in range(kc):
                for t in range(NR):
                    col = j * NR + t
                    out[base + p * NR + t] = B[q * KC + p, col] if col < n else 0.0
    return out


def naive64(m, n, k, a, at, b, bt):
    A = a.reshape(k, m).T if at else a.reshape(m, k)
    B = b.reshape(n, k).T if bt else b.reshape(k, n)
    return (A.astype(np.float64) @ B.astype(np.float64)).ravel()


@pytest.mark.parametrize("m,k", [(7, 19), (6, 256), (13, 300), (1, 1), (32, 288)])
@pytest.mark.parametrize("tr", [False, True])
def test_pack_layouts(orc, m, k, tr):
    a = orc.Rng(m * 7 + k).rand_vec(m * k)
    assert np.array_equal(orc.pack_a(a, m, k, tr), pack_a_def(a, m, k, tr))
    assert np.array_equal(orc.pack_b(a, m, k, tr), pack_b_def(a, m, k, tr))


@pytest.mark.parametrize("kc", [1, 7, 8, 13, 256])
def test_transpose_to_panel(orc, kc):
    lds = 260
    src = orc.Rng(kc).rand_vec(NR * lds)
    got = orc.transpose_to_panel(src, lds, kc)
    want = np.array([src[t * lds + p] for p in range(kc) for t in range(NR)], np.float32)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("simd", [True, False])
@pytest.mark.parametrize("m,n,k", [(23, 37, 19), (64, 48, 96), (7, 16, 259)])
@pytest.mark.parametrize("at", [False, True])
@pytest.mark.parametrize("bt", [False, True])
def test_matmul_vs_f64(orc, simd, m, n, k, at, bt):
    """check.rs:145-161 gemmcheck shapes, all four transposes, both the AVX2
    and the scalar micro-kernel."""
    old = orc.set_simd(simd)
    try:
        rng = orc.Rng(1234 ^ 0x1234)
        a, b = rng.rand_vec(m * k), rng.rand_vec(k * n)
        got = orc.matmul(m, n, k, a, at, b, bt)
        assert rel_frob(got, naive64(m, n, k, a, at, b, bt)) < 1e-6
    finally:
        orc.set_simd(old)


def test_matmul_integer_exact_and_acc(orc):
    m, n, k = 50, 70, 600
    r = np.random.default_rng(1)
    a = r.integers(-3, 4, m * k).astype(np.float32)
    b = r.integers(-3, 4, k * n).astype(np.float32)
    c0 = r.integers(-3, 4, m * n).astype(np.float32)
    want = naive64(m, n, k, a, False, b, False)
    assert np.array_equal(orc.matmul(m, n, k, a, False, b, False), want.astype(np.float32))
    assert np.array_equal(orc.matmul(m, n, k, a, False, b, False, c0, True),
                          (want + c0).astype(np.float32))


def test_matmul_edge_cases(orc):
    c0 = np.full(12, 7.0, np.float32)
    z = np.zeros(0, np.float32)
    assert np.array_equal(orc.matmul(3, 4, 0, z, False, z, False, c0, False), np.zeros(12))
    assert np.array_equal(orc.matmul(3, 4, 0, z, False, z, False, c0, True), c0)
    assert np.array_equal(orc.gemm_small(3, 4, 0, z, False, z, False, c0, False), c0)


def test_matmul_threads_do_not_change_bits(orc):
    m, n, k = 300, 200, 700
    rng = orc.Rng(3)
    a, b = rng.rand_vec(m * k), rng.rand_vec(k * n)
    one = orc.matmul(m, n, k, a, False, b, True)
    with orc.threads(4):
        four = orc.matmul(m, n, k, a, False, b, True)
    assert np.array_equal(one, four)


@pytest.mark.parametrize("m,n,k", [(5, 6, 3), (6, 5, 600), (40, 72, 1000), (768, 32, 300)])
def test_matmul_dw_vs_f64(orc, m, n, k):
    rng = orc.Rng(m + n + k)
    a, b, c0 = rng.rand_vec(k * m), rng.rand_vec(k * n), rng.rand_vec(m * n)
    want = naive64(m, n, k, a, True, b, False) + c0
    assert rel_frob(orc.matmul_dw(m, n, k, a, b, c0), want) < 1e-6


def test_fold_leaves_one_thread_splits_in_half(orc):
    assert orc.fold_leaves(1, 1) == [(0, 1)]
    assert orc.fold_leaves(5, 1) == [(0, 2), (2, 5)]
    assert orc.fold_leaves(128, 1) == [(0, 64), (64, 128)]
    assert orc.fold_leaves(10, 4) == [(0, 2), (2, 5), (5, 7), (7, 10)]


@pytest.mark.parametrize("rows,fin,fout", [(27, 8, 24), (300, 64, 17)])
def test_linear_vs_f64(orc, rows, fin, fout):
    rng = orc.Rng(rows)
    x, w, b = rng.rand_vec(rows * fin), rng.rand_vec(fout * fin), rng.rand_vec(fout)
    dy, dw0, db0 = rng.rand_vec(rows * fout), rng.rand_vec(fout * fin), rng.rand_vec(fout)
    X, W, DY = (v.astype(np.float64) for v in (x.reshape(rows, fin), w.reshape(fout, fin),
                                               dy.reshape(rows, fout)))
    y = orc.linear_forward(rows, fin, fout, x, w, b)
    assert rel_frob(y, (X @ W.T + b).ravel()) < 1e-6
    dw, db, dx = orc.linear_backward(rows, fin, fout, dy, x, w, dw0, db0)
    assert rel_frob(dw, (DY.T @ X).ravel() + dw0) < 1e-6
    assert rel_frob(db, DY.sum(0) + db0) < 1e-6
    assert rel_frob(dx, (DY @ W).ravel()) < 1e-6
