"""GPU parity: dense GEMM drivers (gemm.rs matmul / gemm_small / matmul_dw),
the Linear layer (linear.rs) and the PackedA/PackedB layouts, through the C ABI,
against the CPU oracle (restated reference) on identical seeded inputs."""
import numpy as np
import pytest

from conftest import TOL, rel_frob, to_dev, to_host

pytestmark = pytest.mark.gpu

# check.rs:147 gemmcheck shapes: partial 6x16 tiles and a K>256 block split
GEMMCHECK = [(23, 37, 19), (64, 48, 96), (7, 16, 259)]


def naive64(m, n, k, a, at, b, bt):
    A = a.reshape(k, m).T if at else a.reshape(m, k)
    B = b.reshape(n, k).T if bt else b.reshape(k, n)
    return (A.astype(np.float64) @ B.astype(np.float64)).ravel()


@pytest.mark.parametrize("m,n,k", GEMMCHECK)
@pytest.mark.parametrize("at", [False, True])
@pytest.mark.parametrize("bt", [False, True])
def test_matmul_gemmcheck(rnn, orc, m, n, k, at, bt):
    rng = orc.Rng(1234 ^ 0x1234)
    a, b = rng.rand_vec(m * k), rng.rand_vec(k * n)
    want = orc.matmul(m, n, k, a, at, b, bt)
    c = to_dev(np.zeros(m * n, np.float32))
    rnn.matmul(m, n, k, to_dev(a), at, to_dev(b), bt, c)
    got = to_host(c)
    assert rel_frob(got, want) < TOL
    assert rel_frob(got, naive64(m, n, k, a, at, b, bt)) < TOL
    # check.rs max_rel metric, tolerance 5e-3
    assert np.abs(got - want).max() / max(np.abs(want).max(), 1e-6) < 5e-3


@pytest.mark.parametrize("at,bt", [(False, False), (False, True), (True, False), (True, True)])
def test_matmul_integer_bit_exact(rnn, orc, at, bt):
    m, n, k = 133, 97, 300
    r = np.random.default_rng(5)
    a = r.integers(-3, 4, m * k).astype(np.float32)
    b = r.integers(-3, 4, k * n).astype(np.float32)
    c0 = r.integers(-3, 4, m * n).astype(np.float32)
    for acc in (False, True):
        want = orc.matmul(m, n, k, a, at, b, bt, c0, acc)
        c = to_dev(c0.copy())
        rnn.matmul(m, n, k, to_dev(a), at, to_dev(b), bt, c, acc)
        assert np.array_equal(to_host(c), want)


def test_matmul_edge_cases(rnn, orc):
    c0 = np.full(12, 7.0, np.float32)
    # k == 0: C zeroed unless acc (gemm.rs:449-454)
    c = to_dev(c0.copy())
    rnn.matmul(3, 4, 0, to_dev(np.zeros(1, np.float32)), False, to_dev(np.zeros(1, np.float32)),
               False, c, False)
    assert np.array_equal(to_host(c), np.zeros(12, np.float32))
    c = to_dev(c0.copy())
    rnn.matmul(3, 4, 0, to_dev(np.zeros(1, np.float32)), False, to_dev(np.zeros(1, np.float32)),
               False, c, True)
    assert np.array_equal(to_host(c), c0)
    # m == 0 / n == 0: untouched
    c = to_dev(c0.copy())
    rnn.matmul(0, 4, 3, to_dev(np.ones(12, np.float32)), False, to_dev(np.ones(12, np.float32)),
               False, c, False)
    assert np.array_equal(to_host(c), c0)


@pytest.mark.parametrize("m,n,k,at,bt", [
    (16384, 768, 256, False, True),    # bench.rs:18 S3 qkv fwd
    (16384, 256, 768, False, False),   # bench.rs:20 S3 qkv dX
    (768, 256, 16384, True, False),    # bench.rs:21 S3 qkv dW (matmul with at)
    (4096, 384, 1024, False, True),    # bench.rs:23 merge fwd
])
def test_matmul_gemmbench_shapes(rnn, orc, m, n, k, at, bt):
    rng = orc.Rng(7)
    a, b = rng.rand_vec(m * k), rng.rand_vec(k * n)
    with orc.threads(8):
        want = orc.matmul(m, n, k, a, at, b, bt)
    c = to_dev(np.zeros(m * n, np.float32))
    rnn.matmul(m, n, k, to_dev(a), at, to_dev(b), bt, c)
    assert rel_frob(to_host(c), want) < TOL


def test_gemm_small_batched_attention_shapes(rnn, orc):
    # 512 (image, head) problems: QK^T (bt), PV, P^T dO (at)
    cnt = 512
    rng = orc.Rng(11)
    for (m, n, k, at, bt) in [(64, 64, 32, False, True), (64, 32, 64, False, False),
                              (64, 32, 64, True, False), (9, 9, 4, False, True)]:
        a = rng.rand_vec(cnt * m * k)
        b = rng.rand_vec(cnt * k * n)
        c = to_dev(np.zeros(cnt * m * n, np.float32))
        rnn.gemm_small_batched(cnt, m, n, k, to_dev(a), m * k, at, to_dev(b), k * n, bt, c, m * n)
        got = to_host(c).reshape(cnt, m * n)
        for i in (0, 1, 255, cnt - 1):
            want = orc.gemm_small(m, n, k, a[i * m * k:(i + 1) * m * k], at,
                                  b[i * k * n:(i + 1) * k * n], bt)
            assert rel_frob(got[i], want) < TOL


def test_gemm_small_k0_leaves_c(rnn, orc):
    c0 = np.arange(8, dtype=np.float32)
    c = to_dev(c0.copy())
    one = to_dev(np.ones(8, np.float32))
    rnn.gemm_small_batched(2, 2, 2, 0, one, 0, False, one, 0, False, c, 4)
    assert np.array_equal(to_host(c), c0)
    assert np.array_equal(orc.gemm_small(2, 2, 0, np.zeros(0, np.float32), False,
                                         np.zeros(0, np.float32), False, c0[:4]), c0[:4])


@pytest.mark.parametrize("m,n,k", [(768, 256, 8192), (5, 6, 3), (64, 700, 1000), (300, 40, 257)])
def test_matmul_dw(rnn, orc, m, n, k):
    rng = orc.Rng(3)
    a, b, c0 = rng.rand_vec(k * m), rng.rand_vec(k * n), rng.rand_vec(m * n)
    with orc.threads(8):
        want = orc.matmul_dw(m, n, k, a, b, c0)
    c = to_dev(c0.copy())
    rnn.matmul_dw(m, n, k, to_dev(a), to_dev(b), c)
    got = to_host(c)
    assert rel_frob(got, want) < TOL
    # deterministic: same inputs, same bits
    c2 = to_dev(c0.copy())
    rnn.matmul_dw(m, n, k, to_dev(a), to_dev(b), c2)
    assert np.array_equal(to_host(c2), got)


def test_matmul_dw_integer_exact(rnn, orc):
    m, n, k = 40, 72, 5000
    r = np.random.default_rng(9)
    a = r.integers(-2, 3, k * m).astype(np.float32)
    b = r.integers(-2, 3, k * n).astype(np.float32)
    c0 = r.integers(-2, 3, m * n).astype(np.float32)
    want = orc.matmul_dw(m, n, k, a, b, c0)
    c = to_dev(c0.copy())
    rnn.matmul_dw(m, n, k, to_dev(a), to_dev(b), c)
    assert np.array_equal(to_host(c), want)


# db is summed by the dW GEMM itself on its direct-to-LDS path (fout and fin
# multiples of 4): split-K (8192 rows; 4096 rows with a partial last row
# tile), one launch (27 rows), 128 x 128 tiles (4096 x 4096); fout = 30 takes
# the column-sum kernels.
@pytest.mark.parametrize("rows,fin,fout,bias", [(8192, 256, 768, True), (27, 8, 24, True),
                                                 (64, 384, 1024, False), (4096, 36, 100, True),
                                                 (64, 4096, 4096, True), (100, 64, 30, True)])
def test_linear(rnn, orc, rows, fin, fout, bias):
    rng = orc.Rng(21)
    x, w = rng.rand_vec(rows * fin), rng.rand_vec(fout * fin) * np.float32(0.02)
    b = rng.rand_vec(fout) if bias else None
    dy = rng.rand_vec(rows * fout)
    dw0, db0 = rng.rand_vec(fout * fin), (rng.rand_vec(fout) if bias else None)
    with orc.threads(8):
        y_want = orc.linear_forward(rows, fin, fout, x, w, b)
        dw_want, db_want, dx_want = orc.linear_backward(rows, fin, fout, dy, x, w, dw0, db0)
    y = rnn.linear_forward(rows, fin, fout, to_dev(x), to_dev(w), to_dev(b) if bias else None)
    assert rel_frob(to_host(y), y_want) < TOL
    dw = to_dev(dw0.copy())
    db = to_dev(db0.copy()) if bias else None
    dx = rnn.linear_backward(rows, fin, fout, to_dev(dy), to_dev(x), to_dev(w), dw, db)
    assert rel_frob(to_host(dw), dw_want) < TOL
    assert rel_frob(to_host(dx), dx_want) < TOL
    if bias:
        assert rel_frob(to_host(db), db_want) < TOL


@pytest.mark.parametrize("rows,fin,fout", [(8192, 256, 768), (100, 64, 30), (27, 6, 10)])
def test_linear_backward_acc(rnn, orc, rows, fin, fout):
    """rnn_linear_backward_ex with RNN_LINEAR_ACC_DX: dx0 + the dx that
    rnn_linear_backward writes, bit for bit (dW and db as the plain call's,
    bit for bit), and within TOL of the oracle."""
    rng = orc.Rng(22)
    x, w = rng.rand_vec(rows * fin), rng.rand_vec(fout * fin) * np.float32(0.02)
    dy, dx0 = rng.rand_vec(rows * fout), rng.rand_vec(rows * fin)
    X, W, DY = to_dev(x), to_dev(w), to_dev(dy)
    dw1, db1 = to_dev(np.zeros(fout * fin, np.float32)), to_dev(np.zeros(fout, np.float32))
    dx = to_host(rnn.linear_backward(rows, fin, fout, DY, X, W, dw1, db1))
    dw2, db2 = to_dev(np.zeros(fout * fin, np.float32)), to_dev(np.zeros(fout, np.float32))
    DX = to_dev(dx0.copy())
    out = rnn.linear_backward(rows, fin, fout, DY, X, W, dw2, db2, dx=DX, acc_dx=True)
    assert out is DX
    assert np.array_equal(to_host(DX), (dx0 + dx).astype(np.float32))
    assert np.array_equal(to_host(dw1), to_host(dw2)) and np.array_equal(to_host(db1), to_host(db2))
    with orc.threads(8):
        _, _, dx_want = orc.linear_backward(rows, fin, fout, dy, x, w, np.zeros(fout * fin, np.float32),
                                            np.zeros(fout, np.float32))
    assert rel_frob(to_host(DX) - dx0, dx_want) < TOL


@pytest.mark.parametrize("rows,fin,fout,rpi,masked", [(8192, 352, 256, 64, True),
                                                      (2048, 256, 384, 16, False),
                                                      (300, 40, 36, 10, True),
                                                      (96, 6, 20, 32, True)])
def test_linear_forward_residual(rnn, orc, rows, fin, fout, rpi, masked):
    """rnn_linear_forward_residual == rnn_linear_forward then
    rnn_residual_add_scaled(out, y, ...), bit for bit (rpi 10: the two-pass
    fallback; fin 6: the register-staged GEMM's epilogue), y within TOL of the
    oracle."""
    import ctypes as C
    from rustnn_amd import _ptr, lib
    rng = orc.Rng(23)
    x, w = rng.rand_vec(rows * fin), rng.rand_vec(fout * fin) * np.float32(0.05)
    b, l, out0 = rng.rand_vec(fout), rng.rand_vec(fout), rng.rand_vec(rows * fout)
    n = rows // rpi
    mask = np.where(np.arange(n) % 3 == 1, 0.0, 1.25).astype(np.float32)
    X, W, B, L = to_dev(x), to_dev(w), to_dev(b), to_dev(l)
    M = to_dev(mask) if masked else None
    y1 = rnn.linear_forward(rows, fin, fout, X, W, B)
    O1 = to_dev(out0.copy())
    ctx = rnn.default_ctx()
    ctx.check(lib().rnn_residual_add_scaled(ctx.h, rows, fout, _ptr(O1, rows * fout, "x"),
                                            _ptr(y1, rows * fout, "a"), _ptr(L, fout, "l"),
                                            _ptr(M, n, "m") if masked else None, rpi,
                                            _ptr(O1, rows * fout, "y")))
    O2 = to_dev(out0.copy())
    y2 = rnn.linear_forward_residual(rows, fin, fout, X, W, B, O2, L, M, rpi)
    assert np.array_equal(to_host(y1), to_host(y2))
    assert np.array_equal(to_host(O1), to_host(O2))
    with orc.threads(8):
        yw = orc.linear_forward(rows, fin, fout, x, w, b)
    assert rel_frob(to_host(y2), yw) < TOL


@pytest.mark.parametrize("m,k", [(32, 288), (288, 32), (7, 259), (1, 1), (13, 600)])
@pytest.mark.parametrize("tr", [False, True])
def test_pack_bit_exact(rnn, orc, m, k, tr):
    rng = orc.Rng(m * 1000 + k)
    a = rng.rand_vec(m * k)
    assert np.array_equal(to_host(rnn.dbg_pack_a(to_dev(a), m, k, tr)), orc.pack_a(a, m, k, tr))
    assert np.array_equal(to_host(rnn.dbg_pack_b(to_dev(a), m, k, tr)), orc.pack_b(a, m, k, tr))


def test_destroy_flushes_deferred_reductions(rnn, orc):
    """A context destroyed with deferral on and reductions still queued runs
    them first: the Linear backward's dW (split over rows) and bias
    gradient equal the immediate path's, bit for bit."""
    rows, fin, fout = 8192, 64, 96
    rng = orc.Rng(31)
    x, dy = to_dev(rng.rand_vec(rows * fin)), to_dev(rng.rand_vec(rows * fout))
    w = to_dev(rng.rand_vec(fout * fin))
    got = []
    for defer in (False, True):
        ctx = rnn.Context(0)
        dw = to_dev(np.zeros(fout * fin, np.float32))
        db = to_dev(np.zeros(fout, np.float32))
        ctx.set_defer(defer)
        rnn.linear_backward(rows, fin, fout, dy, x, w, dw, db, ctx=ctx)
        ctx.close()  # no flush: destroy runs what is queued
        got.append((to_host(dw), to_host(db)))
    assert np.array_equal(got[0][0], got[1][0])
    assert np.array_equal(got[0][1], got[1][1])
    assert got[1][1].any()
