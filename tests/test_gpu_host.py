"""GPU: the host-slice entry points of the Rust shim (rnn_*_host) through the
C ABI on numpy buffers, against the device entry points they wrap on the
same data (bit for bit: the same kernels run on a staged copy) and, for one
shape each, against the oracle at the parity tolerance.  Covers the
accumulating outputs (acc, dW, dq / dkv / dtau / drel), the k = 0 quirk of
gemm_small, a fused QKV buffer passed as both q and kv, and dq == dkv."""
import ctypes as C

import numpy as np
import pytest

from conftest import TOL, rel_frob, to_dev, to_host

pytestmark = pytest.mark.gpu


def _p(a):
    return C.c_void_p(a.ctypes.data) if a is not None else None


def _d(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


@pytest.mark.parametrize("m,n,k,at,bt,acc", [(96, 80, 300, 0, 1, 0), (33, 70, 129, 1, 0, 1),
                                             (64, 64, 0, 0, 0, 0), (5, 7, 0, 0, 0, 1)])
def test_matmul_host(rnn, orc, m, n, k, at, bt, acc):
    L, ctx = rnn.lib(), rnn.Context(0)
    rng = orc.Rng(1 + m)
    a, b, c0 = rng.rand_vec(m * k), rng.rand_vec(k * n), rng.rand_vec(m * n)
    c = c0.copy()
    ctx.check(L.rnn_matmul_host(ctx.h, m, n, k, _p(a), at, _p(b), bt, _p(c), acc))
    A, B, Cd = to_dev(a), to_dev(b), to_dev(c0.copy())
    ctx.check(L.rnn_matmul(ctx.h, m, n, k, _d(A), at, _d(B), bt, _d(Cd), acc))
    assert np.array_equal(c, to_host(Cd))
    if k:
        want = orc.matmul(m, n, k, a, at, b, bt) + (c0 if acc else 0)
        assert rel_frob(c, want) < TOL
    else:
        assert np.array_equal(c, c0 if acc else np.zeros_like(c0))
    ctx.close()


def test_gemm_small_and_matmul_dw_host(rnn, orc):
    L, ctx = rnn.lib(), rnn.Context(0)
    rng = orc.Rng(7)
    cnt, m, n, k = 6, 64, 32, 64
    a, b = rng.rand_vec(cnt * m * k), rng.rand_vec(cnt * k * n)
    c0 = rng.rand_vec(cnt * m * n)
    for kk, acc in ((k, 1), (0, 0)):
        c = c0.copy()
        ctx.check(L.rnn_gemm_small_batched_host(ctx.h, cnt, m, n, kk, _p(a), m * k, 1, _p(b),
                                                k * n, 0, _p(c), m * n, acc))
        # the device operands stay referenced until the call has run
        A, B, Cd = to_dev(a), to_dev(b), to_dev(c0.copy())
        ctx.check(L.rnn_gemm_small_batched(ctx.h, cnt, m, n, kk, _d(A), m * k, 1, _d(B), k * n,
                                           0, _d(Cd), m * n, acc))
        assert np.array_equal(c, to_host(Cd))
        if kk == 0:
            assert np.array_equal(c, c0)  # gemm_small's k = 0 leaves C untouched
    mm, nn, kk = 48, 72, 1000
    a, b, c0 = rng.rand_vec(kk * mm), rng.rand_vec(kk * nn), rng.rand_vec(mm * nn)
    c = c0.copy()
    ctx.check(L.rnn_matmul_dw_host(ctx.h, mm, nn, kk, _p(a), _p(b), _p(c)))
    A, B, Cd = to_dev(a), to_dev(b), to_dev(c0.copy())
    ctx.check(L.rnn_matmul_dw(ctx.h, mm, nn, kk, _d(A), _d(B), _d(Cd)))
    assert np.array_equal(c, to_host(Cd))
    assert rel_frob(c - c0, orc.matmul(mm, nn, kk, a, 1, b, 0)) < TOL
    ctx.close()


@pytest.mark.parametrize("n,cin,cout,k,s,p,h", [(8, 32, 32, 3, 1, 1, 32), (4, 16, 32, 3, 2, 1, 16),
                                                (4, 32, 64, 1, 2, 0, 16)])
def test_conv_host(rnn, orc, n, cin, cout, k, s, p, h):
    L, ctx = rnn.lib(), rnn.Context(0)
    sp = orc.ConvSpec.make(cin, cout, k, s, p, h, h)
    gsp = rnn.ConvSpec.make(cin, cout, k, s, p, h, h)
    rng = orc.Rng(20 + cin)
    x, dy = rng.rand_vec(n * cin * h * h), rng.rand_vec(n * cout * sp.hw)
    w, dw0 = rng.rand_vec(cout * sp.ckk), rng.rand_vec(cout * sp.ckk)
    y, dx, dw = np.empty(n * cout * sp.hw, np.float32), np.empty_like(x), dw0.copy()
    ctx.check(L.rnn_conv2d_forward_host(ctx.h, C.byref(gsp), n, _p(x), _p(w), _p(y)))
    ctx.check(L.rnn_conv2d_backward_x_host(ctx.h, C.byref(gsp), n, _p(dy), _p(w), _p(dx)))
    ctx.check(L.rnn_conv2d_backward_w_host(ctx.h, C.byref(gsp), n, _p(dy), _p(x), _p(dw)))
    X, W, DY = to_dev(x), to_dev(w), to_dev(dy)
    Y, DX, DW = to_dev(np.empty_like(y)), to_dev(np.empty_like(x)), to_dev(dw0.copy())
    ctx.check(L.rnn_conv2d_forward(ctx.h, C.byref(gsp), n, _d(X), _d(W), _d(Y)))
    ctx.check(L.rnn_conv2d_backward_x(ctx.h, C.byref(gsp), n, _d(DY), _d(W), _d(DX)))
    ctx.check(L.rnn_conv2d_backward_w(ctx.h, C.byref(gsp), n, _d(DY), _d(X), _d(DW)))
    assert np.array_equal(y, to_host(Y))
    assert np.array_equal(dx, to_host(DX))
    assert np.array_equal(dw, to_host(DW))
    assert rel_frob(y, orc.conv2d_forward(sp, n, x, w)) < TOL
    assert rel_frob(dx, orc.conv2d_backward_x(sp, n, dy, w)) < TOL
    assert rel_frob(dw - dw0, orc.conv2d_backward_w(sp, n, dy, x)) < TOL
    ctx.close()


def test_attention_host(rnn, orc):
    """SelfAttn's fused QKV buffer as both q and kv, dq == dkv accumulating
    into one buffer, dtau / drel accumulating (attn.rs:387-438)."""
    L, ctx = rnn.lib(), rnn.Context(0)
    n, hh, dh, t = 8, 4, 32, 64
    c = hh * dh
    relidx, nrel = rnn.rel_index(8, 8, 8, 8)
    rng = orc.Rng(11)
    qkv = rng.rand_vec(n * t * 3 * c) * np.float32(1 / np.sqrt(dh))
    tau = np.full(hh, 1 / np.sqrt(dh), np.float32)
    rel, dout = rng.rand_vec(hh * nrel), rng.rand_vec(n * t * c)
    dab0, dtau0, drel0 = rng.rand_vec(qkv.size), rng.rand_vec(hh), rng.rand_vec(hh * nrel)
    core = rnn.Core(hh, dh, t, t, relidx, nrel, True, ctx=ctx)
    d = core.desc(3 * c, 0, 3 * c, c, 2 * c)
    p, o = np.empty(n * hh * t * t, np.float32), np.empty(n * t * c, np.float32)
    ctx.check(L.rnn_attn_forward_host(ctx.h, C.byref(d), n, _p(qkv), _p(qkv), _p(tau), _p(rel),
                                      _p(p), _p(o)))
    dab, dtau, drel = dab0.copy(), dtau0.copy(), drel0.copy()
    ctx.check(L.rnn_attn_backward_host(ctx.h, C.byref(d), n, _p(qkv), _p(qkv), _p(tau), _p(p),
                                       _p(dout), _p(dab), _p(dab), _p(dtau), _p(drel)))
    Q = to_dev(qkv)
    P, O = core.forward(n, Q, 3 * c, 0, Q, 3 * c, c, 2 * c, to_dev(tau), to_dev(rel))
    DAB, DT, DR = to_dev(dab0.copy()), to_dev(dtau0.copy()), to_dev(drel0.copy())
    core.backward(n, Q, 3 * c, 0, Q, 3 * c, c, 2 * c, to_dev(tau), P, to_dev(dout), DAB, DAB,
                  DT, DR)
    assert np.array_equal(p, to_host(P)) and np.array_equal(o, to_host(O))
    assert np.array_equal(dab, to_host(DAB))
    assert np.array_equal(dtau, to_host(DT)) and np.array_equal(drel, to_host(DR))
    od = orc.attn_desc(hh, dh, t, t, 3 * c, 0, 3 * c, c, 2 * c, relidx, nrel, True)
    p_w, o_w = orc.attn_forward(od, n, qkv, qkv, tau, rel)
    z = np.zeros(qkv.size, np.float32)
    dq_w, dkv_w, dtau_w, drel_w = orc.attn_backward(od, n, qkv, qkv, tau, p_w, dout, z, z,
                                                    np.zeros(hh, np.float32),
                                                    np.zeros(hh * nrel, np.float32))
    assert rel_frob(p, p_w) < TOL and rel_frob(o, o_w) < TOL
    assert rel_frob(dab - dab0, dq_w + dkv_w) < TOL
    assert rel_frob(dtau - dtau0, dtau_w) < TOL and rel_frob(drel - drel0, drel_w) < TOL
    ctx.close()


@pytest.mark.parametrize("bias", [True, False])
def test_linear_host(rnn, orc, bias):
    L, ctx = rnn.lib(), rnn.Context(0)
    rows, fin, fout = 4096, 96, 160
    rng = orc.Rng(40)
    x, w = rng.rand_vec(rows * fin), rng.rand_vec(fout * fin)
    b = rng.rand_vec(fout) if bias else None
    dy, dw0 = rng.rand_vec(rows * fout), rng.rand_vec(fout * fin)
    db0 = rng.rand_vec(fout) if bias else None
    y = np.empty(rows * fout, np.float32)
    ctx.check(L.rnn_linear_forward_host(ctx.h, rows, fin, fout, _p(x), _p(w), _p(b), _p(y)))
    dw, db, dx = dw0.copy(), db0.copy() if bias else None, np.empty_like(x)
    ctx.check(L.rnn_linear_backward_host(ctx.h, rows, fin, fout, _p(dy), _p(x), _p(w), _p(dw),
                                         _p(db), _p(dx)))
    X, W, DY = to_dev(x), to_dev(w), to_dev(dy)
    B = to_dev(b) if bias else None
    Y, DX = to_dev(np.empty_like(y)), to_dev(np.empty_like(x))
    DW, DB = to_dev(dw0.copy()), to_dev(db0.copy()) if bias else None
    ctx.check(L.rnn_linear_forward(ctx.h, rows, fin, fout, _d(X), _d(W), _d(B), _d(Y)))
    ctx.check(L.rnn_linear_backward(ctx.h, rows, fin, fout, _d(DY), _d(X), _d(W), _d(DW), _d(DB),
                                    _d(DX)))
    assert np.array_equal(y, to_host(Y)) and np.array_equal(dx, to_host(DX))
    assert np.array_equal(dw, to_host(DW))
    if bias:
        assert np.array_equal(db, to_host(DB))
    yw = orc.matmul(rows, fout, fin, x, 0, w, 1).reshape(rows, fout)
    if bias:
        yw = yw + b[None, :]
    assert rel_frob(y, yw.ravel()) < TOL
    ctx.close()


def test_host_null_context_and_operands(rnn):
    """No GPU work: a null context or a missing operand is an error code."""
    L = rnn.lib()
    assert L.rnn_matmul_host(None, 1, 1, 1, None, 0, None, 0, None, 0) == rnn.RNN_E_NULL
    ctx = rnn.Context(0)
    assert L.rnn_matmul_host(ctx.h, 2, 2, 2, None, 0, None, 0, None, 0) == rnn.RNN_E_NULL
    ctx.close()
