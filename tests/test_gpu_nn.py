"""GPU parity: the ResNet layers around the convs (nn.rs:102-110, 253-637)
through the C ABI against the CPU oracle on identical seeded inputs, and the
reference's layercheck (check.rs:548-670) through the HIP path.

Bit-exact where the reference's order is reproduced exactly (gap, classifier
Linear, SGD, ReLU / add helpers, BN apply given the same statistics); within
1e-5 relative Frobenius where sums run in a different order (BN statistics and
dgamma / dbeta: f64 tree sums here, sequential f64 / f32 in the reference) or
libm differs (softmax_ce: expf / logf)."""
import numpy as np
import pytest

from conftest import TOL, rel_frob, to_dev, to_host

import refcheck

pytestmark = pytest.mark.gpu

BN_SHAPES = [(128, 32, 32 * 32), (128, 128, 64), (7, 5, 25), (3, 4, 25), (2, 3, 6)]


def _bn_data(orc, n, c, hw, seed):
    rng = orc.Rng(seed)
    x = (rng.rand_vec(n * c * hw) * np.float32(1.7) + np.float32(0.3)).reshape(n, c, hw)
    g = (np.float32(0.5) + rng.uniform_vec(c)).astype(np.float32)
    b = rng.rand_vec(c)
    return rng, x, g, b


@pytest.mark.parametrize("n,c,hw", BN_SHAPES)
@pytest.mark.parametrize("relu", [0, 1])
def test_bn_forward_train(rnn, orc, n, c, hw, relu):
    import rustnn_amd as R
    _, x, g, b = _bn_data(orc, n, c, hw, 100 + c)
    rm0 = np.linspace(-0.3, 0.3, c).astype(np.float32)
    rv0 = np.linspace(0.7, 1.3, c).astype(np.float32)
    y_want = x.copy()
    rm_w, rv_w = rm0.copy(), rv0.copy()
    with orc.threads(8):
        _, mean_w, inv_w = orc.bn_train_forward(y_want, g, b, rm_w, rv_w, relu=bool(relu))
    X, Y = to_dev(x), to_dev(np.zeros_like(x))
    RM, RV = to_dev(rm0), to_dev(rv0)
    M, IS = to_dev(np.zeros(c, np.float32)), to_dev(np.zeros(c, np.float32))
    G, B = to_dev(g), to_dev(b)  # held for the call: freed tensors may share memory
    ctx = R.default_ctx()
    ctx.check(R.lib().rnn_bn_forward_train(ctx.h, n, c, hw, R._ptr(X, 0, "x"), R._ptr(Y, 0, "y"),
                                           R._ptr(G, c, "g"), R._ptr(B, c, "b"),
                                           R._ptr(RM, c, "rm"), R._ptr(RV, c, "rv"),
                                           R._ptr(M, c, "m"), R._ptr(IS, c, "is"), 0.1, 1e-5,
                                           relu))
    assert rel_frob(to_host(M), mean_w) < 1e-6
    assert rel_frob(to_host(IS), inv_w) < 1e-6
    assert rel_frob(to_host(Y), y_want) < TOL
    assert rel_frob(to_host(RM), rm_w) < 1e-6
    assert rel_frob(to_host(RV), rv_w) < 1e-6


@pytest.mark.parametrize("n,c,hw", [(128, 64, 256), (7, 5, 25)])
def test_bn_forward_eval(rnn, orc, n, c, hw):
    import rustnn_amd as R
    _, x, g, b = _bn_data(orc, n, c, hw, 7)
    rm = np.linspace(-0.3, 0.3, c).astype(np.float32)
    rv = np.linspace(0.7, 1.3, c).astype(np.float32)
    y_want = x.copy()
    orc.bn_eval_forward(y_want, g, b, rm, rv, relu=True)
    X = to_dev(x)
    G, B, RM, RV = to_dev(g), to_dev(b), to_dev(rm), to_dev(rv)
    ctx = R.default_ctx()
    ctx.check(R.lib().rnn_bn_forward_eval(ctx.h, n, c, hw, R._ptr(X, 0, "x"), R._ptr(X, 0, "y"),
                                          R._ptr(G, c, "g"), R._ptr(B, c, "b"),
                                          R._ptr(RM, c, "rm"), R._ptr(RV, c, "rv"), 1e-5, 1))
    assert np.array_equal(to_host(X), y_want)  # same formula, same rounding


@pytest.mark.parametrize("n,c,hw", BN_SHAPES)
@pytest.mark.parametrize("masked", [False, True])
def test_bn_backward(rnn, orc, n, c, hw, masked):
    from rustnn_amd.nn import BatchNorm2d
    rng, x, g, b = _bn_data(orc, n, c, hw, 300 + c)
    dy = rng.rand_vec(x.size).reshape(x.shape)
    relu_out = rng.rand_vec(x.size).reshape(x.shape)  # about half <= 0
    y = x.copy()
    with orc.threads(8):
        xhat, _, invstd = orc.bn_train_forward(y, g, b, np.zeros(c, np.float32),
                                               np.ones(c, np.float32))
        dyw = np.where(relu_out <= 0, np.float32(0), dy).astype(np.float32) if masked else dy
        dg_w, db_w = np.full(c, 0.25, np.float32), np.full(c, -0.5, np.float32)
        dx_w = orc.bn_backward(dyw, xhat, g, invstd, dg_w, db_w)
    bn = BatchNorm2d(c)
    bn.g.v.copy_(to_dev(g))
    bn.b.v.copy_(to_dev(b))
    bn.g.g.fill_(0.25)
    bn.b.g.fill_(-0.5)
    bn.forward(to_dev(x), True)
    dx = bn.backward(to_dev(dy), to_dev(relu_out) if masked else None)
    assert rel_frob(to_host(dx), dx_w) < TOL
    assert rel_frob(to_host(bn.g.g), dg_w) < TOL
    assert rel_frob(to_host(bn.b.g), db_w) < TOL


def test_elementwise_bit_exact(rnn, orc):
    from rustnn_amd import nn
    rng = orc.Rng(21)
    for n in (1, 5, 4096, 100003):
        a, b = rng.rand_vec(n), rng.rand_vec(n)
        A, B = to_dev(a), to_dev(b)
        nn.add_relu_(A, B)
        w = a.copy()
        orc.add_relu(w, b)
        assert np.array_equal(to_host(A), w)
        A = to_dev(a)
        nn.add_(A, B)
        w = a.copy()
        orc.add_(w, b)
        assert np.array_equal(to_host(A), w)
        D = to_dev(b)
        nn.relu_back_(D, to_dev(a))
        w = b.copy()
        orc.relu_back(w, a)
        assert np.array_equal(to_host(D), w)
        # add_relu_back_: add_(a, relu_back_(b, y)) with b unchanged (n = 5
        # and 100003 leave a ragged tail past the float4 items)
        y = rng.rand_vec(n)
        A, B = to_dev(a), to_dev(b)
        nn.add_relu_back_(A, B, to_dev(y))
        m, w = b.copy(), a.copy()
        orc.relu_back(m, y)
        orc.add_(w, m)
        assert np.array_equal(to_host(A), w)
        assert np.array_equal(to_host(B), b)


@pytest.mark.parametrize("n,c,h,w", [(128, 128, 8, 8), (3, 5, 7, 3), (2, 4, 4, 4)])
def test_gap_bit_exact(rnn, orc, n, c, h, w):
    from rustnn_amd import nn
    x = orc.Rng(23).rand_vec(n * c * h * w).reshape(n, c, h, w)
    y = nn.gap_forward(to_dev(x))
    yw = orc.gap_forward(x)
    assert np.array_equal(to_host(y), yw)
    dx = nn.gap_backward(y, h, w)
    assert np.array_equal(to_host(dx), orc.gap_backward(yw, h, w))


@pytest.mark.parametrize("rows,fin,fout", [(128, 128, 100), (3, 6, 5), (17, 33, 9)])
def test_fc_bit_exact(rnn, orc, rows, fin, fout):
    from rustnn_amd import nn
    rng = orc.Rng(29)
    x = rng.rand_vec(rows * fin).reshape(rows, fin)
    w = rng.rand_vec(fout * fin)
    b = rng.rand_vec(fout)
    dy = rng.rand_vec(rows * fout).reshape(rows, fout)
    dy[::3, ::2] = 0.0  # the reference skips zero gradients
    lin = nn.Linear(fin, fout, to_dev(w), to_dev(b))
    lin.w.g.copy_(to_dev(np.linspace(-1, 1, fin * fout).astype(np.float32)))
    lin.b.g.fill_(0.125)
    y = lin.forward(to_dev(x))
    assert np.array_equal(to_host(y), orc.fc_forward(x, w, b, fout))
    dx = lin.backward(to_dev(dy))
    dw_w = np.linspace(-1, 1, fin * fout).astype(np.float32)
    db_w = np.full(fout, 0.125, np.float32)
    dx_w = orc.fc_backward(dy, x, w, dw_w, db_w)
    assert np.array_equal(to_host(dx), dx_w)
    assert np.array_equal(to_host(lin.w.g), dw_w)
    assert np.array_equal(to_host(lin.b.g), db_w)


@pytest.mark.parametrize("rows,nclass", [(128, 100), (4, 7), (300, 10)])
@pytest.mark.parametrize("smooth", [0.0, 0.1])
def test_softmax_ce(rnn, orc, rows, nclass, smooth):
    import torch
    from rustnn_amd import nn
    rng = orc.Rng(31)
    z = rng.rand_vec(rows * nclass).reshape(rows, nclass) * np.float32(2.5)
    labels = np.array([rng.below(nclass) for _ in range(rows)], np.uint32)
    lw, cw, dw = orc.softmax_ce(z, labels, smooth)
    loss, corr, d = nn.softmax_ce(to_dev(z), torch.from_numpy(labels.astype(np.int32)).cuda(),
                                  smooth)
    assert abs(float(to_host(loss)[0]) - lw) <= 1e-5 * max(1.0, abs(lw))
    assert int(to_host(corr)[0]) == cw
    assert rel_frob(to_host(d), dw) < TOL


def test_sgd_bit_exact(rnn, orc):
    from rustnn_amd.nn import Param
    rng = orc.Rng(37)
    for n, decay in ((1000, True), (77, False)):
        v, g, m = rng.rand_vec(n), rng.rand_vec(n), rng.rand_vec(n)
        p = Param(to_dev(v), decay)
        p.g.copy_(to_dev(g))
        p.m.copy_(to_dev(m))
        p.step(0.2, 0.9, 5e-4)
        orc.sgd_step(v, g, m, 0.2, 0.9, 5e-4 if decay else 0.0)
        assert np.array_equal(to_host(p.v), v)
        assert np.array_equal(to_host(p.m), m)
        assert not to_host(p.g).any()


def test_layercheck_nn_gpu(rnn, orc):
    """check.rs:548-670 through the HIP path (tolerance 5e-3)."""
    from oracle import pymodel
    res = refcheck.nn_layercheck(orc, refcheck.GpuNN(pymodel))
    bad = [(t, e) for t, e in res if not e < refcheck.TOL]
    assert not bad, bad
