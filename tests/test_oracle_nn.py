"""Pins of the oracle's ResNet layers (oracle/orc_nn.c, oracle/pymodel.py).

Each layer is checked against something other than its own formula:
  * BatchNorm2d train forward / backward: torch-CPU float64 batch_norm and
    autograd (an independent library), f64 running-statistics update, and the
    reference's own layercheck dircheck at its shape (check.rs:548-598);
  * gap: f64 mean and the exact sequential f32 sum;
  * the classifier Linear: f64 matmul and integer-valued inputs (exact);
  * softmax_ce: torch-CPU float64 cross_entropy with label smoothing, and
    the reference's dircheck (check.rs:659-670);
  * SGD: the closed form in f64, decay vs no decay;
  * ResNet: the reference's full-network gradcheck (check.rs:727-775, seed
    1234, tolerance 5e-3), its block dircheck (check.rs:625-657), parameter
    count and ResNet::flops of ResNet-20.
A planted mistake in the oracle (dropped mean in the BN backward) must fail
the torch pin."""
import numpy as np
import pytest

from conftest import rel_frob

import refcheck


def _torch():
    return pytest.importorskip("torch")


def bn_inputs(orc, n=3, c=4, hw=25, seed=11):
    rng = orc.Rng(seed)
    x = (rng.rand_vec(n * c * hw) * np.float32(2.0) + np.float32(1.0)).reshape(n, c, hw)
    g = (np.float32(0.5) + rng.uniform_vec(c)).astype(np.float32)
    b = rng.rand_vec(c)
    return x, g, b


def test_bn_forward_matches_torch_f64(orc):
    torch = _torch()
    x, g, b = bn_inputs(orc, 4, 6, 49)
    y = x.copy()
    rm = np.linspace(-0.5, 0.5, 6).astype(np.float32)
    rv = np.linspace(0.5, 1.5, 6).astype(np.float32)
    rm0, rv0 = rm.copy(), rv.copy()
    xhat, mean, invstd = orc.bn_train_forward(y, g, b, rm, rv, relu=False)
    xt = torch.from_numpy(x.astype(np.float64))
    rmt, rvt = torch.from_numpy(rm0.astype(np.float64)), torch.from_numpy(rv0.astype(np.float64))
    want = torch.nn.functional.batch_norm(xt, rmt, rvt, torch.from_numpy(g.astype(np.float64)),
                                          torch.from_numpy(b.astype(np.float64)), training=True,
                                          momentum=0.1, eps=1e-5).numpy()
    assert rel_frob(y, want) < 1e-6
    # torch updates the running variance with the unbiased estimate too
    assert np.allclose(rm, rmt.numpy(), rtol=1e-6, atol=1e-7)
    assert np.allclose(rv, rvt.numpy(), rtol=1e-6, atol=1e-7)
    # ReLU variant
    y2 = x.copy()
    orc.bn_train_forward(y2, g, b, rm0.copy(), rv0.copy(), relu=True)
    assert np.array_equal(y2, np.maximum(y, 0))


def test_bn_eval_matches_closed_form(orc):
    x, g, b = bn_inputs(orc)
    rm = np.array([0.1, -0.2, 0.3, 0.0], np.float32)
    rv = np.array([1.5, 0.5, 2.0, 1.0], np.float32)
    y = x.copy()
    orc.bn_eval_forward(y, g, b, rm, rv, relu=False)
    want = (x.astype(np.float64) - rm[None, :, None]) / np.sqrt(rv[None, :, None] + 1e-5) \
        * g[None, :, None] + b[None, :, None]
    assert rel_frob(y, want) < 1e-6


def test_bn_backward_matches_torch_autograd(orc):
    torch = _torch()
    x, g, b = bn_inputs(orc, 4, 5, 36)
    dy = orc.Rng(3).rand_vec(x.size).reshape(x.shape)
    y = x.copy()
    xhat, _, invstd = orc.bn_train_forward(y, g, b, np.zeros(5, np.float32),
                                           np.ones(5, np.float32))
    dg, db = np.zeros(5, np.float32), np.zeros(5, np.float32)
    dx = orc.bn_backward(dy, xhat, g, invstd, dg, db)
    xt = torch.from_numpy(x.astype(np.float64)).requires_grad_()
    gt = torch.from_numpy(g.astype(np.float64)).requires_grad_()
    bt = torch.from_numpy(b.astype(np.float64)).requires_grad_()
    out = torch.nn.functional.batch_norm(xt, None, None, gt, bt, training=True, eps=1e-5)
    out.backward(torch.from_numpy(dy.astype(np.float64)))
    assert rel_frob(dx, xt.grad.numpy()) < 1e-5
    assert rel_frob(dg, gt.grad.numpy()) < 1e-5
    assert rel_frob(db, bt.grad.numpy()) < 1e-6


def test_planted_bn_mistake_fails_torch_pin(orc):
    """Dropping the dbeta term of the BN backward (a plausible slip) is caught."""
    torch = _torch()
    x, g, b = bn_inputs(orc, 4, 5, 36)
    dy = orc.Rng(3).rand_vec(x.size).reshape(x.shape)
    y = x.copy()
    xhat, _, invstd = orc.bn_train_forward(y, g, b, np.zeros(5, np.float32),
                                           np.ones(5, np.float32))
    dg, db = np.zeros(5, np.float32), np.zeros(5, np.float32)
    dx = orc.bn_backward(dy, xhat, g, invstd, dg, db)
    m = x.shape[0] * x.shape[2]
    planted = dx + (g * invstd / m)[None, :, None] * db[None, :, None]
    xt = torch.from_numpy(x.astype(np.float64)).requires_grad_()
    out = torch.nn.functional.batch_norm(xt, None, None, torch.from_numpy(g.astype(np.float64)),
                                         torch.from_numpy(b.astype(np.float64)), training=True,
                                         eps=1e-5)
    out.backward(torch.from_numpy(dy.astype(np.float64)))
    assert rel_frob(planted, xt.grad.numpy()) > 1e-3


def test_gap_and_elementwise(orc):
    rng = orc.Rng(5)
    x = rng.rand_vec(2 * 3 * 7 * 5).reshape(2, 3, 7, 5)
    y = orc.gap_forward(x)
    assert rel_frob(y, x.astype(np.float64).mean(axis=(2, 3))) < 1e-6
    seq = np.zeros((2, 3), np.float32)
    for i in range(2):
        for c in range(3):
            s = np.float32(0)
            for v in x[i, c].ravel():
                s = np.float32(s + v)
            seq[i, c] = s / np.float32(35)
    assert np.array_equal(y, seq)
    dx = orc.gap_backward(y, 7, 5)
    assert np.array_equal(dx, np.broadcast_to((y / np.float32(35))[:, :, None, None], dx.shape))
    a = rng.rand_vec(100)
    b = rng.rand_vec(100)
    a1 = a.copy()
    orc.add_relu(a1, b)
    assert np.array_equal(a1, np.maximum(a + b, 0))
    a2 = a.copy()
    orc.add_(a2, b)
    assert np.array_equal(a2, a + b)
    d = b.copy()
    orc.relu_back(d, a)
    assert np.array_equal(d, np.where(a <= 0, 0, b))


def test_fc_matches_f64_and_integers(orc):
    rng = orc.Rng(9)
    x = rng.rand_vec(5 * 7).reshape(5, 7)
    w = rng.rand_vec(3 * 7)
    b = rng.rand_vec(3)
    y = orc.fc_forward(x, w, b, 3)
    want = x.astype(np.float64) @ w.reshape(3, 7).T.astype(np.float64) + b
    assert rel_frob(y, want) < 1e-6
    dy = rng.rand_vec(5 * 3).reshape(5, 3)
    dy[1, 2] = 0.0
    dw, db = np.zeros(21, np.float32), np.zeros(3, np.float32)
    dx = orc.fc_backward(dy, x, w, dw, db)
    assert rel_frob(dw, (dy.T.astype(np.float64) @ x).ravel()) < 1e-6
    assert rel_frob(db, dy.astype(np.float64).sum(0)) < 1e-6
    assert rel_frob(dx, dy.astype(np.float64) @ w.reshape(3, 7)) < 1e-6
    xi = np.round(x * 4).astype(np.float32)
    wi = np.round(w * 4).astype(np.float32)
    yi = orc.fc_forward(xi, wi, np.zeros(3, np.float32), 3)
    assert np.array_equal(yi, (xi.astype(np.float64) @ wi.reshape(3, 7).T).astype(np.float32))


def test_softmax_ce_matches_torch(orc):
    torch = _torch()
    rng = orc.Rng(13)
    z = rng.rand_vec(6 * 10).reshape(6, 10) * np.float32(3)
    labels = np.array([rng.below(10) for _ in range(6)], np.uint32)
    for smooth in (0.0, 0.1):
        loss, correct, d = orc.softmax_ce(z, labels, smooth)
        zt = torch.from_numpy(z.astype(np.float64)).requires_grad_()
        lt = torch.nn.functional.cross_entropy(zt, torch.from_numpy(labels.astype(np.int64)),
                                               label_smoothing=smooth)
        lt.backward()
        assert abs(loss - lt.item()) < 1e-5 * max(1.0, abs(lt.item()))
        assert rel_frob(d, zt.grad.numpy()) < 1e-5
        assert correct == int((z.argmax(1) == labels).sum())


def test_sgd_closed_form(orc):
    rng = orc.Rng(17)
    v, g, m = rng.rand_vec(50), rng.rand_vec(50), rng.rand_vec(50)
    for wd in (0.0, 5e-4):
        vv, gg, mm = v.copy(), g.copy(), m.copy()
        orc.sgd_step(vv, gg, mm, 0.2, 0.9, wd)
        g64 = g.astype(np.float64) + wd * v
        m64 = 0.9 * m.astype(np.float64) + g64
        assert rel_frob(mm, m64) < 1e-6
        assert rel_frob(vv, v - 0.2 * (g64 + 0.9 * m64)) < 1e-6
        assert not gg.any()


def test_layercheck_bn_linear_block_ce_oracle(orc):
    """check.rs:548-670 (after the conv shapes, in the reference's draw order)."""
    from oracle import pymodel
    res = refcheck.nn_layercheck(orc, refcheck.OracleNN(orc, pymodel))
    for tag, err in res:
        assert err < refcheck.TOL, (tag, err)


def test_resnet_gradcheck_oracle(orc):
    """check.rs:727-775: ResNet(1, 4, 10, 1234), batch 8 at 16x16, smooth 0."""
    from oracle import pymodel
    err = refcheck.resnet_gradcheck(orc, refcheck.OracleResNet(pymodel))
    assert err < refcheck.TOL, err


def test_resnet20_size_and_flops(orc):
    from oracle import pymodel
    net = pymodel.ResNet(3, 32, 100, 0)
    nparams = sum(p.v.size for p in net.params())
    assert abs(nparams - 1.10e6) / 1.10e6 < 0.01
    assert abs(net.flops(32, 32) - 324.76e6) / 324.76e6 < 1e-3
