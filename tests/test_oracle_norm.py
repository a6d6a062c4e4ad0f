"""Pins of the oracle's norm.rs layers (oracle/orc_norm.c).

Each layer is checked against an independent statement of the same function:
torch-CPU float64 (layer_norm, silu, a grouped conv2d, softmax pooling) and
its autograd for every gradient, plus the reference's own normcheck
(check.rs:182-291: dircheck at n=3, t=9, c=8, SwiGlu h=16, DwConv3 on 3x3
tokens; eps 3e-4, tolerance 5e-3).  A planted mistake in a restatement (a
dropped xhat term in the LayerNorm backward, a transposed depthwise tap)
must fail its pin."""
import numpy as np
import pytest

from conftest import rel_frob

import refcheck


def _torch():
    return pytest.importorskip("torch")


def _r(shape, seed, scale=1.0, shift=0.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale + shift).astype(np.float32)


def test_layernorm_matches_torch_f64(orc):
    torch = _torch()
    rows, c = 37, 48
    x = _r((rows, c), 1, 2.0, 0.5)
    g, b = _r(c, 2, 0.2, 1.0), _r(c, 3)
    y, xhat, invstd = orc.ln_forward(x, g, b)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    gt = torch.tensor(g, dtype=torch.float64, requires_grad=True)
    bt = torch.tensor(b, dtype=torch.float64, requires_grad=True)
    yt = torch.nn.functional.layer_norm(xt, (c,), gt, bt, 1e-5)
    assert rel_frob(y, yt.detach().numpy()) < 1e-6
    assert np.array_equal(orc.ln_forward(x, g, b, train=False), y)  # eval == train output
    dy = _r((rows, c), 4)
    yt.backward(torch.tensor(dy, dtype=torch.float64))
    dg, db = np.zeros(c, np.float32), np.zeros(c, np.float32)
    dx = orc.ln_backward(dy, xhat, invstd, g, dg, db)
    assert rel_frob(dx, xt.grad.numpy()) < 1e-5
    assert rel_frob(dg, gt.grad.numpy()) < 1e-5
    assert rel_frob(db, bt.grad.numpy()) < 1e-6
    # planted: the xhat * m2 term dropped from dx
    d = dy * g
    bad = invstd[:, None] * (d - d.mean(1, keepdims=True))
    assert rel_frob(bad, xt.grad.numpy()) > 1e-2


def test_layernorm_constant_row(orc):
    """var clamps at 0: a constant row normalises to 0 with invstd 1/sqrt(eps)."""
    x = np.full((2, 16), 3.25, np.float32)
    g, b = np.ones(16, np.float32), _r(16, 5)
    y, xhat, invstd = orc.ln_forward(x, g, b)
    assert not xhat.any()
    assert np.array_equal(y, np.broadcast_to(b, y.shape))
    assert np.allclose(invstd, 1.0 / np.sqrt(np.float32(1e-5)))


def test_layerscale_closed_form(orc):
    x, l, dy = _r((20, 12), 6), _r(12, 7), _r((20, 12), 8)
    assert np.array_equal(orc.layerscale_forward(x, l), x * l)
    dl = np.ones(12, np.float32)
    dx = orc.layerscale_backward(dy, x, l, dl)
    assert np.array_equal(dx, dy * l)
    assert rel_frob(dl - 1.0, (dy.astype(np.float64) * x).sum(0)) < 1e-6


def test_swiglu_matches_torch_f64(orc):
    torch = _torch()
    rows, h = 30, 20
    ab = _r((rows, 2 * h), 9, 2.0)
    u = orc.swiglu_forward(ab, h)
    at = torch.tensor(ab, dtype=torch.float64, requires_grad=True)
    ut = torch.nn.functional.silu(at[:, :h]) * at[:, h:]
    assert rel_frob(u, ut.detach().numpy()) < 1e-6
    du = _r((rows, h), 10)
    ut.backward(torch.tensor(du, dtype=torch.float64))
    assert rel_frob(orc.swiglu_backward(du, ab, h), at.grad.numpy()) < 1e-6


def _dw_torch(x, w, b, n, th, tw, torch):
    """Depthwise 3x3 pad 1 as torch's grouped conv2d on NCHW, float64."""
    c = b.size
    xt = torch.tensor(x.reshape(n, th, tw, c), dtype=torch.float64).permute(0, 3, 1, 2)
    xt = xt.contiguous().requires_grad_(True)
    wt = torch.tensor(w.reshape(3, 3, c), dtype=torch.float64).permute(2, 0, 1)
    wt = wt.reshape(c, 1, 3, 3).contiguous().requires_grad_(True)
    bt = torch.tensor(b, dtype=torch.float64, requires_grad=True)
    yt = torch.nn.functional.conv2d(xt, wt, bt, padding=1, groups=c)
    return xt, wt, bt, yt


def test_dwconv3_matches_torch_f64(orc):
    torch = _torch()
    n, th, tw, c = 3, 5, 4, 12
    x, w, b = _r((n, th * tw, c), 11), _r((9, c), 12, 0.3), _r(c, 13)
    y = orc.dwconv3_forward(x, w, b, n, th, tw)
    xt, wt, bt, yt = _dw_torch(x, w, b, n, th, tw, torch)
    want = yt.detach().permute(0, 2, 3, 1).reshape(n, th * tw, c).numpy()
    assert rel_frob(y, want) < 1e-6
    dy = _r((n, th * tw, c), 14)
    yt.backward(torch.tensor(dy.reshape(n, th, tw, c), dtype=torch.float64).permute(0, 3, 1, 2))
    dw, db = np.zeros((9, c), np.float32), np.zeros(c, np.float32)
    dx = orc.dwconv3_backward(dy, x, w, n, th, tw, dw, db)
    assert rel_frob(dx, xt.grad.permute(0, 2, 3, 1).reshape(n, th * tw, c).numpy()) < 1e-6
    assert rel_frob(dw, wt.grad.reshape(c, 9).T.numpy()) < 1e-6
    assert rel_frob(db, bt.grad.numpy()) < 1e-6
    # planted: taps transposed (w read as [kx][ky])
    bad = orc.dwconv3_forward(x, w.reshape(3, 3, c).transpose(1, 0, 2).copy(), b, n, th, tw)
    assert rel_frob(bad, want) > 1e-2


def test_seqpool_matches_torch_f64(orc):
    torch = _torch()
    n, t, c = 4, 9, 16
    x, p = _r((n, t, c), 15), _r(c, 16, 0.5)
    z, w = orc.seqpool_forward(x, p, n, t)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    pt = torch.tensor(p, dtype=torch.float64, requires_grad=True)
    wt = torch.softmax(xt @ pt, dim=1)
    zt = (wt[:, :, None] * xt).sum(1)
    assert rel_frob(w, wt.detach().numpy()) < 1e-6
    assert rel_frob(z, zt.detach().numpy()) < 1e-6
    dz = _r((n, c), 17)
    zt.backward(torch.tensor(dz, dtype=torch.float64))
    dp = np.zeros(c, np.float32)
    dx = orc.seqpool_backward(dz, w, x, p, n, t, dp)
    assert rel_frob(dx, xt.grad.numpy()) < 1e-6
    assert rel_frob(dp, pt.grad.numpy()) < 1e-5


class OracleNorm:
    """normcheck backend on the CPU oracle (float32 numpy arrays)."""

    def __init__(self, orc):
        self.o = orc

    def ln(self, x, g, b, dy):
        y, xh, iv = self.o.ln_forward(x, g, b)
        dg, db = np.zeros_like(g), np.zeros_like(b)
        dx = self.o.ln_backward(dy, xh, iv, g, dg, db)
        return y, dx, np.concatenate([dg, db])

    def ln_y(self, x, g, b):
        return self.o.ln_forward(x, g, b, train=False)

    def dw(self, x, w, b, n, th, tw, dy):
        y = self.o.dwconv3_forward(x, w, b, n, th, tw)
        dw, db = np.zeros_like(w), np.zeros_like(b)
        dx = self.o.dwconv3_backward(dy, x, w, n, th, tw, dw, db)
        return y, dx, np.concatenate([dw.ravel(), db])

    def dw_y(self, x, w, b, n, th, tw):
        return self.o.dwconv3_forward(x, w, b, n, th, tw)

    def sp(self, x, p, n, t, dz):
        z, w = self.o.seqpool_forward(x, p, n, t)
        dp = np.zeros_like(p)
        dx = self.o.seqpool_backward(dz, w, x, p, n, t, dp)
        return z, dx, dp

    def sp_z(self, x, p, n, t):
        return self.o.seqpool_forward(x, p, n, t)[0]

    def sw(self, x, wg, bg, wd, bd, h, dy):
        """SwiGlu through the oracle's Linear and gate; returns y, dx and the
        parameter gradients in for_each_param order."""
        o = self.o
        rows, c = x.shape
        ab = o.linear_forward(rows, c, 2 * h, x, wg, bg)
        u = o.swiglu_forward(ab, h)
        y = o.linear_forward(rows, h, c, u, wd, bd)
        dwd, dbd, du = o.linear_backward(rows, h, c, dy, u, wd, np.zeros_like(wd),
                                         np.zeros_like(bd))
        dab = o.swiglu_backward(du, ab, h)
        dwg, dbg, dx = o.linear_backward(rows, c, 2 * h, dab, x, wg, np.zeros_like(wg),
                                         np.zeros_like(bg))
        return y, dx.reshape(x.shape), np.concatenate([dwg.ravel(), dbg, dwd.ravel(), dbd])

    def sw_y(self, x, wg, bg, wd, bd, h):
        o = self.o
        rows, c = x.shape
        u = o.swiglu_forward(o.linear_forward(rows, c, 2 * h, x, wg, bg), h)
        return o.linear_forward(rows, h, c, u, wd, bd)


def normcheck(orc, be, rng=None, x=None, r=None):
    """check.rs:182-291 on a backend: dx and the parameters of each layer by
    dircheck at the reference's fixture (n=3, t=9, c=8), with the layers'
    weights drawn as the reference's constructors draw them (SwiGlu::new(c,
    16, 2), DwConv3::new, SeqPool::new: Param::trunc_normal).  Without rng /
    x / r it starts its own stream (Rng::new(1234 ^ 0x1234), gemmcheck's
    draws skipped, as vitcheck does).  Returns {name: relative error}."""
    f = np.float32
    n, t, c = 3, 9, 8
    if rng is None:
        rng = orc.Rng(1234 ^ 0x1234)
        refcheck.skip_gemmcheck_draws(rng)
        x = rng.rand_vec(n * t * c)
        r = rng.rand_vec(n * t * c)
    eps = refcheck.gc_eps()
    X = lambda v: v.reshape(n * t, c)
    d32 = refcheck.dot32
    dc = lambda base, grad, fn: refcheck.dircheck(base, np.asarray(grad).ravel(), eps, rng, fn)
    out = {}
    # 2. LayerNorm: g = 1 + 0.2 v, b = v
    g = f(1.0) + f(0.2) * rng.rand_vec(c)
    b = rng.rand_vec(c)
    _, dx, dgb = be.ln(X(x), g, b, X(r))
    out["layernorm dx"] = dc(x, dx, lambda v: d32(be.ln_y(X(v), g, b), r))
    out["layernorm dparams"] = dc(np.concatenate([g, b]), dgb,
                                  lambda v: d32(be.ln_y(X(x), v[:c].copy(), v[c:].copy()), r))
    # 3. SwiGlu::new(c, 16, 2): wg Linear(c, 32, 0.02), wd Linear::scaled(16, c, depth 2)
    h = 16
    wg = rng.trunc_normal(2 * h * c, f(0.02))
    bg = np.zeros(2 * h, np.float32)
    wd = rng.trunc_normal(c * h, f(0.02) / np.sqrt(f(2.0) * f(2.0)))
    bd = np.zeros(c, np.float32)
    _, dx, dps = be.sw(X(x), wg, bg, wd, bd, h, X(r))
    out["swiglu dx"] = dc(x, dx, lambda v: d32(be.sw_y(X(v), wg, bg, wd, bd, h), r))
    cut = np.cumsum([wg.size, bg.size, wd.size])

    def sw_p(v):
        a, bb, cc, dd = np.split(v, cut)
        return d32(be.sw_y(X(x), a.copy(), bb.copy(), cc.copy(), dd.copy(), h), r)
    out["swiglu dparams"] = dc(np.concatenate([wg, bg, wd, bd]), dps, sw_p)
    # 4. DwConv3::new(c, 3, 3): w trunc_normal(0.1); then b = v
    w = rng.trunc_normal(9 * c, f(0.1)).reshape(9, c)
    bb = rng.rand_vec(c)
    _, dx, dwb = be.dw(X(x), w, bb, n, 3, 3, X(r))
    out["dwconv3x3 dx"] = dc(x, dx, lambda v: d32(be.dw_y(X(v), w, bb, n, 3, 3), r))
    out["dwconv3x3 dparams"] = dc(
        np.concatenate([w.ravel(), bb]), dwb,
        lambda v: d32(be.dw_y(X(x), v[:9 * c].reshape(9, c).copy(), v[9 * c:].copy(), n, 3, 3),
                      r))
    # 5. SeqPool::new(c): p trunc_normal(0.02); rz = v
    p = rng.trunc_normal(c, f(0.02))
    rz = rng.rand_vec(n * c)
    T = lambda v: v.reshape(n, t, c)
    _, dx, dp = be.sp(T(x), p, n, t, rz)
    out["seqpool dx"] = dc(x, dx, lambda v: d32(be.sp_z(T(v), p, n, t), rz))
    out["seqpool dparams"] = dc(p, dp, lambda v: d32(be.sp_z(T(x), v, n, t), rz))
    return out


def test_reference_normcheck_on_oracle(orc):
    errs = normcheck(orc, OracleNorm(orc))
    bad = {k: v for k, v in errs.items() if not v < refcheck.TOL}
    assert not bad, errs
