"""GPU parity: norm.rs on the device (rustnn_amd/norm.py over norm.hip)
against the CPU oracle (oracle/orc_norm.c) on identical seeded inputs.

Bars:
* bit-exact where the kernels keep the reference's per-element operation
  order and no transcendental is involved: the depthwise forward and dX, the
  LayerScale outputs;
* LayerNorm y / xhat / invstd: relative 1e-6 (the f64 row sums are added in
  another order, which can move mu or var by one f32 ulp), and at least 99%
  of the elements bit-identical;
* SwiGLU and SeqPool forward: relative 1e-6 (the device's expf);
* every gradient (column reductions in another order, f64 here): 1e-5
  relative Frobenius (TOL);
* the reference's normcheck (check.rs:182-291) through the GPU path."""
import numpy as np
import pytest

from conftest import TOL, rel_frob, to_dev, to_host

import refcheck
from test_oracle_norm import normcheck

pytestmark = pytest.mark.gpu


def _r(shape, seed, scale=1.0, shift=0.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale + shift).astype(np.float32)


def _dev(a):
    import torch
    return to_dev(np.ascontiguousarray(a, np.float32)).reshape(torch.Size(a.shape))


@pytest.mark.parametrize("rows,c", [(4096, 256), (1024, 384), (300, 1024), (33, 7), (1, 64)])
def test_layernorm(rnn, orc, rows, c):
    from rustnn_amd.norm import LayerNorm
    x = _r((rows, c), rows + c, 1.5, 0.3)
    g, b = _r(c, 1, 0.2, 1.0), _r(c, 2)
    dy = _r((rows, c), 3)
    ln = LayerNorm(c)
    ln.g.v.copy_(to_dev(g))
    ln.b.v.copy_(to_dev(b))
    y = to_host(ln.forward(_dev(x), True))
    want, xh, iv = orc.ln_forward(x, g, b)
    assert rel_frob(y, want) < 1e-6
    assert np.mean(y.ravel() == want.ravel()) >= 0.99
    assert rel_frob(to_host(ln.xhat), xh) < 1e-6
    assert rel_frob(to_host(ln.invstd), iv) < 1e-6
    ye = to_host(ln.forward(_dev(x), False))  # eval: same output, nothing kept
    assert rel_frob(ye, want) < 1e-6
    ln.forward(_dev(x), True)
    dx = to_host(ln.backward(_dev(dy)))
    dg, db = np.zeros(c, np.float32), np.zeros(c, np.float32)
    # the oracle's backward on the device's xhat / invstd, so only the
    # backward's own arithmetic is compared
    wdx = orc.ln_backward(dy, to_host(ln.xhat).reshape(rows, c), to_host(ln.invstd), g, dg, db)
    assert rel_frob(dx, wdx) < TOL
    assert rel_frob(to_host(ln.g.g), dg) < TOL
    assert rel_frob(to_host(ln.b.g), db) < TOL


@pytest.mark.parametrize("rows,c", [(300, 256), (37, 1024)])
def test_layernorm_backward_add(rnn, orc, rows, c):
    """rnn_ln_backward_add == rnn_ln_backward then add_, bit for bit, into a
    new tensor and in place on the addend (one pass for c <= 512, the
    two-kernel path above)."""
    from rustnn_amd.norm import LayerNorm
    x, dy, r = _r((rows, c), 31, 2.0, 0.5), _r((rows, c), 32), _r((rows, c), 33)
    ln = LayerNorm(c)
    ln.g.v.copy_(to_dev(_r(c, 34, 0.2, 1.0)))
    ln.forward(_dev(x), True)
    plain = to_host(ln.backward(_dev(dy))).reshape(rows, c)
    dg, db = to_host(ln.g.g).copy(), to_host(ln.b.g).copy()
    want = (plain + r).astype(np.float32)
    got = to_host(ln.backward(_dev(dy), add=_dev(r))).reshape(rows, c)
    assert np.array_equal(got, want)
    R = _dev(r)
    ln.backward(_dev(dy), add=R, out=R)
    assert np.array_equal(to_host(R).reshape(rows, c), want)
    # the parameter gradients accumulate as the plain backward's did
    assert rel_frob(to_host(ln.g.g), 3 * dg) < TOL and rel_frob(to_host(ln.b.g), 3 * db) < TOL


@pytest.mark.parametrize("n,t,c,masked", [(8, 64, 256, True), (3, 5, 384, False),
                                          (2, 9, 600, True)])
def test_layernorm_backward_add_ls(rnn, orc, n, t, c, masked):
    """rnn_ln_backward_add_ls == rnn_ln_backward_add then the DropPath +
    LayerScale backward of its dx (rnn_drop_layerscale_backward), bit for
    bit: dx, the LayerScale's input gradient, dgamma / dbeta and dl (c 600:
    the separate passes; 3 x 5 rows leave a partial row block)."""
    from rustnn_amd.norm import LayerNorm, LayerScale
    rows = n * t
    x, dy, r, lx = (_r((rows, c), 41 + i, 1.5 if i == 0 else 1.0) for i in range(4))
    mask = ((np.random.default_rng(45).random(n) < 0.7) / 0.7).astype(np.float32) if masked \
        else None
    outs = []
    for fused in (False, True):
        ln, ls = LayerNorm(c), LayerScale(c, 0.3)
        ln.g.v.copy_(to_dev(_r(c, 46, 0.2, 1.0)))
        ls.l.v.copy_(to_dev(_r(c, 47, 0.1, 0.4)))
        ln.forward(_dev(x), True)
        ls.x = _dev(lx)
        M = to_dev(mask) if masked else None
        R = _dev(r)
        if fused:
            dx, ldx = ln.backward(_dev(dy), add=R, out=R, ls=(ls, M))
        else:
            dx = ln.backward(_dev(dy), add=R, out=R)
            ldx = ls.backward(dx, M)
        outs.append([to_host(v).ravel() for v in (dx, ldx, ln.g.g, ln.b.g, ls.l.g)])
    for a, b in zip(*outs):
        assert np.array_equal(a, b)
    assert outs[1][4].any()


def test_layerscale(rnn, orc):
    from rustnn_amd.norm import LayerScale
    rows, c = 2048, 384
    x, l, dy = _r((rows, c), 4), _r(c, 5, 1e-2), _r((rows, c), 6)
    ls = LayerScale(c, 1e-4)
    ls.l.v.copy_(to_dev(l))
    y = to_host(ls.forward(_dev(x), True))
    assert np.array_equal(y.reshape(rows, c), orc.layerscale_forward(x, l))
    dl = np.zeros(c, np.float32)
    wdx = orc.layerscale_backward(dy, x, l, dl)
    dx = to_host(ls.backward(_dev(dy)))
    assert np.array_equal(dx.reshape(rows, c), wdx)
    assert rel_frob(to_host(ls.l.g), dl) < TOL


@pytest.mark.parametrize("n,t,c,masked", [(16, 64, 256, True), (3, 7, 33, True),
                                           (5, 16, 384, False)])
def test_residual_add_scaled(rnn, orc, n, t, c, masked):
    """rnn_residual_add_scaled == x + DropPath(LayerScale(a)) composed from
    the oracle's LayerScale forward, the per-image mask and add_, bit for
    bit, out of place and in place; a is left unchanged."""
    import ctypes as C
    from rustnn_amd import _ptr, lib
    rows = n * t
    x, a, l = _r((rows, c), 24), _r((rows, c), 25), _r(c, 26, 1e-2)
    keep = np.float32(0.8)
    mask = np.where(np.arange(n) % 3 == 1, np.float32(0.0), np.float32(1.0) / keep).astype(np.float32)
    t_ = orc.layerscale_forward(a, l).reshape(n, t, c)
    if masked:
        t_ = np.where(mask[:, None, None] == 1.0, t_, t_ * mask[:, None, None]).astype(np.float32)
    want = (x.reshape(n, t, c) + t_).astype(np.float32).reshape(rows, c)
    ctx = rnn.default_ctx()
    X, A, L = _dev(x), _dev(a), to_dev(l)
    M = to_dev(mask) if masked else None
    for inplace in (False, True):
        Y = X.clone() if inplace else _dev(np.zeros((rows, c), np.float32))
        src = Y if inplace else X
        ctx.check(lib().rnn_residual_add_scaled(
            ctx.h, rows, c, _ptr(src, rows * c, "x"), _ptr(A, rows * c, "a"), _ptr(L, c, "l"),
            _ptr(M, n, "m") if masked else None, t, _ptr(Y, rows * c, "y")))
        assert np.array_equal(to_host(Y).reshape(rows, c), want)
    assert np.array_equal(to_host(A).reshape(rows, c), a.reshape(rows, c))


@pytest.mark.parametrize("n,t,c", [(16, 64, 256), (3, 7, 33)])
def test_drop_layerscale_backward(rnn, orc, n, t, c):
    """rnn_drop_layerscale_backward == DropPath::backward (dy times the
    image's mask) then LayerScale::backward, dy left unchanged."""
    from rustnn_amd.norm import LayerScale
    rows = n * t
    x, l, dy = _r((rows, c), 14), _r(c, 15, 1e-2), _r((rows, c), 16)
    keep = np.float32(0.8)
    mask = np.where(np.arange(n) % 3 == 1, np.float32(0.0), np.float32(1.0) / keep)
    mask = mask.astype(np.float32)
    ls = LayerScale(c, 1e-4)
    ls.l.v.copy_(to_dev(l))
    ls.forward(_dev(x), True)
    g = (dy.reshape(n, t, c) * mask[:, None, None]).reshape(rows, c).astype(np.float32)
    dl = np.zeros(c, np.float32)
    wdx = orc.layerscale_backward(g, x, l, dl)
    DY = _dev(dy)
    dx = to_host(ls.backward(DY, to_dev(mask)))
    assert np.array_equal(dx.reshape(rows, c), wdx)
    assert rel_frob(to_host(ls.l.g), dl) < TOL
    assert np.array_equal(to_host(DY).reshape(rows, c), dy.reshape(rows, c))


@pytest.mark.parametrize("n,t,c,cross,masked", [(8, 64, 256, True, (True, True)),
                                                (8, 64, 256, False, (True, False)),
                                                (3, 5, 200, True, (False, True)),
                                                (2, 9, 600, True, (True, True)),
                                                (4, 16, 384, True, (False, False))])
def test_block_branch_backward(rnn, orc, n, t, c, cross, masked):
    """rnn_block_branch_backward equals the separate calls it fuses, bit for
    bit: lsm's and ls1's DropPath + LayerScale backward, then the gamma
    gate's LayerScale backward over da (c = 600 takes the separate passes
    themselves; 3 x 5 = 15 rows leave a partial row block)."""
    import torch
    from rustnn_amd import default_ctx, lib, _ptr
    rows = n * t
    dy, a, dwo, cm = (_dev(_r((rows, c), 40 + i)) for i in range(4))
    l1, gam, lm = (_dev(_r(c, 50 + i, 0.3, 0.5)) for i in range(3))
    mk = lambda s: _dev((np.random.default_rng(s).random(n) < 0.7).astype(np.float32) / 0.7)
    m1 = mk(60) if masked[0] else None
    m2 = mk(61) if masked[1] and cross else None
    dl0 = [_dev(_r(c, 70 + i)) for i in range(3)]
    ctx = default_ctx()
    L = lib()
    P = lambda x, k: _ptr(x, k, "x")
    # the separate calls
    dl1, dg, dlm = (d.clone() for d in dl0)
    da, ddw, dc = (torch.empty_like(dy) for _ in range(3))
    if cross:
        ctx.check(L.rnn_drop_layerscale_backward(ctx.h, rows, c, P(dy, rows * c), P(cm, rows * c),
                                                 P(lm, c), P(m2, n), t, P(dc, rows * c),
                                                 P(dlm, c)))
    ctx.check(L.rnn_drop_layerscale_backward(ctx.h, rows, c, P(dy, rows * c), P(a, rows * c),
                                             P(l1, c), P(m1, n), t, P(da, rows * c), P(dl1, c)))
    ctx.check(L.rnn_layerscale_backward(ctx.h, rows, c, P(da, rows * c), P(dwo, rows * c),
                                        P(gam, c), P(ddw, rows * c), P(dg, c)))
    # the fused pass
    fl1, fg, flm = (d.clone() for d in dl0)
    fa, fw, fc = (torch.full_like(dy, 7.0) for _ in range(3))
    ctx.check(L.rnn_block_branch_backward(
        ctx.h, rows, c, P(dy, rows * c), P(a, rows * c), P(l1, c), P(m1, n), P(dwo, rows * c),
        P(gam, c), P(cm, rows * c) if cross else None, P(lm, c) if cross else None, P(m2, n), t,
        P(fa, rows * c), P(fl1, c), P(fw, rows * c), P(fg, c),
        P(fc, rows * c) if cross else None, P(flm, c) if cross else None))
    pairs = [(fa, da), (fw, ddw), (fl1, dl1), (fg, dg)]
    if cross:
        pairs += [(fc, dc), (flm, dlm)]
    else:
        assert np.all(to_host(fc) == 7.0) and np.array_equal(to_host(flm), to_host(dl0[2]))
    for got, want in pairs:
        assert np.array_equal(to_host(got), to_host(want))
    assert to_host(fl1).any() and to_host(fw).any()


@pytest.mark.parametrize("rows,h", [(4096, 352), (1000, 512), (7, 5)])
def test_swiglu_gate(rnn, orc, rows, h):
    import torch
    from rustnn_amd import default_ctx, lib, _ptr
    ab = _r((rows, 2 * h), rows + h, 2.0)
    du = _r((rows, h), 7)
    ctx = default_ctx()
    u = torch.empty(rows * h, device="cuda")
    dab = torch.empty(rows * 2 * h, device="cuda")
    A, D = to_dev(ab), to_dev(du)
    ctx.check(lib().rnn_swiglu_forward(ctx.h, rows, h, _ptr(A, ab.size, "ab"),
                                       _ptr(u, rows * h, "u")))
    ctx.check(lib().rnn_swiglu_backward(ctx.h, rows, h, _ptr(D, du.size, "du"),
                                        _ptr(A, ab.size, "ab"), _ptr(dab, ab.size, "dab")))
    assert rel_frob(to_host(u), orc.swiglu_forward(ab, h)) < 1e-6
    assert rel_frob(to_host(dab), orc.swiglu_backward(du, ab, h)) < 1e-6
    if h % 4 == 0:
        # operands one float off 16-byte alignment take the one-element
        # kernels: the four-column kernels equal them bit for bit
        A1, D1 = torch.zeros(ab.size + 1, device="cuda"), torch.zeros(du.size + 1, device="cuda")
        A1[1:].copy_(A.reshape(-1))
        D1[1:].copy_(D.reshape(-1))
        u1 = torch.empty(rows * h + 1, device="cuda")
        dab1 = torch.empty(rows * 2 * h + 1, device="cuda")
        ctx.check(lib().rnn_swiglu_forward(ctx.h, rows, h, A1[1:].data_ptr(), u1[1:].data_ptr()))
        ctx.check(lib().rnn_swiglu_backward(ctx.h, rows, h, D1[1:].data_ptr(), A1[1:].data_ptr(),
                                            dab1[1:].data_ptr()))
        assert np.array_equal(to_host(u1[1:]), to_host(u))
        assert np.array_equal(to_host(dab1[1:]), to_host(dab))


def test_swiglu_layer(rnn, orc):
    """SwiGlu (wg, gate, wd) at the rustvit's stage-3 shape vs the oracle."""
    from rustnn_amd.norm import SwiGlu
    rows, c, h = 2048, 256, 352
    x, dy = _r((rows, c), 8), _r((rows, c), 9)
    wg, bg = _r(2 * h * c, 10, 0.02), _r(2 * h, 11, 0.1)
    wd, bd = _r(c * h, 12, 0.02), _r(c, 13, 0.1)
    sw = SwiGlu(c, h, to_dev(wg), to_dev(bg), to_dev(wd), to_dev(bd))
    y = to_host(sw.forward(_dev(x), True))
    ab = orc.linear_forward(rows, c, 2 * h, x, wg, bg)
    u = orc.swiglu_forward(ab, h)
    assert rel_frob(y, orc.linear_forward(rows, h, c, u, wd, bd)) < TOL
    dx = to_host(sw.backward(_dev(dy)))
    dwd, dbd, du = orc.linear_backward(rows, h, c, dy, u, wd, np.zeros_like(wd), np.zeros_like(bd))
    dab = orc.swiglu_backward(du, ab, h)
    dwg, dbg, wdx = orc.linear_backward(rows, c, 2 * h, dab, x, wg, np.zeros_like(wg),
                                        np.zeros_like(bg))
    assert rel_frob(dx, wdx) < TOL
    got = []
    sw.for_each_param(lambda p: got.append(to_host(p.g)))
    for g_, w_ in zip(got, (dwg, dbg, dwd, dbd)):
        assert rel_frob(g_, w_) < TOL


@pytest.mark.parametrize("n,th,tw,c", [(64, 8, 8, 256), (16, 4, 4, 384), (3, 5, 4, 12),
                                       (2, 1, 7, 5)])
def test_dwconv3(rnn, orc, n, th, tw, c):
    from rustnn_amd.norm import DwConv3
    x, dy = _r((n, th * tw, c), n + c), _r((n, th * tw, c), 14)
    w, b = _r((9, c), 15, 0.1), _r(c, 16)
    dw = DwConv3(c, th, tw, to_dev(w.ravel()), to_dev(b))
    y = to_host(dw.forward(_dev(x), True))
    assert np.array_equal(y.reshape(x.shape), orc.dwconv3_forward(x, w, b, n, th, tw))
    gw, gb = np.zeros((9, c), np.float32), np.zeros(c, np.float32)
    wdx = orc.dwconv3_backward(dy, x, w, n, th, tw, gw, gb)
    dx = to_host(dw.backward(_dev(dy)))
    assert np.array_equal(dx.reshape(x.shape), wdx)
    assert rel_frob(to_host(dw.w.g), gw) < TOL
    assert rel_frob(to_host(dw.b.g), gb) < TOL


@pytest.mark.parametrize("n,th,tw,c,masked", [(64, 8, 8, 256, True), (16, 4, 4, 384, False),
                                               (3, 5, 4, 12, True), (2, 1, 7, 5, True)])
def test_dwconv3_branch_forward(rnn, orc, n, th, tw, c, masked):
    """rnn_dwconv3_branch_forward == the oracle's DwConv3 forward, then
    a + gamma d and x + DropPath(LayerScale(a)) (vit.rs:150-160) composed in
    numpy f32, bit for bit; out of place and with y = x (c = 5: the unfused
    fallback)."""
    from rustnn_amd.norm import DwConv3
    t = th * tw
    h, a, x = _r((n, t, c), 30), _r((n, t, c), 31), _r((n, t, c), 32)
    w, b, gam, l = _r((9, c), 33, 0.1), _r(c, 34), _r(c, 35, 0.5), _r(c, 36, 1e-2)
    keep = np.float32(0.8)
    mask = np.where(np.arange(n) % 3 == 1, np.float32(0.0), np.float32(1.0) / keep).astype(np.float32)
    wd = orc.dwconv3_forward(h, w, b, n, th, tw).reshape(n, t, c)
    wa = (a + gam * wd).astype(np.float32)
    ts = orc.layerscale_forward(wa.reshape(-1, c), l).reshape(n, t, c)
    if masked:
        ts = (ts * mask[:, None, None]).astype(np.float32)
    wy = (x + ts).astype(np.float32)
    dw = DwConv3(c, th, tw, to_dev(w.ravel()), to_dev(b))
    for inplace in (False, True):
        H, A, X = _dev(h), _dev(a), _dev(x)
        Y = X if inplace else _dev(np.zeros((n, t, c), np.float32))
        M = to_dev(mask) if masked else None
        D = dw.forward_branch(H, A, to_dev(gam), X, to_dev(l), M, Y, True)
        assert np.array_equal(to_host(D).reshape(n, t, c), wd)
        assert np.array_equal(to_host(A).reshape(n, t, c), wa)
        assert np.array_equal(to_host(Y).reshape(n, t, c), wy)
        assert dw.x is H and dw.n == n


@pytest.mark.parametrize("n,th,tw,c", [(64, 8, 8, 256), (2, 1, 7, 5)])
def test_dwconv3_backward_acc(rnn, orc, n, th, tw, c):
    """rnn_dwconv3_backward_ex with RNN_DW3_ACC_DX: dx0 + the oracle's input
    gradient, bit for bit (c = 5: the scalar kernel)."""
    from rustnn_amd.norm import DwConv3
    x, dy, dx0 = _r((n, th * tw, c), 40), _r((n, th * tw, c), 41), _r((n, th * tw, c), 42)
    w, b = _r((9, c), 43, 0.1), _r(c, 44)
    dw = DwConv3(c, th, tw, to_dev(w.ravel()), to_dev(b))
    dw.forward(_dev(x), True)
    gw, gb = np.zeros((9, c), np.float32), np.zeros(c, np.float32)
    wdx = orc.dwconv3_backward(dy, x, w, n, th, tw, gw, gb).reshape(x.shape)
    DX = _dev(dx0)
    out = dw.backward(_dev(dy), acc_dx=DX)
    assert out is DX
    assert np.array_equal(to_host(DX).reshape(x.shape), (dx0 + wdx).astype(np.float32))
    assert rel_frob(to_host(dw.w.g), gw) < TOL


@pytest.mark.parametrize("n,t,c", [(256, 16, 384), (64, 64, 256), (3, 9, 8), (5, 1, 33)])
def test_seqpool(rnn, orc, n, t, c):
    from rustnn_amd.norm import SeqPool
    x, p, dz = _r((n, t, c), n + t), _r(c, 17, 0.3), _r((n, c), 18)
    sp = SeqPool(c, to_dev(p))
    z = to_host(sp.forward(_dev(x), True))
    wz, ww = orc.seqpool_forward(x, p, n, t)
    assert rel_frob(z, wz) < 1e-6
    assert rel_frob(to_host(sp.w), ww) < 1e-6
    dp = np.zeros(c, np.float32)
    # the oracle's backward on the device's softmax weights
    wdx = orc.seqpool_backward(dz, to_host(sp.w), x, p, n, t, dp)
    dx = to_host(sp.backward(_dev(dz)))
    assert rel_frob(dx, wdx) < TOL
    assert rel_frob(to_host(sp.p.g), dp) < TOL


class GpuNorm:
    """normcheck backend on the device layers (numpy in and out)."""

    def ln(self, x, g, b, dy):
        from rustnn_amd.norm import LayerNorm
        ln = LayerNorm(g.size)
        ln.g.v.copy_(to_dev(g))
        ln.b.v.copy_(to_dev(b))
        y = ln.forward(_dev(x), True)
        dx = ln.backward(_dev(dy))
        return to_host(y), to_host(dx), np.concatenate([to_host(ln.g.g), to_host(ln.b.g)])

    def ln_y(self, x, g, b):
        from rustnn_amd.norm import LayerNorm
        ln = LayerNorm(g.size)
        ln.g.v.copy_(to_dev(g))
        ln.b.v.copy_(to_dev(b))
        return to_host(ln.forward(_dev(x), False))

    def _sw(self, wg, bg, wd, bd, h):
        from rustnn_amd.norm import SwiGlu
        return SwiGlu(wd.size // h, h, to_dev(wg), to_dev(bg), to_dev(wd), to_dev(bd))

    def sw(self, x, wg, bg, wd, bd, h, dy):
        sw = self._sw(wg, bg, wd, bd, h)
        y = sw.forward(_dev(x), True)
        dx = sw.backward(_dev(dy))
        g = []
        sw.for_each_param(lambda p: g.append(to_host(p.g)))
        return to_host(y), to_host(dx), np.concatenate(g)

    def sw_y(self, x, wg, bg, wd, bd, h):
        return to_host(self._sw(wg, bg, wd, bd, h).forward(_dev(x), False))

    def dw(self, x, w, b, n, th, tw, dy):
        from rustnn_amd.norm import DwConv3
        d = DwConv3(b.size, th, tw, to_dev(w.ravel()), to_dev(b))
        y = d.forward(_dev(x), True)
        dx = d.backward(_dev(dy))
        return to_host(y), to_host(dx), np.concatenate([to_host(d.w.g), to_host(d.b.g)])

    def dw_y(self, x, w, b, n, th, tw):
        from rustnn_amd.norm import DwConv3
        return to_host(DwConv3(b.size, th, tw, to_dev(w.ravel()), to_dev(b)).forward(_dev(x),
                                                                                      False))

    def sp(self, x, p, n, t, dz):
        from rustnn_amd.norm import SeqPool
        s = SeqPool(p.size, to_dev(p))
        z = s.forward(_dev(x), True)
        dx = s.backward(to_dev(dz))
        return to_host(z), to_host(dx), to_host(s.p.g)

    def sp_z(self, x, p, n, t):
        from rustnn_amd.norm import SeqPool
        return to_host(SeqPool(p.size, to_dev(p)).forward(_dev(x), False))


def test_reference_normcheck_on_gpu(rnn, orc):
    errs = normcheck(orc, GpuNorm())
    bad = {k: v for k, v in errs.items() if not v < refcheck.TOL}
    assert not bad, errs
