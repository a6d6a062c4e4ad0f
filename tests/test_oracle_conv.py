"""Pins the oracle's convolution (conv.rs + Conv2d drivers, nn.rs:166-250) on
the CPU: torch-CPU golden fixtures, an f64 direct convolution, the adjoint
identities that tie forward, dX and dW together, integer exactness, im2col
against its closed form, and the reference's own conv gradcheck."""
import glob
import os

import numpy as np
import pytest

from conftest import rel_frob
import refcheck

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def conv64(x, w, n, cin, cout, k, s, p, h, wd):
    """Direct convolution in f64 (definition)."""
    X = np.pad(x.reshape(n, cin, h, wd).astype(np.float64), ((0, 0), (0, 0), (p, p), (p, p)))
    W = w.reshape(cout, cin, k, k).astype(np.float64)
    oh, ow = (h + 2 * p - k) // s + 1, (wd + 2 * p - k) // s + 1
    Y = np.zeros((n, cout, oh, ow))
    for kh in range(k):
        for kw in range(k):
            patch = X[:, :, kh:kh + s * (oh - 1) + 1:s, kw:kw + s * (ow - 1) + 1:s]
            Y += np.einsum("nchw,oc->nohw", patch, W[:, :, kh, kw])
    return Y


def conv64_dx(dy, w, n, cin, cout, k, s, p, h, wd):
    oh, ow = (h + 2 * p - k) // s + 1, (wd + 2 * p - k) // s + 1
    DY = dy.reshape(n, cout, oh, ow).astype(np.float64)
    W = w.reshape(cout, cin, k, k).astype(np.float64)
    DX = np.zeros((n, cin, h + 2 * p, wd + 2 * p))
    for kh in range(k):
        for kw in range(k):
            DX[:, :, kh:kh + s * (oh - 1) + 1:s, kw:kw + s * (ow - 1) + 1:s] += np.einsum(
                "nohw,oc->nchw", DY, W[:, :, kh, kw])
    return DX[:, :, p:p + h, p:p + wd]


def conv64_dw(dy, x, n, cin, cout, k, s, p, h, wd):
    X = np.pad(x.reshape(n, cin, h, wd).astype(np.float64), ((0, 0), (0, 0), (p, p), (p, p)))
    oh, ow = (h + 2 * p - k) // s + 1, (wd + 2 * p - k) // s + 1
    DY = dy.reshape(n, cout, oh, ow).astype(np.float64)
    DW = np.zeros((cout, cin, k, k))
    for kh in range(k):
        for kw in range(k):
            patch = X[:, :, kh:kh + s * (oh - 1) + 1:s, kw:kw + s * (ow - 1) + 1:s]
            DW[:, :, kh, kw] = np.einsum("nohw,nchw->oc", DY, patch)
    return DW


SHAPES = [(2, 3, 4, 3, 1, 1, 6), (2, 4, 6, 1, 2, 0, 8), (2, 4, 5, 3, 2, 1, 7),
          (3, 32, 32, 3, 1, 1, 16), (2, 32, 64, 3, 2, 1, 16), (2, 64, 128, 1, 2, 0, 16),
          (2, 5, 7, 3, 2, 1, 9), (1, 300, 20, 3, 1, 1, 5)]


@pytest.mark.parametrize("n,cin,cout,k,s,p,h", SHAPES)
def test_conv_vs_f64_direct(orc, n, cin, cout, k, s, p, h):
    sp = orc.ConvSpec.make(cin, cout, k, s, p, h, h)
    rng = orc.Rng(cin * 100 + cout)
    x = rng.rand_vec(n * cin * h * h)
    w = rng.rand_vec(cout * sp.ckk)
    dy = rng.rand_vec(n * cout * sp.hw)
    assert rel_frob(orc.conv2d_forward(sp, n, x, w), conv64(x, w, n, cin, cout, k, s, p, h, h)) < 1e-6
    assert rel_frob(orc.conv2d_backward_x(sp, n, dy, w),
                    conv64_dx(dy, w, n, cin, cout, k, s, p, h, h)) < 1e-6
    assert rel_frob(orc.conv2d_backward_w(sp, n, dy, x),
                    conv64_dw(dy, x, n, cin, cout, k, s, p, h, h)) < 1e-6


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLD, "conv_*.npz"))),
                         ids=lambda p: os.path.basename(p))
def test_conv_golden(orc, path):
    """Oracle against torch-CPU float64 fixtures (tests/golden/make_golden.py)."""
    z = np.load(path)
    n, cin, cout, k, s, p, h = (int(v) for v in z["spec"])
    sp = orc.ConvSpec.make(cin, cout, k, s, p, h, h)
    assert rel_frob(orc.conv2d_forward(sp, n, z["x"], z["w"]), z["y"]) < 1e-6
    assert rel_frob(orc.conv2d_backward_x(sp, n, z["dy"], z["w"]), z["dx"]) < 1e-6
    assert rel_frob(orc.conv2d_backward_w(sp, n, z["dy"], z["x"]), z["dw"]) < 1e-6
    # the f64 definition used above agrees with torch too
    assert rel_frob(conv64(z["x"], z["w"], n, cin, cout, k, s, p, h, h), z["y"]) < 1e-12


@pytest.mark.parametrize("n,cin,cout,k,s,p,h", SHAPES[:4])
def test_adjoint_identities(orc, n, cin, cout, k, s, p, h):
    """<conv(x), dy> = <x, dX(dy)> = <w, dW(dy, x)>: dX and dW are the exact
    adjoints of the forward map (catches flipped taps, swapped channels)."""
    sp = orc.ConvSpec.make(cin, cout, k, s, p, h, h)
    rng = orc.Rng(77)
    x, w, dy = rng.rand_vec(n * cin * h * h), rng.rand_vec(cout * sp.ckk), rng.rand_vec(n * cout * sp.hw)
    y = orc.conv2d_forward(sp, n, x, w).astype(np.float64).ravel()
    dx = orc.conv2d_backward_x(sp, n, dy, w).astype(np.float64).ravel()
    dw = orc.conv2d_backward_w(sp, n, dy, x).astype(np.float64).ravel()
    a = y @ dy
    assert abs(a - x @ dx) <= 1e-5 * (abs(a) + 1)
    assert abs(a - w @ dw) <= 1e-5 * (abs(a) + 1)


def test_conv_integer_exact_and_threads(orc):
    n, cin, cout, k, s, p, h = 6, 32, 64, 3, 2, 1, 16
    sp = orc.ConvSpec.make(cin, cout, k, s, p, h, h)
    r = np.random.default_rng(0)
    x = r.integers(-2, 3, n * cin * h * h).astype(np.float32)
    w = r.integers(-2, 3, cout * sp.ckk).astype(np.float32)
    dy = r.integers(-2, 3, n * cout * sp.hw).astype(np.float32)
    y = orc.conv2d_forward(sp, n, x, w)
    assert np.array_equal(y, conv64(x, w, n, cin, cout, k, s, p, h, h).astype(np.float32))
    dw1 = orc.conv2d_backward_w(sp, n, dy, x)
    with orc.threads(4):
        dw4 = orc.conv2d_backward_w(sp, n, dy, x)
        y4 = orc.conv2d_forward(sp, n, x, w)
    assert np.array_equal(dw1, dw4) and np.array_equal(y, y4)
    assert np.array_equal(dw1, conv64_dw(dy, x, n, cin, cout, k, s, p, h, h).reshape(cout, -1))


@pytest.mark.parametrize("cin,k,s,p,h", [(3, 3, 1, 1, 6), (4, 1, 2, 0, 8), (4, 3, 2, 1, 7),
                                         (2, 3, 1, 1, 5)])
def test_im2col_closed_form(orc, cin, k, s, p, h):
    """gather_span (conv.rs:68-120) == the im2col definition, bit for bit."""
    sp = orc.ConvSpec.make(cin, 1, k, s, p, h, h)
    x = orc.Rng(1).rand_vec(cin * h * h)
    X = x.reshape(cin, h, h)
    want = np.zeros((sp.ckk, sp.hw), np.float32)
    for ci in range(cin):
        for kh in range(k):
            for kw in range(k):
                for oy in range(sp.oh):
                    for ox in range(sp.ow):
                        iy, ix = oy * s + kh - p, ox * s + kw - p
                        if 0 <= iy < h and 0 <= ix < h:
                            want[(ci * k + kh) * k + kw, oy * sp.ow + ox] = X[ci, iy, ix]
    assert np.array_equal(orc.im2col(sp, x), want)
    rm = orc.rowmap(sp)
    assert [tuple(r) for r in rm] == [(ci, kh, kw) for ci in range(cin) for kh in range(k)
                                      for kw in range(k)]


def test_reference_conv_gradcheck_on_oracle(orc):
    """check.rs:510-546 at seed 1234 through the oracle: every dircheck < 5e-3."""
    res = refcheck.conv_layercheck(orc.Rng, refcheck.OracleConv(orc))
    assert len(res) == 6
    for tag, err in res:
        assert err < refcheck.TOL, (tag, err)


def test_planted_mistake_is_caught(orc):
    """A plausible oracle bug -- dropping one tap of dX -- fails the f64 pin."""
    n, cin, cout, k, s, p, h = 2, 3, 4, 3, 1, 1, 6
    sp = orc.ConvSpec.make(cin, cout, k, s, p, h, h)
    rng = orc.Rng(2)
    dy, w = rng.rand_vec(n * cout * sp.hw), rng.rand_vec(cout * sp.ckk)
    w_bad = w.reshape(cout, cin, k, k).copy()
    w_bad[:, :, 0, 0] = 0.0
    bad = orc.conv2d_backward_x(sp, n, dy, w_bad.ravel())
    assert rel_frob(bad, conv64_dx(dy, w, n, cin, cout, k, s, p, h, h)) > 1e-2
