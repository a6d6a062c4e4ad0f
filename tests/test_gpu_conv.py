"""GPU parity: implicit-GEMM convolution (conv.rs forward_image / dx_image /
dw_image through the Conv2d batch drivers, nn.rs:166-250) against the CPU
oracle on identical seeded inputs, at the BASELINE config shapes and at the
reference's gradcheck shapes (check.rs:505-509)."""
import zlib

import numpy as np
import pytest

from conftest import TOL, rel_frob, to_dev, to_host

pytestmark = pytest.mark.gpu

# (name, n, cin, cout, k, stride, pad, h)
SHAPES = [
    ("cfg0_3x3s1_32to32_32", 128, 32, 32, 3, 1, 1, 32),
    ("cfg1_3x3s2_32to64_32", 128, 32, 64, 3, 2, 1, 32),
    ("cfg1_3x3s1_64to64_16", 128, 64, 64, 3, 1, 1, 16),
    ("cfg1_3x3s2_64to128_16", 128, 64, 128, 3, 2, 1, 16),
    ("cfg1_3x3s1_128to128_8", 128, 128, 128, 3, 1, 1, 8),
    ("cfg1_1x1s2_32to64_32", 128, 32, 64, 1, 2, 0, 32),
    ("cfg1_1x1s2_64to128_16", 128, 64, 128, 1, 2, 0, 16),
    ("stem_3x3s1_3to32_32", 16, 3, 32, 3, 1, 1, 32),
    ("gc_3x3s1_3to4_6", 2, 3, 4, 3, 1, 1, 6),
    ("gc_1x1s2_4to6_8", 2, 4, 6, 1, 2, 0, 8),
    ("gc_3x3s2_4to5_7", 2, 4, 5, 3, 2, 1, 7),
    ("odd_3x3s1_5to40_9", 3, 5, 40, 3, 1, 1, 9),
    ("odd_3x3s2_34to33_11", 5, 34, 33, 3, 2, 1, 11),
    # the few-input-channel dW kernel: cin 1 and 2, pad 0, a partial last
    # tile of output rows (20 rows in tiles of 12) with 16-byte dY loads
    ("smallc_3x3s1_1to8_20", 3, 1, 8, 3, 1, 1, 20),
    ("smallc_3x3s1_2to40_22_p0", 3, 2, 40, 3, 1, 0, 22),
    # strided forward whose quarter-of-channels chunk (24) does not fit LDS
    # at 64 positions: the plan falls back to 8-channel chunks
    ("tok_3x3s2_96to256_16", 4, 96, 256, 3, 2, 1, 16),
]


def inputs(orc, sp, n, seed=7):
    """BASELINE config 0 draw order: x ~ N(0,1), W Kaiming-normal, dY ~ N(0,1)."""
    rng = orc.Rng(seed)
    x = rng.rand_vec(n * sp.cin * sp.h * sp.w)
    w = rng.rand_vec(sp.cout * sp.ckk) * np.float32(np.sqrt(2.0 / sp.ckk))
    dy = rng.rand_vec(n * sp.cout * sp.hw)
    return x, w, dy


@pytest.mark.parametrize("name,n,cin,cout,k,s,p,h", SHAPES, ids=[s[0] for s in SHAPES])
def test_conv_parity(rnn, orc, name, n, cin, cout, k, s, p, h):
    sp = orc.ConvSpec.make(cin, cout, k, s, p, h, h)
    gsp = rnn.ConvSpec.make(cin, cout, k, s, p, h, h)
    x, w, dy = inputs(orc, sp, n)
    dw0 = np.linspace(-1, 1, sp.cout * sp.ckk).astype(np.float32)
    with orc.threads(8):
        y_want = orc.conv2d_forward(sp, n, x, w)
        dx_want = orc.conv2d_backward_x(sp, n, dy, w)
        dw_want = orc.conv2d_backward_w(sp, n, dy, x, dw0).ravel()
    X, W, DY = to_dev(x), to_dev(w), to_dev(dy)
    y = rnn.conv2d_forward(gsp, n, X, W)
    dx = rnn.conv2d_backward_x(gsp, n, DY, W)
    dw = to_dev(dw0.copy())
    rnn.conv2d_backward_w(gsp, n, DY, X, dw)
    assert rel_frob(to_host(y), y_want) < TOL, "forward"
    assert rel_frob(to_host(dx), dx_want) < TOL, "dx"
    assert rel_frob(to_host(dw) - dw0, dw_want - dw0) < TOL, "dw"


@pytest.mark.parametrize("name,n,cin,cout,k,s,p,h", SHAPES, ids=[s[0] for s in SHAPES])
def test_conv_integer_bit_exact(rnn, orc, name, n, cin, cout, k, s, p, h):
    """Integer-valued fp32 inputs make every sum exact, so any summation order
    must reproduce the oracle bit for bit."""
    sp = orc.ConvSpec.make(cin, cout, k, s, p, h, h)
    gsp = rnn.ConvSpec.make(cin, cout, k, s, p, h, h)
    r = np.random.default_rng(zlib.crc32(name.encode()))
    x = r.integers(-2, 3, n * cin * h * h).astype(np.float32)
    w = r.integers(-2, 3, sp.cout * sp.ckk).astype(np.float32)
    dy = r.integers(-2, 3, n * sp.cout * sp.hw).astype(np.float32)
    with orc.threads(8):
        y_want = orc.conv2d_forward(sp, n, x, w)
        dx_want = orc.conv2d_backward_x(sp, n, dy, w)
        dw_want = orc.conv2d_backward_w(sp, n, dy, x)
    X, W, DY = to_dev(x), to_dev(w), to_dev(dy)
    assert np.array_equal(to_host(rnn.conv2d_forward(gsp, n, X, W)).ravel(), y_want.ravel())
    assert np.array_equal(to_host(rnn.conv2d_backward_x(gsp, n, DY, W)).ravel(), dx_want.ravel())
    dw = to_dev(np.zeros(sp.cout * sp.ckk, np.float32))
    rnn.conv2d_backward_w(gsp, n, DY, X, dw)
    assert np.array_equal(to_host(dw), dw_want.ravel())


@pytest.mark.parametrize("name,n,cin,cout,k,s,p,h", SHAPES, ids=[s[0] for s in SHAPES])
def test_conv_packed_weights_bit_exact(rnn, orc, name, n, cin, cout, k, s, p, h):
    """rnn_conv2d_forward_packed / _backward_x_packed (weights in the kernels'
    slab order, zero-padded) give the same bits as the unpacked calls: the
    same values reach the same LDS slabs.  The packed copy itself is checked
    element by element against W at sampled positions of the layout."""
    import rustnn_amd as R
    sp = R.ConvSpec.make(cin, cout, k, s, p, h, h)
    x, w, dy = inputs(orc, sp, n, seed=23)
    X, W, DY = to_dev(x), to_dev(w), to_dev(dy)
    for dx in (0, 1):
        wp = R.conv_pack_weights(sp, dx, W)
        if (k, s, p) not in ((3, 1, 1), (3, 2, 1), (1, 2, 0), (1, 1, 0)):
            assert wp is None  # no specialised kernel for this (k, stride, pad): nothing to pack
            return
        assert wp is not None
        if dx == 0:
            want = to_host(R.conv2d_forward(sp, n, X, W))
            got = to_host(R.conv2d_forward_packed(sp, n, X, W, wp))
        else:
            want = to_host(R.conv2d_backward_x(sp, n, DY, W))
            got = to_host(R.conv2d_backward_x_packed(sp, n, DY, W, wp))
        assert np.array_equal(got, want), (name, dx)
        # layout: [mblk][chunk][q][tap][lane][4]; find CH from the size
        kk = k * k
        cs, cd = (cout, cin) if dx else (cin, cout)
        hp = to_host(wp)
        nmblk = (cd + 31) // 32
        per_ch = hp.size // (nmblk * kk * 32)  # nchunks * CH
        W3 = w.reshape(cout, cin, kk)
        nz = int(np.count_nonzero(hp))
        assert nz == int(np.count_nonzero(W3)), (name, dx, nz)
        assert np.isclose(np.sort(np.abs(hp[hp != 0])), np.sort(np.abs(W3[W3 != 0]))).all()
        assert per_ch >= cs


@pytest.mark.parametrize("name,n,cin,cout,k,s,p,h", SHAPES, ids=[s[0] for s in SHAPES])
def test_conv_dw_slabs(rnn, orc, name, n, cin, cout, k, s, p, h):
    """rnn_conv2d_backward_w_slabs: nz partial slabs whose sum is the batch
    dW.  Integer-valued inputs: the slab sum equals the oracle bit for bit;
    seeded normal inputs: within TOL of the oracle, and the slab-order sum
    matches what rnn_conv2d_backward_w adds."""
    sp = orc.ConvSpec.make(cin, cout, k, s, p, h, h)
    gsp = rnn.ConvSpec.make(cin, cout, k, s, p, h, h)
    floats = rnn.conv2d_backward_w_slab_floats(gsp, n)
    ln = sp.cout * sp.ckk
    assert floats > 0 and floats % ln == 0, (floats, ln)
    r = np.random.default_rng(zlib.crc32(name.encode()) + 1)
    xi = r.integers(-2, 3, n * cin * h * h).astype(np.float32)
    dyi = r.integers(-2, 3, n * sp.cout * sp.hw).astype(np.float32)
    xg, _, dyg = inputs(orc, sp, n, seed=31)
    for x, dy, exact in ((xi, dyi, True), (xg, dyg, False)):
        with orc.threads(8):
            want = orc.conv2d_backward_w(sp, n, dy, x).ravel()
        X, DY = to_dev(x), to_dev(dy)
        slabs = to_dev(np.full(floats, np.nan, np.float32))
        nz = rnn.conv2d_backward_w_slabs(gsp, n, DY, X, slabs)
        assert 1 <= nz <= floats // ln
        sl = to_host(slabs)[: nz * ln].reshape(nz, ln)
        assert np.isfinite(sl).all(), "every slab element is written"
        got = sl.astype(np.float64).sum(axis=0)
        if exact:
            assert np.array_equal(got.astype(np.float32), want), name
        else:
            assert rel_frob(got, want) < TOL, name
            dw = to_dev(np.zeros(ln, np.float32))
            rnn.conv2d_backward_w(gsp, n, DY, X, dw)
            assert rel_frob(to_host(dw), got) < 1e-6, name


@pytest.mark.parametrize("cin,p,h", [(3, 1, 32), (2, 0, 22)])
def test_conv_dw_smallc_unaligned_dy(rnn, orc, cin, p, h):
    """The few-input-channel dW kernel reads dY with 16-byte loads only when
    dY is 16-byte aligned: a dY starting 4 bytes into its buffer takes the
    scalar path and gives the same sums."""
    n, cout = 4, 32
    sp = orc.ConvSpec.make(cin, cout, 3, 1, p, h, h)
    gsp = rnn.ConvSpec.make(cin, cout, 3, 1, p, h, h)
    x, _, dy = inputs(orc, sp, n, seed=41)
    with orc.threads(8):
        want = orc.conv2d_backward_w(sp, n, dy, x).ravel()
    buf = to_dev(np.concatenate([np.zeros(1, np.float32), dy]))
    DY = buf[1:]
    assert DY.data_ptr() % 16 != 0
    got = []
    for d in (DY, to_dev(dy)):
        dw = to_dev(np.zeros(sp.cout * sp.ckk, np.float32))
        rnn.conv2d_backward_w(gsp, n, d, to_dev(x), dw)
        got.append(to_host(dw))
    assert rel_frob(got[0], want) < TOL
    assert np.array_equal(got[0], got[1])


def test_conv_packs_object(rnn, orc):
    """rnn_conv_packs_*: Conv2d layers on one ConvPacks give the unpacked
    calls' forward and dX bit for bit -- before and after an in-place weight
    change followed by update() -- and within TOL of the oracle; a shape with
    no packed form (3x3 pad 0) keeps the plain path; a layer whose weights moved
    makes update() raise."""
    import torch
    ctx = rnn.default_ctx()
    shapes = [(3, 32, 3, 1, 1, 32), (32, 96, 3, 2, 1, 32), (32, 96, 1, 2, 0, 32),
              (16, 24, 3, 1, 0, 12), (96, 64, 3, 1, 1, 16)]
    n = 4
    rng = orc.Rng(77)
    layers = []
    for (cin, cout, k, s_, p, h) in shapes:
        w = to_dev(rng.rand_vec(cout * cin * k * k) * np.float32(0.1))
        layers.append((rnn.Conv2d(cin, cout, k, s_, p, w, ctx=ctx), h))
    packs = rnn.ConvPacks([(c, h, h) for c, h in layers], ctx=ctx)
    assert layers[3][0].packed[1] is None and layers[3][0].packed[2] is None  # pad 0
    assert all(c.packed[1] for c, _ in layers[:3] + layers[4:])

    def run(c, h, x, dy):
        y = c.forward(x, n, h, h, True)
        dx = c.backward(dy)
        return to_host(y), to_host(dx)

    for step in range(2):
        for c, h in layers:
            sp = c.spec(h, h)
            x = to_dev(rng.rand_vec(n * c.cin * h * h))
            dy = to_dev(rng.rand_vec(n * c.cout * sp.hw))
            got = run(c, h, x, dy)
            keep, c.packed = c.packed, None
            want = run(c, h, x, dy)
            c.packed = keep
            assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
            osp = orc.ConvSpec.make(c.cin, c.cout, c.k, c.stride, c.pad, h, h)
            assert rel_frob(got[0], orc.conv2d_forward(osp, n, to_host(x), to_host(c.w))) < TOL
        for c, _ in layers:  # an optimiser step: W changes in place
            c.w.mul_(0.5).add_(0.01)
        packs.update()
    c0 = layers[0][0]
    c0.w = c0.w.clone()
    with pytest.raises(RuntimeError):
        packs.update()
    packs.close()
    assert all(c.packed is None for c, _ in layers)


def test_conv_deterministic(rnn, orc):
    sp = rnn.ConvSpec.make(32, 32, 3, 1, 1, 32, 32)
    x, w, dy = inputs(orc, sp, 128, seed=99)
    X, W, DY = to_dev(x), to_dev(w), to_dev(dy)
    outs = []
    for _ in range(2):
        dw = to_dev(np.zeros(sp.cout * sp.ckk, np.float32))
        rnn.conv2d_backward_w(sp, 128, DY, X, dw)
        outs.append((to_host(rnn.conv2d_forward(sp, 128, X, W)),
                     to_host(rnn.conv2d_backward_x(sp, 128, DY, W)), to_host(dw)))
    for a, b in zip(*outs):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("cin,cout,k,s,p,h", [(3, 4, 3, 1, 1, 6), (4, 6, 1, 2, 0, 8),
                                              (4, 5, 3, 2, 1, 7), (32, 32, 3, 1, 1, 32)])
def test_dbg_im2col_export_bit_exact(rnn, orc, cin, cout, k, s, p, h):
    """rnn_dbg_im2col, the debug export of the RowMap / gather_span layout
    (conv.rs:68-120), equals the oracle's im2col.  The export is its own
    small kernel: the conv kernels stage their windows by DMA instead, and
    that indexing is pinned by test_conv_integer_bit_exact (every sum exact,
    so any misplaced tap or halo element changes the result)."""
    sp = orc.ConvSpec.make(cin, cout, k, s, p, h, h)
    gsp = rnn.ConvSpec.make(cin, cout, k, s, p, h, h)
    x = orc.Rng(5).rand_vec(cin * h * h)
    got = to_host(rnn.dbg_im2col(gsp, to_dev(x))).reshape(sp.ckk, sp.hw)
    assert np.array_equal(got, orc.im2col(sp, x))


def test_conv_bad_spec_raises(rnn):
    sp = rnn.ConvSpec.make(4, 4, 3, 1, 1, 8, 8)
    bad = rnn.ConvSpec()
    for f in ("cin", "cout", "k", "stride", "pad", "h", "w", "oh", "ow"):
        setattr(bad, f, getattr(sp, f))
    bad.oh = 9  # does not match Conv2d::out_dim
    x = to_dev(np.zeros(4 * 64, np.float32))
    w = to_dev(np.zeros(4 * 36, np.float32))
    with pytest.raises(rnn.RnnError):
        rnn.conv2d_forward(bad, 1, x, w, y=to_dev(np.zeros(4 * 81, np.float32)))


def test_conv_layercheck_gpu(rnn, orc):
    """The reference's conv gradcheck (check.rs:503-546: 3x3/s1, 1x1/s2 and
    3x3/s2, dx and dw by dircheck at seed 1234, tolerance 5e-3) through the
    HIP conv path, in the reference's Rng draw order."""
    import refcheck
    res = refcheck.conv_layercheck(orc.Rng, refcheck.GpuConv(rnn))
    assert len(res) == 6
    bad = [(t, e) for t, e in res if not e < refcheck.TOL]
    assert not bad, res
