"""Restatement of the reference's gradient-check harness (check.rs), run
against a pluggable backend (the CPU oracle or the HIP path).

* dircheck (check.rs:16-40): central difference along a random direction v
  drawn from the same Rng, relative error |num - ana| / (|num| + |ana| + 1e-6).
* conv_layercheck (check.rs:503-546): the three conv layer shapes at seed 1234
  in the reference's exact Rng draw order (Kaiming W, x, r, then one direction
  per dircheck), tolerance 5e-3, eps = GC_EPS or 3e-4 (check.rs:55-60).
* nn_layercheck (check.rs:548-670): batchnorm dx / dgamma / dbeta, linear dx /
  dw, the two BasicBlock shapes (dx, dparams) and softmax_ce dlogits, drawing
  from the same Rng after the conv shapes.
* resnet_gradcheck (check.rs:727-775): ResNet(1, 4, 10, seed), parameters
  perturbed by 0.3*normal, batch 8 at 16x16, smooth 0, one dircheck over every
  parameter.
"""
import os

import numpy as np

TOL = 5e-3  # check.rs:42-44
SEED = 1234  # check.rs:778
CONV_SHAPES = [  # check.rs:505-509
    (3, 4, 3, 1, 1, 6, "conv 3x3/s1"),
    (4, 6, 1, 2, 0, 8, "conv 1x1/s2"),
    (4, 5, 3, 2, 1, 7, "conv 3x3/s2"),
]


def gc_eps():
    try:
        return float(os.environ.get("GC_EPS", "3e-4"))
    except ValueError:
        return 3e-4


def dircheck(base, grad, eps, rng, lossf):
    """check.rs:19-40 (f32 perturbation, as the reference)."""
    n = base.size
    v = rng.rand_vec(n)
    e = np.float32(eps)
    lp = np.float32(lossf((base + e * v).astype(np.float32)))
    lm = np.float32(lossf((base - e * v).astype(np.float32)))
    num = (lp - lm) / (np.float32(2.0) * e)
    ana = np.float32(np.dot(grad.astype(np.float64), v.astype(np.float64)))
    return float(abs(num - ana) / (abs(num) + abs(ana) + 1e-6))


def dot32(a, b):
    return np.float32(np.dot(np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()))


class OracleConv:
    """Conv backend on the CPU oracle."""

    def __init__(self, orc):
        self.o = orc

    def spec(self, cin, cout, k, s, p, h):
        return self.o.ConvSpec.make(cin, cout, k, s, p, h, h)

    def forward(self, sp, n, x, w):
        return self.o.conv2d_forward(sp, n, x, w).ravel()

    def backward(self, sp, n, dy, x, w, dw):
        dw = self.o.conv2d_backward_w(sp, n, dy, x, dw).ravel()
        return self.o.conv2d_backward_x(sp, n, dy, w).ravel(), dw


class GpuConv:
    """Conv backend on the HIP path (C ABI through rustnn_amd)."""

    def __init__(self, rnn):
        import torch
        self.r = rnn
        self.t = torch

    def _d(self, a):
        return self.t.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()

    def _h(self, t):
        self.t.cuda.synchronize()
        return t.cpu().numpy().ravel()

    def spec(self, cin, cout, k, s, p, h):
        return self.r.ConvSpec.make(cin, cout, k, s, p, h, h)

    def forward(self, sp, n, x, w):
        return self._h(self.r.conv2d_forward(sp, n, self._d(x), self._d(w)))

    def backward(self, sp, n, dy, x, w, dw):
        DW = self._d(dw)
        self.r.conv2d_backward_w(sp, n, self._d(dy), self._d(x), DW)
        dx = self.r.conv2d_backward_x(sp, n, self._d(dy), self._d(w))
        return self._h(dx), self._h(DW)


def conv_layercheck(rng_cls, backend):
    """Returns [(tag, err)] for dx and dw of each conv shape (check.rs:510-546)."""
    rng = rng_cls(SEED)
    eps = gc_eps()
    out = []
    for cin, cout, k, s, p, hh, tag in CONV_SHAPES:
        fan_in = cin * k * k
        sc = np.float32(np.sqrt(np.float32(2.0) / np.float32(fan_in)))  # nn.rs:95-100
        w = (rng.rand_vec(cout * fan_in) * sc).astype(np.float32)
        x = rng.rand_vec(2 * cin * hh * hh)
        sp = backend.spec(cin, cout, k, s, p, hh)
        y0 = backend.forward(sp, 2, x, w)
        r = rng.rand_vec(y0.size)
        dx, dw = backend.backward(sp, 2, r, x, w, np.zeros(w.size, np.float32))
        e = dircheck(x, dx, eps, rng, lambda c: dot32(backend.forward(sp, 2, c, w), r))
        out.append((f"{tag} dx", e))
        e = dircheck(w, dw, eps, rng, lambda c: dot32(backend.forward(sp, 2, x, c), r))
        out.append((f"{tag} dw", e))
    return out


# ------------------------------------------------------------- nn.rs layers
def _skip_conv_draws(rng):
    """Advances the Rng past conv_layercheck's draws (W, x, r, two directions)."""
    for cin, cout, k, s, p, hh, _ in CONV_SHAPES:
        oh = (hh + 2 * p - k) // s + 1
        ckk = cin * k * k
        rng.rand_vec(cout * ckk)
        rng.rand_vec(2 * cin * hh * hh)
        rng.rand_vec(2 * cout * oh * oh)
        rng.rand_vec(2 * cin * hh * hh)
        rng.rand_vec(cout * ckk)


def nn_layercheck(orc, be):
    """check.rs:548-670 on backend `be`; returns [(tag, err)]."""
    rng = orc.Rng(SEED)
    eps = gc_eps()
    _skip_conv_draws(rng)
    out = []
    # batchnorm (check.rs:548-598)
    c = 4
    g = (np.float32(0.5) + rng.uniform_vec(c)).astype(np.float32)
    b = rng.rand_vec(c)
    x = (rng.rand_vec(3 * c * 25) * np.float32(2.0) + np.float32(1.0)).reshape(3, c, 5, 5)
    bn = be.bn(c, g, b)
    y0 = bn.forward(x)
    r = rng.rand_vec(y0.size)
    dx = bn.backward(r.reshape(x.shape))
    dg, db = bn.grads()
    out.append(("batchnorm dx", dircheck(x.ravel(), dx, eps, rng,
                                         lambda cc: dot32(bn.forward(cc.reshape(x.shape)), r))))
    out.append(("batchnorm dgamma", dircheck(g, dg, eps, rng,
                                             lambda cc: dot32(bn.with_gamma(cc, x), r))))
    out.append(("batchnorm dbeta", dircheck(b, db, eps, rng,
                                            lambda cc: dot32(bn.with_beta(cc, x), r))))
    # linear (check.rs:600-624)
    lin = be.linear(6, 5, rng)
    lin.set_bias(rng.rand_vec(5))
    x = rng.rand_vec(3 * 6).reshape(3, 6)
    y0 = lin.forward(x)
    r = rng.rand_vec(y0.size)
    dx = lin.backward(r.reshape(y0.shape))
    dw = lin.dw()
    out.append(("linear dx", dircheck(x.ravel(), dx, eps, rng,
                                      lambda cc: dot32(lin.forward(cc.reshape(x.shape)), r))))
    w0 = lin.weight()
    out.append(("linear dw", dircheck(w0, dw, eps, rng, lambda cc: dot32(lin.with_weight(cc, x),
                                                                         r))))
    # BasicBlock (check.rs:625-657)
    for cin, cout, stride, tag in ((4, 4, 1, "block id/s1"), (4, 8, 2, "block down/s2")):
        blk = be.block(cin, cout, stride, rng)
        base = blk.params()
        base = (base + np.float32(0.3) * rng.rand_vec(base.size)).astype(np.float32)
        blk.set_params(base)
        x = rng.rand_vec(2 * cin * 64).reshape(2, cin, 8, 8)
        y0 = blk.forward(x)
        r = rng.rand_vec(y0.size)
        dx = blk.backward(r.reshape(y0.shape))
        out.append((f"{tag} dx", dircheck(x.ravel(), dx, eps, rng,
                                          lambda cc: dot32(blk.forward(cc.reshape(x.shape)), r))))
        grad = blk.grads()

        def lossp(cc):
            blk.set_params(cc)
            return dot32(blk.forward(x), r)
        out.append((f"{tag} dparams", dircheck(base, grad, eps, rng, lossp)))
        blk.set_params(base)
    # softmax_ce (check.rs:659-670)
    n, nc = 4, 7
    z = rng.rand_vec(n * nc).reshape(n, nc)
    labels = np.array([rng.below(nc) for _ in range(n)], np.uint32)
    _, d = be.softmax_ce(z, labels, 0.1)
    out.append(("softmax_ce dlogits", dircheck(z.ravel(), d, eps, rng,
                                               lambda cc: be.softmax_ce(cc.reshape(n, nc), labels,
                                                                        0.1)[0])))
    return out


def resnet_gradcheck(orc, be, seed=SEED):
    """check.rs:727-775 on backend `be` (a ResNet factory); returns the error."""
    NC, BS = 10, 8
    eps = gc_eps()
    net = be.resnet(1, 4, NC, seed)
    rng = orc.Rng(seed ^ 0x5EED)
    base = net.params()
    base = (base + np.float32(0.3) * rng.rand_vec(base.size)).astype(np.float32)
    net.set_params(base)
    x = rng.rand_vec(BS * 3 * 16 * 16).reshape(BS, 3, 16, 16)
    labels = np.array([rng.below(NC) for _ in range(BS)], np.uint32)
    logits = net.forward(x)
    _, dl = be.softmax_ce(logits, labels, 0.0)
    net.backward(dl.reshape(BS, NC))
    grad = net.grads()

    def lossf(cc):
        net.set_params(cc)
        return be.softmax_ce(net.forward(x), labels, 0.0)[0]
    return dircheck(base, grad, eps, rng, lossf)


class _OracleBn:
    def __init__(self, M, c, g, b):
        self.bn = M.BatchNorm2d(c)
        self.bn.g.v[:] = g
        self.bn.b.v[:] = b

    def forward(self, x):
        return self.bn.forward(np.ascontiguousarray(x, np.float32), True)

    def backward(self, dy):
        return self.bn.backward(np.ascontiguousarray(dy, np.float32)).ravel()

    def grads(self):
        return self.bn.g.g.copy(), self.bn.b.g.copy()

    def with_gamma(self, g, x):
        old = self.bn.g.v.copy()
        self.bn.g.v[:] = g
        y = self.forward(x)
        self.bn.g.v[:] = old
        return y

    def with_beta(self, b, x):
        old = self.bn.b.v.copy()
        self.bn.b.v[:] = b
        y = self.forward(x)
        self.bn.b.v[:] = old
        return y


class _OracleLinear:
    def __init__(self, M, fin, fout, rng):
        self.l = M.Linear(fin, fout, rng)

    def set_bias(self, b):
        self.l.b.v[:] = b

    def forward(self, x):
        return self.l.forward(x, True)

    def backward(self, dy):
        return self.l.backward(dy).ravel()

    def dw(self):
        return self.l.w.g.copy()

    def weight(self):
        return self.l.w.v.copy()

    def with_weight(self, w, x):
        old = self.l.w.v.copy()
        self.l.w.v[:] = w
        y = self.l.forward(x, False)
        self.l.w.v[:] = old
        return y


class _OracleBlock:
    def __init__(self, M, cin, cout, stride, rng):
        self.b = M.BasicBlock(cin, cout, stride, rng)

    def params(self):
        return np.concatenate([p.v for p in self.b.params()])

    def grads(self):
        return np.concatenate([p.g for p in self.b.params()])

    def set_params(self, flat):
        off = 0
        for p in self.b.params():
            p.v[:] = flat[off:off + p.v.size]
            off += p.v.size

    def forward(self, x):
        return self.b.forward(np.ascontiguousarray(x, np.float32), True)

    def backward(self, dy):
        return self.b.backward(dy).ravel()


class _OracleNet:
    def __init__(self, M, depth, width, nc, seed):
        self.n = M.ResNet(depth, width, nc, seed)

    def params(self):
        return np.concatenate([p.v for p in self.n.params()])

    def grads(self):
        return np.concatenate([p.g for p in self.n.params()])

    def set_params(self, flat):
        off = 0
        for p in self.n.params():
            p.v[:] = flat[off:off + p.v.size]
            off += p.v.size

    def forward(self, x):
        return self.n.forward(x, True)

    def backward(self, dl):
        self.n.backward(dl)


class OracleNN:
    """Layer factory on the CPU oracle (oracle/pymodel.py)."""

    def __init__(self, orc, pymodel):
        self.o, self.M = orc, pymodel

    def bn(self, c, g, b):
        return _OracleBn(self.M, c, g, b)

    def linear(self, fin, fout, rng):
        return _OracleLinear(self.M, fin, fout, rng)

    def block(self, cin, cout, stride, rng):
        return _OracleBlock(self.M, cin, cout, stride, rng)

    def softmax_ce(self, z, labels, smooth):
        loss, _, d = self.o.softmax_ce(z, labels, smooth)
        return loss, d.ravel()


class OracleResNet(OracleNN):
    def __init__(self, pymodel):
        from oracle import pyorc
        super().__init__(pyorc, pymodel)

    def resnet(self, depth, width, nc, seed):
        return _OracleNet(self.M, depth, width, nc, seed)


# ---------------------------------------------------------------- GPU side
def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def _host(t):
    import torch
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


class _GpuBn:
    def __init__(self, rnn, c, g, b):
        from rustnn_amd.nn import BatchNorm2d
        self.bn = BatchNorm2d(c)
        self.bn.g.v.copy_(_dev(g))
        self.bn.b.v.copy_(_dev(b))

    def forward(self, x):
        return _host(self.bn.forward(_dev(x), True))

    def backward(self, dy):
        return _host(self.bn.backward(_dev(dy))).ravel()

    def grads(self):
        return _host(self.bn.g.g).copy(), _host(self.bn.b.g).copy()

    def with_gamma(self, g, x):
        old = self.bn.g.v.clone()
        self.bn.g.v.copy_(_dev(g))
        y = self.forward(x)
        self.bn.g.v.copy_(old)
        return y

    def with_beta(self, b, x):
        old = self.bn.b.v.clone()
        self.bn.b.v.copy_(_dev(b))
        y = self.forward(x)
        self.bn.b.v.copy_(old)
        return y


class _GpuLinear:
    def __init__(self, M, fin, fout, rng):
        from rustnn_amd.nn import Linear
        ref = M.Linear(fin, fout, rng)  # the reference's Kaiming draws
        self.l = Linear(fin, fout, _dev(ref.w.v))

    def set_bias(self, b):
        self.l.b.v.copy_(_dev(b))

    def forward(self, x):
        return _host(self.l.forward(_dev(x), True))

    def backward(self, dy):
        return _host(self.l.backward(_dev(dy))).ravel()

    def dw(self):
        return _host(self.l.w.g).copy()

    def weight(self):
        return _host(self.l.w.v).copy()

    def with_weight(self, w, x):
        old = self.l.w.v.clone()
        self.l.w.v.copy_(_dev(w))
        y = _host(self.l.forward(_dev(x), False))
        self.l.w.v.copy_(old)
        return y


class _GpuBlock:
    def __init__(self, M, cin, cout, stride, rng):
        from rustnn_amd.model import BasicBlock
        ref = M.BasicBlock(cin, cout, stride, rng)  # the reference's draws
        wd = _dev(ref.down[0].w.v) if ref.down is not None else None
        self.b = BasicBlock(cin, cout, stride, _dev(ref.c1.w.v), _dev(ref.c2.w.v), wd)

    def params(self):
        return np.concatenate([_host(v).ravel() for v, _ in self.b.params()])

    def grads(self):
        return np.concatenate([_host(g).ravel() for _, g in self.b.params()])

    def set_params(self, flat):
        off = 0
        for v, _ in self.b.params():
            v.copy_(_dev(flat[off:off + v.numel()]))
            off += v.numel()

    def forward(self, x):
        return _host(self.b.forward(_dev(x), True))

    def backward(self, dy):
        return _host(self.b.backward(_dev(dy))).ravel()


class _GpuNet:
    def __init__(self, depth, width, nc, seed):
        from rustnn_amd.model import ResNet
        self.n = ResNet(depth, width, nc, seed)

    def params(self):
        return _host(self.n.params())

    def grads(self):
        return _host(self.n.grads())

    def set_params(self, flat):
        self.n.set_params(_dev(flat))

    def forward(self, x):
        return _host(self.n.forward(_dev(x), True))

    def backward(self, dl):
        self.n.backward(_dev(dl))


class GpuNN:
    """Layer / network factory on the HIP path (C ABI through rustnn_amd)."""

    def __init__(self, pymodel):
        self.M = pymodel

    def bn(self, c, g, b):
        return _GpuBn(None, c, g, b)

    def linear(self, fin, fout, rng):
        return _GpuLinear(self.M, fin, fout, rng)

    def block(self, cin, cout, stride, rng):
        return _GpuBlock(self.M, cin, cout, stride, rng)

    def softmax_ce(self, z, labels, smooth):
        import torch
        from rustnn_amd.nn import softmax_ce
        loss, _, d = softmax_ce(_dev(z), torch.from_numpy(labels.astype(np.int32)).cuda(), smooth)
        return float(_host(loss)[0]), _host(d).ravel()

    def resnet(self, depth, width, nc, seed):
        return _GpuNet(depth, width, nc, seed)


# ------------------------------------------------------------ vitcheck
# vitcheck (check.rs:163-180): one Rng::new(seed ^ 0x1234) through gemmcheck's
# draws, the token fixture (n 3, t 9, c 8), normcheck, attncheck and netcheck.
GEMM_SHAPES = [(23, 37, 19), (64, 48, 96), (7, 16, 259)]  # check.rs:147
VIT_NTC = (3, 9, 8)
NET_CFG = dict(width=4, cmid=6, dim=8, heads=2, depth3=2, dim4=12, heads4=2, depth4=1,
               mem_at=(1,), droppath=0.2, img=16)  # check.rs:401-413
NET_PARENT = [0, 0, 1, 1, 2, 2]


def skip_gemmcheck_draws(rng):
    """gemmcheck (check.rs:145-161) draws a then b for each shape and each of
    the four transpose combinations."""
    for m, n, k in GEMM_SHAPES:
        for _ in range(4):
            rng.rand_vec(m * k)
            rng.rand_vec(k * n)


def check_params(layer, eps, rng, loss):
    """check_params! (check.rs:75-99): one dircheck over every parameter of
    `layer` (an adapter), the values restored afterwards."""
    base, grad = layer.values(), layer.grads()

    def lossp(v):
        layer.set_values(v)
        return loss()
    e = dircheck(base, grad, eps, rng, lossp)
    layer.set_values(base)
    return e


def attncheck(be, rng, x, r, n, c, eps):
    """attncheck (check.rs:294-395) on backend `be`: SelfAttn (random rel),
    CrossAttn over a 6x6 memory (dx, dmem, dparams) and a reader Block with
    DropPath 0.2 and parameters perturbed by 0.2 N(0,1).  Returns
    {tag: relative error}."""
    out = {}
    # 6. self-attention with LSA and the relative bias
    at = be.self_attn(c, 2, 3, 3, 2, rng)
    at.set_rel(rng.rand_vec(at.rel_len()))
    at.fwd(x)
    dx = at.bwd(r)
    out["selfattn dx"] = dircheck(x, dx, eps, rng, lambda v: dot32(at.fwd(v), r))
    at.zero_grads()
    at.fwd(x)
    at.bwd(r)
    out["selfattn dparams"] = check_params(at, eps, rng, lambda: dot32(at.fwd(x), r))
    # 7. cross-attention on the memory
    mh = 6
    cr = be.cross_attn(c, 2, 3, 3, mh, mh, 2, rng)
    cr.set_rel(rng.rand_vec(cr.rel_len()))
    mem = rng.rand_vec(n * mh * mh * 2 * c)
    cr.fwd(x, mem)
    dx, dmem = cr.bwd(r, mem)
    out["crossattn dx"] = dircheck(x, dx, eps, rng, lambda v: dot32(cr.fwd(v, mem), r))
    out["crossattn dmem"] = dircheck(mem, dmem, eps, rng, lambda v: dot32(cr.fwd(x, v), r))
    cr.zero_grads()
    cr.fwd(x, mem)
    cr.bwd(r, mem)
    out["crossattn dparams"] = check_params(cr, eps, rng, lambda: dot32(cr.fwd(x, mem), r))
    # 8. the whole Block, with the memory and seeded stochastic depth
    blk = be.block(c, 2, 3, 3, (mh, mh), 2, 0.2, 7, 0.3, rng)
    v0 = blk.values()
    blk.set_values((v0 + np.float32(0.2) * rng.rand_vec(v0.size)).astype(np.float32))
    mem = rng.rand_vec(n * mh * mh * 2 * c)
    blk.fwd(x, mem, 99)
    dx, _ = blk.bwd(r, mem)
    out["block dx"] = dircheck(x, dx, eps, rng, lambda v: dot32(blk.fwd(v, mem, 99), r))
    blk.zero_grads()
    blk.fwd(x, mem, 99)
    blk.bwd(r, mem)
    out["block dparams"] = check_params(blk, eps, rng, lambda: dot32(blk.fwd(x, mem, 99), r))
    return out


def netcheck(be, rng, eps, seed=SEED):
    """netcheck (check.rs:396-460): the small RustViT of
    RustViT::new(cfg, parent, 3, seed ^ 0xBEEF) with parameters perturbed by
    0.15 N(0,1), batch 3, loss = <outputs, g> over the three heads, both
    hints and the pooled feature; one dircheck over every parameter."""
    net = be.rustvit(NET_CFG, NET_PARENT, 3, seed ^ 0xBEEF, 4242)
    v0 = net.values()
    net.set_values((v0 + np.float32(0.15) * rng.rand_vec(v0.size)).astype(np.float32))
    bs, nf = 3, len(NET_PARENT)
    x = rng.rand_vec(bs * 3 * 16 * 16)
    keys = ("logits", "coarse", "e1", "e2", "h1", "h2", "hfinal")
    sizes = (bs * nf, bs * 3, bs * nf, bs * nf, bs * 12, bs * 12, bs * 12)
    g = {k: rng.rand_vec(s) for k, s in zip(keys, sizes)}

    def lin(o):
        return (dot32(o["logits"], g["logits"]) + dot32(o["coarse"], g["coarse"]) +
                dot32(o["e1"], g["e1"]) + dot32(o["e2"], g["e2"]) + dot32(o["h1"], g["h1"]) +
                dot32(o["h2"], g["h2"]) + dot32(o["feat"], g["hfinal"]))

    net.fwd(x)
    net.bwd(g)
    return check_params(net, eps, rng, lambda: lin(net.fwd(x)))


def vitcheck(orc, norm_be, attn_be, seed=SEED):
    """vitcheck (check.rs:163-180) on the given backends: {tag: error}."""
    from test_oracle_norm import normcheck
    rng = orc.Rng(seed ^ 0x1234)
    eps = gc_eps()
    skip_gemmcheck_draws(rng)
    n, t, c = VIT_NTC
    x = rng.rand_vec(n * t * c)
    r = rng.rand_vec(n * t * c)
    out = dict(normcheck(orc, norm_be, rng, x, r))
    out.update(attncheck(attn_be, rng, x, r, n, c, eps))
    out["rustvit (all parameters)"] = netcheck(attn_be, rng, eps, seed)
    return out


class _Layer:
    """Adapter over a layer whose parameters are Param objects with v / g
    (oracle: numpy arrays; device: CUDA tensors)."""

    def __init__(self, obj, params, to_np, from_np):
        self.o, self.ps, self.h, self.d = obj, params, to_np, from_np

    def values(self):
        return np.concatenate([self.h(p.v).ravel() for p in self.ps]).astype(np.float32)

    def grads(self):
        return np.concatenate([self.h(p.g).ravel() for p in self.ps]).astype(np.float32)

    def set_values(self, v):
        off = 0
        for p in self.ps:
            k = p.v.size if isinstance(p.v, np.ndarray) else p.v.numel()
            part = np.ascontiguousarray(v[off:off + k], np.float32)
            if isinstance(p.v, np.ndarray):
                p.v[:] = part
            else:
                p.v.copy_(self.d(part))
            off += k

    def zero_grads(self):
        for p in self.ps:
            if isinstance(p.g, np.ndarray):
                p.g[:] = 0
            else:
                p.g.zero_()

    def rel_len(self):
        return self.o.rel.v.size if isinstance(self.o.rel.v, np.ndarray) else self.o.rel.v.numel()

    def set_rel(self, v):
        if isinstance(self.o.rel.v, np.ndarray):
            self.o.rel.v[:] = v
        else:
            self.o.rel.v.copy_(self.d(v))


class OracleAttn:
    """attncheck / netcheck backend on the CPU oracle (oracle/pyvit.py)."""

    def __init__(self):
        from oracle import pyvit
        self.V = pyvit

    def _wrap(self, obj, kind, n, t, c):
        L = _Layer(obj, obj.params(), lambda a: np.asarray(a), lambda a: a)
        sh = lambda v: np.asarray(v, np.float32).reshape(n, t, c)
        if kind == "self":
            L.fwd = lambda x: obj.forward(sh(x), True).ravel()
            L.bwd = lambda dy: obj.backward(sh(dy)).ravel()
        else:
            def bwd(dy, mem):
                dmem = np.zeros(np.size(mem), np.float32)
                if kind == "cross":
                    dx = obj.backward(sh(dy), self._mem(mem, n, c), dmem)
                else:
                    dx = obj.backward(sh(dy), self._mem(mem, n, c), dmem)
                return dx.ravel(), dmem
            if kind == "cross":
                L.fwd = lambda x, mem: obj.forward(sh(x), self._mem(mem, n, c), True).ravel()
            else:
                L.fwd = lambda x, mem, seed: obj.forward(sh(x), self._mem(mem, n, c), True,
                                                         seed).ravel()
            L.bwd = bwd
        return L

    @staticmethod
    def _mem(mem, n, c):
        return np.asarray(mem, np.float32).reshape(n, -1, 2 * c)

    def self_attn(self, c, h, th, tw, depth, rng):
        return self._wrap(self.V.SelfAttn(c, h, th, tw, depth, rng), "self", VIT_NTC[0],
                          th * tw, c)

    def cross_attn(self, c, h, th, tw, mh, mw, depth, rng):
        return self._wrap(self.V.CrossAttn(c, h, th, tw, mh, mw, depth, rng), "cross",
                          VIT_NTC[0], th * tw, c)

    def block(self, c, h, th, tw, mem, depth, drop, idx, ls, rng):
        return self._wrap(self.V.Block(c, h, th, tw, mem, depth, np.float32(drop), idx,
                                       np.float32(ls), rng), "block", VIT_NTC[0], th * tw, c)

    def rustvit(self, cfg, parent, nc, seed, drop_seed):
        net = self.V.RustViT(cfg, parent, nc, seed)
        net.drop_seed = drop_seed
        L = _Layer(net, net.params(), lambda a: np.asarray(a), lambda a: a)
        img = cfg["img"]
        L.fwd = lambda x: {k: np.ravel(v) for k, v in
                           net.forward(np.asarray(x, np.float32).reshape(-1, 3, img, img),
                                       True).items()}
        L.bwd = lambda g: net.backward(g)
        return L


class _SyncedRng:
    """Runs a device constructor on the state of an oracle Rng: the device's
    host generator (rustnn_amd.data.Rng) takes the oracle's state and hands
    it back advanced, so one stream feeds both, as one Rng feeds the
    reference's check."""

    def __init__(self, orng):
        self.o = orng

    def __enter__(self):
        from rustnn_amd.data import Rng
        self.d = Rng(0)
        for i in range(4):
            self.d.state[i] = self.o.st.s[i]
        return self.d

    def __exit__(self, *a):
        for i in range(4):
            self.o.st.s[i] = self.d.state[i]


class GpuAttn:
    """attncheck / netcheck backend on the device layers (rustnn_amd.vit)."""

    def _wrap(self, obj, kind, n, t, c):
        import torch
        ps = []
        obj.for_each_param(ps.append)
        L = _Layer(obj, ps, _host, _dev)
        sh = lambda v: _dev(v).reshape(n, t, c)
        mem_of = lambda mem: _dev(mem).reshape(n, -1, 2 * c)
        if kind == "self":
            L.fwd = lambda x: _host(obj.forward(sh(x), True)).ravel()
            L.bwd = lambda dy: _host(obj.backward(sh(dy))).ravel()
            return L

        def bwd(dy, mem):
            dmem = torch.zeros(np.size(mem), device="cuda")
            dx = obj.backward(sh(dy), mem_of(mem), dmem)
            return _host(dx).ravel(), _host(dmem).ravel()
        if kind == "cross":
            L.fwd = lambda x, mem: _host(obj.forward(sh(x), mem_of(mem), True)).ravel()
        else:
            L.fwd = lambda x, mem, seed: _host(obj.forward(sh(x), mem_of(mem), True,
                                                           seed)).ravel()
        L.bwd = bwd
        return L

    def self_attn(self, c, h, th, tw, depth, rng):
        from rustnn_amd.vit import SelfAttn
        with _SyncedRng(rng) as d:
            obj = SelfAttn(c, h, th, tw, depth, d)
        return self._wrap(obj, "self", VIT_NTC[0], th * tw, c)

    def cross_attn(self, c, h, th, tw, mh, mw, depth, rng):
        from rustnn_amd.vit import CrossAttn
        with _SyncedRng(rng) as d:
            obj = CrossAttn(c, h, th, tw, mh, mw, depth, d)
        return self._wrap(obj, "cross", VIT_NTC[0], th * tw, c)

    def block(self, c, h, th, tw, mem, depth, drop, idx, ls, rng):
        from rustnn_amd.vit import Block
        with _SyncedRng(rng) as d:
            obj = Block(c, h, th, tw, mem, depth, float(np.float32(drop)), idx,
                        float(np.float32(ls)), d)
        return self._wrap(obj, "block", VIT_NTC[0], th * tw, c)

    def rustvit(self, cfg, parent, nc, seed, drop_seed):
        from rustnn_amd.vit import RustViT
        par = _dev(np.asarray(parent, np.uint32).view(np.float32)).view(dtype=_i32dtype())
        net = RustViT(cfg, par, nc, seed=seed)
        net.drop_seed = drop_seed
        L = _Layer(net, net.params(), _host, _dev)
        img = cfg["img"]
        L.fwd = lambda x: {k: _host(v).ravel() for k, v in
                           net.forward(_dev(x).reshape(-1, 3, img, img), True).items()}
        L.bwd = lambda g: net.backward({k: _dev(v) for k, v in g.items()})
        return L


def _i32dtype():
    import torch
    return torch.int32
