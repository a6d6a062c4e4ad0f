"""norm.rs on the device: LayerNorm, LayerScale, SwiGlu, DwConv3, SeqPool.

Mirrors the reference's layer interface (norm.rs:17-586) over token tensors:
float32 CUDA tensors of shape [n, t, c] (tok.rs ``Tok``, channel fastest).
``forward(x, train)`` / ``backward(dy)`` as in the reference; parameter
gradients accumulate into ``Param.g`` (``rustnn_amd.optim.Param``, so the
layers feed ``Optim.step_all`` directly).  Every call goes through
librnn.so; there is no CPU fallback.
"""
from __future__ import annotations

from . import RNN_DW3_ACC_DX, Linear, _ptr, default_ctx, lib
from .optim import Param


def _rows_c(x):
    c = x.shape[-1]
    return x.numel() // c, c


class LayerNorm:
    """LayerNorm (norm.rs:17-143): g = 1, b = 0, eps 1e-5, f64 row statistics."""

    def __init__(self, c, device=0, ctx=None):
        import torch
        dev = f"cuda:{device}"
        self.c, self.eps = c, 1e-5
        self.ctx = ctx or default_ctx(device)
        self.g = Param(torch.ones(c, device=dev), False)
        self.b = Param(torch.zeros(c, device=dev), False)
        self.xhat = self.invstd = None

    def forward(self, x, train):
        import torch
        rows, c = _rows_c(x)
        if c != self.c:
            raise ValueError(f"LayerNorm: {c} channels, the layer has {self.c}")
        y = torch.empty_like(x)
        if train:
            self.xhat = torch.empty_like(x)
            self.invstd = torch.empty(rows, device=x.device)
        xh = self.xhat if train else None
        iv = self.invstd if train else None
        self.ctx.check(lib().rnn_ln_forward(
            self.ctx.h, rows, c, _ptr(x, rows * c, "x"), _ptr(self.g.v, c, "g"),
            _ptr(self.b.v, c, "b"), self.eps, _ptr(y, rows * c, "y"),
            _ptr(xh, rows * c, "xhat"), _ptr(iv, rows, "invstd")))
        return y

    def backward(self, dy, add=None, out=None, ls=None):
        """Returns dx; with ``add``, dx + add in the same pass (the add_ that
        follows the norm in Block::backward), written to ``out`` (which may
        be ``add``) or a new tensor.  With ``ls`` = (LayerScale, DropPath
        mask or None) as well, that layer's backward over the returned dx
        runs in the same pass: returns (dx, the LayerScale's input gradient),
        as ``ls[0].backward(dx, ls[1])`` would."""
        import torch
        rows, c = _rows_c(dy)
        dx = out if out is not None else torch.empty_like(dy)
        if ls is not None:
            if add is None:
                raise ValueError("LayerNorm.backward: ls needs add")
            layer, mask = ls
            lsdx = torch.empty_like(dy)
            self.ctx.check(lib().rnn_ln_backward_add_ls(
                self.ctx.h, rows, c, _ptr(dy, rows * c, "dy"), _ptr(self.xhat, rows * c, "xhat"),
                _ptr(self.invstd, rows, "invstd"), _ptr(self.g.v, c, "g"),
                _ptr(add, rows * c, "add"), _ptr(dx, rows * c, "dx"), _ptr(self.g.g, c, "dg"),
                _ptr(self.b.g, c, "db"), _ptr(layer.x, rows * c, "lsx"), _ptr(layer.l.v, c, "l"),
                _ptr(mask, 1, "mask"), rows // mask.numel() if mask is not None else 1,
                _ptr(lsdx, rows * c, "lsdx"), _ptr(layer.l.g, c, "dl")))
            return dx, lsdx
        if add is None:
            self.ctx.check(lib().rnn_ln_backward(
                self.ctx.h, rows, c, _ptr(dy, rows * c, "dy"), _ptr(self.xhat, rows * c, "xhat"),
                _ptr(self.invstd, rows, "invstd"), _ptr(self.g.v, c, "g"),
                _ptr(dx, rows * c, "dx"), _ptr(self.g.g, c, "dg"), _ptr(self.b.g, c, "db")))
        else:
            self.ctx.check(lib().rnn_ln_backward_add(
                self.ctx.h, rows, c, _ptr(dy, rows * c, "dy"), _ptr(self.xhat, rows * c, "xhat"),
                _ptr(self.invstd, rows, "invstd"), _ptr(self.g.v, c, "g"),
                _ptr(add, rows * c, "add"), _ptr(dx, rows * c, "dx"), _ptr(self.g.g, c, "dg"),
                _ptr(self.b.g, c, "db")))
        return dx

    def for_each_param(self, f):
        f(self.g)
        f(self.b)


class LayerScale:
    """LayerScale (norm.rs:147-217): y = lambda x, lambda = init per channel."""

    def __init__(self, c, init, device=0, ctx=None):
        import torch
        self.c = c
        self.ctx = ctx or default_ctx(device)
        self.l = Param(torch.full((c,), float(init), device=f"cuda:{device}"), False)
        self.x = None

    def forward(self, x, train):
        """y = x lambda.  Training keeps x for the backward (the caller must
        not change it) and returns a new tensor; eval scales x in place, as
        the reference consumes its input."""
        import torch
        rows, c = _rows_c(x)
        if c != self.c:
            raise ValueError(f"LayerScale: {c} channels, the layer has {self.c}")
        y = torch.empty_like(x) if train else x
        if train:
            self.x = x
        self.ctx.check(lib().rnn_layerscale_forward(self.ctx.h, rows, c, _ptr(x, rows * c, "x"),
                                                    _ptr(self.l.v, c, "l"),
                                                    _ptr(y, rows * c, "y")))
        return y

    def backward(self, dy, mask=None):
        """norm.rs:182-212, after DropPath::backward's per-image mask when
        one is given (vit.rs:61-73): returns a new dx; dy is not changed."""
        import torch
        rows, c = _rows_c(dy)
        dx = torch.empty_like(dy)
        rpi = rows // mask.numel() if mask is not None else 1
        self.ctx.check(lib().rnn_drop_layerscale_backward(
            self.ctx.h, rows, c, _ptr(dy, rows * c, "dy"), _ptr(self.x, rows * c, "x"),
            _ptr(self.l.v, c, "l"), _ptr(mask, mask.numel(), "mask") if mask is not None else None,
            rpi, _ptr(dx, rows * c, "dx"), _ptr(self.l.g, c, "dl")))
        return dx

    def for_each_param(self, f):
        f(self.l)


def _linear_param(lin):
    """A Linear's weight and bias as optim Params sharing its buffers; the
    weight is a [fout x fin] matrix (linear.rs:25-33)."""
    w = Param.__new__(Param)
    w.v, w.g = lin.w, lin.gw
    import torch
    w.m, w.v2 = torch.zeros_like(lin.w), torch.zeros_like(lin.w)
    w.decay, w.rows, w.cols = True, lin.fout, lin.fin
    out = [w]
    if lin.b is not None:
        b = Param.__new__(Param)
        b.v, b.g = lin.b, lin.gb
        b.m, b.v2 = torch.zeros_like(lin.b), torch.zeros_like(lin.b)
        b.decay, b.rows, b.cols = False, 0, 0
        out.append(b)
    return out


class SwiGlu:
    """SwiGlu (norm.rs:221-294): wg Linear(c, 2h) -> u = silu(a) b -> wd
    Linear(h, c).  wg / wd take the given weights (or 0.02 normals)."""

    def __init__(self, c, h, wg=None, bg=None, wd=None, bd=None, device=0, ctx=None):
        self.c, self.h = c, h
        self.ctx = ctx or default_ctx(device)
        self.wg = Linear(c, 2 * h, True, wg, bg, device, self.ctx)
        self.wd = Linear(h, c, True, wd, bd, device, self.ctx)
        self._params = _linear_param(self.wg) + _linear_param(self.wd)
        self.ab = None
        self.rows = 0

    def forward(self, x, train, residual=None):
        """residual = (out, l, mask, rows per image): the down projection also
        adds out += (y l) mask[image] (Linear.forward)."""
        import torch
        rows, c = _rows_c(x)
        h = self.h
        ab = self.wg.forward(x.reshape(-1), rows, train)
        u = torch.empty(rows * h, device=x.device)
        self.ctx.check(lib().rnn_swiglu_forward(self.ctx.h, rows, h, _ptr(ab, rows * 2 * h, "ab"),
                                                _ptr(u, rows * h, "u")))
        if train:
            self.ab, self.rows = ab, rows
        return self.wd.forward(u, rows, train, residual).view(x.shape)

    def backward(self, dy):
        import torch
        rows, h = self.rows, self.h
        du = self.wd.backward(dy.reshape(-1))
        dab = torch.empty(rows * 2 * h, device=dy.device)
        self.ctx.check(lib().rnn_swiglu_backward(self.ctx.h, rows, h, _ptr(du, rows * h, "du"),
                                                 _ptr(self.ab, rows * 2 * h, "ab"),
                                                 _ptr(dab, rows * 2 * h, "dab")))
        return self.wg.backward(dab).view(dy.shape)

    def for_each_param(self, f):
        for p in self._params:
            f(p)


class DwConv3:
    """DwConv3 (norm.rs:296-457): depthwise 3x3, pad 1, on th x tw tokens;
    w [9, c] tap-major, b [c]."""

    def __init__(self, c, th, tw, w=None, b=None, device=0, ctx=None):
        import torch
        dev = f"cuda:{device}"
        self.c, self.th, self.tw = c, th, tw
        self.ctx = ctx or default_ctx(device)
        self.w = Param(w if w is not None else torch.randn(9 * c, device=dev) * 0.1, False)
        self.b = Param(b if b is not None else torch.zeros(c, device=dev), False)
        self.x, self.n = None, 0

    def _images(self, x):
        img = self.th * self.tw * self.c
        if x.numel() % img:
            raise ValueError(f"DwConv3: {x.numel()} elements is not a whole number of "
                             f"{self.th}x{self.tw}x{self.c} images")
        return x.numel() // img

    def forward(self, x, train):
        import torch
        n, c = self._images(x), self.c
        need = n * self.th * self.tw * c
        y = torch.empty_like(x)
        self.ctx.check(lib().rnn_dwconv3_forward(
            self.ctx.h, n, self.th, self.tw, c, _ptr(x, need, "x"), _ptr(self.w.v, 9 * c, "w"),
            _ptr(self.b.v, c, "b"), _ptr(y, need, "y")))
        if train:
            self.x, self.n = x, n
        return y

    def forward_branch(self, h, a, gamma, x, l, mask, y, train):
        """Block::forward's first branch (vit.rs:150-160) in one pass: d =
        forward(h) (returned), a += gamma d in place, y = x + (a l) m with m
        the DropPath mask per image (None: 1) -- rnn_dwconv3_branch_forward."""
        import torch
        n, c = self._images(h), self.c
        need = n * self.th * self.tw * c
        d = torch.empty_like(h)
        self.ctx.check(lib().rnn_dwconv3_branch_forward(
            self.ctx.h, n, self.th, self.tw, c, _ptr(h, need, "h"), _ptr(self.w.v, 9 * c, "w"),
            _ptr(self.b.v, c, "b"), _ptr(d, need, "d"), _ptr(a, need, "a"),
            _ptr(gamma, c, "gamma"), _ptr(x, need, "x"), _ptr(l, c, "l"),
            _ptr(mask, n, "mask") if mask is not None else None, _ptr(y, need, "y")))
        if train:
            self.x, self.n = h, n
        return d

    def backward(self, dy, acc_dx=None):
        """dx, or acc_dx += dx (returned) when given."""
        import torch
        c = self.c
        if self._images(dy) != self.n:
            raise ValueError("DwConv3.backward: dy does not match the forward's input")
        need = self.n * self.th * self.tw * c
        dx = torch.empty_like(dy) if acc_dx is None else acc_dx
        self.ctx.check(lib().rnn_dwconv3_backward_ex(
            self.ctx.h, self.n, self.th, self.tw, c, _ptr(dy, need, "dy"),
            _ptr(self.x, need, "x"), _ptr(self.w.v, 9 * c, "w"), _ptr(dx, need, "dx"),
            _ptr(self.w.g, 9 * c, "dw"), _ptr(self.b.g, c, "db"),
            0 if acc_dx is None else RNN_DW3_ACC_DX))
        return dx

    def for_each_param(self, f):
        f(self.w)
        f(self.b)


class SeqPool:
    """SeqPool (norm.rs:459-586): z = sum_t softmax_t(x p) x_t, [n, c]."""

    def __init__(self, c, p=None, device=0, ctx=None):
        import torch
        self.c = c
        self.ctx = ctx or default_ctx(device)
        self.p = Param(p if p is not None else torch.randn(c, device=f"cuda:{device}") * 0.02,
                       True)
        self.w = self.x = None
        self.n = self.t = 0

    def forward(self, x, train):
        import torch
        n, t, c = x.shape
        if c != self.c:
            raise ValueError(f"SeqPool: {c} channels, the pool has {self.c}")
        z = torch.empty(n, c, device=x.device)
        w = torch.empty(n, t, device=x.device)
        self.ctx.check(lib().rnn_seqpool_forward(self.ctx.h, n, t, c, _ptr(x, n * t * c, "x"),
                                                 _ptr(self.p.v, c, "p"), _ptr(z, n * c, "z"),
                                                 _ptr(w, n * t, "w")))
        if train:
            self.w, self.x, self.n, self.t = w, x, n, t
        return z

    def backward(self, dz):
        import torch
        n, t, c = self.n, self.t, self.c
        dx = torch.empty(n, t, c, device=dz.device)
        self.ctx.check(lib().rnn_seqpool_backward(
            self.ctx.h, n, t, c, _ptr(dz, n * c, "dz"), _ptr(self.w, n * t, "w"),
            _ptr(self.x, n * t * c, "x"), _ptr(self.p.v, c, "p"), _ptr(dx, n * t * c, "dx"),
            _ptr(self.p.g, c, "dp")))
        return dx

    def for_each_param(self, f):
        f(self.p)
