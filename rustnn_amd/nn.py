"""nn.rs on the device: the ResNet layers around the convolutions.

Mirrors the reference's nn.rs interface (nn.rs:37-637) over float32 CUDA
tensors, calling librnn.so through its C ABI:

* ``Param`` (value, gradient, momentum, decay flag) and ``Param.step`` --
  Param::step, Nesterov SGD (nn.rs:102-110)
* ``BatchNorm2d`` (forward / forward_relu in train or eval mode, backward) --
  nn.rs:253-428
* ``relu_back_``, ``add_``, ``add_relu_`` -- nn.rs:430-450
* ``gap_forward`` / ``gap_backward`` -- nn.rs:452-473
* ``Linear`` (the scalar classifier) -- nn.rs:475-564
* ``softmax_ce`` -- nn.rs:566-637

The one interface difference: the reference's BatchNorm2d normalises in place
and keeps xhat for the backward; here the forward writes a new tensor and the
layer keeps its input, from which the backward recomputes xhat bit for bit.
"""
from __future__ import annotations

import math

from . import _new, _ptr, default_ctx, lib


def _dims(x):
    n, c = x.shape[0], x.shape[1]
    return n, c, x.numel() // max(n * c, 1)


class Param:
    """Param (nn.rs:37-111) on the device."""

    def __init__(self, v, decay):
        import torch
        self.v = v.contiguous()
        self.g = torch.zeros_like(self.v)
        self.m = torch.zeros_like(self.v)
        self.decay = decay

    def step(self, lr, mom, wd, ctx=None):
        """Param::step (nn.rs:102-110)."""
        ctx = ctx or default_ctx()
        ctx.check(lib().rnn_sgd_step(ctx.h, self.v.numel(), _ptr(self.v, 0, "v"),
                                     _ptr(self.g, self.v.numel(), "g"),
                                     _ptr(self.m, self.v.numel(), "m"), lr, mom,
                                     wd if self.decay else 0.0))


class BatchNorm2d:
    """BatchNorm2d (nn.rs:253-428): gamma 1, beta 0, running mean 0 / var 1,
    momentum 0.1, eps 1e-5; f64 batch statistics."""

    def __init__(self, c, device=0, ctx=None):
        import torch
        dev = f"cuda:{device}"
        self.c = c
        self.ctx = ctx or default_ctx(device)
        self.g = Param(torch.ones(c, device=dev), False)
        self.b = Param(torch.zeros(c, device=dev), False)
        self.rm = torch.zeros(c, device=dev)
        self.rv = torch.ones(c, device=dev)
        self.mom, self.eps = 0.1, 1e-5
        self.mean = torch.zeros(c, device=dev)
        self.invstd = torch.zeros(c, device=dev)
        self.x = None

    def zero_gamma(self):
        self.g.v.zero_()

    def _run(self, x, train, relu):
        n, c, hw = _dims(x)
        y = _new(x.numel(), x).view(x.shape)
        L, ctx = lib(), self.ctx
        if train:
            ctx.check(L.rnn_bn_forward_train(
                ctx.h, n, c, hw, _ptr(x, n * c * hw, "x"), _ptr(y, n * c * hw, "y"),
                _ptr(self.g.v, c, "gamma"), _ptr(self.b.v, c, "beta"), _ptr(self.rm, c, "rm"),
                _ptr(self.rv, c, "rv"), _ptr(self.mean, c, "mean"),
                _ptr(self.invstd, c, "invstd"), self.mom, self.eps, int(relu)))
            self.x = x
        else:
            ctx.check(L.rnn_bn_forward_eval(
                ctx.h, n, c, hw, _ptr(x, n * c * hw, "x"), _ptr(y, n * c * hw, "y"),
                _ptr(self.g.v, c, "gamma"), _ptr(self.b.v, c, "beta"), _ptr(self.rm, c, "rm"),
                _ptr(self.rv, c, "rv"), self.eps, int(relu)))
        return y

    def forward(self, x, train):
        return self._run(x, train, False)

    def forward_relu(self, x, train):
        return self._run(x, train, True)

    def backward(self, dy, relu_out=None):
        """BatchNorm2d::backward (nn.rs:379-425); relu_out folds relu_back_ of dy in."""
        n, c, hw = _dims(dy)
        dx = _new(dy.numel(), dy).view(dy.shape)
        self.ctx.check(lib().rnn_bn_backward(
            self.ctx.h, n, c, hw, _ptr(dy, n * c * hw, "dy"),
            _ptr(relu_out, n * c * hw, "relu_out"), _ptr(self.x, n * c * hw, "x"),
            _ptr(self.mean, c, "mean"), _ptr(self.invstd, c, "invstd"),
            _ptr(self.g.v, c, "gamma"), _ptr(dx, n * c * hw, "dx"), _ptr(self.g.g, c, "dgamma"),
            _ptr(self.b.g, c, "dbeta")))
        return dx


def relu_back_(d, y, ctx=None):
    ctx = ctx or default_ctx()
    ctx.check(lib().rnn_relu_back(ctx.h, d.numel(), _ptr(d, 0, "d"), _ptr(y, d.numel(), "y")))


def add_(a, b, ctx=None):
    ctx = ctx or default_ctx()
    ctx.check(lib().rnn_add(ctx.h, a.numel(), _ptr(a, 0, "a"), _ptr(b, a.numel(), "b")))


def add_relu_back_(a, b, y, ctx=None):
    """add_(a, relu_back_(b, y)) with b left unchanged (nn.rs:432-443)."""
    ctx = ctx or default_ctx()
    ctx.check(lib().rnn_add_relu_back(ctx.h, a.numel(), _ptr(a, 0, "a"), _ptr(b, a.numel(), "b"),
                                      _ptr(y, a.numel(), "y")))


def add_relu_(a, b, ctx=None):
    ctx = ctx or default_ctx()
    ctx.check(lib().rnn_add_relu(ctx.h, a.numel(), _ptr(a, 0, "a"), _ptr(b, a.numel(), "b")))


def gap_forward(x, ctx=None):
    """gap_forward (nn.rs:455-463): [n, c, h, w] -> [n, c]."""
    ctx = ctx or default_ctx()
    n, c, hw = _dims(x)
    y = _new(n * c, x).view(n, c)
    ctx.check(lib().rnn_gap_forward(ctx.h, n, c, hw, _ptr(x, n * c * hw, "x"), _ptr(y, n * c, "y")))
    return y


def gap_backward(dy, h, w, ctx=None):
    """gap_backward (nn.rs:465-473): [n, c] -> [n, c, h, w]."""
    ctx = ctx or default_ctx()
    n, c = dy.shape[0], dy.numel() // dy.shape[0]
    dx = _new(n * c * h * w, dy).view(n, c, h, w)
    ctx.check(lib().rnn_gap_backward(ctx.h, n, c, h * w, _ptr(dy, n * c, "dy"),
                                     _ptr(dx, n * c * h * w, "dx")))
    return dx


class Linear:
    """nn.rs Linear (nn.rs:475-564), the ResNet classifier: w [fout, fin],
    bias; bit-identical to the reference's scalar loops."""

    def __init__(self, fin, fout, w, b=None, device=0, ctx=None):
        import torch
        self.fin, self.fout = fin, fout
        self.ctx = ctx or default_ctx(device)
        self.w = Param(w, True)
        self.b = Param(b if b is not None else torch.zeros(fout, device=w.device), False)
        self.x, self.n = None, 0

    def forward(self, x, train=True):
        n = x.shape[0]
        y = _new(n * self.fout, x).view(n, self.fout)
        self.ctx.check(lib().rnn_fc_forward(self.ctx.h, n, self.fin, self.fout,
                                            _ptr(x, n * self.fin, "x"),
                                            _ptr(self.w.v, self.fin * self.fout, "w"),
                                            _ptr(self.b.v, self.fout, "b"),
                                            _ptr(y, n * self.fout, "y")))
        if train:
            self.x, self.n = x, n
        return y

    def backward(self, dy):
        """backward_w + backward_x (nn.rs:519-564): returns dx [n, fin]."""
        n = self.n
        dx = _new(n * self.fin, dy).view(n, self.fin)
        self.ctx.check(lib().rnn_fc_backward(self.ctx.h, n, self.fin, self.fout,
                                             _ptr(dy, n * self.fout, "dy"),
                                             _ptr(self.x, n * self.fin, "x"),
                                             _ptr(self.w.v, self.fin * self.fout, "w"),
                                             _ptr(self.w.g, self.fin * self.fout, "dw"),
                                             _ptr(self.b.g, self.fout, "db"),
                                             _ptr(dx, n * self.fin, "dx")))
        return dx


def softmax_ce(logits, labels, smooth, ctx=None):
    """softmax_ce (nn.rs:620-637) -> (loss tensor [1], correct tensor [1] int32,
    dlogits [rows, nclass]).  labels: int32 CUDA tensor."""
    import torch
    ctx = ctx or default_ctx()
    rows = logits.shape[0]
    nclass = logits.numel() // rows
    d = _new(rows * nclass, logits).view(rows, nclass)
    loss = torch.zeros(1, device=logits.device)
    corr = torch.zeros(1, dtype=torch.int32, device=logits.device)
    ctx.check(lib().rnn_softmax_ce(ctx.h, rows, nclass, _ptr(logits, rows * nclass, "logits"),
                                   _ptr(labels, rows, "labels"), float(smooth),
                                   _ptr(d, rows * nclass, "dlogits"), _ptr(loss, 1, "loss"),
                                   _ptr(corr, 1, "correct")))
    return loss, corr, d


def kaiming_std(fan_in):
    """Param::kaiming scale (nn.rs:95-100)."""
    return math.sqrt(2.0 / fan_in)
