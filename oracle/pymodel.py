"""CPU oracle of the reference ResNet (model.rs, nn.rs) built on liborc.so.

TEST INFRASTRUCTURE ONLY (see pyorc.py): a restatement of the reference's
CIFAR ResNet train step used to check the device-resident ResNet of
rustnn_amd and to time the reference-style CPU step as a baseline.  Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg may
import it.

Structure and order follow the reference:
  * Param (nn.rs:37-111): value, gradient, momentum, decay flag; Kaiming init
    w = normal() * sqrt(2 / fan_in) (nn.rs:95-100); Nesterov step (102-110).
  * Conv2d (nn.rs:113-250), BatchNorm2d (nn.rs:253-428, gamma 1, beta 0,
    running mean 0 / var 1, momentum 0.1, eps 1e-5), the scalar classifier
    Linear (nn.rs:475-564, Kaiming * 0.5, zero bias).
  * BasicBlock (model.rs:10-101): conv-BN-ReLU, conv-BN with zero-init gamma,
    1x1/s2 conv-BN shortcut when the shape changes, add + ReLU.
  * ResNet (model.rs:103-209): blocks are created (and draw from the Rng)
    before the stem and the classifier; parameters are visited stem, stem BN,
    blocks (c1, b1, c2, b2, down conv, down BN), fc w, fc b.
"""
from __future__ import annotations

import numpy as np

from . import pyorc as O


class Param:
    def __init__(self, v, decay):
        self.v = np.ascontiguousarray(v, np.float32)
        self.g = np.zeros_like(self.v)
        self.m = np.zeros_like(self.v)
        self.decay = decay

    @classmethod
    def kaiming(cls, fan_in, n, rng):
        s = np.float32(np.sqrt(np.float32(2.0) / np.float32(fan_in)))
        return cls((rng.rand_vec(n) * s).astype(np.float32), True)

    def step(self, lr, mom, wd):
        O.sgd_step(self.v, self.g, self.m, lr, mom, wd if self.decay else 0.0)


class Conv2d:
    def __init__(self, cin, cout, k, stride, pad, rng):
        self.cin, self.cout, self.k, self.stride, self.pad = cin, cout, k, stride, pad
        self.w = Param.kaiming(cin * k * k, cout * cin * k * k, rng)
        self.x = None

    def spec(self, h, w):
        return O.ConvSpec.make(self.cin, self.cout, self.k, self.stride, self.pad, h, w)

    def forward(self, x, train):
        n, _, h, w = x.shape
        sp = self.spec(h, w)
        if train:
            self.x = x
        return np.ascontiguousarray(O.conv2d_forward(sp, n, x, self.w.v))

    def backward_w(self, dy):
        n, _, h, w = self.x.shape
        sp = self.spec(h, w)
        self.w.g[:] = O.conv2d_backward_w(sp, n, dy, self.x, self.w.g).ravel()

    def backward(self, dy):
        self.backward_w(dy)
        n, _, h, w = self.x.shape
        return np.ascontiguousarray(O.conv2d_backward_x(self.spec(h, w), n, dy, self.w.v))


class BatchNorm2d:
    def __init__(self, c):
        self.g = Param(np.ones(c, np.float32), False)
        self.b = Param(np.zeros(c, np.float32), False)
        self.rm = np.zeros(c, np.float32)
        self.rv = np.ones(c, np.float32)
        self.mom, self.eps = 0.1, 1e-5
        self.xhat = self.invstd = None

    def _run(self, y, train, relu):
        y = np.ascontiguousarray(y, np.float32).copy()
        if train:
            self.xhat, _, self.invstd = O.bn_train_forward(y, self.g.v, self.b.v, self.rm,
                                                           self.rv, self.mom, self.eps, relu)
        else:
            O.bn_eval_forward(y, self.g.v, self.b.v, self.rm, self.rv, self.eps, relu)
        return y

    def forward(self, y, train):
        return self._run(y, train, False)

    def forward_relu(self, y, train):
        return self._run(y, train, True)

    def backward(self, dy):
        return O.bn_backward(np.ascontiguousarray(dy, np.float32), self.xhat, self.g.v,
                             self.invstd, self.g.g, self.b.g)


class Linear:
    """nn.rs Linear (the ResNet classifier)."""

    def __init__(self, fin, fout, rng):
        self.fin, self.fout = fin, fout
        self.w = Param.kaiming(fin, fin * fout, rng)
        self.w.v *= np.float32(0.5)
        self.b = Param(np.zeros(fout, np.float32), False)
        self.x = None

    def forward(self, x, train):
        x = np.ascontiguousarray(x, np.float32).reshape(x.shape[0], -1)
        if train:
            self.x = x.copy()
        return O.fc_forward(x, self.w.v, self.b.v, self.fout)

    def backward(self, dy):
        return O.fc_backward(dy, self.x, self.w.v, self.w.g, self.b.g)


class BasicBlock:
    def __init__(self, cin, cout, stride, rng):
        self.b2 = BatchNorm2d(cout)
        self.b2.g.v[:] = 0.0  # zero_gamma (model.rs:22-23)
        self.c1 = Conv2d(cin, cout, 3, stride, 1, rng)
        self.b1 = BatchNorm2d(cout)
        self.c2 = Conv2d(cout, cout, 3, 1, 1, rng)
        self.down = None
        if stride != 1 or cin != cout:
            self.down = (Conv2d(cin, cout, 1, stride, 0, rng), BatchNorm2d(cout))

    def forward(self, x, train):
        h = self.b1.forward_relu(self.c1.forward(x, train), train)
        y = self.b2.forward(self.c2.forward(h, train), train)
        if self.down is not None:
            c, b = self.down
            s = b.forward(c.forward(x, train), train)
            O.add_relu(y, s)
        else:
            O.add_relu(y, x)
        if train:
            self.h1, self.out = h, y
        return y

    def backward(self, d):
        d = np.ascontiguousarray(d, np.float32).copy()
        O.relu_back(d, self.out)
        dmain = self.c2.backward(self.b2.backward(d))
        O.relu_back(dmain, self.h1)
        dx = self.c1.backward(self.b1.backward(dmain))
        if self.down is not None:
            c, b = self.down
            ds = c.backward(b.backward(d))
            O.add_(dx, ds)
        else:
            O.add_(dx, d)
        return dx

    def params(self):
        ps = [self.c1.w, self.b1.g, self.b1.b, self.c2.w, self.b2.g, self.b2.b]
        if self.down is not None:
            c, b = self.down
            ps += [c.w, b.g, b.b]
        return ps

    def buffers(self):
        bs = [self.b1.rm, self.b1.rv, self.b2.rm, self.b2.rv]
        if self.down is not None:
            bs += [self.down[1].rm, self.down[1].rv]
        return bs


class ResNet:
    """ResNet::new(depth_n, width, nclass, seed) (model.rs:113-135)."""

    def __init__(self, depth_n, width, nclass, seed):
        rng = O.Rng(seed)
        widths = [width, width * 2, width * 4]
        self.blocks = []
        cin = width
        for s, w in enumerate(widths):
            for b in range(depth_n):
                stride = 2 if s > 0 and b == 0 else 1
                self.blocks.append(BasicBlock(cin, w, stride, rng))
                cin = w
        self.stem = Conv2d(3, width, 3, 1, 1, rng)
        self.stem_bn = BatchNorm2d(width)
        self.fc = Linear(width * 4, nclass, rng)
        self.nclass = nclass

    def forward(self, x, train):
        h = self.stem_bn.forward_relu(self.stem.forward(np.ascontiguousarray(x, np.float32),
                                                        train), train)
        if train:
            self.stem_out = h
        for b in self.blocks:
            h = b.forward(h, train)
        self.feat_hw = (h.shape[2], h.shape[3])
        return self.fc.forward(O.gap_forward(h), train)

    def backward(self, dlogits):
        dpool = self.fc.backward(dlogits)
        d = O.gap_backward(dpool.reshape(dpool.shape[0], -1), *self.feat_hw)
        for b in reversed(self.blocks):
            d = b.backward(d)
        O.relu_back(d, self.stem_out)
        d = self.stem_bn.backward(d)
        self.stem.backward_w(d)

    def params(self):
        ps = [self.stem.w, self.stem_bn.g, self.stem_bn.b]
        for b in self.blocks:
            ps += b.params()
        return ps + [self.fc.w, self.fc.b]

    def buffers(self):
        bs = [self.stem_bn.rm, self.stem_bn.rv]
        for b in self.blocks:
            bs += b.buffers()
        return bs

    def step(self, lr, mom, wd):
        for p in self.params():
            p.step(lr, mom, wd)

    def flops(self, h, w):
        """ResNet::flops (model.rs:179-198): forward FLOP per image."""
        f = 2 * 3 * 9 * self.stem.cout * h * w
        hw = (h, w)
        c = self.stem.cout
        for b in self.blocks:
            s = b.c1.stride
            oh, ow = hw[0] // s, hw[1] // s
            f += 2 * b.c1.cin * 9 * b.c1.cout * oh * ow
            f += 2 * b.c2.cin * 9 * b.c2.cout * oh * ow
            if b.down is not None:
                f += 2 * b.down[0].cin * b.down[0].cout * oh * ow
            hw = (oh, ow)
            c = b.c2.cout
        return f + 2 * c * self.fc.fout

    def train_step(self, x, labels, smooth, lr, mom, wd):
        """One bench/train step (train.rs:686-699): forward, softmax-CE,
        backward, SGD.  Returns (loss, correct, logits)."""
        logits = self.forward(x, True)
        loss, correct, dl = O.softmax_ce(logits, labels, smooth)
        self.backward(dl)
        self.step(lr, mom, wd)
        return loss, correct, logits
