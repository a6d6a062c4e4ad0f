"""model.rs on the device: the CIFAR ResNet train step.

``ResNet`` mirrors the reference's ResNet (model.rs:103-209) over the native
runtime of librnn.so (``rnn_resnet_*``): parameters, gradients, momenta, BN
running statistics and activations stay on the device for the whole step;
``train_step`` runs forward, softmax cross-entropy, backward and the Nesterov
SGD step (train.rs:686-699) and is replayed from a hipGraph after its first
call for a shape.
"""
from __future__ import annotations

import ctypes as C

from . import RnnError, _ptr, _sz, _i, _vp, default_ctx, lib


class _DevArray:
    """Device memory owned by the library, exposed to torch.as_tensor through
    the CUDA array interface (no copy)."""

    def __init__(self, ptr, shape, typestr):
        self.__cuda_array_interface__ = {"shape": shape, "typestr": typestr, "data": (ptr, False),
                                         "strides": None, "version": 2}


class ResNet:
    """ResNet::new(depth_n, width, nclass, seed) (model.rs:113-135)."""

    def __init__(self, depth_n, width, nclass, seed, device=0, ctx=None):
        self.ctx = ctx or default_ctx(device)
        self.depth_n, self.width, self.nclass = depth_n, width, nclass
        self.device = device
        h = _vp()
        self.ctx.check(lib().rnn_resnet_create(self.ctx.h, depth_n, width, nclass,
                                               C.c_uint64(seed & 0xFFFFFFFFFFFFFFFF), C.byref(h)))
        self.h = h
        self.name = f"resnet{6 * depth_n + 2}-w{width}"

    # ---- state
    def num_params(self):
        return int(lib().rnn_resnet_num_params(self.h))

    def num_buffers(self):
        return int(lib().rnn_resnet_num_buffers(self.h))

    def tensor_lens(self):
        """(len, decay) of each parameter in for_each_param order."""
        out = []
        for i in range(int(lib().rnn_resnet_num_tensors(self.h))):
            n, d = _sz(), _i()
            self.ctx.check(lib().rnn_resnet_tensor_len(self.h, i, C.byref(n), C.byref(d)))
            out.append((int(n.value), bool(d.value)))
        return out

    def _get(self, which, count):
        import torch
        t = torch.empty(count, dtype=torch.float32, device=f"cuda:{self.device}")
        self.ctx.check(lib().rnn_resnet_copy(self.h, which, _ptr(t, count, "dst"), None))
        return t

    def _set(self, which, src, count):
        self.ctx.check(lib().rnn_resnet_copy(self.h, which, None, _ptr(src.contiguous(), count,
                                                                        "src")))

    def params(self):
        """Flat values in for_each_param order (model.rs:164-175)."""
        return self._get(0, self.num_params())

    def grads(self):
        return self._get(1, self.num_params())

    def momenta(self):
        return self._get(2, self.num_params())

    def buffers(self):
        """BN running mean / var in for_each_buffer order (model.rs:177-184)."""
        return self._get(3, self.num_buffers())

    def set_params(self, v):
        self._set(0, v, self.num_params())

    def set_grads(self, g):
        self._set(1, g, self.num_params())

    def set_buffers(self, b):
        self._set(3, b, self.num_buffers())

    # ---- model.rs
    def forward(self, x, train=True):
        """ResNet::forward (model.rs:138-150): x [n, 3, h, w] -> logits [n, nclass]."""
        import torch
        n, _, h, w = x.shape
        lg = torch.empty(n, self.nclass, dtype=torch.float32, device=x.device)
        self.ctx.check(lib().rnn_resnet_forward(self.h, n, h, w, _ptr(x, n * 3 * h * w, "x"),
                                                int(train), _ptr(lg, n * self.nclass, "logits")))
        return lg

    def backward(self, dlogits):
        """ResNet::backward (model.rs:152-162): gradients accumulate."""
        self.ctx.check(lib().rnn_resnet_backward(self.h, _ptr(dlogits, dlogits.numel(), "dl")))

    def step(self, lr, mom, wd):
        """ResNet::step (model.rs:205-207)."""
        self.ctx.check(lib().rnn_resnet_step(self.h, lr, mom, wd))

    def train_step(self, x, labels, smooth, lr, mom, wd, loss=None, correct=None):
        """forward + softmax_ce + backward + step (train.rs:686-699).  loss /
        correct: optional CUDA tensors ([1] float32 / [1] int32).  x and
        labels None: the batch already written into ``inputs()``."""
        if x is None and labels is None:
            n, h, w = self._in_shape
            xp = lp = None
        else:
            n, _, h, w = x.shape
            xp, lp = _ptr(x, n * 3 * h * w, "x"), _ptr(labels, n, "labels")
        self.ctx.check(lib().rnn_resnet_train_step(
            self.h, n, h, w, xp, lp, float(smooth), float(lr), float(mom), float(wd),
            _ptr(loss, 1, "loss"), _ptr(correct, 1, "correct")))

    def inputs(self, n, h, w):
        """The network's input slots for n x 3 x h x w batches as CUDA tensors
        (x float32 [n, 3, h, w], labels int32 [n]) over device memory the
        network owns: fill them in place, then ``train_step(None, None, ...)``.
        Valid until the shape changes or the network is closed."""
        import torch
        xp, lp = _vp(), _vp()
        self.ctx.check(lib().rnn_resnet_inputs(self.h, n, h, w, C.byref(xp), C.byref(lp)))
        self._in_shape = (n, h, w)
        dev = torch.device("cuda", self.device)
        return (torch.as_tensor(_DevArray(xp.value, (n, 3, h, w), "<f4"), device=dev),
                torch.as_tensor(_DevArray(lp.value, (n,), "<i4"), device=dev))

    def dbg_buffer(self, block, which):
        """A copy of one of the buffers the step keeps for `block`
        (rnn_dbg_resnet_buffer: 0 y1, 1 h, 2 y2, 3 ys, 4 out, 5-7 the c1 / c2
        / shortcut output gradients, 8 / 9 b1 / b2 mean then invstd, 10 the
        block's input)."""
        import torch
        p, n = _vp(), C.c_size_t()
        self.ctx.check(lib().rnn_dbg_resnet_buffer(self.h, block, which, C.byref(p), C.byref(n)))
        dev = torch.device("cuda", self.device)
        return torch.as_tensor(_DevArray(p.value, (n.value,), "<f4"), device=dev).clone()

    def dw_group(self, launch=True):
        """The algorithmic FLOP of the step's grouped weight-gradient launch,
        enqueued once more over the last backward's buffers when `launch`
        (rnn_dbg_resnet_dw_group; 0.0 without a grouped launch)."""
        f = C.c_double()
        self.ctx.check(lib().rnn_dbg_resnet_dw_group(self.h, int(bool(launch)), C.byref(f)))
        return f.value

    def set_graph(self, on):
        self.ctx.check(lib().rnn_resnet_set_graph(self.h, int(bool(on))))

    def graph_state(self):
        why = C.c_char_p()
        st = lib().rnn_resnet_graph_state(self.h, C.byref(why))
        if st < 0:
            raise RnnError(st, "graph_state")
        return bool(st), (why.value or b"").decode()

    def flops(self, h, w):
        """ResNet::flops (model.rs:179-198): forward FLOP per image."""
        return int(lib().rnn_resnet_flops(self.h, h, w))

    def close(self):
        if getattr(self, "h", None):
            lib().rnn_resnet_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class BasicBlock:
    """BasicBlock (model.rs:10-101) composed from the layer entry points of
    the C ABI (conv, BatchNorm2d, add / ReLU), with caller-supplied weights
    (w1, w2 and, with a shortcut, wd, as [cout, cin*k*k] CUDA tensors).  BN
    gamma starts at 1, 0 for the second BN (model.rs:22-23)."""

    def __init__(self, cin, cout, stride, w1, w2, wd=None, device=0, ctx=None):
        from . import Conv2d
        from .nn import BatchNorm2d
        self.ctx = ctx or default_ctx(device)
        self.cin, self.cout, self.stride = cin, cout, stride
        self.c1 = Conv2d(cin, cout, 3, stride, 1, w=w1, device=device, ctx=self.ctx)
        self.b1 = BatchNorm2d(cout, device, self.ctx)
        self.c2 = Conv2d(cout, cout, 3, 1, 1, w=w2, device=device, ctx=self.ctx)
        self.b2 = BatchNorm2d(cout, device, self.ctx)
        self.b2.zero_gamma()
        self.down = None
        if stride != 1 or cin != cout:
            self.down = (Conv2d(cin, cout, 1, stride, 0, w=wd, device=device, ctx=self.ctx),
                         BatchNorm2d(cout, device, self.ctx))

    def forward(self, x, train=True):
        """BasicBlock::forward (model.rs:39-57); x [n, cin, h, w]."""
        from .nn import add_relu_
        n, _, h, w = x.shape
        y1 = self.c1.forward(x.reshape(-1), n, h, w, train)
        sp = self.c1.spec(h, w)
        hh = self.b1.forward_relu(y1.view(n, self.cout, sp.oh, sp.ow), train)
        y = self.b2.forward(self.c2.forward(hh.reshape(-1), n, sp.oh, sp.ow, train)
                            .view(n, self.cout, sp.oh, sp.ow), train)
        if self.down is not None:
            c, b = self.down
            s = b.forward(c.forward(x.reshape(-1), n, h, w, train).view(y.shape), train)
            add_relu_(y, s, ctx=self.ctx)
        else:
            add_relu_(y, x, ctx=self.ctx)
        if train:
            self.h1, self.out, self.xshape = hh, y, x.shape
        return y

    def backward(self, d):
        """BasicBlock::backward (model.rs:59-77): returns dx."""
        from .nn import add_, relu_back_
        d = d.clone()
        relu_back_(d, self.out, ctx=self.ctx)
        dmain = self.c2.backward(self.b2.backward(d).reshape(-1)).view(self.h1.shape)
        relu_back_(dmain, self.h1, ctx=self.ctx)
        dx = self.c1.backward(self.b1.backward(dmain).reshape(-1)).view(self.xshape)
        if self.down is not None:
            c, b = self.down
            ds = c.backward(b.backward(d).reshape(-1)).view(self.xshape)
            add_(dx, ds, ctx=self.ctx)
        else:
            add_(dx, d, ctx=self.ctx)
        return dx

    def params(self):
        """(value, grad) tensors in for_each_param order (model.rs:79-91)."""
        ps = [(self.c1.w, self.c1.g), (self.b1.g.v, self.b1.g.g), (self.b1.b.v, self.b1.b.g),
              (self.c2.w, self.c2.g), (self.b2.g.v, self.b2.g.g), (self.b2.b.v, self.b2.b.g)]
        if self.down is not None:
            c, b = self.down
            ps += [(c.w, c.g), (b.g.v, b.g.g), (b.b.v, b.b.g)]
        return ps
