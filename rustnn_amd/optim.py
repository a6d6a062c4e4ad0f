"""optim.rs on the device: Muon (Newton-Schulz over the batched GEMM core),
AdamW, the global-norm clip and the weight EMA.

Mirrors the reference's interface (optim.rs:124-317): ``newton_schulz``,
``Optim(muon, ns_steps).step_all(params, lr, wd)``, ``clip_(params, max)``
and ``Ema(d).update / swap_in / swap_out``, over ``Param`` objects holding
CUDA tensors (nn.rs Param, nn.rs:43-75).  Every call goes through librnn.so;
there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import RnnError, _ptr, _sz, _vp, default_ctx, lib


class RnnParam(C.Structure):
    _fields_ = [("v", _vp), ("g", _vp), ("m", _vp), ("v2", _vp), ("len", _sz), ("rows", _sz),
                ("cols", _sz), ("decay", C.c_int)]


class Param:
    """nn.rs Param (nn.rs:43-75): value, gradient, momentum and AdamW's second
    moment on the device; rows/cols mark a [rows x cols] matrix (Muon)."""

    def __init__(self, v, decay, rows=0, cols=0):
        import torch
        self.v = v.contiguous().reshape(-1)
        self.g = torch.zeros_like(self.v)
        self.m = torch.zeros_like(self.v)
        self.v2 = torch.zeros_like(self.v)
        self.decay = bool(decay)
        self.rows, self.cols = int(rows), int(cols)

    def __setattr__(self, name, value):
        # any change of a buffer or of the shape drops the cached C view
        object.__setattr__(self, name, value)
        if name != "_cs":
            object.__setattr__(self, "_cs", None)

    def shaped(self, rows, cols):
        """Param::shaped (nn.rs:69-74)."""
        assert rows * cols == self.v.numel()
        self.rows, self.cols = int(rows), int(cols)
        return self

    def _c(self):
        if self._cs is None:
            n = self.v.numel()
            self._cs = RnnParam(_ptr(self.v, n, "v"), _ptr(self.g, n, "g"), _ptr(self.m, n, "m"),
                                _ptr(self.v2, n, "v2"), n, self.rows, self.cols, int(self.decay))
        return self._cs


class _ParamList:
    """The C array of a parameter list, rebuilt only when one of the
    parameters' C views changed."""

    def __init__(self):
        self.key, self.arr = None, None

    def __call__(self, params):
        cs = [p._c() for p in params]
        key = tuple(map(id, cs))
        if key != self.key:
            self.arr = (RnnParam * len(cs))(*cs)
            self.key = key
        return self.arr


def newton_schulz(g, rows, cols, steps, ctx=None):
    """newton_schulz (optim.rs:124-145) in place on g: [rows*cols] or
    [count, rows*cols] (same-shape matrices orthogonalised together)."""
    ctx = ctx or default_ctx()
    count = g.numel() // (rows * cols)
    ctx.check(lib().rnn_newton_schulz(ctx.h, count, rows, cols, steps,
                                      _ptr(g, count * rows * cols, "g"), rows * cols))
    return g


class Optim:
    """Optim (optim.rs:147-235): Muon for matrices with both sides > 1 (when
    ``muon``), AdamW for the rest; ``t`` counts steps."""

    def __init__(self, muon=True, ns_steps=3, ctx=None):
        self.ctx = ctx or default_ctx()
        h = _vp()
        self.ctx.check(lib().rnn_optim_create(self.ctx.h, int(bool(muon)), ns_steps, C.byref(h)))
        self.h = h
        self.muon, self.ns_steps = bool(muon), ns_steps
        self.mom, self.b1, self.b2, self.eps = 0.95, 0.9, 0.999, 1e-8
        self._list = _ParamList()

    @property
    def t(self):
        return int(lib().rnn_optim_t(self.h))

    def set(self, mom=None, b1=None, b2=None, eps=None, t=None):
        self.mom = self.mom if mom is None else mom
        self.b1 = self.b1 if b1 is None else b1
        self.b2 = self.b2 if b2 is None else b2
        self.eps = self.eps if eps is None else eps
        self.ctx.check(lib().rnn_optim_set(self.h, self.mom, self.b1, self.b2, self.eps,
                                           self.t if t is None else t))

    def step_all(self, params, lr, wd):
        """Optim::step_all (optim.rs:177-205)."""
        arr = self._list(params)
        self.ctx.check(lib().rnn_optim_step(self.h, len(params), C.cast(arr, _vp), float(lr),
                                            float(wd)))

    def close(self):
        if getattr(self, "h", None):
            lib().rnn_optim_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


_clip_list = _ParamList()


def clip_(params, max_norm, ctx=None, norm=None):
    """clip_ (optim.rs:237-251): the global gradient norm over every
    parameter's gradient and, above ``max_norm``, every gradient scaled by
    max / norm.  Returns the norm as a float (one device sync), or, when
    ``norm`` (a 1-element device tensor) is given, leaves it there and
    returns ``norm`` without synchronising."""
    import torch
    ctx = ctx or default_ctx()
    sync = norm is None
    if norm is None:
        norm = torch.zeros(1, dtype=torch.float32, device="cuda")
    arr = _clip_list(params)
    ctx.check(lib().rnn_clip_params(ctx.h, len(params), C.cast(arr, _vp), float(max_norm),
                                    _ptr(norm, 1, "norm")))
    return float(norm.item()) if sync else norm


class Ema:
    """Ema (optim.rs:253-317): the exponential average of the weights."""

    def __init__(self, d, ctx=None):
        self.ctx = ctx or default_ctx()
        self.d = np.float32(d)
        self.w = []
        self.ready = False
        self.t = 0
        self._list = _ParamList()

    def update(self, params):
        """Ema::update (optim.rs:270-288): one launch over the whole list."""
        self.t += 1
        if not self.ready:
            self.w = [p.v.clone() for p in params]
            self._wp = (C.c_void_p * len(self.w))(*[e.data_ptr() for e in self.w])
            self.ready = True
            return
        if len(params) != len(self.w):
            raise RnnError(-2, f"EMA with {len(self.w)} tensors for {len(params)} parameters")
        for e, p in zip(self.w, params):
            if e.numel() != p.v.numel():
                raise RnnError(-2, "EMA tensor and parameter differ in length")
        t = np.float32(self.t)
        d = min(self.d, (np.float32(1.0) + t) / (np.float32(10.0) + t))
        arr = self._list(params)
        self.ctx.check(lib().rnn_ema_update_params(self.ctx.h, len(params), C.cast(self._wp, _vp),
                                                   C.cast(arr, _vp), float(d)))

    def swap_in(self, params):
        """Ema::swap_in (optim.rs:290-305): the model takes the average's
        weights; returns the originals."""
        if not (self.ready and len(self.w) == len(params)):
            raise RnnError(-2, f"EMA with {len(self.w)} tensors for {len(params)} parameters")
        old = []
        for p, e in zip(params, self.w):
            old.append(p.v.clone())
            p.v.copy_(e)
        return old

    @staticmethod
    def swap_out(params, old):
        """Ema::swap_out (optim.rs:307-316)."""
        if len(params) != len(old):
            raise RnnError(-2, "swap_out with a different number of tensors than swap_in")
        for p, o in zip(params, old):
            p.v.copy_(o)
