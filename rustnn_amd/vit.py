"""vit.rs / attn.rs call sites on the device: SelfAttn, CrossAttn, DropPath,
the pre-LN Block, token merge, TaxoHead and Exit.

Mirrors the reference's layer interface (attn.rs:346-560, vit.rs:25-353)
over token tensors [n, t, c] (float32 CUDA, channel fastest):
``forward(x, ..., train)`` / ``backward(dy, ...)``; parameter gradients
accumulate into ``rustnn_amd.optim.Param.g`` and ``for_each_param`` walks
the parameters in the reference's order, so a list of them feeds
``Optim.step_all`` / ``clip_`` / ``Ema`` directly.  Initial values are drawn
with torch's generator (truncated normal as Param::trunc_normal), not with
the reference's Rng stream.  Every compute call goes through librnn.so.
"""
from __future__ import annotations

import math

from . import Core, Linear, _ptr, default_ctx, lib, rel_index
from .norm import DwConv3, LayerNorm, LayerScale, SeqPool, SwiGlu, _linear_param
from .optim import Param


def _trunc_normal(n, std, gen, device):
    """Param::trunc_normal (nn.rs:77-89) in distribution: N(0, 1) clamped to
    +-2 (the reference redraws up to 8 times first), times std."""
    import torch
    z = torch.randn(n, generator=gen, device=device)
    for _ in range(8):
        bad = z.abs() > 2.0
        if not bool(bad.any()):
            break
        z = torch.where(bad, torch.randn(n, generator=gen, device=device), z)
    return z.clamp(-2.0, 2.0) * std


def _linear(fin, fout, bias, std, gen, device, ctx):
    w = _trunc_normal(fin * fout, std, gen, device)
    return Linear(fin, fout, bias, w, None, 0, ctx)


def _scaled_std(depth):
    """Linear::scaled (linear.rs:37-41)."""
    return 0.02 / math.sqrt(2.0 * depth)


def _add_(a, b, ctx):
    ctx.check(lib().rnn_add(ctx.h, a.numel(), _ptr(a, a.numel(), "a"), _ptr(b, a.numel(), "b")))
    return a


class SelfAttn:
    """SelfAttn (attn.rs:346-448): fused qkv Linear(c, 3c) -> Core (masked
    diagonal) -> proj Linear::scaled; tau = 1/sqrt(dh), rel = 0."""

    def __init__(self, c, h, th, tw, depth, gen=None, device=0, ctx=None):
        import torch
        dev = f"cuda:{device}"
        self.ctx = ctx or default_ctx(device)
        gen = gen or torch.Generator(device=dev).manual_seed(0)
        self.c, self.h, self.dh, self.t = c, h, c // h, th * tw
        relidx, nrel = rel_index(th, tw, th, tw)
        self.qkv = _linear(c, 3 * c, True, 0.02, gen, dev, self.ctx)
        self.proj = _linear(c, c, True, _scaled_std(depth), gen, dev, self.ctx)
        self.tau = Param(torch.full((h,), 1.0 / math.sqrt(self.dh), device=dev), False)
        self.rel = Param(torch.zeros(h * nrel, device=dev), False)
        self.core = Core(h, self.dh, self.t, self.t, relidx, nrel, True, ctx=self.ctx)
        self._lin = _linear_param(self.qkv) + _linear_param(self.proj)
        self.ab = self.p = None
        self.n = 0

    def forward(self, x, train):
        n, t, c = x.shape
        ab = self.qkv.forward(x.reshape(-1), n * t, train)
        p, o = self.core.forward(n, ab, 3 * c, 0, ab, 3 * c, c, 2 * c, self.tau.v, self.rel.v)
        y = self.proj.forward(o, n * t, train)
        if train:
            self.ab, self.p, self.n = ab, p, n
        return y.view(n, t, c)

    def backward(self, dy):
        import torch
        n, t, c = self.n, self.t, self.c
        do = self.proj.backward(dy.reshape(-1))
        # dq and dk/dv land in one fused-QKV gradient (attn.rs:418-438)
        dab = torch.zeros(n * t * 3 * c, device=dy.device)
        self.core.backward(n, self.ab, 3 * c, 0, self.ab, 3 * c, c, 2 * c, self.tau.v, self.p,
                           do, dab, dab, self.tau.g, self.rel.g)
        return self.qkv.backward(dab).view(n, t, c)

    def for_each_param(self, f):
        for p in self._lin:
            f(p)
        f(self.tau)
        f(self.rel)


class CrossAttn:
    """CrossAttn (attn.rs:450-560): wq Linear(c, c) -> Core over the memory
    [n, mh*mw, 2c] (K at 0, V at c), no mask -> proj Linear::scaled."""

    def __init__(self, c, h, th, tw, mh, mw, depth, gen=None, device=0, ctx=None):
        import torch
        dev = f"cuda:{device}"
        self.ctx = ctx or default_ctx(device)
        gen = gen or torch.Generator(device=dev).manual_seed(0)
        self.c, self.h, self.dh = c, h, c // h
        self.tq, self.tk = th * tw, mh * mw
        relidx, nrel = rel_index(th, tw, mh, mw)
        self.wq = _linear(c, c, True, 0.02, gen, dev, self.ctx)
        self.proj = _linear(c, c, True, _scaled_std(depth), gen, dev, self.ctx)
        self.tau = Param(torch.full((h,), 1.0 / math.sqrt(self.dh), device=dev), False)
        self.rel = Param(torch.zeros(h * nrel, device=dev), False)
        self.core = Core(h, self.dh, self.tq, self.tk, relidx, nrel, False, ctx=self.ctx)
        self._lin = _linear_param(self.wq) + _linear_param(self.proj)
        self.q = self.p = None
        self.n = 0

    def forward(self, x, mem, train):
        n, t, c = x.shape
        q = self.wq.forward(x.reshape(-1), n * t, train)
        p, o = self.core.forward(n, q, c, 0, mem, 2 * c, 0, c, self.tau.v, self.rel.v)
        y = self.proj.forward(o, n * t, train)
        if train:
            self.q, self.p, self.n = q, p, n
        return y.view(n, t, c)

    def backward(self, dy, mem, dmem):
        """Returns dx; dmem ([n, tk, 2c]) accumulates."""
        import torch
        n, t, c = self.n, self.tq, self.c
        do = self.proj.backward(dy.reshape(-1))
        dq = torch.zeros(n * t * c, device=dy.device)
        self.core.backward(n, self.q, c, 0, mem, 2 * c, 0, c, self.tau.v, self.p, do, dq, dmem,
                           self.tau.g, self.rel.g)
        return self.wq.backward(dq).view(n, t, c)

    def for_each_param(self, f):
        for p in self._lin:
            f(p)
        f(self.tau)
        f(self.rel)


class DropPath:
    """DropPath (vit.rs:25-74): the whole branch of an image dropped with
    probability p; the mask comes from Rng::new(seed), drawn on the device."""

    def __init__(self, p, ctx=None):
        self.p = float(p)
        self.ctx = ctx or default_ctx()
        self.mask = None

    def forward(self, x, train, seed):
        import torch
        if not train or self.p <= 0.0:
            self.mask = None
            return x
        n = x.shape[0]
        self.mask = torch.empty(n, device=x.device)
        self.ctx.check(lib().rnn_drop_path_forward(self.ctx.h, n, x.numel() // n,
                                                   _ptr(x, x.numel(), "x"), self.p,
                                                   seed & 0xFFFFFFFFFFFFFFFF,
                                                   _ptr(self.mask, n, "mask")))
        return x

    def backward(self, dy):
        if self.mask is None:
            return dy
        n = dy.shape[0]
        self.ctx.check(lib().rnn_drop_path_backward(self.ctx.h, n, dy.numel() // n,
                                                    _ptr(dy, dy.numel(), "dy"),
                                                    _ptr(self.mask, n, "mask")))
        return dy


class Block:
    """Block (vit.rs:76-250), pre-LN with three branches from one norm:
    h = LN(x); x += ls1 * dp1(SelfAttn(h) + gamma * DwConv3(h));
    x += lsm * dp2(CrossAttn(h, mem)) (reader blocks); x += ls2 * dp3(SwiGlu(LN(x)))."""

    def __init__(self, c, h, th, tw, mem, depth, drop, idx, ls_init, gen=None, device=0,
                 ctx=None):
        import torch
        dev = f"cuda:{device}"
        self.ctx = ctx or default_ctx(device)
        gen = gen or torch.Generator(device=dev).manual_seed(int(idx))
        self.c, self.idx = c, int(idx)
        hidden = -(-(4 * c // 3) // 16) * 16
        self.n1 = LayerNorm(c, device, self.ctx)
        self.attn = SelfAttn(c, h, th, tw, depth, gen, device, self.ctx)
        self.dw = DwConv3(c, th, tw, _trunc_normal(9 * c, 0.1, gen, dev), None, device, self.ctx)
        self.gamma = Param(torch.full((c,), 0.5, device=dev), False)
        self.ls1 = LayerScale(c, ls_init, device, self.ctx)
        self.cross = (CrossAttn(c, h, th, tw, mem[0], mem[1], depth, gen, device, self.ctx)
                      if mem else None)
        self.lsm = LayerScale(c, ls_init, device, self.ctx) if mem else None
        self.n2 = LayerNorm(c, device, self.ctx)
        wg = _trunc_normal(2 * hidden * c, 0.02, gen, dev)
        wd = _trunc_normal(hidden * c, _scaled_std(depth), gen, dev)
        self.mlp = SwiGlu(c, hidden, wg, None, wd, None, device, self.ctx)
        self.ls2 = LayerScale(c, ls_init, device, self.ctx)
        self.dp1, self.dp2, self.dp3 = (DropPath(drop, self.ctx), DropPath(drop, self.ctx),
                                        DropPath(drop, self.ctx))
        self.dwo = None

    def forward(self, x, mem, train, seed):
        import torch
        L, ctx, c = lib(), self.ctx, self.c
        h = self.n1.forward(x, train)
        a = self.attn.forward(h, train)
        d = self.dw.forward(h, train)
        rows = a.numel() // c
        ctx.check(L.rnn_axpy_cols(ctx.h, rows, c, _ptr(a, rows * c, "a"),
                                  _ptr(self.gamma.v, c, "gamma"), _ptr(d, rows * c, "d")))
        if train:
            self.dwo = d
        a = self.dp1.forward(self.ls1.forward(a, train), train, seed ^ self.idx)
        y = torch.clone(x)
        _add_(y, a, ctx)
        if self.cross is not None:
            if mem is None:
                raise ValueError("Block: a reader block needs the memory")
            cm = self.cross.forward(h, mem, train)
            cm = self.dp2.forward(self.lsm.forward(cm, train), train, seed ^ self.idx ^ 0x5151)
            _add_(y, cm, ctx)
        h2 = self.n2.forward(y, train)
        m = self.mlp.forward(h2, train)
        m = self.dp3.forward(self.ls2.forward(m, train), train, seed ^ self.idx ^ 0xA2A2)
        _add_(y, m, ctx)
        return y

    def backward(self, dz, mem=None, dmem=None):
        """Returns dx; dmem accumulates the memory's gradient (vit.rs:175-249)."""
        import torch
        L, ctx, c = lib(), self.ctx, self.c
        dm = self.ls2.backward(self.dp3.backward(dz.clone()))
        dh2 = self.mlp.backward(dm)
        dy = dz.clone()
        _add_(dy, self.n2.backward(dh2), ctx)
        dh = torch.zeros_like(dy)
        if self.cross is not None:
            dc = self.lsm.backward(self.dp2.backward(dy.clone()))
            _add_(dh, self.cross.backward(dc, mem, dmem), ctx)
        da = self.ls1.backward(self.dp1.backward(dy.clone()))
        # gamma.g += sum da * dwo; ddw = gamma * da: the LayerScale backward
        rows = da.numel() // c
        ddw = torch.empty_like(da)
        ctx.check(L.rnn_layerscale_backward(ctx.h, rows, c, _ptr(da, rows * c, "da"),
                                            _ptr(self.dwo, rows * c, "dwo"),
                                            _ptr(self.gamma.v, c, "gamma"),
                                            _ptr(ddw, rows * c, "ddw"),
                                            _ptr(self.gamma.g, c, "dgamma")))
        _add_(dh, self.attn.backward(da), ctx)
        _add_(dh, self.dw.backward(ddw), ctx)
        _add_(dy, self.n1.backward(dh), ctx)
        return dy

    def for_each_param(self, f):
        """Block::for_each_param (vit.rs:234-249)."""
        self.n1.for_each_param(f)
        self.attn.for_each_param(f)
        self.dw.for_each_param(f)
        f(self.gamma)
        self.ls1.for_each_param(f)
        if self.cross is not None:
            self.cross.for_each_param(f)
            self.lsm.for_each_param(f)
        self.n2.for_each_param(f)
        self.mlp.for_each_param(f)
        self.ls2.for_each_param(f)


def token_merge(z, th, ctx=None):
    """token_merge (vit.rs:612-630): [n, th*th, c] -> [n, (th/2)^2, 4c]."""
    import torch
    ctx = ctx or default_ctx()
    n, t, c = z.shape
    y = torch.empty(n, t // 4, 4 * c, device=z.device)
    ctx.check(lib().rnn_token_merge(ctx.h, n, th, c, _ptr(z, z.numel(), "z"),
                                    _ptr(y, z.numel(), "y")))
    return y


def token_merge_back(dy, th, c, ctx=None):
    """token_merge_back (vit.rs:632-650)."""
    import torch
    ctx = ctx or default_ctx()
    n = dy.shape[0]
    dz = torch.empty(n, th * th, c, device=dy.device)
    ctx.check(lib().rnn_token_merge_backward(ctx.h, n, th, c, _ptr(dy, dz.numel(), "dy"),
                                             _ptr(dz, dz.numel(), "dz")))
    return dz


class TaxoHead:
    """TaxoHead (vit.rs:254-318): coarse Linear(c, nc), resid Linear(c, nf);
    fine logits z_f[j] = z_c[parent[j]] + r[j].  parent: CUDA int32/uint32."""

    def __init__(self, c, parent, nc, gen=None, device=0, ctx=None):
        import torch
        dev = f"cuda:{device}"
        self.ctx = ctx or default_ctx(device)
        gen = gen or torch.Generator(device=dev).manual_seed(1)
        self.parent, self.nc, self.nf = parent, nc, parent.numel()
        self.coarse = _linear(c, nc, True, 0.02, gen, dev, self.ctx)
        self.resid = _linear(c, self.nf, True, 0.02, gen, dev, self.ctx)
        self._params = _linear_param(self.coarse) + _linear_param(self.resid)
        self.n = 0

    def forward(self, f, n, train):
        zc = self.coarse.forward(f.reshape(-1), n, train)
        zf = self.resid.forward(f.reshape(-1), n, train)
        self.ctx.check(lib().rnn_taxo_head_combine(
            self.ctx.h, n, self.nf, self.nc, _ptr(self.parent, self.nf, "parent"),
            _ptr(zf, n * self.nf, "zf"), _ptr(zc, n * self.nc, "zc")))
        self.n = n
        return zf.view(n, self.nf), zc.view(n, self.nc)

    def backward(self, dzf, dzc):
        import torch
        n = self.n
        dc = torch.empty(n * self.nc, device=dzf.device)
        self.ctx.check(lib().rnn_taxo_head_combine_backward(
            self.ctx.h, n, self.nf, self.nc, _ptr(self.parent, self.nf, "parent"),
            _ptr(dzf, n * self.nf, "dzf"), _ptr(dzc, n * self.nc, "dzc"),
            _ptr(dc, n * self.nc, "dc")))
        df = self.resid.backward(dzf.reshape(-1))
        _add_(df, self.coarse.backward(dc), self.ctx)
        return df

    def for_each_param(self, f):
        for p in self._params:
            f(p)


class Exit:
    """Exit (vit.rs:320-353): fc Linear(cin, nclass) and hint Linear(cin,
    chint, no bias) over the same feature."""

    def __init__(self, cin, nclass, chint, gen=None, device=0, ctx=None):
        import torch
        dev = f"cuda:{device}"
        self.ctx = ctx or default_ctx(device)
        gen = gen or torch.Generator(device=dev).manual_seed(2)
        self.fc = _linear(cin, nclass, True, 0.02, gen, dev, self.ctx)
        self.hint = _linear(cin, chint, False, 0.02, gen, dev, self.ctx)
        self._params = _linear_param(self.fc) + _linear_param(self.hint)
        self.n = 0

    def forward(self, f, n, train):
        self.n = n
        return (self.fc.forward(f.reshape(-1), n, train).view(n, -1),
                self.hint.forward(f.reshape(-1), n, train).view(n, -1))

    def backward(self, dz, dh):
        d = self.fc.backward(dz.reshape(-1))
        return _add_(d, self.hint.backward(dh.reshape(-1)), self.ctx)

    def for_each_param(self, f):
        for p in self._params:
            f(p)


def nchw_to_tokens(x, ctx=None):
    """Tok::from_tensor (tok.rs): [n, c, h, w] -> [n, h*w, c]."""
    import torch
    ctx = ctx or default_ctx()
    n, c, hh, ww = x.shape
    t = torch.empty(n, hh * ww, c, device=x.device)
    ctx.check(lib().rnn_nchw_to_tokens(ctx.h, n, c, hh * ww, _ptr(x, x.numel(), "x"),
                                       _ptr(t, x.numel(), "t")))
    return t


def tokens_to_nchw(t, hh, ww, ctx=None):
    """Tok::to_tensor (tok.rs): [n, h*w, c] -> [n, c, h, w]."""
    import torch
    ctx = ctx or default_ctx()
    n, hw, c = t.shape
    x = torch.empty(n, c, hh, ww, device=t.device)
    ctx.check(lib().rnn_tokens_to_nchw(ctx.h, n, c, hw, _ptr(t, t.numel(), "t"),
                                       _ptr(x, t.numel(), "x")))
    return x
