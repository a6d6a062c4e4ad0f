"""vit.rs / attn.rs call sites on the device: SelfAttn, CrossAttn, DropPath,
the pre-LN Block, token merge, TaxoHead and Exit.

Mirrors the reference's layer interface (attn.rs:346-560, vit.rs:25-353)
over token tensors [n, t, c] (float32 CUDA, channel fastest):
``forward(x, ..., train)`` / ``backward(dy, ...)``; parameter gradients
accumulate into ``rustnn_amd.optim.Param.g`` and ``for_each_param`` walks
the parameters in the reference's order, so a list of them feeds
``Optim.step_all`` / ``clip_`` / ``Ema`` directly.  Initial values come from
the reference's generator (rng.rs, ``rustnn_amd.data.Rng``) in the
reference's draw order, so a network built from a seed holds the same
weights as the reference's built from that seed, bit for bit.  Every compute
call goes through librnn.so.
"""
from __future__ import annotations


import numpy as np

from . import Core, Linear, _ptr, default_ctx, lib, linear_backward, linear_forward, rel_index
from .data import Rng
from .norm import DwConv3, LayerNorm, LayerScale, SeqPool, SwiGlu, _linear_param
from .optim import Param


def _rng(rng, seed):
    """A generator argument: an Rng, a seed, or None (Rng::new(seed))."""
    if rng is None:
        return Rng(seed)
    return Rng(rng) if isinstance(rng, int) else rng


def _trunc_normal(n, std, rng, device):
    """Param::trunc_normal (nn.rs:77-89) from the reference's generator: a
    normal redrawn up to 8 times while |z| > 2, clamped to [-2, 2], times
    std (an f32)."""
    import torch
    return torch.from_numpy(rng.trunc_normal(n, std)).to(device)


def _kaiming(fan_in, n, rng, device):
    """Param::kaiming (nn.rs:95-100): normal() * sqrt(2 / fan_in) in f32."""
    import torch
    s = np.sqrt(np.float32(2.0) / np.float32(fan_in))
    return torch.from_numpy(rng.normal_vec(n, s)).to(device)


def _linear(fin, fout, bias, std, rng, device, ctx):
    """Linear::new (linear.rs:25-35): w [fout, fin] trunc_normal(std), b 0."""
    w = _trunc_normal(fin * fout, std, rng, device)
    return Linear(fin, fout, bias, w, None, 0, ctx)


def _inv_sqrt(dh):
    """1 / sqrt(dh) in f32: tau's initial value (attn.rs:371, 479)."""
    return float(np.float32(1.0) / np.sqrt(np.float32(dh)))


def _scaled_std(depth):
    """Linear::scaled (linear.rs:37-41): 0.02 / sqrt(2 depth), in f32."""
    return np.float32(0.02) / np.sqrt(np.float32(2.0) * np.float32(depth))


class SelfAttn:
    """SelfAttn (attn.rs:346-448): fused qkv Linear(c, 3c) -> Core (masked
    diagonal) -> proj Linear::scaled; tau = 1/sqrt(dh), rel = 0."""

    def __init__(self, c, h, th, tw, depth, rng=None, device=0, ctx=None):
        import torch
        dev = f"cuda:{device}"
        self.ctx = ctx or default_ctx(device)
        rng = _rng(rng, 0)
        self.c, self.h, self.dh, self.t = c, h, c // h, th * tw
        relidx, nrel = rel_index(th, tw, th, tw)
        self.qkv = _linear(c, 3 * c, True, 0.02, rng, dev, self.ctx)
        self.proj = _linear(c, c, True, _scaled_std(depth), rng, dev, self.ctx)
        self.tau = Param(torch.full((h,), _inv_sqrt(self.dh), device=dev), False)
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

    def backward(self, dy, acc_dx=None):
        """dx, or acc_dx += dx (returned) when given."""
        import torch
        n, t, c = self.n, self.t, self.c
        do = self.proj.backward(dy.reshape(-1))
        # dq and dk/dv land in one fused-QKV gradient (attn.rs:418-438: zeroed
        # buffers, accumulated into; here written directly)
        dab = torch.empty(n * t * 3 * c, device=dy.device)
        self.core.backward(n, self.ab, 3 * c, 0, self.ab, 3 * c, c, 2 * c, self.tau.v, self.p,
                           do, dab, dab, self.tau.g, self.rel.g, set_dq=True, set_dkv=True)
        acc = acc_dx.reshape(-1) if acc_dx is not None else None
        return self.qkv.backward(dab, acc_dx=acc).view(n, t, c)

    def for_each_param(self, f):
        for p in self._lin:
            f(p)
        f(self.tau)
        f(self.rel)


class CrossAttn:
    """CrossAttn (attn.rs:450-560): wq Linear(c, c) -> Core over the memory
    [n, mh*mw, 2c] (K at 0, V at c), no mask -> proj Linear::scaled."""

    def __init__(self, c, h, th, tw, mh, mw, depth, rng=None, device=0, ctx=None):
        import torch
        dev = f"cuda:{device}"
        self.ctx = ctx or default_ctx(device)
        rng = _rng(rng, 0)
        self.c, self.h, self.dh = c, h, c // h
        self.tq, self.tk = th * tw, mh * mw
        relidx, nrel = rel_index(th, tw, mh, mw)
        self.wq = _linear(c, c, True, 0.02, rng, dev, self.ctx)
        self.proj = _linear(c, c, True, _scaled_std(depth), rng, dev, self.ctx)
        self.tau = Param(torch.full((h,), _inv_sqrt(self.dh), device=dev), False)
        self.rel = Param(torch.zeros(h * nrel, device=dev), False)
        self.core = Core(h, self.dh, self.tq, self.tk, relidx, nrel, False, ctx=self.ctx)
        self._lin = _linear_param(self.wq) + _linear_param(self.proj)
        self.q = self.p = None
        self.n = 0

    def forward(self, x, mem, train, residual=None):
        """residual = (out, l, mask): the projection also adds
        out += (y l) mask[image] (Linear.forward)."""
        n, t, c = x.shape
        q = self.wq.forward(x.reshape(-1), n * t, train)
        p, o = self.core.forward(n, q, c, 0, mem, 2 * c, 0, c, self.tau.v, self.rel.v)
        res = None if residual is None else (*residual, t)
        y = self.proj.forward(o, n * t, train, res)
        if train:
            self.q, self.p, self.n = q, p, n
        return y.view(n, t, c)

    def backward(self, dy, mem, dmem, set_dmem=False):
        """Returns dx; dmem ([n, tk, 2c]) accumulates (set_dmem: is
        written, what a zeroed dmem would receive)."""
        import torch
        n, t, c = self.n, self.tq, self.c
        do = self.proj.backward(dy.reshape(-1))
        dq = torch.empty(n * t * c, device=dy.device)
        self.core.backward(n, self.q, c, 0, mem, 2 * c, 0, c, self.tau.v, self.p, do, dq, dmem,
                           self.tau.g, self.rel.g, set_dq=True, set_dkv=set_dmem)
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
        # drawn ahead by draw_masks for the next forward: (mask, seed); used
        # only by a forward with that seed and batch
        self.premask = None

    def forward(self, x, train, seed):
        import torch
        if not train or self.p <= 0.0:
            self.mask = self.premask = None
            return x
        n = x.shape[0]
        pre = self._take_premask(n, seed)
        if pre is not None:
            # the draw of Rng::new(seed) already made by draw_masks
            self.mask = pre
            self.ctx.check(lib().rnn_drop_path_backward(self.ctx.h, n, x.numel() // n,
                                                        _ptr(x, x.numel(), "x"),
                                                        _ptr(self.mask, n, "mask")))
            return x
        self.premask = None
        self.mask = torch.empty(n, device=x.device)
        self.ctx.check(lib().rnn_drop_path_forward(self.ctx.h, n, x.numel() // n,
                                                   _ptr(x, x.numel(), "x"), self.p,
                                                   seed & 0xFFFFFFFFFFFFFFFF,
                                                   _ptr(self.mask, n, "mask")))
        return x

    def take_mask(self, n, train, seed, device):
        """This forward's mask without applying it (a fused consumer scales
        by it): the one draw_masks made ahead, else a fresh draw of
        Rng::new(seed); None in eval or when p is 0."""
        import ctypes as C

        import torch
        if not train or self.p <= 0.0:
            self.mask = self.premask = None
            return None
        pre = self._take_premask(n, seed)
        if pre is not None:
            self.mask = pre
            return self.mask
        self.mask = torch.empty(n, device=device)
        self.ctx.check(lib().rnn_drop_path_masks(
            self.ctx.h, 1, n, (C.c_float * 1)(self.p),
            (C.c_uint64 * 1)(seed & 0xFFFFFFFFFFFFFFFF), (C.c_void_p * 1)(self.mask.data_ptr())))
        return self.mask

    def _take_premask(self, n, seed):
        """The mask draw_masks drew ahead, when it was drawn for this seed
        and batch size; it is dropped either way."""
        pre, self.premask = self.premask, None
        if pre is None:
            return None
        m, s = pre
        if s != seed & 0xFFFFFFFFFFFFFFFF or m.numel() != n:
            return None
        return m

    def backward(self, dy):
        if self.mask is None:
            return dy
        n = dy.shape[0]
        self.ctx.check(lib().rnn_drop_path_backward(self.ctx.h, n, dy.numel() // n,
                                                    _ptr(dy, dy.numel(), "dy"),
                                                    _ptr(self.mask, n, "mask")))
        return dy


def draw_masks(layers, n, device, ctx):
    """DropPath::forward's draws (vit.rs:44-51) of several layers in one
    launch: ``layers`` lists (DropPath, seed); every layer with p > 0 gets
    the mask of Rng::new(seed) over n images for its next forward."""
    import ctypes as C

    import torch
    act = [(dp, s) for dp, s in layers if dp.p > 0.0]
    if not act:
        return
    masks = [torch.empty(n, device=device) for _ in act]
    k = len(act)
    p = (C.c_float * k)(*[dp.p for dp, _ in act])
    seeds = (C.c_uint64 * k)(*[s & 0xFFFFFFFFFFFFFFFF for _, s in act])
    ptrs = (C.c_void_p * k)(*[m.data_ptr() for m in masks])
    ctx.check(lib().rnn_drop_path_masks(ctx.h, k, n, p, seeds, ptrs))
    for (dp, s), m in zip(act, masks):
        dp.premask = (m, s & 0xFFFFFFFFFFFFFFFF)


class Block:
    """Block (vit.rs:76-250), pre-LN with three branches from one norm:
    h = LN(x); x += ls1 * dp1(SelfAttn(h) + gamma * DwConv3(h));
    x += lsm * dp2(CrossAttn(h, mem)) (reader blocks); x += ls2 * dp3(SwiGlu(LN(x)))."""

    def __init__(self, c, h, th, tw, mem, depth, drop, idx, ls_init, rng=None, device=0,
                 ctx=None):
        """Block::new (vit.rs:117-143): draws, in order, SelfAttn (qkv, proj),
        DwConv3, CrossAttn (wq, proj) for a reader block, SwiGlu (wg, wd)."""
        import torch
        dev = f"cuda:{device}"
        self.ctx = ctx or default_ctx(device)
        rng = _rng(rng, int(idx))
        self.c, self.idx = c, int(idx)
        hidden = -(-(4 * c // 3) // 16) * 16
        self.n1 = LayerNorm(c, device, self.ctx)
        self.attn = SelfAttn(c, h, th, tw, depth, rng, device, self.ctx)
        self.dw = DwConv3(c, th, tw, _trunc_normal(9 * c, 0.1, rng, dev), None, device, self.ctx)
        self.gamma = Param(torch.full((c,), 0.5, device=dev), False)
        self.ls1 = LayerScale(c, ls_init, device, self.ctx)
        self.cross = (CrossAttn(c, h, th, tw, mem[0], mem[1], depth, rng, device, self.ctx)
                      if mem else None)
        self.lsm = LayerScale(c, ls_init, device, self.ctx) if mem else None
        self.n2 = LayerNorm(c, device, self.ctx)
        wg = _trunc_normal(2 * hidden * c, 0.02, rng, dev)
        wd = _trunc_normal(hidden * c, _scaled_std(depth), rng, dev)
        self.mlp = SwiGlu(c, hidden, wg, None, wd, None, device, self.ctx)
        self.ls2 = LayerScale(c, ls_init, device, self.ctx)
        self.dp1, self.dp2, self.dp3 = (DropPath(drop, self.ctx), DropPath(drop, self.ctx),
                                        DropPath(drop, self.ctx))
        self.dwo = None

    def drop_layers(self, seed):
        """(DropPath, seed) of this block's branches as forward draws them."""
        out = [(self.dp1, seed ^ self.idx)]
        if self.cross is not None:
            out.append((self.dp2, seed ^ self.idx ^ 0x5151))
        return out + [(self.dp3, seed ^ self.idx ^ 0xA2A2)]

    def forward(self, x, mem, train, seed):
        import torch
        L, ctx, c = lib(), self.ctx, self.c
        h = self.n1.forward(x, train)
        a = self.attn.forward(h, train)
        # a += gamma * DwConv3(h); y = x + dp1(ls1(a)) in one pass, then the
        # other branches added in place, each in one pass (vit.rs:150-176)
        mask = self.dp1.take_mask(x.shape[0], train, seed ^ self.idx, x.device)
        y = torch.empty_like(x)
        d = self.dw.forward_branch(h, a, self.gamma.v, x, self.ls1.l.v, mask, y, train)
        if train:
            self.dwo = d
            self.ls1.x = a
        n = x.shape[0]
        if self.cross is not None:
            if mem is None:
                raise ValueError("Block: a reader block needs the memory")
            # y += dp2(lsm(CrossAttn(h, mem))) in the projection's epilogue
            mask = self.dp2.take_mask(n, train, seed ^ self.idx ^ 0x5151, x.device)
            cm = self.cross.forward(h, mem, train, (y, self.lsm.l.v, mask))
            if train:
                self.lsm.x = cm
        h2 = self.n2.forward(y, train)
        # y += dp3(ls2(SwiGlu(h2))) in the down projection's epilogue
        mask = self.dp3.take_mask(n, train, seed ^ self.idx ^ 0xA2A2, x.device)
        m = self.mlp.forward(h2, train, (y, self.ls2.l.v, mask, h2.numel() // (n * self.c)))
        if train:
            self.ls2.x = m
        return y

    def backward(self, dz, mem=None, dmem=None, set_dmem=False):
        """Returns dx; dmem accumulates the memory's gradient (vit.rs:175-249)
        -- set_dmem: is written, as a zeroed dmem would be."""
        return self.backward_fused(dz, mem, dmem, set_dmem)[0]

    def backward_fused(self, dz, mem=None, dmem=None, set_dmem=False, dm=None, nxt=None):
        """Block::backward with the seams between blocks fused: ``dm`` is this
        block's ls2 input gradient when the previous call already computed it
        (else ls2's backward runs here), and with ``nxt`` (the block whose
        backward follows) its ls2 backward runs in this block's last
        LayerNorm pass.  Returns (dx, nxt's ls2 input gradient or None)."""
        import torch
        L, ctx, c = lib(), self.ctx, self.c
        # each branch's DropPath + LayerScale backward reads dz / dy unchanged
        if dm is None:
            dm = self.ls2.backward(dz, self.dp3.mask)
        dh2 = self.mlp.backward(dm)
        dy = self.n2.backward(dh2, add=dz)  # n2's input gradient + dz, a new tensor
        # the first residual's branch gradients in one pass over dy: dc =
        # lsm's DropPath + LayerScale backward (reader blocks), da = ls1's,
        # ddw = gamma * da with gamma.g += sum da * dwo
        rows = dy.numel() // c
        cross = self.cross is not None
        m1, m2 = self.dp1.mask, (self.dp2.mask if cross else None)
        nimg = next((m.numel() for m in (m1, m2) if m is not None), 1)
        da, ddw = torch.empty_like(dy), torch.empty_like(dy)
        dc, cm, lm, dlm = ((torch.empty_like(dy), self.lsm.x, self.lsm.l.v, self.lsm.l.g)
                           if cross else (None, None, None, None))
        ctx.check(L.rnn_block_branch_backward(
            ctx.h, rows, c, _ptr(dy, rows * c, "dy"), _ptr(self.ls1.x, rows * c, "a"),
            _ptr(self.ls1.l.v, c, "l1"), _ptr(m1, nimg, "m1"), _ptr(self.dwo, rows * c, "dwo"),
            _ptr(self.gamma.v, c, "gamma"), _ptr(cm, rows * c, "cm"), _ptr(lm, c, "lm"),
            _ptr(m2, nimg, "m2"), rows // nimg, _ptr(da, rows * c, "da"),
            _ptr(self.ls1.l.g, c, "dl1"), _ptr(ddw, rows * c, "ddw"),
            _ptr(self.gamma.g, c, "dgamma"), _ptr(dc, rows * c, "dc"), _ptr(dlm, c, "dlm")))
        dh = self.cross.backward(dc, mem, dmem, set_dmem) if cross else None
        # the branches' input gradients summed in branch order, each added by
        # the kernel that computes it
        dh = self.attn.backward(da, acc_dx=dh)
        self.dw.backward(ddw, acc_dx=dh)
        if nxt is None:
            self.n1.backward(dh, add=dy, out=dy)  # dy += n1's input gradient
            return dy, None
        # dy += n1's input gradient, and the next block's ls2 backward of it
        _, dm_next = self.n1.backward(dh, add=dy, out=dy, ls=(nxt.ls2, nxt.dp3.mask))
        return dy, dm_next

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

    def __init__(self, c, parent, nc, rng=None, device=0, ctx=None):
        dev = f"cuda:{device}"
        self.ctx = ctx or default_ctx(device)
        rng = _rng(rng, 1)
        self.parent, self.nc, self.nf = parent, nc, parent.numel()
        self.coarse = _linear(c, nc, True, 0.02, rng, dev, self.ctx)
        self.resid = _linear(c, self.nf, True, 0.02, rng, dev, self.ctx)
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
        return self.coarse.backward(dc, acc_dx=df)  # df + the coarse Linear's dx

    def for_each_param(self, f):
        for p in self._params:
            f(p)


class Exit:
    """Exit (vit.rs:320-353): fc Linear(cin, nclass) and hint Linear(cin,
    chint, no bias) over the same feature."""

    def __init__(self, cin, nclass, chint, rng=None, device=0, ctx=None):
        dev = f"cuda:{device}"
        self.ctx = ctx or default_ctx(device)
        rng = _rng(rng, 2)
        self.fc = _linear(cin, nclass, True, 0.02, rng, dev, self.ctx)
        self.hint = _linear(cin, chint, False, 0.02, rng, dev, self.ctx)
        self._params = _linear_param(self.fc) + _linear_param(self.hint)
        self.n = 0

    def forward(self, f, n, train):
        self.n = n
        return (self.fc.forward(f.reshape(-1), n, train).view(n, -1),
                self.hint.forward(f.reshape(-1), n, train).view(n, -1))

    def backward(self, dz, dh):
        d = self.fc.backward(dz.reshape(-1))
        return self.hint.backward(dh.reshape(-1), acc_dx=d)  # d + the hint Linear's dx

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


# ------------------------------------------------------------------ the network
def _optim_param(v, g, decay):
    """An optim Param sharing an existing value / gradient pair."""
    import torch
    p = Param.__new__(Param)
    p.v, p.g = v, g
    p.m, p.v2 = torch.zeros_like(v), torch.zeros_like(v)
    p.decay, p.rows, p.cols = bool(decay), 0, 0
    return p


class _ConvBN:
    """Conv2d (nn.rs:115-250) followed by BatchNorm2d (nn.rs:253-428), NCHW."""

    def __init__(self, cin, cout, k, stride, pad, rng, dev, device, ctx, relu=False):
        from . import Conv2d
        from .nn import BatchNorm2d
        fan = cin * k * k
        w = _kaiming(fan, cout * fan, rng, dev)
        self.conv = Conv2d(cin, cout, k, stride, pad, w, device, ctx)
        self.bn = BatchNorm2d(cout, device, ctx)
        self.relu, self.cout, self.k, self.stride, self.pad = relu, cout, k, stride, pad
        self.wp = _optim_param(self.conv.w, self.conv.g, True)
        self.gp = _optim_param(self.bn.g.v, self.bn.g.g, False)
        self.bp = _optim_param(self.bn.b.v, self.bn.b.g, False)

    def out_hw(self, h, w):
        return ((h + 2 * self.pad - self.k) // self.stride + 1,
                (w + 2 * self.pad - self.k) // self.stride + 1)

    def forward(self, x, train):
        n, _, h, w = x.shape
        oh, ow = self.out_hw(h, w)
        y = self.conv.forward(x, n, h, w, train).view(n, self.cout, oh, ow)
        return self.bn.forward_relu(y, train) if self.relu else self.bn.forward(y, train)

    def backward(self, dy, relu_out=None):
        """dX; dW, dgamma, dbeta accumulate.  relu_out folds relu_back in."""
        n, _, h, w = self.conv.xshape[0], 0, self.conv.xshape[1], self.conv.xshape[2]
        d = self.bn.backward(dy, relu_out)
        return self.conv.backward(d).view(n, -1, h, w)

    def params(self):
        return [self.wp, self.gp, self.bp]


class BasicBlock:
    """BasicBlock (model.rs:10-107): conv-BN-ReLU, conv-BN (gamma 0), a 1x1
    conv-BN shortcut when the shape changes, add + ReLU."""

    def __init__(self, cin, cout, stride, rng, dev, device, ctx):
        """BasicBlock::new (model.rs:20-39): draws c1, c2, then the shortcut."""
        self.ctx = ctx
        self.a = _ConvBN(cin, cout, 3, stride, 1, rng, dev, device, ctx, relu=True)
        self.b = _ConvBN(cout, cout, 3, 1, 1, rng, dev, device, ctx)
        self.b.bn.zero_gamma()
        self.down = (_ConvBN(cin, cout, 1, stride, 0, rng, dev, device, ctx)
                     if stride != 1 or cin != cout else None)
        self.h1 = self.out = None

    def forward(self, x, train):
        from .nn import add_relu_
        h = self.a.forward(x, train)
        y = self.b.forward(h, train)
        add_relu_(y, self.down.forward(x, train) if self.down else x, self.ctx)
        if train:
            self.h1, self.out = h, y
        return y

    def backward(self, d):
        """BasicBlock::backward (model.rs:56-71).  relu_back_ of d by the
        block's output is taken by the kernels that read d (the second BN's
        and the shortcut's backward, or the shortcut's add), so d itself is
        left unchanged."""
        from .nn import add_, add_relu_back_
        dmain = self.b.backward(d, self.out)
        dx = self.a.backward(dmain, self.h1)
        if self.down:
            add_(dx, self.down.backward(d, self.out), self.ctx)
        else:
            add_relu_back_(dx, d, self.out, self.ctx)
        return dx

    def params(self):
        ps = self.a.params() + self.b.params()
        return ps + (self.down.params() if self.down else [])


VIT_DEFAULT = dict(width=32, cmid=96, dim=256, heads=4, depth3=5, dim4=384, heads4=6, depth4=2,
                   mem_at=(1, 3), droppath=0.1, img=32)


class RustViT:
    """RustViT (vit.rs:400-757): convolutional trunk (stem, two BasicBlocks),
    a 16x16 memory of 2*dim channels (1x1 conv + LayerNorm), 8x8 tokens
    (3x3/s2 conv + BN), depth3 Blocks (cross-attention readers at mem_at), a
    2x2 token merge to dim4, depth4 Blocks, LayerNorm + SeqPool + TaxoHead,
    and two exits (GAP of the trunk; SeqPool of the stage-3 tokens).  parent:
    the superclass of each fine class (CUDA int32); seed seeds the weights."""

    def __init__(self, cfg=None, parent=None, ncoarse=20, seed=0, device=0, ctx=None):
        """RustViT::new (vit.rs:432-507): one Rng::new(seed) drawn in the
        reference's order -- the stage-3 blocks, the stage-4 blocks, then the
        stem, c1, c2, the memory conv, the token conv, the merge Linear, the
        pool, the head, exit 1, pool2 and exit 2 -- so the weights equal the
        reference's bit for bit."""
        import torch
        cfg = dict(VIT_DEFAULT, **(cfg or {}))
        dev = f"cuda:{device}"
        self.cfg, self.ctx = cfg, ctx or default_ctx(device)
        rng = Rng(int(seed))
        w, cm, d, d4 = cfg["width"], cfg["cmid"], cfg["dim"], cfg["dim4"]
        self.mh, self.th = cfg["img"] // 2, cfg["img"] // 4
        depth = cfg["depth3"] + cfg["depth4"]
        nf = parent.numel()
        self.nclass, ctx = nf, self.ctx
        self.parent_host = [int(v) for v in parent.cpu().tolist()]  # the checkpoint hash
        # DropPath rate cfg.droppath * i / (max(depth, 2) - 1), in f32
        div = np.float32(max(depth, 2) - 1)
        rate = lambda i: float(np.float32(cfg["droppath"]) * np.float32(i) / div)
        self.blocks3 = [Block(d, cfg["heads"], self.th, self.th,
                              (self.mh, self.mh) if i in cfg["mem_at"] else None, depth,
                              rate(i), i + 1, 1e-4, rng, device, ctx)
                        for i in range(cfg["depth3"])]
        th4 = self.th // 2
        self.blocks4 = [Block(d4, cfg["heads4"], th4, th4, None, depth,
                              rate(cfg["depth3"] + i), cfg["depth3"] + i + 1, 1e-4, rng, device,
                              ctx)
                        for i in range(cfg["depth4"])]
        self.stem = _ConvBN(3, w, 3, 1, 1, rng, dev, device, ctx, relu=True)
        self.c1 = BasicBlock(w, w, 1, rng, dev, device, ctx)
        self.c2 = BasicBlock(w, cm, 2, rng, dev, device, ctx)
        from . import Conv2d
        self.memconv = Conv2d(cm, 2 * d, 1, 1, 0, _kaiming(cm, 2 * d * cm, rng, dev), device, ctx)
        self.memln = LayerNorm(2 * d, device, ctx)
        self.tok = _ConvBN(cm, d, 3, 2, 1, rng, dev, device, ctx)
        self.mergeln = LayerNorm(4 * d, device, ctx)
        self.merge = _linear(4 * d, d4, True, 0.02, rng, dev, ctx)
        self.headln = LayerNorm(d4, device, ctx)
        self.pool = SeqPool(d4, _trunc_normal(d4, 0.02, rng, dev), device, ctx)
        self.head = TaxoHead(d4, parent, ncoarse, rng, device, ctx)
        self.e1 = Exit(cm, nf, d4, rng, device, ctx)
        self.pool2 = SeqPool(d, _trunc_normal(d, 0.02, rng, dev), device, ctx)
        self.e2 = Exit(d, nf, d4, rng, device, ctx)
        self.memw = _optim_param(self.memconv.w, self.memconv.g, True)
        self.mergep = _linear_param(self.merge)
        self.use_exits, self.drop_seed = True, 0
        self.mem = self.c2_out = self.stem_out = self.mem_in = None
        self.n = 0
        self._packs = None

    def _trunk_convs(self):
        """(Conv2d, h, w) of every convolution of the trunk at its input size."""
        s = self.cfg["img"]
        out = [(self.stem.conv, s, s)]
        for b in (self.c1, self.c2):
            out += [(b.a.conv, s, s)]
            if b.down:
                out += [(b.down.conv, s, s)]
            s = b.a.out_hw(s, s)[0]
            out += [(b.b.conv, s, s)]
        return out + [(self.tok.conv, self.mh, self.mh)]

    def _repack(self):
        """The trunk's packed weights from the current ones: one launch per
        forward (the optimiser, EMA or a checkpoint may have changed them)."""
        from . import ConvPacks
        if self._packs is None:
            self._packs = ConvPacks(self._trunk_convs(), self.ctx)
        else:
            self._packs.update()

    def forward(self, x, train):
        """RustViT::forward (vit.rs:510-609): dict with logits, coarse and, in
        training with exits, e1, e2, h1, h2; feat (the pooled feature)."""
        from .nn import gap_forward
        n, cfg, d = x.shape[0], self.cfg, self.cfg["dim"]
        self._repack()
        h = self.stem.forward(x, train)
        if train:
            self.stem_out = h
        h = self.c1.forward(h, train)
        h = self.c2.forward(h, train)
        if train:
            self.c2_out = h
        mh = self.mh
        # the memory's 1x1 conv as the product it is, on the trunk's tokens:
        # [n*mh*mh, cm] x W^T with W = [2d][cm] (the conv's weights)
        cm = self.cfg["cmid"]
        ht = nchw_to_tokens(h, self.ctx)
        memt = linear_forward(n * mh * mh, cm, 2 * d, ht, self.memconv.w, None,
                              ctx=self.ctx).view(n, mh * mh, 2 * d)
        if train:
            self.mem_in = ht
        mem = self.memln.forward(memt, train)
        z = nchw_to_tokens(self.tok.forward(h, train), self.ctx)
        seed = self.drop_seed
        if train:
            # every block's DropPath masks in one launch
            draw_masks([lay for b in self.blocks3 + self.blocks4 for lay in b.drop_layers(seed)],
                       n, x.device, self.ctx)
        for b in self.blocks3:
            z = b.forward(z, mem, train, seed)
        if train:
            self.mem = mem
        out = {}
        if self.use_exits and train:
            f = self.pool2.forward(z, train)
            out["e2"], out["h2"] = self.e2.forward(f, n, train)
        z = token_merge(z, self.th, self.ctx)
        zn = self.mergeln.forward(z, train)
        t4 = zn.shape[1]
        z4 = self.merge.forward(zn.reshape(-1), n * t4, train).view(n, t4, cfg["dim4"])
        for b in self.blocks4:
            z4 = b.forward(z4, None, train, seed)
        zf = self.headln.forward(z4, train)
        feat = self.pool.forward(zf, train)
        out["logits"], out["coarse"] = self.head.forward(feat, n, train)
        out["feat"] = feat
        if self.use_exits and train:
            g = gap_forward(self.c2_out, self.ctx)
            out["e1"], out["h1"] = self.e1.forward(g, n, train)
        self.n = n
        return out

    def backward(self, g):
        """RustViT::backward (vit.rs:628-688) from the output gradients
        (logits, coarse; e1, e2, h1, h2 with exits; hfinal optional)."""
        import torch
        from .nn import add_, gap_backward
        ctx, n, d, cm = self.ctx, self.n, self.cfg["dim"], self.cfg["cmid"]
        dfeat = self.head.backward(g["logits"], g["coarse"])
        if g.get("hfinal") is not None:
            add_(dfeat, g["hfinal"], ctx)
        dzf = self.pool.backward(dfeat)
        dz4 = self.headln.backward(dzf)
        # each block's last LayerNorm pass also runs the next one's ls2
        # backward (Block.backward_fused)
        order, dm = self.blocks4[::-1], None
        for i, b in enumerate(order):
            dz4, dm = b.backward_fused(dz4, dm=dm, nxt=order[i + 1] if i + 1 < len(order) else None)
        t4 = dz4.shape[1]
        dmg = self.merge.backward(dz4.reshape(-1)).view(n, t4, 4 * d)
        dzn = self.mergeln.backward(dmg)
        dz = token_merge_back(dzn, self.th, d, ctx)
        if self.use_exits and g.get("e2") is not None:
            df2 = self.e2.backward(g["e2"], g["h2"])
            add_(dz, self.pool2.backward(df2.view(n, d)), ctx)
        # the memory's gradient: the last reader block (the first in the
        # backward) writes it, the others add to it -- what the reference's
        # zeroed dmem receives (vit.rs:652-655)
        dmem = torch.empty_like(self.mem)
        first = True
        order, dm = self.blocks3[::-1], None
        for i, b in enumerate(order):
            dz, dm = b.backward_fused(dz, self.mem, dmem, first and b.cross is not None, dm,
                                      order[i + 1] if i + 1 < len(order) else None)
            first = first and b.cross is None
        if first:
            dmem.zero_()  # no reader block
        dt = tokens_to_nchw(dz, self.th, self.th, ctx)
        dc2 = self.tok.backward(dt)
        mh = self.mh
        dmemn = self.memln.backward(dmem)
        dht = linear_backward(n * mh * mh, cm, 2 * d, dmemn, self.mem_in, self.memconv.w,
                              self.memconv.g, ctx=ctx)
        add_(dc2, tokens_to_nchw(dht.view(n, mh * mh, cm), mh, mh, ctx), ctx)
        if self.use_exits and g.get("e1") is not None:
            dgv = self.e1.backward(g["e1"], g["h1"])
            add_(dc2, gap_backward(dgv.view(n, cm), mh, mh, ctx), ctx)
        dh = self.c2.backward(dc2)
        dh = self.c1.backward(dh)
        dh = self.stem.bn.backward(dh, self.stem_out)  # relu_back_ folded in
        self.stem.conv.backward_w(dh)

    def for_each_param(self, f):
        """RustViT::for_each_param (vit.rs:690-716)."""
        for p in self.stem.params() + self.c1.params() + self.c2.params():
            f(p)
        f(self.memw)
        self.memln.for_each_param(f)
        for p in self.tok.params():
            f(p)
        for b in self.blocks3:
            b.for_each_param(f)
        self.mergeln.for_each_param(f)
        for p in self.mergep:
            f(p)
        for b in self.blocks4:
            b.for_each_param(f)
        self.headln.for_each_param(f)
        self.pool.for_each_param(f)
        self.head.for_each_param(f)
        if self.use_exits:
            self.e1.for_each_param(f)
            self.pool2.for_each_param(f)
            self.e2.for_each_param(f)

    def params(self):
        ps = []
        self.for_each_param(ps.append)
        return ps


# Config defaults of the rustvit trainer (cli.rs:62-120): loss weights, clip,
# EMA, the optimiser and the learning-rate schedule's budget (ntrain images,
# epochs and warm-up epochs at this batch size).
VIT_TRAIN = dict(smooth=0.1, sib=0.7, coarse_w=0.4, exit_w=(0.3, 0.6), alpha=1.0, temp=3.0,
                 beta=0.03, clip=1.0, ema=0.9998, ema_auto=True, lr=6e-4, lr_min=1e-5, wd=0.06,
                 muon=True, ns=3, no_taxo=False, seed=1234, batch=128, ntrain=50000, epochs=100,
                 warmup=10)


def lr_at(peak, lo, step, total, warm):
    """lr_at (train.rs:21-28), in f32 (rnn_lr_at): linear warm-up, then a
    cosine down to lo."""
    return float(lib().rnn_lr_at(float(np.float32(peak)), float(np.float32(lo)), int(step),
                                 int(total), int(warm)))


class ViTStep:
    """Trainer::step of the rustvit (train.rs:346-387) on the device, from an
    assembled batch: the soft targets of the (possibly mixed) batch and its
    dominant labels (train.rs:121-155, 313-320), DropPath's seed drawn from
    the trainer's generator, forward, build_loss (train.rs:70-118: the fine
    soft-target CE, the coarse CE when coarse_w > 0 and the taxonomy is on,
    the exits' CE, their distillation KL against the final logits and the
    hint MSE to the pooled feature), backward, lr_at, clip_,
    Optim::step_all and the EMA; the step counter advances.

    The trainer's generator is ``self.rng`` = Rng::new(seed ^ 0xABCD)
    (train.rs:260).  A caller that assembles batches as Trainer::make_batch
    does draws the batch seed and the mix plan from it before calling (data
    module: ``make_batch_train(.., seed=step.rng.next_u64())``,
    ``mix_batch(.., step.rng)``) and passes perm and lam; without them the
    batch counts as unmixed.  The losses stay on the device."""

    def __init__(self, net, parent, ncoarse, hp=None):
        from .optim import Ema, Optim
        self.net, self.parent, self.nc = net, parent, ncoarse
        self.hp = hp = dict(VIT_TRAIN, **(hp or {}))
        self.params = net.params()
        self.opt = Optim(hp["muon"], hp["ns"], ctx=net.ctx)
        self.rng = Rng(int(hp["seed"]) ^ 0xABCD)
        # Trainer::new (train.rs:241-259): the schedule's budget and the EMA
        # decay that keeps its window at a tenth of the run
        self.steps_per_epoch = hp["ntrain"] // hp["batch"]
        self.total_steps = self.steps_per_epoch * hp["epochs"]
        self.warm_steps = self.steps_per_epoch * hp["warmup"]
        f = np.float32
        d = f(hp["ema"])
        if hp["ema_auto"] and self.total_steps > 0:
            d = min(f(1.0) - f(10.0) / f(self.total_steps), d)
        self.ema_decay = float(d)
        self.ema = Ema(d, ctx=net.ctx) if d > 0 else None
        self.step = 0
        self.norm = None
        self.lr = None
        # the backward's parameter-gradient reductions queued and run in one
        # launch at its end (rnn_ctx_set_defer; bit-identical results)
        self.defer = True

    def __call__(self, x, labels, coarse, perm=None, lam=None, lr=None, wd=None):
        """One step; returns (total loss, hits against the dominant labels)
        as device tensors.  lr / wd override the schedule and hp["wd"]."""
        total, correct, _ = self.forward_backward(x, labels, coarse, perm, lam)
        self.update(lr, wd)
        return total, correct

    def forward_backward(self, x, labels, coarse, perm=None, lam=None):
        """The first half of Trainer::step (train.rs:348-362): targets, the
        DropPath seed, forward, build_loss, backward (gradients accumulate in
        the parameters).  Returns (total, correct, the output dict)."""
        from .loss import mix_dominant, soft_targets
        hp, net, ctx = self.hp, self.net, self.net.ctx
        nf, n = net.nclass, labels.numel()
        taxo = not hp["no_taxo"]
        tf, tc = soft_targets(labels, nf, hp["smooth"], self.parent if taxo else None,
                              hp["sib"], coarse, self.nc, perm, lam, ctx=ctx)
        dom = labels if perm is None else mix_dominant(labels, perm, lam, ctx=ctx)
        net.drop_seed = self.rng.next_u64()
        if self.defer:
            ctx.set_defer(True)
        try:
            return self._forward_backward(x, labels, coarse, tf, tc, dom, n, taxo)
        finally:
            if self.defer:
                ctx.set_defer(False)  # flushes: every gradient complete

    def _forward_backward(self, x, labels, coarse, tf, tc, dom, n, taxo):
        from .loss import build_loss
        hp, net, ctx = self.hp, self.net, self.net.ctx
        out = net.forward(x, True)
        # build_loss (train.rs:70-118) in one library call: every loss term,
        # the gradients written, the total in the reference's order and
        # grouping (f32)
        g, total, _, correct = build_loss(out, tf, tc if taxo else None, dom,
                                          coarse if taxo else None, net.nclass, self.nc, hp,
                                          ctx=ctx)
        net.backward(g)
        return total, correct, out

    def update(self, lr=None, wd=None):
        """The second half of Trainer::step (train.rs:364-386): lr_at,
        clip_, Optim::step_all, the EMA; the step counter advances."""
        import torch
        from .optim import clip_
        hp, ctx = self.hp, self.net.ctx
        if lr is None:
            lr = lr_at(hp["lr"], hp["lr_min"], self.step, self.total_steps, self.warm_steps)
        self.lr = lr
        if self.norm is None:
            self.norm = torch.zeros(1, device=self.params[0].v.device)
        if hp["clip"] > 0:
            clip_(self.params, hp["clip"], ctx=ctx, norm=self.norm)
        self.opt.step_all(self.params, lr, hp["wd"] if wd is None else wd)
        if self.ema is not None:
            self.ema.update(self.params)
        self.step += 1


FNV_OFFSET = 0xCBF29CE484222325


def fingerprint(step, last_loss):
    """Trainer::fingerprint (train.rs:444-470): FNV-1a over every parameter's
    value, momentum and (for the tensors AdamW has updated) second moment in
    for_each_param order, then the EMA weights, the step count as 8
    little-endian bytes and the last loss.  The state is copied to the host
    and hashed there."""
    import ctypes as C
    import struct

    import numpy as np
    L = lib()

    def fold(h, t):
        a = np.ascontiguousarray(t.detach().cpu().numpy(), np.float32)
        return int(L.rnn_fnv1a_f32(C.c_uint64(h), a.ctypes.data, a.size))

    h = FNV_OFFSET
    opt = step.opt
    for p in step.params:
        adam = not (opt.muon and p.rows > 0 and min(p.rows, p.cols) > 1)
        h = fold(h, p.v)
        h = fold(h, p.m)
        if adam and opt.t > 0:  # v2 exists once AdamW has stepped (optim.rs:208-210)
            h = fold(h, p.v2)
    if step.ema is not None and step.ema.ready:
        for w in step.ema.w:
            h = fold(h, w)
    tb = struct.pack("<Q", int(opt.t))
    h = int(L.rnn_fnv1a_bytes(C.c_uint64(h), C.c_char_p(tb), 8))
    lb = np.array([float(last_loss)], np.float32)
    return int(L.rnn_fnv1a_f32(C.c_uint64(h), lb.ctypes.data, 1))
