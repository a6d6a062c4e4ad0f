"""An independent float64 statement of the reference rustvit network in
torch (CPU autograd), for the parity tests of the oracle and of the device
network.

Written from the reference's definitions, not from either implementation
under test: vit.rs:510-609 (RustViT::forward), the pre-LN Block
(vit.rs:145-173), SelfAttn / CrossAttn / Core (attn.rs:143-223, 387-530),
LayerNorm / LayerScale / SwiGLU / DwConv3 / SeqPool (norm.rs), the conv
trunk (model.rs BasicBlock, nn.rs Conv2d and BatchNorm2d in training mode)
and TaxoHead / Exit (vit.rs:282-345).  DropPath uses the per-image factors
the reference draws from Rng::new(seed) (passed in as `masks`).

``RustViTF64(cfg, nclass, ncoarse, parent)`` consumes a flat list of
parameter arrays in the reference's for_each_param order (vit.rs:690-716),
so the same list read from the oracle or from the device builds it;
``forward(x, masks)`` returns the outputs as a dict like the reference's
``Out``; gradients come from torch autograd.
"""
from __future__ import annotations

import numpy as np
import torch

F = torch.nn.functional
D = torch.float64


def rel_index(th, tw, mh, mw):
    """rel_index (attn.rs:53-72) and the bias-table length."""
    if mh == th:
        sy, sx, s, oy, ox = 2 * th - 1, 2 * tw - 1, 1, th - 1, tw - 1
    else:
        sy, sx, s, oy, ox = 2 * (th - 1) + mh, 2 * (tw - 1) + mw, 2, mh - 1, mw - 1
    idx = [(s * qy - my + oy) * sx + (s * qx - mx + ox)
           for qy in range(th) for qx in range(tw) for my in range(mh) for mx in range(mw)]
    return torch.tensor(idx, dtype=torch.long).view(th * tw, mh * mw), sy * sx


class _Params:
    """Hands out the parameters in for_each_param order."""

    def __init__(self, arrays):
        self.t = [torch.tensor(np.asarray(a, np.float64).ravel(), dtype=D, requires_grad=True)
                  for a in arrays]
        self.i = 0

    def take(self, n):
        p = self.t[self.i]
        assert p.numel() == n, (self.i, p.numel(), n)
        self.i += 1
        return p


def _bn(x, g, b):
    """BatchNorm2d in training mode (nn.rs:297-348): batch mean and biased
    variance over (n, h, w), eps 1e-5."""
    m = x.mean(dim=(0, 2, 3), keepdim=True)
    v = ((x - m) ** 2).mean(dim=(0, 2, 3), keepdim=True)
    return (x - m) / torch.sqrt(v + 1e-5) * g.view(1, -1, 1, 1) + b.view(1, -1, 1, 1)


def _ln(x, g, b):
    return F.layer_norm(x, (x.shape[-1],), g, b, 1e-5)


class _Conv:
    def __init__(self, P, cin, cout, k, s, p):
        self.w = P.take(cout * cin * k * k).view(cout, cin, k, k)
        self.s, self.p = s, p

    def __call__(self, x):
        return F.conv2d(x, self.w, stride=self.s, padding=self.p)


class _ConvBN:
    def __init__(self, P, cin, cout, k, s, p):
        self.conv = _Conv(P, cin, cout, k, s, p)
        self.g, self.b = P.take(cout), P.take(cout)

    def __call__(self, x):
        return _bn(self.conv(x), self.g, self.b)


class _BasicBlock:
    """model.rs:41-56: conv-BN-ReLU, conv-BN, shortcut, add + ReLU."""

    def __init__(self, P, cin, cout, stride):
        self.a = _ConvBN(P, cin, cout, 3, stride, 1)
        self.b = _ConvBN(P, cout, cout, 3, 1, 1)
        self.down = _ConvBN(P, cin, cout, 1, stride, 0) if stride != 1 or cin != cout else None

    def __call__(self, x):
        y = self.b(torch.relu(self.a(x)))
        return torch.relu(y + (self.down(x) if self.down else x))


class _Linear:
    def __init__(self, P, fin, fout, bias=True):
        self.w = P.take(fin * fout).view(fout, fin)
        self.b = P.take(fout) if bias else None

    def __call__(self, x):
        y = x @ self.w.T
        return y + self.b if self.b is not None else y


def _core(q, k, v, tau, rel, relidx, nrel, h, mask):
    """Core::forward (attn.rs:174-223): softmax(tau QK^T + rel[idx]) V per
    head, the diagonal masked when `mask`.  q [n, tq, c], k / v [n, tk, c]."""
    n, tq, c = q.shape
    tk, dh = k.shape[1], c // h
    qh = q.reshape(n, tq, h, dh).permute(0, 2, 1, 3)
    kh = k.reshape(n, tk, h, dh).permute(0, 2, 1, 3)
    vh = v.reshape(n, tk, h, dh).permute(0, 2, 1, 3)
    s = qh @ kh.transpose(-1, -2)
    x = tau.view(1, h, 1, 1) * s + rel.view(h, nrel)[:, relidx].unsqueeze(0)
    if mask:
        x = x.masked_fill(torch.eye(tq, tk, dtype=torch.bool), float("-inf"))
    o = torch.softmax(x, -1) @ vh
    return o.permute(0, 2, 1, 3).reshape(n, tq, c)


class _Block:
    """Block (vit.rs:76-173)."""

    def __init__(self, P, c, h, th, mh, depth_unused=None):
        self.c, self.h, self.th, self.mh = c, h, th, mh
        hidden = -(-(4 * c // 3) // 16) * 16
        t = th * th
        self.n1 = (P.take(c), P.take(c))
        self.qkv, self.proj = _Linear(P, c, 3 * c), _Linear(P, c, c)
        self.tau, self.rel = P.take(h), None
        self.relidx, nrel = rel_index(th, th, th, th)
        self.nrel = nrel
        self.rel = P.take(h * nrel)
        self.dw_w, self.dw_b = P.take(9 * c), P.take(c)
        self.gamma = P.take(c)
        self.ls1 = P.take(c)
        if mh:
            self.wq, self.cproj = _Linear(P, c, c), _Linear(P, c, c)
            self.ctau = P.take(h)
            self.crelidx, self.cnrel = rel_index(th, th, mh, mh)
            self.crel = P.take(h * self.cnrel)
            self.lsm = P.take(c)
        self.n2 = (P.take(c), P.take(c))
        self.wg, self.wd = _Linear(P, c, 2 * hidden), _Linear(P, hidden, c)
        self.ls2 = P.take(c)
        assert t > 0

    def __call__(self, x, mem, masks):
        """masks: (dp1, dp2, dp3) per-image factors or None (DropPath off)."""
        c, h, th = self.c, self.h, self.th
        n, t = x.shape[0], th * th
        mk = lambda i: (1.0 if masks is None or masks[i] is None else
                        torch.tensor(np.asarray(masks[i], np.float64), dtype=D).view(n, 1, 1))
        hh = _ln(x, *self.n1)
        ab = self.qkv(hh)
        sa = self.proj(_core(ab[..., :c], ab[..., c:2 * c], ab[..., 2 * c:], self.tau, self.rel,
                             self.relidx, self.nrel, h, True))
        hi = hh.reshape(n, th, th, c).permute(0, 3, 1, 2)
        wdw = self.dw_w.view(3, 3, c).permute(2, 0, 1).reshape(c, 1, 3, 3)
        dw = F.conv2d(hi, wdw, self.dw_b, padding=1, groups=c).permute(0, 2, 3, 1).reshape(n, t, c)
        y = x + mk(0) * (self.ls1 * (sa + self.gamma * dw))
        if self.mh:
            ca = self.cproj(_core(self.wq(hh), mem[..., :c], mem[..., c:], self.ctau, self.crel,
                                  self.crelidx, self.cnrel, h, False))
            y = y + mk(1) * (self.lsm * ca)
        g2 = self.wg(_ln(y, *self.n2))
        hid = g2.shape[-1] // 2
        m = self.wd(F.silu(g2[..., :hid]) * g2[..., hid:])
        return y + mk(2) * (self.ls2 * m)


def _seqpool(x, p):
    """SeqPool::forward (norm.rs:487-528)."""
    w = torch.softmax(x @ p, dim=1)
    return (w.unsqueeze(-1) * x).sum(dim=1)


def _tokens(x):
    n, c = x.shape[0], x.shape[1]
    return x.reshape(n, c, -1).permute(0, 2, 1)


class RustViTF64:
    """RustViT (vit.rs:400-609) in float64 over parameters given in
    for_each_param order."""

    def __init__(self, cfg, nclass, ncoarse, parent, arrays):
        P = _Params(arrays)
        self.params = P.t
        self.cfg, self.parent = cfg, torch.tensor(np.asarray(parent, np.int64))
        w, cm, d, d4 = cfg["width"], cfg["cmid"], cfg["dim"], cfg["dim4"]
        self.mh, self.th = cfg["img"] // 2, cfg["img"] // 4
        self.stem = _ConvBN(P, 3, w, 3, 1, 1)
        self.c1 = _BasicBlock(P, w, w, 1)
        self.c2 = _BasicBlock(P, w, cm, 2)
        self.memconv = _Conv(P, cm, 2 * d, 1, 1, 0)
        self.memln = (P.take(2 * d), P.take(2 * d))
        self.tok = _ConvBN(P, cm, d, 3, 2, 1)
        self.blocks3 = [_Block(P, d, cfg["heads"], self.th, self.mh if i in cfg["mem_at"] else 0)
                        for i in range(cfg["depth3"])]
        self.mergeln = (P.take(4 * d), P.take(4 * d))
        self.merge = _Linear(P, 4 * d, d4)
        self.blocks4 = [_Block(P, d4, cfg["heads4"], self.th // 2, 0)
                        for _ in range(cfg["depth4"])]
        self.headln = (P.take(d4), P.take(d4))
        self.pool = P.take(d4)
        self.coarse, self.resid = _Linear(P, d4, ncoarse), _Linear(P, d4, nclass)
        self.e1 = (_Linear(P, cm, nclass), _Linear(P, cm, d4, bias=False))
        self.pool2 = P.take(d)
        self.e2 = (_Linear(P, d, nclass), _Linear(P, d, d4, bias=False))
        assert P.i == len(P.t), "parameter list longer than the network"

    def forward(self, x, masks3=None, masks4=None):
        """x [n, 3, img, img] (numpy); masks3 / masks4: per block a tuple of
        three DropPath factor vectors (or None)."""
        cfg = self.cfg
        x = torch.tensor(np.asarray(x, np.float64), dtype=D)
        n, th = x.shape[0], self.th
        h = torch.relu(self.stem(x))
        h = self.c2(self.c1(h))
        mem = _ln(_tokens(self.memconv(h)), *self.memln)
        z = _tokens(self.tok(h))
        for i, b in enumerate(self.blocks3):
            z = b(z, mem, masks3[i] if masks3 else None)
        out = {}
        f2 = _seqpool(z, self.pool2)
        out["e2"], out["h2"] = self.e2[0](f2), self.e2[1](f2)
        c, t2 = cfg["dim"], th // 2
        zm = z.reshape(n, t2, 2, t2, 2, c).permute(0, 1, 3, 2, 4, 5).reshape(n, t2 * t2, 4 * c)
        z4 = self.merge(_ln(zm, *self.mergeln))
        for i, b in enumerate(self.blocks4):
            z4 = b(z4, None, masks4[i] if masks4 else None)
        feat = _seqpool(_ln(z4, *self.headln), self.pool)
        zc = self.coarse(feat)
        out["logits"] = self.resid(feat) + zc[:, self.parent]
        out["coarse"], out["feat"] = zc, feat
        g = h.mean(dim=(2, 3))
        out["e1"], out["h1"] = self.e1[0](g), self.e1[1](g)
        return out
