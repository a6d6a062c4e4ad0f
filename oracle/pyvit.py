"""CPU oracle of the reference rustvit (vit.rs) and of its train step
(train.rs), composed from the liborc.so layers of pyorc.py.

TEST INFRASTRUCTURE ONLY: a restatement of the reference's RustViT network
and Trainer::step used to check the device network of rustnn_amd.vit.  Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg may
import it.  Each layer below is one of the oracle's pinned restatements
(pyorc.py; their pins are in tests/test_oracle_*.py); this file adds only the
wiring, which follows the reference call for call:

* Param::trunc_normal / kaiming / filled (nn.rs:55-100) and Linear::new /
  scaled (linear.rs:25-41), drawn from one Rng::new(seed) in the order of
  RustViT::new (vit.rs:432-507): stage-3 blocks, stage-4 blocks, stem, c1, c2,
  memconv, tokconv, merge, pool, head, exit 1, pool2, exit 2; within a Block
  (vit.rs:117-143): qkv, proj, dw, [wq, proj], wg, wd.
* SelfAttn / CrossAttn forward and backward (attn.rs:387-552): qkv Linear ->
  Core -> proj; the self backward sums separate dq and dkv buffers.
* DropPath (vit.rs:25-74), Block (vit.rs:145-250), TaxoHead (vit.rs:282-312),
  Exit (vit.rs:330-345), token_merge (vit.rs:612-650), RustViT::forward /
  backward (vit.rs:510-688), for_each_param (vit.rs:690-716).
* build_loss (train.rs:70-118), targets (train.rs:121-155), the dominant
  labels (train.rs:313-320), lr_at (train.rs:21-28) and Trainer::step
  (train.rs:346-387) with clip_, Optim::step_all and Ema::update
  (optim.rs:177-288).

Parity of the wiring is pinned by the reference's own netcheck
(check.rs:397-450), run on this oracle in tests/test_oracle_vit_net.py.
"""
from __future__ import annotations

import numpy as np

from . import pymodel as PM
from . import pyorc as O

f32 = np.float32


class Param:
    """nn.rs Param (nn.rs:43-111) with the Muon shape (rows, cols) and
    AdamW's second moment, allocated when AdamW first touches it."""

    def __init__(self, v, decay, rows=0, cols=0):
        self.v = np.ascontiguousarray(v, f32).ravel()
        self.g = np.zeros_like(self.v)
        self.m = np.zeros_like(self.v)
        self.v2 = None
        self.decay, self.rows, self.cols = bool(decay), rows, cols

    @classmethod
    def trunc_normal(cls, n, std, decay, rng):
        return cls(rng.trunc_normal(n, std), decay)

    @classmethod
    def filled(cls, n, val, decay):
        return cls(np.full(n, f32(val), f32), decay)

    @classmethod
    def zeros(cls, n, decay):
        return cls(np.zeros(n, f32), decay)


def scaled_std(depth):
    """Linear::scaled (linear.rs:37-41): 0.02 / sqrt(2 depth) in f32."""
    return f32(0.02) / np.sqrt(f32(2.0) * f32(depth))


class Linear:
    """Linear (linear.rs:14-104): w [fout, fin] (a Muon matrix), bias 0."""

    def __init__(self, fin, fout, bias, std, rng):
        self.fin, self.fout = fin, fout
        self.w = Param.trunc_normal(fin * fout, std, True, rng)
        self.w.rows, self.w.cols = fout, fin
        self.b = Param.zeros(fout, False) if bias else None
        self.x, self.rows = None, 0

    def forward(self, x, rows, train):
        y = O.linear_forward(rows, self.fin, self.fout, x, self.w.v,
                             self.b.v if self.b else None)
        if train:
            self.x, self.rows = np.ascontiguousarray(x, f32).ravel().copy(), rows
        return y

    def backward(self, dy):
        dw, db, dx = O.linear_backward(self.rows, self.fin, self.fout, dy, self.x, self.w.v,
                                       self.w.g, self.b.g if self.b else None)
        self.w.g[:] = dw
        if self.b:
            self.b.g[:] = db
        return dx

    def params(self):
        return [self.w] + ([self.b] if self.b else [])


class LayerNorm:
    """LayerNorm (norm.rs:17-143)."""

    def __init__(self, c):
        self.g, self.b = Param.filled(c, 1.0, False), Param.zeros(c, False)

    def forward(self, x, train):
        if train:
            y, self.xhat, self.invstd = O.ln_forward(x, self.g.v, self.b.v)
            return y
        return O.ln_forward(x, self.g.v, self.b.v, train=False)

    def backward(self, dy):
        return O.ln_backward(dy, self.xhat, self.invstd, self.g.v, self.g.g, self.b.g)

    def params(self):
        return [self.g, self.b]


class LayerScale:
    """LayerScale (norm.rs:151-217)."""

    def __init__(self, c, init):
        self.l = Param.filled(c, init, False)

    def forward(self, x, train):
        if train:
            self.x = np.ascontiguousarray(x, f32).copy()
        return O.layerscale_forward(x, self.l.v)

    def backward(self, dy):
        return O.layerscale_backward(dy, self.x, self.l.v, self.l.g)

    def params(self):
        return [self.l]


class SwiGlu:
    """SwiGlu (norm.rs:231-294): wg Linear(c, 2h), gate, wd Linear::scaled."""

    def __init__(self, c, h, depth, rng):
        self.h = h
        self.wg = Linear(c, 2 * h, True, f32(0.02), rng)
        self.wd = Linear(h, c, True, scaled_std(depth), rng)

    def forward(self, x, train):
        rows = x.size // self.wg.fin
        ab = self.wg.forward(x, rows, train)
        if train:
            self.ab = ab
        return self.wd.forward(O.swiglu_forward(ab, self.h), rows, train).reshape(x.shape)

    def backward(self, dy):
        du = self.wd.backward(dy)
        return self.wg.backward(O.swiglu_backward(du, self.ab, self.h)).reshape(dy.shape)

    def params(self):
        return self.wg.params() + self.wd.params()


class DwConv3:
    """DwConv3 (norm.rs:296-457): w [9, c] trunc_normal(0.1), no decay."""

    def __init__(self, c, th, tw, rng):
        self.th, self.tw = th, tw
        self.w = Param.trunc_normal(9 * c, f32(0.1), False, rng)
        self.b = Param.zeros(c, False)

    def forward(self, x, train):
        if train:
            self.x = np.ascontiguousarray(x, f32).copy()
        return O.dwconv3_forward(x, self.w.v, self.b.v, x.shape[0], self.th, self.tw)

    def backward(self, dy):
        return O.dwconv3_backward(dy, self.x, self.w.v, dy.shape[0], self.th, self.tw, self.w.g,
                                  self.b.g)

    def params(self):
        return [self.w, self.b]


class SeqPool:
    """SeqPool (norm.rs:459-586): p trunc_normal(0.02), decayed."""

    def __init__(self, c, rng):
        self.p = Param.trunc_normal(c, f32(0.02), True, rng)

    def forward(self, x, train):
        n, t = x.shape[0], x.shape[1]
        z, w = O.seqpool_forward(x, self.p.v, n, t)
        if train:
            self.x, self.w, self.n, self.t = np.ascontiguousarray(x, f32).copy(), w, n, t
        return z.reshape(n, -1)

    def backward(self, dz):
        dx = O.seqpool_backward(dz, self.w, self.x, self.p.v, self.n, self.t, self.p.g)
        return dx.reshape(self.x.shape)

    def params(self):
        return [self.p]


def _tau(h, dh):
    return Param.filled(h, f32(1.0) / np.sqrt(f32(dh)), False)


class SelfAttn:
    """SelfAttn (attn.rs:346-448)."""

    def __init__(self, c, h, th, tw, depth, rng):
        self.c, self.h, self.t = c, h, th * tw
        dh = c // h
        relidx, nrel = O.rel_index(th, tw, th, tw)
        self.qkv = Linear(c, 3 * c, True, f32(0.02), rng)
        self.proj = Linear(c, c, True, scaled_std(depth), rng)
        self.tau = _tau(h, dh)
        self.rel = Param.zeros(h * nrel, False)
        self.desc = O.attn_desc(h, dh, self.t, self.t, 3 * c, 0, 3 * c, c, 2 * c, relidx, nrel,
                                True)

    def forward(self, x, train):
        n, t, c = x.shape
        ab = self.qkv.forward(x, n * t, train)
        p, o = O.attn_forward(self.desc, n, ab, ab, self.tau.v, self.rel.v)
        y = self.proj.forward(o, n * t, train)
        if train:
            self.ab, self.p, self.n = ab, p, n
        return y.reshape(n, t, c)

    def backward(self, dy):
        n, t, c = self.n, self.t, self.c
        do = self.proj.backward(dy)
        z = np.zeros(n * t * 3 * c, f32)
        dab, dkv, dtau, drel = O.attn_backward(self.desc, n, self.ab, self.ab, self.tau.v, self.p,
                                               do, z, z, self.tau.g, self.rel.g)
        self.tau.g[:], self.rel.g[:] = dtau, drel
        return self.qkv.backward(dab + dkv).reshape(n, t, c)

    def params(self):
        return self.qkv.params() + self.proj.params() + [self.tau, self.rel]


class CrossAttn:
    """CrossAttn (attn.rs:450-560): queries from x, K / V from the memory
    [n, tk, 2c] (K at column 0, V at c), no mask."""

    def __init__(self, c, h, th, tw, mh, mw, depth, rng):
        self.c, self.h, self.tq = c, h, th * tw
        dh = c // h
        relidx, nrel = O.rel_index(th, tw, mh, mw)
        self.wq = Linear(c, c, True, f32(0.02), rng)
        self.proj = Linear(c, c, True, scaled_std(depth), rng)
        self.tau = _tau(h, dh)
        self.rel = Param.zeros(h * nrel, False)
        self.desc = O.attn_desc(h, dh, self.tq, mh * mw, c, 0, 2 * c, 0, c, relidx, nrel, False)

    def forward(self, x, mem, train):
        n, t, c = x.shape
        q = self.wq.forward(x, n * t, train)
        p, o = O.attn_forward(self.desc, n, q, mem, self.tau.v, self.rel.v)
        y = self.proj.forward(o, n * t, train)
        if train:
            self.q, self.p, self.n = q, p, n
        return y.reshape(n, t, c)

    def backward(self, dy, mem, dmem):
        """Returns dx; dmem (flat) accumulates in place."""
        n, t, c = self.n, self.tq, self.c
        do = self.proj.backward(dy)
        dq0 = np.zeros(n * t * c, f32)
        dq, dm, dtau, drel = O.attn_backward(self.desc, n, self.q, mem, self.tau.v, self.p, do,
                                             dq0, dmem, self.tau.g, self.rel.g)
        dmem[:] = dm
        self.tau.g[:], self.rel.g[:] = dtau, drel
        return self.wq.backward(dq).reshape(n, t, c)

    def params(self):
        return self.wq.params() + self.proj.params() + [self.tau, self.rel]


class DropPath:
    """DropPath (vit.rs:25-74): the mask from Rng::new(seed)."""

    def __init__(self, p):
        self.p = f32(p)
        self.mask = None

    def forward(self, x, train, seed):
        if not train or self.p <= 0:
            return x
        y, self.mask = O.drop_path(x, x.shape[0], float(self.p), seed)
        return y.reshape(x.shape)

    def backward(self, dy):
        if self.mask is None:
            return dy
        return (dy.reshape(dy.shape[0], -1) * self.mask[:, None]).reshape(dy.shape)


class Block:
    """Block (vit.rs:76-250)."""

    def __init__(self, c, h, th, tw, mem, depth, drop, idx, ls_init, rng):
        hidden = -(-(4 * c // 3) // 16) * 16
        self.c, self.idx = c, idx
        self.n1 = LayerNorm(c)
        self.attn = SelfAttn(c, h, th, tw, depth, rng)
        self.dw = DwConv3(c, th, tw, rng)
        self.gamma = Param.filled(c, 0.5, False)
        self.ls1 = LayerScale(c, ls_init)
        self.cross = CrossAttn(c, h, th, tw, mem[0], mem[1], depth, rng) if mem else None
        self.lsm = LayerScale(c, ls_init) if mem else None
        self.n2 = LayerNorm(c)
        self.mlp = SwiGlu(c, hidden, depth, rng)
        self.ls2 = LayerScale(c, ls_init)
        self.dp1, self.dp2, self.dp3 = DropPath(drop), DropPath(drop), DropPath(drop)

    def forward(self, x, mem, train, seed):
        h = self.n1.forward(x, train)
        a = self.attn.forward(h, train)
        d = self.dw.forward(h, train)
        a = a + self.gamma.v * d
        if train:
            self.dwo = d
        a = self.dp1.forward(self.ls1.forward(a, train), train, seed ^ self.idx)
        y = x + a
        if self.cross is not None:
            cm = self.cross.forward(h, mem, train)
            cm = self.dp2.forward(self.lsm.forward(cm, train), train, seed ^ self.idx ^ 0x5151)
            y = y + cm
        m = self.mlp.forward(self.n2.forward(y, train), train)
        m = self.dp3.forward(self.ls2.forward(m, train), train, seed ^ self.idx ^ 0xA2A2)
        return y + m

    def backward(self, dz, mem=None, dmem=None):
        dm = self.ls2.backward(self.dp3.backward(dz.copy()))
        dy = dz + self.n2.backward(self.mlp.backward(dm))
        dh = np.zeros_like(dy)
        if self.cross is not None:
            dc = self.lsm.backward(self.dp2.backward(dy.copy()))
            dh = dh + self.cross.backward(dc, mem, dmem)
        da = self.ls1.backward(self.dp1.backward(dy.copy()))
        # gamma.g += sum da * dwo; ddw = gamma * da (LayerScale's backward)
        ddw = O.layerscale_backward(da, self.dwo, self.gamma.v, self.gamma.g)
        dh = dh + self.attn.backward(da)
        dh = dh + self.dw.backward(ddw)
        return dy + self.n1.backward(dh)

    def params(self):
        ps = self.n1.params() + self.attn.params() + self.dw.params() + [self.gamma]
        ps += self.ls1.params()
        if self.cross is not None:
            ps += self.cross.params() + self.lsm.params()
        return ps + self.n2.params() + self.mlp.params() + self.ls2.params()


class TaxoHead:
    """TaxoHead (vit.rs:254-318)."""

    def __init__(self, c, parent, nc, rng):
        self.parent, self.nc = np.asarray(parent, np.uint32), nc
        self.coarse = Linear(c, nc, True, f32(0.02), rng)
        self.resid = Linear(c, self.parent.size, True, f32(0.02), rng)

    def forward(self, f, n, train):
        zc = self.coarse.forward(f, n, train).reshape(n, self.nc)
        zf = self.resid.forward(f, n, train).reshape(n, -1)
        self.n = n
        return O.taxo_combine(zf, zc, self.parent), zc

    def backward(self, dzf, dzc):
        n = self.n
        dc = O.taxo_combine_backward(np.asarray(dzf, f32).reshape(n, -1),
                                     np.asarray(dzc, f32).reshape(n, self.nc), self.parent)
        df = self.resid.backward(dzf)
        return df + self.coarse.backward(dc)

    def params(self):
        return self.coarse.params() + self.resid.params()


class Exit:
    """Exit (vit.rs:320-353)."""

    def __init__(self, cin, nclass, chint, rng):
        self.fc = Linear(cin, nclass, True, f32(0.02), rng)
        self.hint = Linear(cin, chint, False, f32(0.02), rng)

    def forward(self, f, n, train):
        return (self.fc.forward(f, n, train).reshape(n, -1),
                self.hint.forward(f, n, train).reshape(n, -1))

    def backward(self, dz, dh):
        return self.fc.backward(dz) + self.hint.backward(dh)

    def params(self):
        return self.fc.params() + self.hint.params()


def _tokens(x):
    """Tok::from_tensor (tok.rs): [n, c, h, w] -> [n, h*w, c]."""
    n, c = x.shape[0], x.shape[1]
    return np.ascontiguousarray(x.reshape(n, c, -1).transpose(0, 2, 1))


def _tensor(t, h, w):
    """Tok::to_tensor (tok.rs): [n, h*w, c] -> [n, c, h, w]."""
    n, _, c = t.shape
    return np.ascontiguousarray(t.transpose(0, 2, 1).reshape(n, c, h, w))


def token_merge(z, th):
    n, _, c = z.shape
    return O.token_merge(z, n, th, c).reshape(n, (th // 2) ** 2, 4 * c)


def token_merge_back(dy, th, c):
    """token_merge_back (vit.rs:632-650): the inverse gather."""
    n, t2 = dy.shape[0], th // 2
    return np.ascontiguousarray(
        dy.reshape(n, t2, t2, 2, 2, c).transpose(0, 1, 3, 2, 4, 5).reshape(n, th * th, c))


VIT_DEFAULT = dict(width=32, cmid=96, dim=256, heads=4, depth3=5, dim4=384, heads4=6, depth4=2,
                   mem_at=(1, 3), droppath=0.1, img=32)


class RustViT:
    """RustViT (vit.rs:400-757) with Rng::new(seed) drawn as RustViT::new."""

    def __init__(self, cfg, parent, ncoarse, seed):
        cfg = dict(VIT_DEFAULT, **(cfg or {}))
        rng = O.Rng(seed)
        w, cm, d, d4 = cfg["width"], cfg["cmid"], cfg["dim"], cfg["dim4"]
        self.cfg, self.mh, self.th = cfg, cfg["img"] // 2, cfg["img"] // 4
        depth = cfg["depth3"] + cfg["depth4"]
        div = f32(max(depth, 2) - 1)
        rate = lambda i: f32(cfg["droppath"]) * f32(i) / div
        self.blocks3 = [Block(d, cfg["heads"], self.th, self.th,
                              (self.mh, self.mh) if i in cfg["mem_at"] else None, depth, rate(i),
                              i + 1, f32(1e-4), rng) for i in range(cfg["depth3"])]
        th4 = self.th // 2
        self.blocks4 = [Block(d4, cfg["heads4"], th4, th4, None, depth, rate(cfg["depth3"] + i),
                              cfg["depth3"] + i + 1, f32(1e-4), rng)
                        for i in range(cfg["depth4"])]
        self.stem = PM.Conv2d(3, w, 3, 1, 1, rng)
        self.stem_bn = PM.BatchNorm2d(w)
        self.c1 = PM.BasicBlock(w, w, 1, rng)
        self.c2 = PM.BasicBlock(w, cm, 2, rng)
        self.memconv = PM.Conv2d(cm, 2 * d, 1, 1, 0, rng)
        self.memln = LayerNorm(2 * d)
        self.tokconv = PM.Conv2d(cm, d, 3, 2, 1, rng)
        self.tok_bn = PM.BatchNorm2d(d)
        self.mergeln = LayerNorm(4 * d)
        self.merge = Linear(4 * d, d4, True, f32(0.02), rng)
        self.headln = LayerNorm(d4)
        self.pool = SeqPool(d4, rng)
        self.nclass = len(parent)
        self.head = TaxoHead(d4, parent, ncoarse, rng)
        self.e1 = Exit(cm, self.nclass, d4, rng)
        self.pool2 = SeqPool(d, rng)
        self.e2 = Exit(d, self.nclass, d4, rng)
        self.drop_seed, self.use_exits = 0, True

    def forward(self, x, train):
        """RustViT::forward (vit.rs:510-609): a dict of the outputs."""
        n, d = x.shape[0], self.cfg["dim"]
        x = np.ascontiguousarray(x, f32)
        h = self.stem_bn.forward_relu(self.stem.forward(x, train), train)
        if train:
            self.stem_out = h
        h = self.c1.forward(h, train)
        h = self.c2.forward(h, train)
        if train:
            self.c2_out = h
        mem = self.memln.forward(_tokens(self.memconv.forward(h, train)), train)
        z = _tokens(self.tok_bn.forward(self.tokconv.forward(h, train), train))
        seed = self.drop_seed
        for b in self.blocks3:
            z = b.forward(z, mem, train, seed)
        if train:
            self.mem = mem
        out = {}
        if self.use_exits and train:
            out["e2"], out["h2"] = self.e2.forward(self.pool2.forward(z, train), n, train)
        zn = self.mergeln.forward(token_merge(z, self.th), train)
        t4 = zn.shape[1]
        z4 = self.merge.forward(zn, n * t4, train).reshape(n, t4, self.cfg["dim4"])
        for b in self.blocks4:
            z4 = b.forward(z4, None, train, seed)
        feat = self.pool.forward(self.headln.forward(z4, train), train)
        out["logits"], out["coarse"] = self.head.forward(feat, n, train)
        out["feat"] = feat
        if self.use_exits and train:
            out["e1"], out["h1"] = self.e1.forward(O.gap_forward(self.c2_out), n, train)
        self.n = n
        return out

    def backward(self, g):
        """RustViT::backward (vit.rs:628-688)."""
        n, d, cm, mh, th = self.n, self.cfg["dim"], self.cfg["cmid"], self.mh, self.th
        dfeat = self.head.backward(g["logits"], g["coarse"])
        if g.get("hfinal") is not None:
            dfeat = dfeat + np.asarray(g["hfinal"], f32).ravel()
        dz4 = self.headln.backward(self.pool.backward(dfeat))
        for b in reversed(self.blocks4):
            dz4 = b.backward(dz4)
        t4 = dz4.shape[1]
        dmg = self.merge.backward(dz4).reshape(n, t4, 4 * d)
        dz = token_merge_back(self.mergeln.backward(dmg), th, d)
        if self.use_exits and g.get("e2") is not None:
            dz = dz + self.pool2.backward(self.e2.backward(g["e2"], g["h2"]))
        dmem = np.zeros(self.mem.size, f32)
        for b in reversed(self.blocks3):
            dz = b.backward(dz, self.mem, dmem)
        dtc = self.tokconv.backward(self.tok_bn.backward(_tensor(dz, th, th)))
        dmemn = self.memln.backward(dmem.reshape(n, mh * mh, 2 * d))
        dc2 = dtc + self.memconv.backward(_tensor(dmemn, mh, mh))
        if self.use_exits and g.get("e1") is not None:
            dg = self.e1.backward(g["e1"], g["h1"])
            dc2 = dc2 + O.gap_backward(dg.reshape(n, cm), mh, mh)
        dh = self.c1.backward(self.c2.backward(np.ascontiguousarray(dc2, f32)))
        dh = np.ascontiguousarray(dh, f32)
        O.relu_back(dh, self.stem_out)
        self.stem.backward_w(self.stem_bn.backward(dh))

    def params(self):
        """RustViT::for_each_param (vit.rs:690-716)."""
        ps = [self.stem.w, self.stem_bn.g, self.stem_bn.b] + self.c1.params() + self.c2.params()
        ps += [self.memconv.w] + self.memln.params()
        ps += [self.tokconv.w, self.tok_bn.g, self.tok_bn.b]
        for b in self.blocks3:
            ps += b.params()
        ps += self.mergeln.params() + self.merge.params()
        for b in self.blocks4:
            ps += b.params()
        ps += self.headln.params() + self.pool.params() + self.head.params()
        if self.use_exits:
            ps += self.e1.params() + self.pool2.params() + self.e2.params()
        return ps


# ---------------------------------------------------------------- train.rs
TRAIN_DEFAULT = dict(smooth=0.1, sib=0.7, coarse_w=0.4, exit_w=(0.3, 0.6), alpha=1.0, temp=3.0,
                     beta=0.03, clip=1.0, ema=0.9998, ema_auto=True, lr=6e-4, lr_min=1e-5,
                     wd=0.06, muon=True, ns=3, no_taxo=False, seed=1234, batch=128, ntrain=50000,
                     epochs=100, warmup=10)


def build_loss(out, tf, tc, hard, hardc, hp, n):
    """build_loss (train.rs:70-118): (gradients, total, ce, correct)."""
    nf = out["logits"].shape[1]
    nc = out["coarse"].shape[1]
    ce, correct, dlog = O.ce_soft(out["logits"], tf, hard, 1.0)
    g = {"logits": dlog, "coarse": np.zeros((n, nc), f32)}
    total = f32(ce)
    if hp["coarse_w"] > 0 and not hp["no_taxo"]:
        lc, _, g["coarse"] = O.ce_soft(out["coarse"], tc, hardc, hp["coarse_w"])
        total = total + f32(hp["coarse_w"]) * f32(lc)
    if "e1" in out:
        d4 = out["feat"].size // n
        w1, w2 = f32(hp["exit_w"][0]), f32(hp["exit_w"][1])
        l1, _, de1 = O.ce_soft(out["e1"], tf, hard, float(w1))
        l2, _, de2 = O.ce_soft(out["e2"], tf, hard, float(w2))
        total = total + (w1 * f32(l1) + w2 * f32(l2))
        if hp["alpha"] > 0:
            k1 = O.kl_distill(out["e1"], out["logits"], hp["temp"], hp["alpha"], de1)
            k2 = O.kl_distill(out["e2"], out["logits"], hp["temp"], hp["alpha"], de2)
            total = total + f32(hp["alpha"]) * (f32(k1) + f32(k2))
        dh1, dh2 = np.zeros((n, d4), f32), np.zeros((n, d4), f32)
        if hp["beta"] > 0:
            feat = out["feat"].reshape(n, d4)
            total = total + (f32(O.hint_mse(out["h1"], feat, hp["beta"], dh1)) +
                             f32(O.hint_mse(out["h2"], feat, hp["beta"], dh2)))
        g.update(e1=de1, e2=de2, h1=dh1, h2=dh2)
        assert de1.shape == (n, nf)
    return g, float(total), ce, correct


def dominant(labels, perm, lam):
    """train.rs:313-320."""
    labels = np.asarray(labels, np.uint32)
    return np.where(np.asarray(lam) >= 0.5, labels, labels[np.asarray(perm)]).astype(np.uint32)


class Trainer:
    """Trainer::step (train.rs:346-387) from an assembled batch, with the
    trainer's generator Rng::new(seed ^ 0xABCD) (train.rs:260)."""

    def __init__(self, net, parent, ncoarse, hp=None):
        self.net, self.parent, self.nc = net, np.asarray(parent, np.uint32), ncoarse
        self.hp = hp = dict(TRAIN_DEFAULT, **(hp or {}))
        self.rng = O.Rng(int(hp["seed"]) ^ 0xABCD)
        spe = hp["ntrain"] // hp["batch"]
        self.total_steps, self.warm_steps = spe * hp["epochs"], spe * hp["warmup"]
        d = f32(hp["ema"])
        if hp["ema_auto"] and self.total_steps > 0:
            d = min(f32(1.0) - f32(10.0) / f32(self.total_steps), d)
        self.ema_decay = d
        self.ema_w, self.ema_t = None, 0
        self.t = 0  # Optim::t
        self.step_no = 0

    def targets(self, labels, coarse, perm=None, lam=None):
        nf = self.net.nclass
        taxo = not self.hp["no_taxo"]
        return O.soft_targets(labels, nf, self.hp["smooth"], self.parent if taxo else None,
                              self.hp["sib"], coarse, self.nc, perm, lam)

    def step_all(self, params, lr, wd):
        """Optim::step_all (optim.rs:177-205)."""
        hp = self.hp
        for p in params:
            rows = getattr(p, "rows", 0)
            cols = getattr(p, "cols", 0)
            if hp["muon"] and rows > 0 and min(rows, cols) > 1:
                O.muon_step(p.v, p.g, p.m, rows, cols, p.decay, lr, wd, 0.95, hp["ns"])
            else:
                if getattr(p, "v2", None) is None:
                    p.v2 = np.zeros_like(p.v)
                O.adam_step(p.v, p.g, p.m, p.v2, p.decay, lr, wd, self.t)
        self.t += 1

    def clip(self, params, max_norm):
        """clip_ (optim.rs:237-251) over the list's gradients."""
        g = np.concatenate([p.g.ravel() for p in params]).astype(f32)
        norm = O.clip(g, [p.g.size for p in params], max_norm)
        off = 0
        for p in params:
            p.g.ravel()[:] = g[off:off + p.g.size]
            off += p.g.size
        return norm

    def ema_update(self, params):
        """Ema::update (optim.rs:270-288)."""
        self.ema_t += 1
        if self.ema_w is None:
            self.ema_w = [p.v.copy() for p in params]
            return
        for w, p in zip(self.ema_w, params):
            O.ema_update(w, p.v, float(self.ema_decay), self.ema_t)

    def forward_backward(self, x, labels, coarse, perm=None, lam=None):
        """train.rs:348-362: targets, the DropPath seed, forward, build_loss,
        backward.  Returns (total, ce, correct, the output dict)."""
        n = len(labels)
        tf, tc = self.targets(labels, coarse, perm, lam)
        dom = (np.asarray(labels, np.uint32) if perm is None else dominant(labels, perm, lam))
        self.net.drop_seed = self.rng.next_u64()
        out = self.net.forward(x, True)
        g, total, ce, correct = build_loss(out, tf, tc, dom, np.asarray(coarse, np.uint32),
                                           self.hp, n)
        self.net.backward(g)
        return total, ce, correct, out

    def update(self, lr=None):
        """train.rs:364-386: lr_at, clip_, step_all, the EMA.  Returns lr."""
        hp = self.hp
        if lr is None:
            lr = O.lr_at(hp["lr"], hp["lr_min"], self.step_no, self.total_steps, self.warm_steps)
        params = self.net.params()
        if hp["clip"] > 0:
            self.clip(params, hp["clip"])
        self.step_all(params, lr, hp["wd"])
        if self.ema_decay > 0:
            self.ema_update(params)
        self.step_no += 1
        return lr

    def fingerprint(self, last_loss):
        """Trainer::fingerprint (train.rs:450-470): FNV-1a from the offset
        basis over, per parameter in for_each_param order, its values, then
        its momentum, then its AdamW second moment (empty -- nothing folded
        -- until AdamW first steps the tensor, optim.rs:208-210, and always
        for a Muon matrix); then every EMA tensor (none before the EMA's
        first update, optim.rs:270-276); then Optim::t as 8 little-endian
        bytes; then the last loss as an f32."""
        h = O.FNV_OFFSET
        for p in self.net.params():
            for arr in (p.v, p.m, getattr(p, "v2", None)):
                if arr is not None:
                    h = O.fnv1a_f32(h, arr)
        for w in self.ema_w or []:
            h = O.fnv1a_f32(h, w)
        h = O.fnv1a_bytes(h, int(self.t).to_bytes(8, "little"))
        return O.fnv1a_f32(h, np.float32(last_loss))

    def step(self, x, labels, coarse, perm=None, lam=None, lr=None):
        """One Trainer::step; returns (total, ce, correct, lr, outputs)."""
        total, ce, correct, out = self.forward_backward(x, labels, coarse, perm, lam)
        return total, ce, correct, self.update(lr), out
