"""GPU parity: the vit.rs pieces on the device (rustnn_amd/vit.py over
vit.hip, norm.hip, attn.hip and the GEMM core).

* DropPath (mask from Rng::new(seed) drawn on the device), the token merge,
  TaxoHead's combine and the NCHW <-> token layout: bit-exact against the
  oracle;
* the whole pre-LN Block (self-attention, depthwise gate, cross-attention
  reader, SwiGLU, LayerScales) forward and every gradient -- x, the memory
  and all parameters -- against an independent torch-CPU float64 statement
  of vit.rs:138-250 at the same weights: relative 1e-5 (TOL);
* the reference's block dircheck (check.rs:360-395: dx and dparams of a
  reader block, eps 3e-4, tolerance 5e-3) with DropPath on, whose seeded
  mask keeps the finite difference valid."""
import numpy as np
import pytest

from conftest import TOL, rel_frob, to_dev, to_host

import refcheck

pytestmark = pytest.mark.gpu


def _i32(a):
    return to_dev(np.asarray(a, np.uint32).view(np.int32))


def test_drop_path(rnn, orc):
    import torch
    from rustnn_amd.vit import DropPath
    n, per = 256, 64 * 384
    x = np.random.default_rng(0).standard_normal(n * per).astype(np.float32)
    X = to_dev(x).reshape(n, 64, 384)
    dp = DropPath(0.1)
    seed = 0x1234 ^ 7 ^ 0x5151
    dp.forward(X, True, seed)
    want, mask = orc.drop_path(x, n, 0.1, seed)
    assert np.array_equal(to_host(dp.mask), mask)
    assert np.array_equal(to_host(X).ravel(), want)
    dy = to_dev(x).reshape(n, 64, 384)
    dp.backward(dy)
    assert np.array_equal(to_host(dy).ravel(), want)
    assert dp.forward(X, False, seed) is X and dp.mask is None  # eval: identity


def test_drop_path_masks_batched(rnn, orc):
    """rnn_drop_path_masks: 40 layers' masks (two launches of up to 32) in
    one call equal the oracle's draws, and a DropPath given its mask ahead
    applies it as its own draw would."""
    from rustnn_amd.vit import DropPath, draw_masks
    n, per = 128, 96
    ps = [0.05 + 0.02 * (k % 7) for k in range(40)]
    seeds = [(0xABCDEF0123456789 * (k + 1)) & 0xFFFFFFFFFFFFFFFF for k in range(40)]
    dps = [DropPath(p) for p in ps]
    x = np.random.default_rng(3).standard_normal(n * per).astype(np.float32)
    draw_masks(list(zip(dps, seeds)), n, "cuda", rnn.default_ctx())
    for dp, p, sd in zip(dps, ps, seeds):
        want, mask = orc.drop_path(x, n, p, sd)
        assert np.array_equal(to_host(dp.premask[0]), mask) and dp.premask[1] == sd
    X = to_dev(x).reshape(n, per)
    dps[5].forward(X, True, seeds[5])
    want, mask = orc.drop_path(x, n, ps[5], seeds[5])
    assert dps[5].premask is None and np.array_equal(to_host(dps[5].mask), mask)
    assert np.array_equal(to_host(X).ravel(), want)
    # a mask drawn ahead for another seed is not used: the forward draws
    # Rng::new(seed) itself
    X = to_dev(x).reshape(n, per)
    dps[6].forward(X, True, seeds[7])
    want, mask = orc.drop_path(x, n, ps[6], seeds[7])
    assert dps[6].premask is None and np.array_equal(to_host(dps[6].mask), mask)
    assert np.array_equal(to_host(X).ravel(), want)


@pytest.mark.parametrize("n,th,c", [(16, 8, 256), (3, 4, 6)])
def test_token_merge_and_layout(rnn, orc, n, th, c):
    """token_merge / token_merge_back bit-exact against the oracle (c 256:
    the four-channel kernel; c 6: the one-element kernel), and the NCHW <->
    token layout changes."""
    from rustnn_amd.vit import nchw_to_tokens, token_merge, token_merge_back, tokens_to_nchw
    z = np.random.default_rng(1).standard_normal(n * th * th * c).astype(np.float32)
    y = token_merge(to_dev(z).reshape(n, th * th, c), th)
    assert np.array_equal(to_host(y).ravel(), orc.token_merge(z, n, th, c))
    back = token_merge_back(y, th, c)
    assert np.array_equal(to_host(back).ravel(), z)
    x = np.random.default_rng(2).standard_normal((n, 96, 16, 16)).astype(np.float32)
    t = nchw_to_tokens(to_dev(x).reshape(x.shape))
    assert np.array_equal(to_host(t), x.reshape(n, 96, 256).transpose(0, 2, 1))
    assert np.array_equal(to_host(tokens_to_nchw(t, 16, 16)), x)


def test_taxo_head_combine(rnn, orc):
    from rustnn_amd import default_ctx, lib, _ptr
    rng = np.random.default_rng(3)
    n, nf, nc = 256, 100, 20
    parent = rng.permutation(np.arange(nf) // 5).astype(np.uint32)
    zf = rng.standard_normal((n, nf)).astype(np.float32)
    zc = rng.standard_normal((n, nc)).astype(np.float32)
    ctx = default_ctx()
    # every device buffer bound to a name for the whole call: a temporary
    # would go back to the allocator before the kernel reads it
    ZF, ZC, P = to_dev(zf), to_dev(zc), _i32(parent)
    ctx.check(lib().rnn_taxo_head_combine(ctx.h, n, nf, nc, _ptr(P, nf, "p"), _ptr(ZF, n * nf, "zf"),
                                          _ptr(ZC, n * nc, "zc")))
    assert np.array_equal(to_host(ZF).reshape(n, nf), orc.taxo_combine(zf, zc, parent))
    dzf = rng.standard_normal((n, nf)).astype(np.float32)
    dzc = rng.standard_normal((n, nc)).astype(np.float32)
    DC = to_dev(np.zeros(n * nc, np.float32))
    DZF, DZC = to_dev(dzf), to_dev(dzc)
    ctx.check(lib().rnn_taxo_head_combine_backward(ctx.h, n, nf, nc, _ptr(P, nf, "p"),
                                                   _ptr(DZF, n * nf, "dzf"),
                                                   _ptr(DZC, n * nc, "dzc"),
                                                   _ptr(DC, n * nc, "dc")))
    assert np.array_equal(to_host(DC).reshape(n, nc), orc.taxo_combine_backward(dzf, dzc, parent))


# ------------------------------------------------------------------ Block
def _params_of(obj):
    ps = []
    obj.for_each_param(lambda p: ps.append(p))
    return ps


def _torch_block(x, mem, W, c, h, th, mh, torch, keep=None):
    """vit.rs:138-172 in float64 (DropPath off): h = LN(x); x += l1 (SA(h) +
    g DW(h)); x += lm CA(h, mem); x += l2 SwiGLU(LN(x)).  `keep` (a list)
    receives each core's raw scores S and logits (their gradient after the
    backward is dS), for the conditioning of dtau."""
    F = torch.nn.functional
    dh = c // h
    n, t = x.shape[0], th * th

    def ln(v, g, b):
        return F.layer_norm(v, (c,), g, b, 1e-5)

    def core(q, k, v, tau, rel, relidx, nrel, mask):
        # q [n, tq, h, dh], k/v [n, tk, h, dh]
        s = torch.einsum("nqhd,nkhd->nhqk", q, k)
        bias = rel.view(h, nrel)[:, relidx]  # [h, tq, tk]
        xx = tau.view(1, h, 1, 1) * s + bias.unsqueeze(0)
        if keep is not None:
            xx.retain_grad()
            keep.append((s, xx))
        if mask:
            eye = torch.eye(s.shape[-1], dtype=torch.bool)
            xx = xx.masked_fill(eye, float("-inf"))
        p = torch.softmax(xx, -1)
        return torch.einsum("nhqk,nkhd->nqhd", p, v).reshape(n, -1, c)

    hh = ln(x, W["n1.g"], W["n1.b"])
    ab = hh @ W["qkv.w"].T + W["qkv.b"]
    q, k, v = ab[..., :c], ab[..., c:2 * c], ab[..., 2 * c:]
    sa = core(q.reshape(n, t, h, dh), k.reshape(n, t, h, dh), v.reshape(n, t, h, dh),
              W["tau"], W["rel"], W["relidx"], W["nrel"], True)
    sa = sa @ W["proj.w"].T + W["proj.b"]
    hi = hh.reshape(n, th, th, c).permute(0, 3, 1, 2)
    wdw = W["dw.w"].view(3, 3, c).permute(2, 0, 1).reshape(c, 1, 3, 3)
    dw = F.conv2d(hi, wdw, W["dw.b"], padding=1, groups=c).permute(0, 2, 3, 1).reshape(n, t, c)
    a = sa + W["gamma"] * dw
    y = x + W["ls1"] * a
    cq = hh @ W["wq.w"].T + W["wq.b"]
    tk = mh * mh
    ca = core(cq.reshape(n, t, h, dh), mem[..., :c].reshape(n, tk, h, dh),
              mem[..., c:].reshape(n, tk, h, dh), W["ctau"], W["crel"], W["crelidx"],
              W["cnrel"], False)
    ca = ca @ W["cproj.w"].T + W["cproj.b"]
    y = y + W["lsm"] * ca
    h2 = ln(y, W["n2.g"], W["n2.b"])
    g2 = h2 @ W["wg.w"].T + W["wg.b"]
    hid = g2.shape[-1] // 2
    u = F.silu(g2[..., :hid]) * g2[..., hid:]
    m = u @ W["wd.w"].T + W["wd.b"]
    return y + W["ls2"] * m


@pytest.mark.parametrize("mh", [6, 9])  # memory of 36 tokens (register path), 81 (composed)
def test_block_matches_torch_f64(rnn, orc, mh):
    import torch
    from rustnn_amd.vit import Block
    n, c, h, th, depth = 3, 32, 2, 4, 7
    t, tk = th * th, mh * mh
    blk = Block(c, h, th, th, (mh, mh), depth, 0.0, 2, 1e-4, 5)
    # non-trivial values for the parameters that start at constants
    r = np.random.default_rng(mh)
    for p in _params_of(blk):
        if p.rows == 0:
            p.v.copy_(to_dev((1.0 + 0.3 * r.standard_normal(p.v.numel())).astype(np.float32)))
    x = r.standard_normal((n, t, c)).astype(np.float32)
    mem = r.standard_normal((n, tk, 2 * c)).astype(np.float32)
    dz = r.standard_normal((n, t, c)).astype(np.float32)
    X, MEM = to_dev(x).reshape(n, t, c), to_dev(mem).reshape(n, tk, 2 * c)
    y = blk.forward(X, MEM, True, 99)
    dmem = torch.zeros(n * tk * 2 * c, device="cuda")
    dx = blk.backward(to_dev(dz).reshape(n, t, c), MEM, dmem)

    T = lambda a, g=True: torch.tensor(np.asarray(a, np.float64), requires_grad=g)
    H = lambda tt: to_host(tt).astype(np.float64)
    relidx, nrel = rnn.rel_index(th, th, th, th)
    crelidx, cnrel = rnn.rel_index(th, th, mh, mh)
    W = {"n1.g": T(H(blk.n1.g.v)), "n1.b": T(H(blk.n1.b.v)),
         "qkv.w": T(H(blk.attn.qkv.w).reshape(3 * c, c)), "qkv.b": T(H(blk.attn.qkv.b)),
         "proj.w": T(H(blk.attn.proj.w).reshape(c, c)), "proj.b": T(H(blk.attn.proj.b)),
         "tau": T(H(blk.attn.tau.v)), "rel": T(H(blk.attn.rel.v)),
         "relidx": torch.tensor(relidx.astype(np.int64).reshape(t, t)), "nrel": nrel,
         "dw.w": T(H(blk.dw.w.v)), "dw.b": T(H(blk.dw.b.v)), "gamma": T(H(blk.gamma.v)),
         "ls1": T(H(blk.ls1.l.v)),
         "wq.w": T(H(blk.cross.wq.w).reshape(c, c)), "wq.b": T(H(blk.cross.wq.b)),
         "cproj.w": T(H(blk.cross.proj.w).reshape(c, c)), "cproj.b": T(H(blk.cross.proj.b)),
         "ctau": T(H(blk.cross.tau.v)), "crel": T(H(blk.cross.rel.v)),
         "crelidx": torch.tensor(crelidx.astype(np.int64).reshape(t, tk)), "cnrel": cnrel,
         "lsm": T(H(blk.lsm.l.v)), "n2.g": T(H(blk.n2.g.v)), "n2.b": T(H(blk.n2.b.v)),
         "wg.w": T(H(blk.mlp.wg.w).reshape(-1, c)), "wg.b": T(H(blk.mlp.wg.b)),
         "wd.w": T(H(blk.mlp.wd.w).reshape(c, -1)), "wd.b": T(H(blk.mlp.wd.b)),
         "ls2": T(H(blk.ls2.l.v))}
    xt, mt = T(x), T(mem)
    kept = []
    yt = _torch_block(xt, mt, W, c, h, th, mh, torch, kept)
    assert rel_frob(to_host(y), yt.detach().numpy()) < TOL
    yt.backward(torch.tensor(dz, dtype=torch.float64))
    assert rel_frob(to_host(dx), xt.grad.numpy()) < TOL, "dx"
    assert rel_frob(to_host(dmem), mt.grad.numpy().ravel()) < TOL, "dmem"
    grads = {"n1.g": blk.n1.g.g, "n1.b": blk.n1.b.g, "qkv.w": blk.attn.qkv.gw,
             "qkv.b": blk.attn.qkv.gb, "proj.w": blk.attn.proj.gw, "proj.b": blk.attn.proj.gb,
             "tau": blk.attn.tau.g, "rel": blk.attn.rel.g, "dw.w": blk.dw.w.g,
             "dw.b": blk.dw.b.g, "gamma": blk.gamma.g, "ls1": blk.ls1.l.g,
             "wq.w": blk.cross.wq.gw, "wq.b": blk.cross.wq.gb, "cproj.w": blk.cross.proj.gw,
             "cproj.b": blk.cross.proj.gb, "ctau": blk.cross.tau.g, "crel": blk.cross.rel.g,
             "lsm": blk.lsm.l.g, "n2.g": blk.n2.g.g, "n2.b": blk.n2.b.g,
             "wg.w": blk.mlp.wg.gw, "wg.b": blk.mlp.wg.gb, "wd.w": blk.mlp.wd.gw,
             "wd.b": blk.mlp.wd.gb, "ls2": blk.ls2.l.g}
    # dtau is one number per head: the sum over n*tq*tk products dS*S whose
    # terms cancel (kappa = sum |dS S| / |sum dS S|, from the float64
    # statement, is in the hundreds), so any f32 evaluation carries a relative
    # error of order kappa * 2^-24 -- above 1e-5.  It is held to the oracle's
    # own distance from float64 (the oracle Block at the same weights) and to
    # that conditioning bound: the device no farther than max(TOL, 2 x the
    # oracle, 16 kappa 2^-24).
    kappa = {}
    for name, (sc, xx) in zip(("tau", "ctau"), kept):
        prod = (xx.grad * sc).detach().numpy()
        prod = np.where(np.isfinite(prod), prod, 0.0)
        kappa[name] = float(np.max(np.abs(prod).sum(axis=(0, 2, 3)) /
                                   np.abs(prod.sum(axis=(0, 2, 3)))))
    from oracle import pyvit
    oblk = pyvit.Block(c, h, th, th, (mh, mh), depth, 0.0, 2, np.float32(1e-4), orc.Rng(5))
    for po, pd in zip(oblk.params(), _params_of(blk)):
        po.v[:] = to_host(pd.v).ravel()
    oblk.forward(x.reshape(n, t, c), mem.reshape(n, tk, 2 * c), True, 99)
    oblk.backward(dz.reshape(n, t, c), mem.reshape(n, tk, 2 * c),
                  np.zeros(n * tk * 2 * c, np.float32))
    oracle_g = {"tau": oblk.attn.tau.g, "ctau": oblk.cross.tau.g}
    for k, g in grads.items():
        want = W[k].grad.numpy().ravel()
        err = rel_frob(to_host(g).ravel(), want)
        if k in oracle_g:
            eo = rel_frob(oracle_g[k], want)
            bound = max(TOL, 2 * eo, 16 * kappa[k] * 2.0 ** -24)
            assert err < bound, (k, err, eo, kappa[k])
        else:
            assert err < TOL, (k, err)


def test_reference_block_dircheck(rnn, orc):
    """check.rs:360-395 shape class: a reader block with DropPath on, dx and
    all parameters by dircheck (seed-stable masks)."""
    import torch
    from rustnn_amd.vit import Block
    n, c, h, th, mh = 3, 8, 2, 3, 6
    t, tk = th * th, mh * mh
    blk = Block(c, h, th, th, (mh, mh), 4, 0.3, 1, 0.5, 11)
    rng = orc.Rng(0x1234 ^ 9)
    eps = refcheck.gc_eps()
    x = rng.rand_vec(n * t * c)
    mem = rng.rand_vec(n * tk * 2 * c)
    r = rng.rand_vec(n * t * c)
    MEM = to_dev(mem).reshape(n, tk, 2 * c)
    seed = 77

    def loss(v):
        y = blk.forward(to_dev(v).reshape(n, t, c), MEM, True, seed)
        return refcheck.dot32(to_host(y), r)

    blk.forward(to_dev(x).reshape(n, t, c), MEM, True, seed)
    dmem = torch.zeros(n * tk * 2 * c, device="cuda")
    dx = blk.backward(to_dev(r).reshape(n, t, c), MEM, dmem)
    e = refcheck.dircheck(x, to_host(dx).ravel(), eps, rng, loss)
    assert e < refcheck.TOL, ("block dx", e)
    ps = _params_of(blk)
    for p in ps:
        p.g.zero_()
    blk.forward(to_dev(x).reshape(n, t, c), MEM, True, seed)
    blk.backward(to_dev(r).reshape(n, t, c), MEM, torch.zeros_like(dmem))
    base = np.concatenate([to_host(p.v).ravel() for p in ps])
    grad = np.concatenate([to_host(p.g).ravel() for p in ps])
    sizes = np.cumsum([p.v.numel() for p in ps])[:-1]

    def lossp(v):
        for p, part in zip(ps, np.split(v, sizes)):
            p.v.copy_(to_dev(part))
        return loss(x)

    e = refcheck.dircheck(base, grad, eps, rng, lossp)
    for p, part in zip(ps, np.split(base, sizes)):
        p.v.copy_(to_dev(part))
    assert e < refcheck.TOL, ("block dparams", e)


def test_reference_netcheck_rustvit(rnn, orc):
    """check.rs:397-450: a small RustViT (img 16, width 4, cmid 6, dim 8 x 2
    blocks with a memory reader, dim4 12 x 1, DropPath 0.2) with parameters
    perturbed by 0.15 N(0, 1), batch 3, loss = <outputs, random gradients>
    over the three heads, both hints and the pooled feature; one dircheck
    over every parameter through the device path."""
    import torch
    from rustnn_amd.vit import RustViT
    cfg = dict(width=4, cmid=6, dim=8, heads=2, depth3=2, dim4=12, heads4=2, depth4=1,
               mem_at=(1,), droppath=0.2, img=16)
    parent = _i32(np.array([0, 0, 1, 1, 2, 2], np.uint32))
    net = RustViT(cfg, parent, 3, seed=0x1234 ^ 0xBEEF)
    net.drop_seed = 4242
    rng = orc.Rng(0x1234 ^ 0x77)
    eps = refcheck.gc_eps()
    ps = net.params()
    for p in ps:
        p.v.add_(to_dev(rng.rand_vec(p.v.numel()) * np.float32(0.15)))
    bs, nf = 3, 6
    x = to_dev(rng.rand_vec(bs * 3 * 16 * 16)).reshape(bs, 3, 16, 16)
    g = {"logits": rng.rand_vec(bs * nf), "coarse": rng.rand_vec(bs * 3),
         "e1": rng.rand_vec(bs * nf), "e2": rng.rand_vec(bs * nf), "h1": rng.rand_vec(bs * 12),
         "h2": rng.rand_vec(bs * 12), "hfinal": rng.rand_vec(bs * 12)}
    gd = {k: to_dev(v) for k, v in g.items()}

    def lin(o):
        return (refcheck.dot32(to_host(o["logits"]), g["logits"]) +
                refcheck.dot32(to_host(o["coarse"]), g["coarse"]) +
                refcheck.dot32(to_host(o["e1"]), g["e1"]) + refcheck.dot32(to_host(o["e2"]), g["e2"]) +
                refcheck.dot32(to_host(o["h1"]), g["h1"]) + refcheck.dot32(to_host(o["h2"]), g["h2"]) +
                refcheck.dot32(to_host(o["feat"]), g["hfinal"]))

    net.forward(x, True)
    net.backward(gd)
    base = np.concatenate([to_host(p.v).ravel() for p in ps])
    grad = np.concatenate([to_host(p.g).ravel() for p in ps])
    assert np.isfinite(grad).all() and np.abs(grad).max() > 0
    sizes = np.cumsum([p.v.numel() for p in ps])[:-1]

    def lossp(v):
        for p, part in zip(ps, np.split(v, sizes)):
            p.v.copy_(to_dev(part))
        return lin(net.forward(x, True))

    e = refcheck.dircheck(base, grad, eps, rng, lossp)
    assert e < refcheck.TOL, ("rustvit (all parameters)", e)


def test_fingerprint_reproducible(rnn):
    """Trainer::fingerprint (train.rs:444-470) as the refactoring gate: two
    runs of the same steps give the same hash (every reduction on the device
    has a fixed order), and a different learning rate another one."""
    import torch
    from rustnn_amd.vit import RustViT, ViTStep, fingerprint
    cfg = dict(width=4, cmid=6, dim=8, heads=2, depth3=2, dim4=12, heads4=2, depth4=1,
               mem_at=(1,), droppath=0.2, img=16)
    parent = _i32(np.array([0, 0, 1, 1, 2, 2], np.uint32))

    def run(lr):
        net = RustViT(cfg, parent, 3, seed=5)
        step = ViTStep(net, parent, 3, dict(lr=lr))
        g = torch.Generator(device="cuda").manual_seed(1)
        x = torch.randn(4, 3, 16, 16, device="cuda", generator=g)
        labels = _i32(np.array([0, 3, 5, 1], np.uint32))
        coarse = _i32(np.array([0, 1, 2, 0], np.uint32))
        loss = None
        for i in range(3):
            net.drop_seed = 100 + i
            loss, _ = step(x, labels, coarse)
        return fingerprint(step, float(loss.item())), step.opt.t

    a, t = run(1e-3)
    b, _ = run(1e-3)
    c, _ = run(2e-3)
    assert t == 3 and a == b and a != c


def test_fingerprint_matches_oracle(rnn, orc):
    """The device Trainer::fingerprint (train.rs:450-470) against the
    oracle's restatement over identical states: at initialisation (both
    networks draw bit-identical weights; no second moments, no EMA, t = 0),
    then after two device train steps with the device's values, momenta,
    AdamW second moments, EMA weights and step count copied into the oracle
    trainer."""
    from oracle import pyvit
    from rustnn_amd.vit import RustViT, ViTStep, fingerprint
    cfg = dict(width=4, cmid=6, dim=8, heads=2, depth3=2, dim4=12, heads4=2, depth4=1,
               mem_at=(1,), droppath=0.2, img=16)
    parent = np.array([0, 0, 1, 1, 2, 2], np.uint32)
    hp = dict(ntrain=400, batch=4, epochs=10, warmup=1, seed=77)
    dnet = RustViT(cfg, _i32(parent), 3, seed=5)
    dstep = ViTStep(dnet, _i32(parent), 3, hp)
    onet = pyvit.RustViT(cfg, list(parent), 3, 5)
    otr = pyvit.Trainer(onet, parent, 3, hp)
    assert fingerprint(dstep, 1.25) == otr.fingerprint(1.25)
    rng = orc.Rng(9)
    x = to_dev(rng.rand_vec(4 * 3 * 16 * 16)).reshape(4, 3, 16, 16)
    labels = _i32(np.array([0, 3, 5, 1], np.uint32))
    coarse = _i32(np.array([0, 1, 2, 0], np.uint32))
    loss = None
    for i in range(2):
        dnet.drop_seed = 100 + i
        loss, _ = dstep(x, labels, coarse)
    last = float(loss.item())
    opt = dstep.opt
    for op, dp in zip(onet.params(), dnet.params()):
        op.v[:] = to_host(dp.v).ravel()
        op.m[:] = to_host(dp.m).ravel()
        muon = opt.muon and dp.rows > 0 and min(dp.rows, dp.cols) > 1
        op.v2 = None if muon else to_host(dp.v2).ravel().copy()
    assert dstep.ema is not None and dstep.ema.ready
    otr.ema_w = [to_host(w).ravel().copy() for w in dstep.ema.w]
    otr.t = opt.t
    assert opt.t == 2
    assert fingerprint(dstep, last) == otr.fingerprint(last)
