"""CPU pins of the oracle's rustvit network and train step (oracle/pyvit.py):

* Param::trunc_normal's draw order against the pinned Rng stream;
* lr_at at its closed-form points (warm-up ramp, the cosine's midpoint and
  end);
* the reference's netcheck (check.rs:397-450) on the oracle network: every
  parameter's gradient by a directional derivative;
* the oracle network against an independent torch float64 statement of the
  same network (tests/torch_rustvit.py) at the same weights: all outputs and
  every parameter gradient, with DropPath on (the reference's seeded masks);
* build_loss (train.rs:70-118) against torch float64 autograd of the same
  total loss, with a mixed batch (targets and the dominant labels);
* a planted mistake (a dropped residual term in the Block) fails the torch
  pin.
"""
import numpy as np
import pytest

import refcheck
from conftest import rel_frob

SMALL = dict(width=4, cmid=6, dim=8, heads=2, depth3=2, dim4=12, heads4=2, depth4=1,
             mem_at=(1,), droppath=0.2, img=16)
PARENT6 = [0, 0, 1, 1, 2, 2]


@pytest.fixture(scope="module")
def vit(orc):
    from oracle import pyvit
    return pyvit


def test_trunc_normal_draw_order(orc):
    """Each value is the next normal of the stream, redrawn (at most 8 times)
    while |z| > 2, clamped, times std."""
    std = np.float32(0.7)
    got = orc.Rng(99).trunc_normal(4000, std)
    r = orc.Rng(99)
    want = np.empty(4000, np.float32)
    redraws = 0
    for i in range(4000):
        z = r.normal()
        k = 0
        while abs(z) > 2.0 and k < 8:
            z = r.normal()
            k += 1
        redraws += k
        want[i] = np.float32(min(max(z, -2.0), 2.0)) * std
    assert redraws > 50  # the seed exercises the redraw path (P(|z| > 2) = 4.6%)
    assert np.array_equal(got, want)
    assert np.abs(got).max() <= 2 * std


def test_lr_at_closed_forms(orc):
    peak, lo, total, warm = 6e-4, 1e-5, 1000, 100
    f = np.float32
    assert orc.lr_at(peak, lo, 0, total, warm) == pytest.approx(lo + (peak - lo) / warm, rel=1e-6)
    assert orc.lr_at(peak, lo, 99, total, warm) == pytest.approx(peak, rel=1e-6)
    assert orc.lr_at(peak, lo, 100, total, warm) == pytest.approx(peak, rel=1e-6)
    assert orc.lr_at(peak, lo, 550, total, warm) == pytest.approx((peak + lo) / 2, rel=1e-5)
    assert orc.lr_at(peak, lo, 1000, total, warm) == pytest.approx(lo, rel=1e-5)
    # no warm-up: the cosine starts at the peak
    assert orc.lr_at(peak, lo, 0, total, 0) == f(peak)


def test_reference_netcheck_on_oracle(orc, vit):
    """check.rs:397-450 on the oracle: the reference's small RustViT with
    parameters perturbed by 0.15 N(0,1), batch 3, loss = <outputs, g>."""
    net = vit.RustViT(SMALL, PARENT6, 3, 0x1234 ^ 0xBEEF)
    net.drop_seed = 4242
    rng = orc.Rng(0x1234 ^ 0x77)
    ps = net.params()
    for p in ps:
        p.v += rng.rand_vec(p.v.size) * np.float32(0.15)
    bs, nf = 3, 6
    x = rng.rand_vec(bs * 3 * 16 * 16).reshape(bs, 3, 16, 16)
    g = {"logits": rng.rand_vec(bs * nf), "coarse": rng.rand_vec(bs * 3),
         "e1": rng.rand_vec(bs * nf), "e2": rng.rand_vec(bs * nf), "h1": rng.rand_vec(bs * 12),
         "h2": rng.rand_vec(bs * 12), "hfinal": rng.rand_vec(bs * 12)}

    def lin(o):
        return sum(refcheck.dot32(np.ravel(o[k]), g[k]) for k in
                   ("logits", "coarse", "e1", "e2", "h1", "h2")) + \
            refcheck.dot32(np.ravel(o["feat"]), g["hfinal"])

    net.forward(x, True)
    net.backward(g)
    base = np.concatenate([p.v for p in ps])
    grad = np.concatenate([p.g for p in ps])
    sizes = np.cumsum([p.v.size for p in ps])[:-1]

    def lossp(v):
        for p, part in zip(ps, np.split(v, sizes)):
            p.v[:] = part
        return lin(net.forward(x, True))

    e = refcheck.dircheck(base, grad, refcheck.gc_eps(), rng, lossp)
    assert e < refcheck.TOL, e


def _masks(orc, cfg, n, seed):
    """The DropPath factors the reference draws per block (vit.rs:150-172)."""
    depth = cfg["depth3"] + cfg["depth4"]
    div = np.float32(max(depth, 2) - 1)
    out3, out4 = [], []
    for i in range(depth):
        p = np.float32(cfg["droppath"]) * np.float32(i) / div
        idx = i + 1
        if p > 0:
            ms = tuple(orc.drop_path(np.ones(n, np.float32), n, float(p), seed ^ idx ^ k)[1]
                       for k in (0, 0x5151, 0xA2A2))
        else:
            ms = None
        (out3 if i < cfg["depth3"] else out4).append(ms)
    return out3, out4


def _torch_net(cfg, parent, nc, arrays):
    import torch_rustvit
    return torch_rustvit.RustViTF64(cfg, len(parent), nc, parent, arrays)


def compare_with_f64(orc, cfg, parent, nc, net_params, run, x, g, seed, planted=None):
    """Runs `run()` (forward + backward of the network under test with the
    output gradients g) and the float64 statement at the same weights;
    returns (outputs error per name, gradient error per parameter)."""
    import torch
    out = run()
    arrays = [np.asarray(a, np.float32) for a in net_params()[0]]
    tnet = _torch_net(cfg, parent, nc, arrays)
    if planted:
        planted(tnet)
    n = x.shape[0]
    m3, m4 = _masks(orc, cfg, n, seed)
    to = tnet.forward(x, m3, m4)
    loss = sum((to[k] * torch.tensor(np.asarray(g[k], np.float64).reshape(to[k].shape))).sum()
               for k in ("logits", "coarse", "e1", "e2", "h1", "h2"))
    loss = loss + (to["feat"] * torch.tensor(np.asarray(g["hfinal"], np.float64)
                                             .reshape(to["feat"].shape))).sum()
    loss.backward()
    oerr = {k: rel_frob(np.ravel(out[k]), to[k].detach().numpy().ravel()) for k in to}
    grads = net_params()[1]
    gerr = [rel_frob(np.ravel(gg), t.grad.numpy()) for gg, t in zip(grads, tnet.params)]
    return oerr, gerr


def _small_setup(orc, vit, seed=0x1234 ^ 0xBEEF):
    net = vit.RustViT(SMALL, PARENT6, 3, seed)
    rng = orc.Rng(7)
    for p in net.params():
        p.v += rng.rand_vec(p.v.size) * np.float32(0.15)
    bs = 3
    x = rng.rand_vec(bs * 3 * 16 * 16).reshape(bs, 3, 16, 16)
    g = {"logits": rng.rand_vec(bs * 6), "coarse": rng.rand_vec(bs * 3), "e1": rng.rand_vec(bs * 6),
         "e2": rng.rand_vec(bs * 6), "h1": rng.rand_vec(bs * 12), "h2": rng.rand_vec(bs * 12),
         "hfinal": rng.rand_vec(bs * 12)}
    return net, x, g


def test_oracle_net_matches_torch_f64(orc, vit):
    net, x, g = _small_setup(orc, vit)
    net.drop_seed = 4242

    def run():
        out = net.forward(x, True)
        net.backward(g)
        return out

    ps = net.params()
    oerr, gerr = compare_with_f64(orc, SMALL, PARENT6, 3, lambda: ([p.v for p in ps],
                                                                    [p.g for p in ps]),
                                  run, x, g, 4242)
    # the oracle's f32 arithmetic stays within 1e-5 of float64 on every output
    # and on every parameter's gradient (measured: 4e-7 and 4e-6 at most)
    assert max(oerr.values()) < 1e-5, oerr
    assert max(gerr) < 1e-5, max(gerr)


def test_planted_residual_drop_fails_torch_pin(orc, vit):
    """A Block that forgets its SwiGLU residual: the f64 pin must catch it."""
    net, x, g = _small_setup(orc, vit)
    net.drop_seed = 4242
    blk = net.blocks3[0]
    orig = blk.forward

    def broken(xx, mem, train, seed):
        y = orig(xx, mem, train, seed)
        h2 = blk.n2.forward(y, train)
        return y - blk.dp3.forward(blk.ls2.forward(blk.mlp.forward(h2, train), train), train,
                                   seed ^ blk.idx ^ 0xA2A2) * 0.5
    blk.forward = broken

    def run():
        return net.forward(x, True)

    ps = net.params()
    oerr, _ = compare_with_f64(orc, SMALL, PARENT6, 3, lambda: ([p.v for p in ps],
                                                                 [p.g for p in ps]),
                               run, x, g, 4242)
    assert max(oerr.values()) > 1e-4


def test_build_loss_matches_torch_f64(orc, vit):
    """build_loss with a mixed batch: the total and every output gradient
    against autograd of the same loss in float64."""
    import torch
    n, nf, nc, d4 = 6, 10, 2, 5
    parent = np.array([0, 0, 0, 0, 0, 1, 1, 1, 1, 1], np.uint32)
    r = orc.Rng(11)
    out = {k: r.rand_vec(n * m).reshape(n, m) for k, m in
           (("logits", nf), ("coarse", nc), ("e1", nf), ("e2", nf), ("h1", d4), ("h2", d4),
            ("feat", d4))}
    labels = np.array([r.below(nf) for _ in range(n)], np.uint32)
    coarse = parent[labels]
    perm = np.array([3, 0, 5, 1, 2, 4], np.uint32)
    lam = np.array([1.0, 0.3, 0.7, 0.5, 0.2, 0.9], np.float32)
    hp = dict(vit.TRAIN_DEFAULT)
    tf, tc = orc.soft_targets(labels, nf, hp["smooth"], parent, hp["sib"], coarse, nc, perm, lam)
    dom = vit.dominant(labels, perm, lam)
    assert list(dom) == [labels[0], labels[0], labels[2], labels[3], labels[2], labels[5]]
    g, total, _, _ = vit.build_loss(out, tf, tc, dom, coarse, hp, n)

    T = {k: torch.tensor(v.astype(np.float64), requires_grad=True) for k, v in out.items()}
    tft, tct = torch.tensor(tf, dtype=torch.float64), torch.tensor(tc, dtype=torch.float64)

    def ce(z, t):
        return -(t * torch.log_softmax(z, 1)).sum(1).mean()

    def kl(s, te, temp):
        pt = torch.softmax(te.detach() / temp, 1)
        return (pt * (torch.log(pt) - torch.log_softmax(s / temp, 1))).sum(1).mean() * temp ** 2

    feat = T["feat"].detach()
    tot = ce(T["logits"], tft) + hp["coarse_w"] * ce(T["coarse"], tct)
    tot = tot + hp["exit_w"][0] * ce(T["e1"], tft) + hp["exit_w"][1] * ce(T["e2"], tft)
    tot = tot + hp["alpha"] * (kl(T["e1"], T["logits"], hp["temp"]) +
                               kl(T["e2"], T["logits"], hp["temp"]))
    tot = tot + hp["beta"] * (((T["h1"] - feat) ** 2).mean() + ((T["h2"] - feat) ** 2).mean())
    tot.backward()
    assert abs(total - tot.item()) / abs(tot.item()) < 1e-5
    for k in ("logits", "coarse", "e1", "e2", "h1", "h2"):
        assert rel_frob(g[k], T[k].grad.numpy()) < 1e-5, k


def test_reference_vitcheck_on_oracle(orc, vit):
    """vitcheck (check.rs:163-180) on the oracle: normcheck, attncheck and
    netcheck on one Rng stream, every check under the reference's 5e-3."""
    from test_oracle_norm import OracleNorm
    errs = refcheck.vitcheck(orc, OracleNorm(orc), refcheck.OracleAttn())
    assert len(errs) == 16  # 8 norm, 7 attention, 1 network
    bad = {k: v for k, v in errs.items() if not v < refcheck.TOL}
    assert not bad, errs


def test_fnv1a_oracle_published_vectors(orc):
    """The oracle's FNV-1a 64 (train.rs:474-484) against the published
    FNV-1a 64 test vectors, and fnv_f32 as the 4 little-endian bytes of each
    float's bit pattern (a big-endian fold gives another hash)."""
    import struct
    off = orc.FNV_OFFSET
    assert orc.fnv1a_bytes(off, b"") == 0xCBF29CE484222325
    assert orc.fnv1a_bytes(off, b"a") == 0xAF63DC4C8601EC8C
    assert orc.fnv1a_bytes(off, b"foobar") == 0x85944171F73967E8
    v = np.array([1.0, -2.5, 3.0e-7, np.inf], np.float32)
    le = b"".join(struct.pack("<f", float(x)) for x in v)
    be = b"".join(struct.pack(">f", float(x)) for x in v)
    assert orc.fnv1a_f32(off, v) == orc.fnv1a_bytes(off, le)
    assert orc.fnv1a_f32(off, v) != orc.fnv1a_bytes(off, be)
    # continuing from a hash = hashing the concatenation
    assert orc.fnv1a_f32(orc.fnv1a_bytes(off, b"ab"), v) == orc.fnv1a_bytes(off, b"ab" + le)


def test_oracle_fingerprint_composition(orc, vit):
    """Trainer::fingerprint (train.rs:450-470) on the oracle trainer: the
    hash of the byte stream [v, m, v2 of each parameter in for_each_param
    order][every EMA tensor][Optim::t as u64 LE][last loss as f32 LE], where
    v2 is empty until AdamW steps a tensor and always for a Muon matrix, and
    the EMA has no tensors before its first update.  Checked before and after
    one step; dropping or reordering a part changes the hash."""
    import struct
    net = vit.RustViT(SMALL, PARENT6, 3, 5)
    tr = vit.Trainer(net, PARENT6, 3, dict(ntrain=400, batch=4, epochs=10, warmup=1, seed=77))
    off = orc.FNV_OFFSET

    def stream(params, ema, t, loss, order=("v", "m", "v2")):
        parts = []
        for p in params:
            for k in order:
                a = getattr(p, k, None)
                if a is not None:
                    parts.append(np.asarray(a, np.float32).tobytes())
        for w in ema or []:
            parts.append(np.asarray(w, np.float32).tobytes())
        parts.append(struct.pack("<Q", t))
        parts.append(struct.pack("<f", loss))
        return b"".join(parts)

    ps = net.params()
    assert all(getattr(p, "v2", None) is None for p in ps) and tr.ema_w is None
    h0 = tr.fingerprint(1.25)
    assert h0 == orc.fnv1a_bytes(off, stream(ps, None, 0, 1.25))
    rng = orc.Rng(5)
    x = rng.rand_vec(4 * 3 * 16 * 16).reshape(4, 3, 16, 16)
    labels = np.array([0, 3, 5, 1], np.uint32)
    coarse = np.array(PARENT6, np.uint32)[labels]
    total, _, _, _, _ = tr.step(x, labels, coarse)
    muon = [p for p in ps if getattr(p, "rows", 0) > 0 and min(p.rows, p.cols) > 1]
    assert muon and all(getattr(p, "v2", None) is None for p in muon)
    adam = [p for p in ps if p not in muon]
    assert adam and all(p.v2 is not None for p in adam) and any(p.v2.any() for p in adam)
    assert tr.t == 1 and tr.ema_w is not None
    h1 = tr.fingerprint(total)
    assert h1 == orc.fnv1a_bytes(off, stream(ps, tr.ema_w, 1, np.float32(total)))
    # planted mistakes: each changes the hash
    assert h1 != orc.fnv1a_bytes(off, stream(ps, tr.ema_w, 1, np.float32(total),
                                             order=("m", "v", "v2")))
    assert h1 != orc.fnv1a_bytes(off, stream(ps, None, 1, np.float32(total)))
    assert h1 != orc.fnv1a_bytes(off, stream(ps, tr.ema_w, 0, np.float32(total)))
