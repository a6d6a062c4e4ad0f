"""Pins the oracle's attention core (attn.rs:21-343) on the CPU: rel_index
against its closed form and the reference's RelGeom cases, forward/backward
against torch-autograd float64 fixtures and an f64 closed form, and dtau /
drel against finite differences."""
import glob
import os

import numpy as np
import pytest

from conftest import rel_frob

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def rel_index_def(th, tw, mh, mw):
    if mh == th:
        sy, sx, scale, oy, ox = 2 * th - 1, 2 * tw - 1, 1, th - 1, tw - 1
    else:
        sy, sx, scale, oy, ox = 2 * (th - 1) + mh, 2 * (tw - 1) + mw, 2, mh - 1, mw - 1
    idx = [(scale * qy - my + oy) * sx + (scale * qx - mx + ox)
           for qy in range(th) for qx in range(tw) for my in range(mh) for mx in range(mw)]
    return np.array(idx, np.uint32), sy * sx


@pytest.mark.parametrize("th,tw,mh,mw", [(8, 8, 8, 8), (8, 8, 16, 16), (4, 4, 4, 4), (3, 3, 6, 6),
                                         (3, 3, 3, 3), (2, 5, 4, 10)])
def test_rel_index(orc, th, tw, mh, mw):
    idx, nrel = orc.rel_index(th, tw, mh, mw)
    want, nrel_w = rel_index_def(th, tw, mh, mw)
    assert nrel == nrel_w and np.array_equal(idx, want)
    assert idx.max() < nrel
    # self attention: the table depends only on the offset q - m; centre = diagonal
    if mh == th:
        assert all(idx[i * th * tw + i] == (th - 1) * (2 * tw - 1) + tw - 1 for i in range(th * tw))


def attn64(q, k, v, tau, rel, idx, mask, dout):
    """Closed form in f64: q [n,h,tq,dh], k/v [n,h,tk,dh] -> p, o and grads."""
    q, k, v, dout = (a.astype(np.float64) for a in (q, k, v, dout))
    n, h, tq, dh = q.shape
    tk = k.shape[2]
    S = q @ k.transpose(0, 1, 3, 2)
    bias = rel.astype(np.float64)[:, idx.reshape(tq, tk)]
    X = tau.astype(np.float64)[None, :, None, None] * S + bias[None]
    if mask:
        X = np.where(np.eye(tq, tk, dtype=bool)[None, None], -np.inf, X)
    X = X - X.max(-1, keepdims=True)
    E = np.exp(X)
    P = E / E.sum(-1, keepdims=True)
    O = P @ v
    dV = P.transpose(0, 1, 3, 2) @ dout
    dP = dout @ v.transpose(0, 1, 3, 2)
    dS = P * (dP - (dP * P).sum(-1, keepdims=True))
    dtau = (dS * S).sum((0, 2, 3))
    drel = np.zeros(rel.shape)
    for hh in range(h):
        np.add.at(drel[hh], idx, dS[:, hh].sum(0).ravel())
    dS = dS * tau.astype(np.float64)[None, :, None, None]
    return P, O, dS @ k, dS.transpose(0, 1, 3, 2) @ q, dV, dtau, drel


def run_oracle(orc, z):
    n, h, dh, th, tw, mh, mw, mask = (int(v) for v in z["dims"])
    tq, tk, c = th * tw, mh * mw, h * dh
    idx, nrel = z["relidx"], int(z["nrel"])
    qb = z["q"].transpose(0, 2, 1, 3).reshape(n, tq, c)
    kvb = np.concatenate([z["k"].transpose(0, 2, 1, 3).reshape(n, tk, c),
                          z["v"].transpose(0, 2, 1, 3).reshape(n, tk, c)], axis=2)
    d = orc.attn_desc(h, dh, tq, tk, c, 0, 2 * c, 0, c, idx, nrel, bool(mask))
    p, o = orc.attn_forward(d, n, qb, kvb, z["tau"], z["rel"])
    dq, dkv, dtau, drel = orc.attn_backward(d, n, qb, kvb, z["tau"], p, z["dout"].transpose(
        0, 2, 1, 3).reshape(n, tq, c), np.zeros(qb.size, np.float32), np.zeros(kvb.size, np.float32),
        np.zeros(h, np.float32), np.zeros(h * nrel, np.float32))
    unq = lambda a, t: a.reshape(n, t, h, dh).transpose(0, 2, 1, 3)
    dkv = dkv.reshape(n, tk, 2 * c)
    return dict(p=p.reshape(n, h, tq, tk), o=unq(o, tq), dq=unq(dq, tq),
                dk=unq(dkv[:, :, :c].copy(), tk), dv=unq(dkv[:, :, c:].copy(), tk), dtau=dtau,
                drel=drel.reshape(h, nrel))


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLD, "attn_*.npz"))),
                         ids=lambda p: os.path.basename(p))
def test_attn_golden(orc, path):
    """Oracle against torch-autograd float64 fixtures (tests/golden/make_golden.py)."""
    z = np.load(path)
    got = run_oracle(orc, z)
    for key in ("p", "o", "dq", "dk", "dv", "dtau", "drel"):
        assert rel_frob(got[key], z[key]) < 1e-5, key
    # the closed form used below agrees with autograd too
    ref = attn64(z["q"], z["k"], z["v"], z["tau"], z["rel"], z["relidx"], bool(z["dims"][7]),
                 z["dout"])
    for key, r in zip(("p", "o", "dq", "dk", "dv", "dtau", "drel"), ref):
        assert rel_frob(r, z[key]) < 1e-10, key


def test_attn_finite_difference_tau_rel(orc):
    """dtau and drel against central differences of L = <O, dout> in f64 (the
    closed form is the checker; the oracle matches it above)."""
    z = np.load(os.path.join(GOLD, "attn_gc_cross.npz"))
    args = [z[k] for k in ("q", "k", "v", "tau", "rel")]
    idx, mask, dout = z["relidx"], bool(z["dims"][7]), z["dout"].astype(np.float64)
    _, _, _, _, _, dtau, drel = attn64(*args, idx, mask, dout)

    def loss(tau, rel):
        o = attn64(args[0], args[1], args[2], tau, rel, idx, mask, dout)[1]
        return float((o * dout).sum())

    e = 1e-6
    tau64, rel64 = args[3].astype(np.float64), args[4].astype(np.float64)
    for hh in range(tau64.size):
        tp, tm = tau64.copy(), tau64.copy()
        tp[hh] += e
        tm[hh] -= e
        assert abs((loss(tp, rel64) - loss(tm, rel64)) / (2 * e) - dtau[hh]) < 1e-6
    for j in (0, 5, 17, rel64.shape[1] - 1):
        rp, rm = rel64.copy(), rel64.copy()
        rp[1, j] += e
        rm[1, j] -= e
        assert abs((loss(tau64, rp) - loss(tau64, rm)) / (2 * e) - drel[1, j]) < 1e-6


def test_attn_oracle_threads_forward_bits(orc):
    """Forward is per (image, head); worker count must not change its bits."""
    z = np.load(os.path.join(GOLD, "attn_cfg2_small.npz"))
    a = run_oracle(orc, z)
    with orc.threads(4):
        b = run_oracle(orc, z)
    assert np.array_equal(a["p"], b["p"]) and np.array_equal(a["o"], b["o"])
    assert np.array_equal(a["dq"], b["dq"]) and np.array_equal(a["dk"], b["dk"])
