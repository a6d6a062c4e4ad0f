"""Pins of the oracle's loss.rs (oracle/orc_loss.c).

* taxo_target / uniform_target / the batch targets: closed forms written out
  in numpy (sibling share, far share, the label's 1 - eps, rows summing to 1,
  the mixup blend) including a singleton group and a one-group taxonomy;
* ce_soft: torch-CPU float64 cross_entropy with probability targets and its
  autograd, argmax hits;
* kl_distill: torch-CPU float64 kl_div(log_softmax(zs/T), softmax(zt/T)) T^2
  with the teacher detached, and its autograd;
* hint_mse: float64 closed form;
* the reference's loss dirchecks (check.rs:688-722: ce_soft and kl_distill at
  n=4, nc=7, eps 3e-4, tolerance 5e-3).
A planted mistake (the sibling share spread over k instead of k - 1) must
fail the closed form."""
import numpy as np
import pytest

from conftest import rel_frob

import refcheck


def _torch():
    return pytest.importorskip("torch")


def _parent(nf=100, nc=20, seed=0):
    """A CIFAR-100-like taxonomy: nc superclasses of nf / nc classes each."""
    return np.random.default_rng(seed).permutation(np.arange(nf) // (nf // nc)).astype(np.uint32)


def taxo_closed(y, parent, eps, sib, share_div=None):
    nf = parent.size
    grp = parent == parent[y]
    k = int(grp.sum())
    out = np.full(nf, eps * (1 - sib) / (nf - k) if nf > k else 0.0)
    if k > 1:
        out[grp] = eps * sib / (share_div(k) if share_div else k - 1)
    out[y] = 1 - eps
    return out


def test_taxo_target_closed_form(orc):
    parent = _parent()
    for y in (0, 17, 99):
        got = orc.taxo_target(y, parent, 0.1, 0.5)
        want = taxo_closed(y, parent, 0.1, 0.5)
        assert np.allclose(got, want, rtol=1e-6, atol=0)
        assert abs(got.astype(np.float64).sum() - 1.0) < 1e-6
        bad = taxo_closed(y, parent, 0.1, 0.5, share_div=lambda k: k)  # planted
        assert not np.allclose(got, bad, rtol=1e-6, atol=0)
    single = parent.copy()
    single[5] = 99  # class 5 alone in its group: no sibling share
    got = orc.taxo_target(5, single, 0.2, 0.5)
    assert got[5] == np.float32(0.8)
    assert np.allclose(np.delete(got, 5), 0.2 * 0.5 / 99, rtol=1e-6)
    one = np.zeros(10, np.uint32)  # one group holding every class: off_far = 0
    got = orc.taxo_target(3, one, 0.1, 0.5)
    assert got[3] == np.float32(0.9) and np.allclose(np.delete(got, 3), 0.1 * 0.5 / 9)


def test_uniform_target(orc):
    got = orc.uniform_target(4, 20, 0.1)
    want = np.full(20, np.float32(0.1) / np.float32(20))
    want[4] += np.float32(0.9)
    assert np.array_equal(got, want)


def test_soft_targets_mixup_blend(orc):
    rng = np.random.default_rng(1)
    n, nf, nc = 16, 100, 20
    parent = _parent()
    labels = rng.integers(0, nf, n).astype(np.uint32)
    coarse = parent[labels]
    perm = rng.permutation(n).astype(np.uint32)
    lam = rng.uniform(0, 1, n).astype(np.float32)
    tf, tc = orc.soft_targets(labels, nf, 0.1, parent, 0.5, coarse, nc, perm, lam)
    for i in range(n):
        a, b = taxo_closed(labels[i], parent, 0.1, 0.5), taxo_closed(labels[perm[i]], parent,
                                                                      0.1, 0.5)
        assert np.allclose(tf[i], lam[i] * a + (1 - lam[i]) * b, rtol=1e-5, atol=1e-7)
        ca = np.full(nc, 0.1 / nc)
        ca[coarse[i]] += 0.9
        cb = np.full(nc, 0.1 / nc)
        cb[coarse[perm[i]]] += 0.9
        assert np.allclose(tc[i], lam[i] * ca + (1 - lam[i]) * cb, rtol=1e-5, atol=1e-7)
    assert np.allclose(tf.sum(1), 1.0, atol=1e-5) and np.allclose(tc.sum(1), 1.0, atol=1e-5)
    tu, none = orc.soft_targets(labels, nf, 0.1)  # no taxonomy, no mixup
    assert none is None
    for i in range(n):
        assert np.array_equal(tu[i], orc.uniform_target(int(labels[i]), nf, 0.1))


def test_ce_soft_matches_torch_f64(orc):
    torch = _torch()
    rng = np.random.default_rng(2)
    n, nc = 32, 100
    z = (rng.standard_normal((n, nc)) * 3).astype(np.float32)
    t = rng.uniform(0.1, 1.1, (n, nc)).astype(np.float32)
    t /= t.sum(1, keepdims=True)
    hard = rng.integers(0, nc, n).astype(np.uint32)
    hard[:5] = z[:5].argmax(1)
    loss, correct, dz = orc.ce_soft(z, t, hard, 0.7)
    zt = torch.tensor(z, dtype=torch.float64, requires_grad=True)
    lt = torch.nn.functional.cross_entropy(zt, torch.tensor(t, dtype=torch.float64))
    lt.backward()
    assert abs(loss - lt.item()) <= 1e-6 * abs(lt.item())
    assert rel_frob(dz, 0.7 * zt.grad.numpy()) < 1e-6
    assert correct == int((z.argmax(1) == hard).sum()) and correct >= 5


def test_kl_distill_matches_torch_f64(orc):
    torch = _torch()
    rng = np.random.default_rng(3)
    n, nc, temp = 32, 100, 2.0
    zs = rng.standard_normal((n, nc)).astype(np.float32)
    zt_ = rng.standard_normal((n, nc)).astype(np.float32)
    dz = np.zeros((n, nc), np.float32)
    loss = orc.kl_distill(zs, zt_, temp, 0.5, dz)
    acc = np.full((n, nc), 0.25, np.float32)  # the gradient accumulates
    orc.kl_distill(zs, zt_, temp, 0.5, acc)
    assert np.array_equal(acc, np.float32(0.25) + dz)
    s = torch.tensor(zs, dtype=torch.float64, requires_grad=True)
    pt = torch.softmax(torch.tensor(zt_, dtype=torch.float64) / temp, 1)
    kl = torch.nn.functional.kl_div(torch.log_softmax(s / temp, 1), pt,
                                    reduction="batchmean") * temp * temp
    kl.backward()
    assert abs(loss - kl.item()) <= 1e-5 * abs(kl.item())
    assert rel_frob(dz, 0.5 * s.grad.numpy()) < 1e-5


def test_hint_mse_closed_form(orc):
    rng = np.random.default_rng(4)
    n, c = 16, 384
    p = rng.standard_normal((n, c)).astype(np.float32)
    t = rng.standard_normal((n, c)).astype(np.float32)
    dz = np.zeros((n, c), np.float32)
    loss = orc.hint_mse(p, t, 0.3, dz)
    e = p.astype(np.float64) - t
    assert abs(loss - 0.3 * (e * e).mean()) <= 1e-6 * loss
    assert rel_frob(dz, 2 * e / (n * c) * 0.3) < 1e-6


def losscheck(orc, be):
    """check.rs:688-722 on a backend: ce_soft and kl_distill dlogits by
    dircheck at n=4, nc=7 with soft targets; returns {name: error}."""
    rng = orc.Rng(1234)
    eps = refcheck.gc_eps()
    n, nc = 4, 7
    z = rng.rand_vec(n * nc)
    labels = np.array([rng.below(nc) for _ in range(n)], np.uint32)
    t = np.empty(n * nc, np.float32)
    for i in range(n):
        row = np.array([rng.uniform() + np.float32(0.1) for _ in range(nc)], np.float32)
        s = np.float32(0.0)
        for v in row:
            s = np.float32(s + v)
        t[i * nc:(i + 1) * nc] = row / s
    Z = lambda v: v.reshape(n, nc)
    T = t.reshape(n, nc)
    d = be.ce_soft(Z(z), T, labels, 1.0)[2]
    out = {"ce_soft dlogits": refcheck.dircheck(
        z, np.asarray(d).ravel(), eps, rng, lambda c: be.ce_soft(Z(c), T, labels, 1.0)[0])}
    teach = rng.rand_vec(n * nc).reshape(n, nc)
    d = be.kl_distill(Z(z), teach, 2.0, 1.0)[1]
    out["kl_distill dlogits"] = refcheck.dircheck(
        z, np.asarray(d).ravel(), eps, rng, lambda c: be.kl_distill(Z(c), teach, 2.0, 1.0)[0])
    return out


class OracleLoss:
    def __init__(self, orc):
        self.o = orc

    def ce_soft(self, z, t, hard, scale):
        return self.o.ce_soft(z, t, hard, scale)

    def kl_distill(self, zs, zt, temp, scale):
        dz = np.zeros(zs.shape, np.float32)
        return self.o.kl_distill(zs, zt, temp, scale, dz), dz


def test_reference_losscheck_on_oracle(orc):
    errs = losscheck(orc, OracleLoss(orc))
    assert all(v < refcheck.TOL for v in errs.values()), errs
