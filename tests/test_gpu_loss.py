"""GPU parity: loss.rs on the device (rustnn_amd/loss.py over loss.hip)
against the CPU oracle (oracle/orc_loss.c) on identical seeded inputs.

Bars: the soft targets are bit-exact (same arithmetic, no transcendental);
ce_soft / kl_distill / hint_mse gradients and losses within 1e-6 relative
(the device's expf / logf), hits exact; the reference's loss dirchecks
(check.rs:688-722) through the device path."""
import numpy as np
import pytest

from conftest import rel_frob, to_dev, to_host

import refcheck
from test_oracle_loss import _parent, losscheck

pytestmark = pytest.mark.gpu


def _i32(a):
    return to_dev(np.asarray(a, np.uint32).view(np.int32))


@pytest.mark.parametrize("taxo", [True, False])
def test_soft_targets(rnn, orc, taxo):
    from rustnn_amd.loss import soft_targets
    rng = np.random.default_rng(5)
    n, nf, nc = 256, 100, 20
    parent = _parent()
    labels = rng.integers(0, nf, n).astype(np.uint32)
    coarse = parent[labels]
    perm = rng.permutation(n).astype(np.uint32)
    lam = rng.uniform(0, 1, n).astype(np.float32)
    tf, tc = soft_targets(_i32(labels), nf, 0.1, _i32(parent) if taxo else None, 0.5,
                          _i32(coarse), nc, _i32(perm), to_dev(lam))
    wf, wc = orc.soft_targets(labels, nf, 0.1, parent if taxo else None, 0.5, coarse, nc, perm,
                              lam)
    assert np.array_equal(to_host(tf), wf)
    assert np.array_equal(to_host(tc), wc)
    tf1, none = soft_targets(_i32(labels), nf, 0.1, _i32(parent) if taxo else None, 0.5)
    assert none is None
    assert np.array_equal(to_host(tf1), orc.soft_targets(labels, nf, 0.1,
                                                         parent if taxo else None, 0.5)[0])


def test_soft_targets_bad_label_is_nan(rnn):
    from rustnn_amd.loss import soft_targets
    labels = np.array([3, 100, 7], np.uint32)  # 100 is out of range for nf = 100
    tf, _ = soft_targets(_i32(labels), 100, 0.1, _i32(_parent()), 0.5)
    t = to_host(tf)
    assert np.isnan(t[1]).all() and not np.isnan(t[[0, 2]]).any()


@pytest.mark.parametrize("n,nc", [(256, 100), (256, 20), (5, 7)])
def test_ce_soft(rnn, orc, n, nc):
    from rustnn_amd.loss import ce_soft
    rng = np.random.default_rng(n + nc)
    z = (rng.standard_normal((n, nc)) * 3).astype(np.float32)
    t = rng.uniform(0.1, 1.1, (n, nc)).astype(np.float32)
    t /= t.sum(1, keepdims=True)
    hard = rng.integers(0, nc, n).astype(np.uint32)
    hard[: n // 3] = z[: n // 3].argmax(1)
    loss, correct, dz = ce_soft(to_dev(z), to_dev(t), _i32(hard), 0.5)
    wl, wc, wdz = orc.ce_soft(z, t, hard, 0.5)
    assert abs(float(to_host(loss)[0]) - wl) <= 1e-6 * abs(wl)
    assert int(to_host(correct)[0]) == wc
    assert rel_frob(to_host(dz), wdz) < 1e-6


def test_kl_distill_and_hint(rnn, orc):
    from rustnn_amd.loss import hint_mse, kl_distill
    rng = np.random.default_rng(6)
    n, nc, c = 256, 100, 384
    zs, zt = (rng.standard_normal((n, nc)) * 2).astype(np.float32), \
        (rng.standard_normal((n, nc)) * 2).astype(np.float32)
    ZS, ZT = to_dev(zs).reshape(n, nc), to_dev(zt).reshape(n, nc)
    dz = to_dev(np.zeros((n, nc), np.float32)).reshape(n, nc)
    loss = kl_distill(ZS, ZT, 2.0, 0.5, dz)
    wd = np.zeros((n, nc), np.float32)
    wl = orc.kl_distill(zs, zt, 2.0, 0.5, wd)
    assert abs(float(to_host(loss)[0]) - wl) <= 1e-6 * abs(wl)
    assert rel_frob(to_host(dz), wd) < 1e-5
    # the gradient accumulates: on top of d0 it is d0 + (the same increment)
    d0 = rng.standard_normal((n, nc)).astype(np.float32)
    acc = to_dev(d0).reshape(n, nc)
    kl_distill(ZS, ZT, 2.0, 0.5, acc)
    assert np.array_equal(to_host(acc), d0 + to_host(dz))
    p, t = rng.standard_normal((n, c)).astype(np.float32), rng.standard_normal((n, c)).astype(
        np.float32)
    h0 = rng.standard_normal((n, c)).astype(np.float32)
    dh = to_dev(h0).reshape(n, c)
    loss = hint_mse(to_dev(p).reshape(n, c), to_dev(t).reshape(n, c), 0.3, dh)
    wh = h0.copy()
    wl = orc.hint_mse(p, t, 0.3, wh)
    assert abs(float(to_host(loss)[0]) - wl) <= 1e-6 * abs(wl)
    assert np.array_equal(to_host(dh), wh)  # no transcendental: bit-exact


class GpuLoss:
    def ce_soft(self, z, t, hard, scale):
        from rustnn_amd.loss import ce_soft
        loss, correct, dz = ce_soft(to_dev(z), to_dev(t), _i32(hard), scale)
        return float(to_host(loss)[0]), int(to_host(correct)[0]), to_host(dz)

    def kl_distill(self, zs, zt, temp, scale):
        import torch
        from rustnn_amd.loss import kl_distill
        dz = torch.zeros(zs.shape, device="cuda")
        loss = kl_distill(to_dev(zs), to_dev(zt), temp, scale, dz)
        return float(to_host(loss)[0]), to_host(dz)


def test_reference_losscheck_on_gpu(rnn, orc):
    errs = losscheck(orc, GpuLoss())
    assert all(v < refcheck.TOL for v in errs.values()), errs


@pytest.mark.parametrize("variant", ["default", "no_taxo", "no_alpha_beta"])
def test_build_loss_matches_oracle(rnn, orc, variant):
    """rnn_build_loss (train.rs:70-118 in one call) against the oracle's
    build_loss on the same heads and targets: the total, ce and hits, and
    every gradient; the branches without the coarse term (no_taxo, whose
    coarse gradient must be zeros) and without distillation / hints (the
    hint gradients zeros)."""
    import torch
    from oracle import pyvit
    from rustnn_amd.loss import build_loss, soft_targets
    n, nf, nc, d4 = 64, 100, 20, 384
    rng = orc.Rng(77)
    hp = dict(pyvit.TRAIN_DEFAULT)
    if variant == "no_taxo":
        hp["no_taxo"] = True
    if variant == "no_alpha_beta":
        hp["alpha"], hp["beta"] = 0.0, 0.0
    parent = np.arange(nf, dtype=np.uint32) // 5
    labels = np.array([rng.below(nf) for _ in range(n)], np.uint32)
    coarse = parent[labels]
    out = {k: rng.rand_vec(n * m).reshape(n, m) * np.float32(2.0) for k, m in
           (("logits", nf), ("coarse", nc), ("e1", nf), ("e2", nf), ("h1", d4), ("h2", d4),
            ("feat", d4))}
    taxo = not hp["no_taxo"]
    tf_w, tc_w = orc.soft_targets(labels, nf, hp["smooth"], parent if taxo else None, hp["sib"],
                                  coarse, nc)
    g_w, total_w, ce_w, corr_w = pyvit.build_loss(out, tf_w, tc_w, labels, coarse, hp, n)
    dev = {k: to_dev(v) for k, v in out.items()}
    L, Cc = _i32(labels), _i32(coarse)
    tf, tc = soft_targets(L, nf, hp["smooth"], _i32(parent) if taxo else None, hp["sib"], Cc, nc)
    g, total, ce, corr = build_loss(dev, tf, tc if taxo else None, L, Cc if taxo else None, nf, nc,
                                    hp)
    assert abs(float(to_host(total)[0]) - total_w) <= 1e-5 * abs(total_w), variant
    assert abs(float(to_host(ce)[0]) - ce_w) <= 1e-5 * abs(ce_w), variant
    assert int(to_host(corr)[0]) == corr_w
    for k, want in g_w.items():
        got = to_host(g[k]).reshape(want.shape)
        if not np.any(want):
            assert not np.any(got), (variant, k)
        else:
            assert rel_frob(got, want) < 1e-5, (variant, k)
