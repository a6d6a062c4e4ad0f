"""GPU parity of the whole rustvit network and train step
against the CPU oracle (oracle/pyvit.py, itself pinned to an independent
torch float64 statement of the network and to the reference's netcheck):

* RustViT::new's initial weights from Rng::new(seed), bit for bit, for the
  reference's netcheck network and for the default network;
* forward outputs and every parameter gradient of the netcheck network (with
  its 0.15 N(0,1) perturbation and DropPath on) against the oracle;
* three Trainer::steps of that network (the second on a mixed batch) against
  the oracle's: the loss, the hits, every gradient and the updated weights;
* one Trainer::step of the DEFAULT network at batch 128 on the config-4
  inputs (images uniform in [0, 1] normalised, labels uniform over 100, a
  seeded 5-per-superclass taxonomy) against the oracle.

Tolerance: 1e-5 relative Frobenius (north_star) per output, per gradient
tensor and for the loss; a gradient tensor above it would have to be no
farther from the float64 statement than twice the oracle's own distance (and
at most 1e-4) -- none is (measured: 7e-6 at most at the default size).  The
learning rate and the step count are exact.  The new weights are checked
against a float64 update (clip_ + Muon / AdamW) from each implementation's
own pre-update state, as a fraction of the float64 change: Newton-Schulz
amplifies f32 rounding, and a weight whose change is small next to its value
holds that change only to its f32 spacing, so the device must be within
max(1e-5, 2 x the oracle's distance) -- measured equal to the oracle's, at
the f32 spacing of the weights."""
import numpy as np
import pytest

from conftest import TOL, rel_frob, to_dev, to_host

pytestmark = pytest.mark.gpu

SMALL = dict(width=4, cmid=6, dim=8, heads=2, depth3=2, dim4=12, heads4=2, depth4=1,
             mem_at=(1,), droppath=0.2, img=16)
PARENT6 = [0, 0, 1, 1, 2, 2]
CIFAR_MEAN = (0.5071, 0.4865, 0.4409)  # data.rs:13-14
CIFAR_STD = (0.2673, 0.2564, 0.2762)


def _i32(a):
    return to_dev(np.asarray(a, np.uint32).view(np.int32))


def _shuffle(rng, v):
    """Rng::shuffle (rng.rs:61-65)."""
    v = list(v)
    for i in range(len(v) - 1, 0, -1):
        j = rng.below(i + 1)
        v[i], v[j] = v[j], v[i]
    return v


def config4_inputs(orc, n, seed):
    """Config-4 batch: images uniform in [0, 1] normalised per channel
    (data.rs:96-98), labels uniform over 100, parent = a seeded shuffle of
    the 5-per-superclass assignment."""
    rng = orc.Rng(seed)
    parent = np.array(_shuffle(rng, np.arange(100) // 5), np.uint32)
    u = rng.uniform_vec(n * 3 * 32 * 32).reshape(n, 3, 32, 32)
    mean = np.array(CIFAR_MEAN, np.float32).reshape(1, 3, 1, 1)
    std = np.array(CIFAR_STD, np.float32).reshape(1, 3, 1, 1)
    x = ((u - mean) / std).astype(np.float32)
    labels = np.array([rng.below(100) for _ in range(n)], np.uint32)
    return x, labels, parent[labels].astype(np.uint32), parent


@pytest.fixture(scope="module")
def vit(orc):
    from oracle import pyvit
    return pyvit


def _check_init(dnet, onet):
    dps, ops = dnet.params(), onet.params()
    assert len(dps) == len(ops)
    for i, (d, o) in enumerate(zip(dps, ops)):
        assert np.array_equal(to_host(d.v).ravel(), o.v), f"parameter {i} differs"
        assert (d.decay, d.rows, d.cols) == (o.decay, o.rows if hasattr(o, "rows") else 0,
                                             o.cols if hasattr(o, "cols") else 0), i


@pytest.mark.parametrize("which", ["netcheck", "default"])
def test_init_bit_exact(rnn, orc, vit, which):
    from rustnn_amd.vit import RustViT
    if which == "netcheck":
        cfg, parent, nc, seed = SMALL, PARENT6, 3, 0x1234 ^ 0xBEEF
    else:
        cfg, parent, nc, seed = None, list(np.arange(100) // 5), 20, 1234
    dnet = RustViT(cfg, _i32(parent), nc, seed=seed)
    onet = vit.RustViT(cfg, parent, nc, seed)
    _check_init(dnet, onet)


def _errs(dev, orc_arrays):
    return [rel_frob(to_host(d).ravel(), np.ravel(o)) for d, o in zip(dev, orc_arrays)]


def _grad_check(dps, ops, f64_err_orc=None, f64_err_dev=None, what=""):
    """Every gradient within TOL of the oracle's, or (a cancelling sum) no
    farther from float64 than twice the oracle."""
    errs = _errs([p.g for p in dps], [p.g for p in ops])
    for i, e in enumerate(errs):
        if e < TOL:
            continue
        assert f64_err_orc is not None, f"{what} gradient {i} ({ops[i].v.size}): {e}"
        eo, ed = f64_err_orc[i], f64_err_dev[i]
        assert ed < max(2 * eo, TOL) and ed < 1e-4, (what, i, e, eo, ed)
    return errs


def test_forward_backward_netcheck_net(rnn, orc, vit):
    """The netcheck network (check.rs:397-450): outputs and every parameter
    gradient, against the oracle and the float64 statement."""
    import torch
    import test_oracle_vit_net as T
    from rustnn_amd.vit import RustViT
    onet, x, g = T._small_setup(orc, vit)
    dnet = RustViT(SMALL, _i32(PARENT6), 3, seed=0x1234 ^ 0xBEEF)
    ops, dps = onet.params(), dnet.params()
    for d, o in zip(dps, ops):
        d.v.copy_(to_dev(o.v))
    onet.drop_seed = dnet.drop_seed = 4242
    out_o = onet.forward(x, True)
    onet.backward(g)
    out_d = dnet.forward(to_dev(x).reshape(x.shape), True)
    dnet.backward({k: to_dev(v) for k, v in g.items()})
    for k in out_o:
        assert rel_frob(to_host(out_d[k]), out_o[k]) < TOL, k
    # float64 distances of both, for the cancelling sums
    _, eo = T.compare_with_f64(orc, SMALL, PARENT6, 3,
                               lambda: ([p.v for p in ops], [p.g for p in ops]),
                               lambda: out_o, x, g, 4242)
    _, ed = T.compare_with_f64(orc, SMALL, PARENT6, 3,
                               lambda: ([to_host(p.v) for p in dps], [to_host(p.g) for p in dps]),
                               lambda: {k: to_host(v) for k, v in out_d.items()}, x, g, 4242)
    errs = _grad_check(dps, ops, eo, ed, "netcheck")
    print("worst gradient errors vs oracle:", sorted(errs)[-5:])
    assert rel_frob(np.concatenate([to_host(p.g) for p in dps]),
                    np.concatenate([p.g for p in ops])) < TOL


def _mixed(n, seed):
    r = np.random.default_rng(seed)
    perm = r.permutation(n).astype(np.uint32)
    lam = r.uniform(0, 1, n).astype(np.float32)
    return perm, lam


def _state(ps, host):
    """(v, g, m, v2, decay, rows, cols) of each parameter, on the host."""
    out = []
    for p in ps:
        v2 = getattr(p, "v2", None)
        arr = [host(p.v), host(p.g), host(p.m),
               np.zeros_like(host(p.v)) if v2 is None else host(v2)]
        out.append(arr + [bool(p.decay), getattr(p, "rows", 0), getattr(p, "cols", 0)])
    return out


def update_f64(state, lr, wd, t, clip=1.0, mom=0.95, b1=0.9, b2=0.999, eps=1e-8, ns=3):
    """clip_ + Optim::step_all (optim.rs:177-251) in float64 from an f32
    state: returns the new weights."""
    from test_oracle_optim import ns_f64
    norm = np.sqrt(sum(float((s[1].astype(np.float64) ** 2).sum()) for s in state))
    sc = clip / norm if norm > clip else 1.0
    out = []
    for v, g, m, v2, decay, rows, cols in state:
        v, g, m, v2 = (a.astype(np.float64) for a in (v, g, m, v2))
        g = g * sc
        wdp = wd if decay else 0.0
        if rows > 0 and min(rows, cols) > 1:
            m = mom * m + g
            x = ns_f64(g + mom * m, rows, cols, ns)
            out.append(v - lr * (0.2 * np.sqrt(max(rows, cols)) * x + wdp * v))
        else:
            c1, c2 = 1 - b1 ** (t + 1), 1 - b2 ** (t + 1)
            m = b1 * m + (1 - b1) * g
            v2 = b2 * v2 + (1 - b2) * g * g
            out.append(v - lr * ((m / c1) / (np.sqrt(v2 / c2) + eps) + wdp * v))
    return out


def _update_check(before_d, before_o, after_d, after_o, lr, wd, t, what):
    """Each implementation's new weights against the float64 update from its
    own pre-update state, as a fraction of the float64 change: the device no
    farther from float64 than max(TOL, 2 x the oracle).  Newton-Schulz
    amplifies f32 rounding in the small singular directions of the momentum,
    and a weight whose change is small next to its value (BN gammas near 1
    move by about lr) holds that change only to its f32 spacing; `floor` is
    that spacing as a fraction of the change, which bounds how well any f32
    implementation can do, and the absolute cap allows 4 x it."""
    ref_d = update_f64(before_d, lr, wd, t)
    ref_o = update_f64(before_o, lr, wd, t)
    worst = (0.0, 0.0, 0.0)
    for i, (bd, bo, ad, ao, rd, ro) in enumerate(zip(before_d, before_o, after_d, after_o,
                                                      ref_d, ref_o)):
        chg = np.linalg.norm(rd - bd[0])
        if chg == 0:
            assert np.array_equal(ad, bd[0]), (what, i)
            continue
        ed = np.linalg.norm(ad - rd) / chg
        eo = np.linalg.norm(ao - ro) / np.linalg.norm(ro - bo[0])
        floor = np.linalg.norm(np.spacing(rd.astype(np.float32))) / chg
        assert ed < max(TOL, 2 * eo) and ed < max(1e-3, 4 * floor), (what, i, ed, eo, floor)
        if floor < 1e-3:  # the change is resolved in f32: report its error
            worst = max(worst, (ed, eo, floor))
    # the two weight changes against each other, whole vector
    dd = np.concatenate([a - b[0] for a, b in zip(after_d, before_d)])
    do = np.concatenate([a - b[0] for a, b in zip(after_o, before_o)])
    e = rel_frob(dd, do)
    assert e < 1e-3, (what, e)
    return worst, e


def test_trainer_steps_netcheck_net(rnn, orc, vit):
    """Three Trainer::steps (the second on a mixed batch): loss, hits, every
    gradient before each update, the learning rate, each weight change
    against float64 and the EMA."""
    from rustnn_amd.vit import RustViT, ViTStep
    nc, n = 3, 4
    hp = dict(ntrain=400, batch=n, epochs=10, warmup=1, seed=77)
    onet = vit.RustViT(SMALL, PARENT6, nc, 0x1234 ^ 0xBEEF)
    dnet = RustViT(SMALL, _i32(PARENT6), nc, seed=0x1234 ^ 0xBEEF)
    otr = vit.Trainer(onet, PARENT6, nc, hp)
    dtr = ViTStep(dnet, _i32(PARENT6), nc, hp)
    ops, dps = onet.params(), dnet.params()
    rng = orc.Rng(5)
    host_d = lambda t: to_host(t).ravel().copy()
    host_o = lambda a: np.array(a, np.float32).ravel()
    for step in range(3):
        x = rng.rand_vec(n * 3 * 16 * 16).reshape(n, 3, 16, 16)
        labels = np.array([rng.below(6) for _ in range(n)], np.uint32)
        coarse = np.array(PARENT6, np.uint32)[labels]
        perm, lam = _mixed(n, step) if step == 1 else (None, None)
        t_o, _, c_o, _ = otr.forward_backward(x, labels, coarse, perm, lam)
        t_d, c_d, _ = dtr.forward_backward(
            to_dev(x).reshape(x.shape), _i32(labels), _i32(coarse),
            None if perm is None else _i32(perm), None if lam is None else to_dev(lam))
        assert abs(float(t_d.item()) - t_o) <= TOL * abs(t_o), (step, float(t_d.item()), t_o)
        assert int(c_d.item()) == c_o
        errs = _grad_check(dps, ops, what=f"step {step}")
        before_d, before_o = _state(dps, host_d), _state(ops, host_o)
        t_opt = otr.t
        lr_o = otr.update()
        dtr.update()
        assert dtr.lr == lr_o and dtr.opt.t == otr.t
        worst, e = _update_check(before_d, before_o, [host_d(p.v) for p in dps],
                                 [host_o(p.v) for p in ops], lr_o, hp.get("wd", 0.06), t_opt,
                                 f"step {step}")
        print(f"step {step}: worst gradient {max(errs):.2e}; worst update vs f64 (device, "
              f"oracle, f32 floor) {worst[0]:.2e} {worst[1]:.2e} {worst[2]:.2e}; device vs "
              f"oracle {e:.2e}")
        assert rel_frob(np.concatenate([host_d(p.v) for p in dps]),
                        np.concatenate([p.v for p in ops])) < TOL
    ema_d = [to_host(w).ravel() for w in dtr.ema.w]
    assert max(rel_frob(a, b) for a, b in zip(ema_d, otr.ema_w)) < TOL


def test_trainer_step_default_batch128(rnn, orc, vit):
    """one Trainer::step of the default network at batch
    128 on the device against the oracle (outputs, loss, hits, every
    gradient, every weight's change)."""
    from rustnn_amd.vit import RustViT, ViTStep
    n = 128
    x, labels, coarse, parent = config4_inputs(orc, n, 2026)
    onet = vit.RustViT(None, list(parent), 20, 1234)
    dnet = RustViT(None, _i32(parent), 20, seed=1234)
    otr = vit.Trainer(onet, parent, 20)
    dtr = ViTStep(dnet, _i32(parent), 20)
    ops, dps = onet.params(), dnet.params()
    with orc.threads(16):
        t_o, _, c_o, out_o = otr.forward_backward(x, labels, coarse)
    t_d, c_d, out_d = dtr.forward_backward(to_dev(x).reshape(x.shape), _i32(labels),
                                           _i32(coarse))
    for k in out_o:
        e = rel_frob(to_host(out_d[k]), out_o[k])
        assert e < TOL, (k, e)
    assert abs(float(t_d.item()) - t_o) <= TOL * abs(t_o)
    assert int(c_d.item()) == c_o
    errs = _grad_check(dps, ops, what="default")
    host_d = lambda t: to_host(t).ravel().copy()
    host_o = lambda a: np.array(a, np.float32).ravel()
    before_d, before_o = _state(dps, host_d), _state(ops, host_o)
    with orc.threads(16):
        lr = otr.update()
    dtr.update()
    assert dtr.lr == lr
    worst, e = _update_check(before_d, before_o, [host_d(p.v) for p in dps],
                             [host_o(p.v) for p in ops], lr, 0.06, 0, "default")
    print(f"default: worst gradient {max(errs):.2e}; worst update vs f64 (device, oracle, "
          f"f32 floor) {worst[0]:.2e} {worst[1]:.2e} {worst[2]:.2e}; device vs oracle {e:.2e}")
    # the updated weights, whole vector (train.rs:346-387), and the EMA
    e_v = rel_frob(np.concatenate([host_d(p.v) for p in dps]),
                   np.concatenate([host_o(p.v) for p in ops]))
    print(f"default: updated weights device vs oracle {e_v:.2e}")
    assert e_v < TOL
    ema_d = [to_host(w).ravel() for w in dtr.ema.w]
    assert max(rel_frob(a, b) for a, b in zip(ema_d, otr.ema_w)) < TOL


def test_deferred_reductions_bit_identical(rnn, orc, vit):
    """ViTStep queues its backward's parameter-gradient reductions and runs
    them in one launch (rnn_ctx_set_defer / rnn_ctx_flush): every gradient
    equals the immediate path's bit for bit (default network, batch 128)."""
    from rustnn_amd.vit import RustViT, ViTStep
    n = 128
    x, labels, coarse, parent = config4_inputs(orc, n, 2027)
    grads = []
    for defer in (False, True):
        net = RustViT(None, _i32(parent), 20, seed=99)
        tr = ViTStep(net, _i32(parent), 20)
        tr.defer = defer
        tr.forward_backward(to_dev(x).reshape(x.shape), _i32(labels), _i32(coarse))
        grads.append([to_host(p.g).ravel().copy() for p in net.params()])
    assert len(grads[0]) == len(grads[1])
    for i, (a, b) in enumerate(zip(*grads)):
        assert np.array_equal(a, b), i


def test_reference_vitcheck_on_gpu(rnn, orc, vit):
    """vitcheck (check.rs:163-180) through the device layers: normcheck,
    attncheck (SelfAttn, CrossAttn over a 6x6 memory with dmem, a reader Block
    with DropPath) and netcheck, on one Rng stream that feeds the device
    constructors too, every check under the reference's 5e-3."""
    import refcheck
    from test_gpu_norm import GpuNorm
    errs = refcheck.vitcheck(orc, GpuNorm(), refcheck.GpuAttn())
    assert len(errs) == 16
    bad = {k: v for k, v in errs.items() if not v < refcheck.TOL}
    assert not bad, errs
