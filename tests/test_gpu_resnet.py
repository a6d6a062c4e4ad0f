"""GPU parity: the device-resident ResNet train step (model.rs, nn.rs,
train.rs:686-699) through the C ABI (rnn_resnet_*) against the CPU oracle's
ResNet (oracle/pymodel.py) on identical seeded inputs.

* initialisation: ResNet::new's Kaiming draws and BN / classifier init,
  bit-exact, in for_each_param / for_each_buffer order;
* one train step at BASELINE config 3 (ResNet-20 W32, batch 128, 32x32,
  smooth 0.1, SGD 0.2 / 0.9 / 5e-4): logits, loss, gradients, updated
  parameters, momenta and running statistics;
* the reference's full-network gradcheck (check.rs:727-775) through the GPU;
* the recorded hipGraph replays bit-identically to eager execution, with eager
  work and synchronisation between the replays."""
import numpy as np
import pytest

from conftest import rel_frob, to_dev, to_host

import refcheck

pytestmark = pytest.mark.gpu

# Tolerances of the whole-network comparison (relative Frobenius): 1e-5 for
# the logits, the loss, the whole gradient vector and every gradient tensor.
# A tensor above 1e-5 against the oracle must be no farther from an
# independent float64 statement of the network (tests/torch_resnet.py) than
# twice the oracle's own distance: the oracle itself sits up to 2.8e-5 from
# float64 on the betas of the BNs whose gradient sums cancel (zero-initialised
# gamma), so no f32 summation order can promise 1e-5 against it there.
TOL_FWD = 1e-5
TOL_GRAD = 1e-5


def _cfg3_inputs(orc, n, seed=2026):
    """Config 3: images uniform in [0, 1] normalised per channel with the
    reference's MEAN / STD (data.rs:13-14, 96-98); labels uniform in 0..99."""
    rng = orc.Rng(seed)
    u = rng.uniform_vec(n * 3 * 32 * 32).reshape(n, 3, 32, 32)
    mean = np.array([0.5071, 0.4865, 0.4409], np.float32)[None, :, None, None]
    std = np.array([0.2673, 0.2564, 0.2762], np.float32)[None, :, None, None]
    x = ((u - mean) / std).astype(np.float32)
    labels = np.array([rng.below(100) for _ in range(n)], np.uint32)
    return x, labels


def _oracle_flat(net, attr):
    return np.concatenate([getattr(p, attr).ravel() for p in net.params()])


def test_init_bit_exact(rnn, orc):
    from oracle import pymodel
    from rustnn_amd.model import ResNet
    for depth, width, nc, seed in ((3, 32, 100, 0), (1, 4, 10, 1234)):
        want = pymodel.ResNet(depth, width, nc, seed)
        got = ResNet(depth, width, nc, seed)
        lens = got.tensor_lens()
        assert [n for n, _ in lens] == [p.v.size for p in want.params()]
        assert [d for _, d in lens] == [p.decay for p in want.params()]
        assert np.array_equal(to_host(got.params()), _oracle_flat(want, "v"))
        assert np.array_equal(to_host(got.buffers()), np.concatenate(want.buffers()))
        assert not to_host(got.grads()).any() and not to_host(got.momenta()).any()
        assert got.flops(32, 32) == want.flops(32, 32)
        got.close()


def test_train_step_config3(rnn, orc):
    """One BASELINE config-3 step on the device vs the oracle."""
    import torch
    from oracle import pymodel
    from rustnn_amd.model import ResNet
    n = 128
    x, labels = _cfg3_inputs(orc, n)
    want = pymodel.ResNet(3, 32, 100, 7)
    got = ResNet(3, 32, 100, 7)
    with orc.threads(16):
        lg_w = want.forward(x, True)
        loss_w, corr_w, dl_w = orc.softmax_ce(lg_w, labels, 0.1)
        want.backward(dl_w)
    X = to_dev(x)
    L = torch.from_numpy(labels.astype(np.int32)).cuda()
    lg = got.forward(X, True)
    from rustnn_amd.nn import softmax_ce
    loss, corr, dl = softmax_ce(lg, L, 0.1)
    got.backward(dl)
    print("logits err", rel_frob(to_host(lg), lg_w), "grad err",
          rel_frob(to_host(got.grads()), _oracle_flat(want, "g")))
    assert rel_frob(to_host(lg), lg_w) < TOL_FWD
    assert abs(float(to_host(loss)[0]) - loss_w) < 1e-5 * abs(loss_w)
    assert int(to_host(corr)[0]) == corr_w
    g_got, g_want = to_host(got.grads()), _oracle_flat(want, "g")
    import torch_resnet
    torch.set_num_threads(16)
    z64, l64, g64 = torch_resnet.resnet_f64([p.v for p in want.params()], 3, 32, 100, x, labels,
                                            0.1)
    assert rel_frob(lg_w, z64) < TOL_FWD and abs(loss_w - l64) < 1e-5 * abs(l64)
    off = 0
    above = []
    for i, (p, gf) in enumerate(zip(want.params(), g64)):
        gd = g_got[off:off + p.v.size]
        off += p.v.size
        e = rel_frob(gd, p.g)
        if e < TOL_GRAD:
            continue
        ed, eo = rel_frob(gd, gf), rel_frob(p.g, gf)
        above.append((i, p.v.size, e, ed, eo))
        assert ed < max(TOL_GRAD, 2 * eo), (i, p.v.size, e, ed, eo)
    print("tensors above 1e-5 vs the oracle (index, size, vs oracle, device vs f64, oracle "
          "vs f64):", above)
    assert rel_frob(g_got, g_want) < TOL_GRAD
    assert rel_frob(to_host(got.buffers()), np.concatenate(want.buffers())) < 1e-6
    # the SGD step on those gradients
    with orc.threads(16):
        want.step(0.2, 0.9, 5e-4)
    got.step(0.2, 0.9, 5e-4)
    assert rel_frob(to_host(got.params()), _oracle_flat(want, "v")) < 1e-6
    assert rel_frob(to_host(got.momenta()), _oracle_flat(want, "m")) < TOL_GRAD
    assert not to_host(got.grads()).any()
    got.close()


def test_bn_stats_in_conv_store_pass(rnn, orc, monkeypatch):
    """The batch statistics taken in the forward convs' store passes (the
    default) == the same network with the statistics in passes of their own
    (RNN_BN_PASSES=separate).  Only the order of the f64 partial sums
    differs, so the steps agree to f32 rounding."""
    import torch
    from rustnn_amd.model import ResNet
    n = 64
    fused = ResNet(3, 32, 100, 13)
    monkeypatch.setenv("RNN_BN_PASSES", "separate")
    sep = ResNet(3, 32, 100, 13)
    monkeypatch.delenv("RNN_BN_PASSES")
    for net in (fused, sep):
        net.set_graph(False)
    la, lb = torch.zeros(1, device="cuda"), torch.zeros(1, device="cuda")
    for step in range(3):
        x, labels = _cfg3_inputs(orc, n, seed=300 + step)
        X = to_dev(x)
        L = torch.from_numpy(labels.astype(np.int32)).cuda()
        fused.train_step(X, L, 0.1, 0.2, 0.9, 5e-4, la)
        sep.train_step(X, L, 0.1, 0.2, 0.9, 5e-4, lb)
        assert abs(float(to_host(la)[0]) - float(to_host(lb)[0])) < 1e-6 * abs(
            float(to_host(lb)[0])), step
        assert rel_frob(to_host(fused.momenta()), to_host(sep.momenta())) < 1e-6, step
        assert rel_frob(to_host(fused.params()), to_host(sep.params())) < 1e-6, step
        assert rel_frob(to_host(fused.buffers()), to_host(sep.buffers())) < 1e-6, step
    fused.close()
    sep.close()


def _relu_flips(got, want):
    """The ReLU masks the backward reads (every block's h and output, and
    the stem's output as block 0's input) on the device against the
    oracle's, after a train forward of both: [(array, flat index, device
    value, oracle value, rms of the tensor)] for the elements where exactly
    one of the two is > 0; `array` is the oracle's saved activation."""
    out = []
    for k, ob in enumerate(want.blocks):
        pairs = [(1, ob.h1), (4, ob.out)] + ([(10, want.stem_out)] if k == 0 else [])
        for which, ref in pairs:
            dv, rv = to_host(got.dbg_buffer(k, which)), ref.reshape(-1)
            rms = float(np.sqrt(np.mean(rv.astype(np.float64) ** 2)))
            for i in np.flatnonzero((dv > 0) != (rv > 0)):
                out.append((ref, int(i), float(dv[i]), float(rv[i]), rms))
    return out


def test_fused_step_batch128_vs_oracle(rnn, orc):
    """The benchmarked path itself: rnn_resnet_train_step at BASELINE config
    3's batch of 128, driven as bench.py drives it (the batch written into
    the network's input slots, eager steps with the weight gradients on the
    second stream, BN statistics in the forward convs' store passes, the
    batch-128 dW tile plans) for three steps against the oracle's step
    (train.rs:686-699; model.rs:39-71, nn.rs:102-110): loss, hits, updated
    parameters, momenta and running statistics after each step.

    Each step starts both from the same state: the oracle takes the device's
    parameters, momenta and running statistics first (they start
    bit-identical).  The momenta hold the step's gradient; where a tensor's
    is more than 1e-5 from the oracle's, the device's must be no farther
    from a float64 statement of the same step (tests/torch_resnet.py from the
    same state) than twice the oracle's own distance; the same for the whole
    vector.

    ReLU ties: the convolutions add in another order than the reference's
    K-blocked chains, so their outputs differ in the last bits, and a ReLU
    input within that distance of zero can land on the other side: the
    backward then passes (or drops) one more gradient element, which the
    BatchNorm backward of that block amplifies (its gradient is what is left
    after removing the per-channel mean and xhat components) -- by about 2e-3
    on one block's gradients for one such element.  Every mask the backward
    reads is compared with the oracle's; each differing element must be a
    tie to within 1e-6 of the tensor's rms, and the oracle's backward then
    takes the device's value there (so both drop or pass the same elements)
    before the gradients are compared."""
    import torch
    import torch_resnet
    from oracle import pymodel
    from rustnn_amd.model import ResNet
    torch.set_num_threads(16)
    n, lr, mom, wd, smooth = 128, 0.2, 0.9, 5e-4, 0.1
    want = pymodel.ResNet(3, 32, 100, 7)
    got = ResNet(3, 32, 100, 7)
    active, _ = got.graph_state()
    assert not active  # the default: eager steps on two streams
    lens = got.tensor_lens()
    offs = np.cumsum([0] + [k for k, _ in lens])
    decay = np.concatenate([np.full(k, float(d)) for k, d in lens])
    xs, ls = got.inputs(n, 32, 32)
    loss = torch.zeros(1, device="cuda")
    corr = torch.zeros(1, dtype=torch.int32, device="cuda")
    ties = 0
    for step in range(3):
        v0, m0 = to_host(got.params()).copy(), to_host(got.momenta()).copy()
        if step:
            for arrs, flat in (([p.v for p in want.params()], v0),
                               ([p.m for p in want.params()], m0),
                               (want.buffers(), to_host(got.buffers()))):
                off = 0
                for a in arrs:
                    np.copyto(a, flat[off:off + a.size].reshape(a.shape))
                    off += a.size
                assert off == flat.size
        x, labels = _cfg3_inputs(orc, n, seed=2026 + step)
        xs.copy_(to_dev(x).reshape(xs.shape))
        ls.copy_(torch.from_numpy(labels.astype(np.int32)).cuda())
        got.train_step(None, None, smooth, lr, mom, wd, loss, corr)
        with orc.threads(16):
            lg_w = want.forward(x, True)
            flips = _relu_flips(got, want)
            for ref, i, dv, ov, rms in flips:
                assert abs(dv) <= 1e-6 * rms and abs(ov) <= 1e-6 * rms, (step, i, dv, ov, rms)
                ref.reshape(-1)[i] = dv  # the oracle's backward follows the device here
            ties += len(flips)
            loss_w, corr_w, dl_w = orc.softmax_ce(lg_w, labels, smooth)
            want.backward(dl_w)
            want.step(lr, mom, wd)
        m_d, m_o = to_host(got.momenta()), _oracle_flat(want, "m")
        e_loss = abs(float(to_host(loss)[0]) - loss_w) / abs(loss_w)
        e_v = rel_frob(to_host(got.params()), _oracle_flat(want, "v"))
        e_m = rel_frob(m_d, m_o)
        e_b = rel_frob(to_host(got.buffers()), np.concatenate(want.buffers()))
        print(f"step {step}: loss {e_loss:.2e} params {e_v:.2e} momenta {e_m:.2e} "
              f"buffers {e_b:.2e}; ReLU ties {[(i, dv, ov) for _, i, dv, ov, _ in flips]}")
        assert e_loss < 1e-5, step
        assert int(to_host(corr)[0]) == corr_w, step
        assert e_v < 1e-6, step
        assert e_b < 1e-6, step
        errs = [rel_frob(m_d[offs[i]:offs[i + 1]], m_o[offs[i]:offs[i + 1]])
                for i in range(len(lens))]
        if e_m < TOL_GRAD and max(errs) < TOL_GRAD:
            continue
        _, _, g64 = torch_resnet.resnet_f64([v0[offs[i]:offs[i + 1]] for i in range(len(lens))],
                                            3, 32, 100, x, labels, smooth)
        m64 = mom * m0.astype(np.float64) + np.concatenate([g.ravel() for g in g64]) + \
            wd * decay * v0.astype(np.float64)
        for i in range(len(lens)):
            sl = slice(int(offs[i]), int(offs[i + 1]))
            ed, eo = rel_frob(m_d[sl], m64[sl]), rel_frob(m_o[sl], m64[sl])
            assert errs[i] < TOL_GRAD or ed < max(TOL_GRAD, 2 * eo), (step, i, errs[i], ed, eo)
        ed, eo = rel_frob(m_d, m64), rel_frob(m_o, m64)
        print(f"step {step}: momenta vs float64: device {ed:.2e}, oracle {eo:.2e}")
        assert e_m < TOL_GRAD or ed < max(TOL_GRAD, 2 * eo), step
    print("ReLU ties over the three steps:", ties)
    assert not got.graph_state()[0]
    got.close()


@pytest.mark.parametrize("n", [32, 128])
def test_fused_train_step_matches_layer_calls(rnn, orc, n):
    """rnn_resnet_train_step (eager, then graph) == forward + softmax_ce +
    backward + step called one by one, bit for bit, at batch 32 and at the
    benchmark's batch of 128 (whose dW tile plans differ)."""
    import torch
    from rustnn_amd.model import ResNet
    from rustnn_amd.nn import softmax_ce
    a, b = ResNet(3, 32, 100, 11), ResNet(3, 32, 100, 11)
    a.set_graph(True)  # b's backward runs its weight gradients on the side stream
    loss = torch.zeros(1, device="cuda")
    corr = torch.zeros(1, dtype=torch.int32, device="cuda")
    for step in range(4):
        x, labels = _cfg3_inputs(orc, n, seed=50 + step)
        X = to_dev(x)
        L = torch.from_numpy(labels.astype(np.int32)).cuda()
        a.train_step(X, L, 0.1, 0.2, 0.9, 5e-4, loss, corr)
        lg = b.forward(X, True)
        lb, cb, dl = softmax_ce(lg, L, 0.1)
        b.backward(dl)
        b.step(0.2, 0.9, 5e-4)
        assert float(to_host(loss)[0]) == float(to_host(lb)[0]), step
        assert int(to_host(corr)[0]) == int(to_host(cb)[0]), step
        assert np.array_equal(to_host(a.params()), to_host(b.params())), step
        assert np.array_equal(to_host(a.momenta()), to_host(b.momenta())), step
        assert np.array_equal(to_host(a.buffers()), to_host(b.buffers())), step
    active, why = a.graph_state()
    assert active, why
    a.close()
    b.close()


def test_train_step_from_input_slots(rnn, orc):
    """rnn_resnet_inputs: batches written in place into the network's input
    slots and stepped with x = labels = NULL == the same batches passed by
    pointer, bit for bit, through eager, recording and replay calls."""
    import torch
    from rustnn_amd.model import ResNet
    n = 32
    a, b = ResNet(3, 32, 100, 5), ResNet(3, 32, 100, 5)
    a.set_graph(True)
    xs, ls = a.inputs(n, 32, 32)
    assert tuple(xs.shape) == (n, 3, 32, 32) and tuple(ls.shape) == (n,)
    la, lb = torch.zeros(1, device="cuda"), torch.zeros(1, device="cuda")
    for step in range(4):
        x, labels = _cfg3_inputs(orc, n, seed=120 + step)
        X = to_dev(x)
        L = torch.from_numpy(labels.astype(np.int32)).cuda()
        xs.copy_(X)
        ls.copy_(L)
        a.train_step(None, None, 0.1, 0.2, 0.9, 5e-4, la)
        b.train_step(X, L, 0.1, 0.2, 0.9, 5e-4, lb)
        assert float(to_host(la)[0]) == float(to_host(lb)[0]), step
        assert np.array_equal(to_host(a.params()), to_host(b.params())), step
        assert np.array_equal(to_host(a.buffers()), to_host(b.buffers())), step
    assert a.graph_state()[0]
    a.close()
    b.close()


def test_graph_replays_match_eager(rnn, orc):
    """Graph replays (one stream) with eager work and synchronisation in
    between, each checked against an eager network stepping on the same
    inputs (weight gradients on the side stream), bit for bit."""
    import torch
    from rustnn_amd.model import ResNet
    n = 64
    g, e = ResNet(3, 32, 100, 3), ResNet(3, 32, 100, 3)
    g.set_graph(True)
    e.set_graph(False)
    for step in range(5):
        x, labels = _cfg3_inputs(orc, n, seed=80 + step)
        X = to_dev(x)
        L = torch.from_numpy(labels.astype(np.int32)).cuda()
        g.train_step(X, L, 0.1, 0.2, 0.9, 5e-4)
        junk = torch.randn(1 << 20, device="cuda")  # unrelated eager work
        junk.mul_(2.0).sum().item()
        e.train_step(X, L, 0.1, 0.2, 0.9, 5e-4)
        torch.cuda.synchronize()
        assert np.array_equal(to_host(g.params()), to_host(e.params())), step
        assert np.array_equal(to_host(g.buffers()), to_host(e.buffers())), step
    assert g.graph_state()[0] and not e.graph_state()[0]
    g.close()
    e.close()


def test_resnet_gradcheck_gpu(rnn, orc):
    """check.rs:727-775 through the device ResNet (tolerance 5e-3)."""
    from oracle import pymodel
    err = refcheck.resnet_gradcheck(orc, refcheck.GpuNN(pymodel))
    assert err < refcheck.TOL, err


def test_gradcheck_net_matches_oracle(rnn, orc):
    """The gradcheck network (ResNet(1, 4, 10), batch 8 at 16x16) step by
    step against the oracle: logits, gradients, updated parameters."""
    import torch
    from oracle import pymodel
    from rustnn_amd.model import ResNet
    from rustnn_amd.nn import softmax_ce
    want, got = pymodel.ResNet(1, 4, 10, 1234), ResNet(1, 4, 10, 1234)
    rng = orc.Rng(99)
    for step in range(3):
        x = rng.rand_vec(8 * 3 * 16 * 16).reshape(8, 3, 16, 16)
        labels = np.array([rng.below(10) for _ in range(8)], np.uint32)
        lw, _, _ = want.train_step(x, labels, 0.1, 0.2, 0.9, 5e-4)
        lg = got.forward(to_dev(x), True)
        loss, _, dl = softmax_ce(lg, torch.from_numpy(labels.astype(np.int32)).cuda(), 0.1)
        got.backward(dl)
        got.step(0.2, 0.9, 5e-4)
        assert abs(float(to_host(loss)[0]) - lw) < 1e-5 * abs(lw), step
        assert rel_frob(to_host(got.params()), _oracle_flat(want, "v")) < 1e-5, step
        assert rel_frob(to_host(got.buffers()), np.concatenate(want.buffers())) < 1e-5, step
    got.close()
