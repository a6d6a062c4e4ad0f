"""GPU parity: batched small attention (attn.rs Core forward/backward and
rel_index) against the CPU oracle, at BASELINE config 2 and at the reference's
attention gradcheck shapes (check.rs:294-358)."""
import numpy as np
import pytest

from conftest import TOL, rel_frob, to_dev, to_host

pytestmark = pytest.mark.gpu


def make_case(orc, n, h, dh, th, tw, mh, mw, variant, seed):
    """Self attention (mh == th): SelfAttn buffer [n, t, 3c] with q/k/v at
    0/c/2c (attn.rs:393-404).  Cross: q [n, tq, c], memory [n, tk, 2c] with
    K at 0, V at c (attn.rs:508-519)."""
    rng = orc.Rng(seed)
    c = h * dh
    tq, tk = th * tw, mh * mw
    relidx, nrel = orc.rel_index(th, tw, mh, mw)
    selfattn = (mh == th and mw == tw)
    scale = np.float32(1.0 / np.sqrt(dh))
    if selfattn:
        qkv = rng.rand_vec(n * tq * 3 * c) * scale
        q, kv = qkv, qkv
        geo = dict(qstride=3 * c, qoff=0, kvstride=3 * c, koff=c, voff=2 * c)
    else:
        q = rng.rand_vec(n * tq * c) * scale
        kv = rng.rand_vec(n * tk * 2 * c) * scale
        geo = dict(qstride=c, qoff=0, kvstride=2 * c, koff=0, voff=c)
    if variant == "plain":   # BASELINE config 2 as specified
        tau = np.ones(h, np.float32)
        rel = np.zeros(h * nrel, np.float32)
        mask = False
    else:                    # SelfAttn/CrossAttn defaults + random rel (check.rs:300, 334)
        tau = np.full(h, 1.0 / np.sqrt(dh), np.float32)
        rel = rng.rand_vec(h * nrel)
        mask = selfattn
    dout = rng.rand_vec(n * tq * c)
    return dict(q=q, kv=kv, geo=geo, tau=tau, rel=rel, mask=mask, relidx=relidx, nrel=nrel,
                dout=dout, tq=tq, tk=tk, selfattn=selfattn)


CASES = [
    # name, n, h, dh, th, tw, mh, mw, variant
    ("cfg2_plain", 128, 4, 32, 8, 8, 8, 8, "plain"),
    ("cfg2_lsa", 128, 4, 32, 8, 8, 8, 8, "lsa"),
    ("gc_self", 3, 2, 4, 3, 3, 3, 3, "lsa"),
    ("gc_cross", 3, 2, 4, 3, 3, 6, 6, "lsa"),
    ("dh64_t16", 16, 6, 64, 4, 4, 4, 4, "lsa"),
    ("dh64_t64", 8, 4, 64, 8, 8, 8, 8, "lsa"),
    # tq or tk above 64: the composed path (batched GEMMs + row kernels)
    # tq <= 64 and tk 128 / 256 with dh 32 / 64: one fused workgroup per
    # (image, head) (attn_fwd_long_kernel) in the forward
    ("cross_tk256", 8, 4, 64, 8, 8, 16, 16, "lsa"),   # the rustvit's cross-attention
    ("cross_tk128_dh32_tq49", 4, 3, 32, 7, 7, 8, 16, "lsa"),
    ("cross_tk256_dh32_tq36", 4, 2, 32, 6, 6, 16, 16, "plain"),
    ("self_t100", 4, 2, 48, 10, 10, 10, 10, "lsa"),   # masked self-attention, 100 tokens
    ("cross_tk81_dh80", 3, 2, 80, 3, 3, 9, 9, "lsa"),
]


@pytest.mark.parametrize("name,n,h,dh,th,tw,mh,mw,variant", CASES, ids=[c[0] for c in CASES])
def test_attn_parity(rnn, orc, name, n, h, dh, th, tw, mh, mw, variant):
    cs = make_case(orc, n, h, dh, th, tw, mh, mw, variant, seed=7)
    g = cs["geo"]
    d = orc.attn_desc(h, dh, cs["tq"], cs["tk"], g["qstride"], g["qoff"], g["kvstride"],
                      g["koff"], g["voff"], cs["relidx"], cs["nrel"], cs["mask"])
    with orc.threads(8):
        p_want, o_want = orc.attn_forward(d, n, cs["q"], cs["kv"], cs["tau"], cs["rel"])
    core = rnn.Core(h, dh, cs["tq"], cs["tk"], cs["relidx"], cs["nrel"], cs["mask"])
    Q = to_dev(cs["q"])
    KV = Q if cs["selfattn"] else to_dev(cs["kv"])
    TAU, REL = to_dev(cs["tau"]), to_dev(cs["rel"])
    P, O = core.forward(n, Q, g["qstride"], g["qoff"], KV, g["kvstride"], g["koff"], g["voff"],
                        TAU, REL)
    assert rel_frob(to_host(P), p_want) < TOL, "p"
    assert rel_frob(to_host(O), o_want) < TOL, "o"

    # backward: separate dq / dkv buffers with non-zero initial content (+=)
    nq, nkv = cs["q"].size, cs["kv"].size
    r = np.random.default_rng(3)
    dq0 = r.standard_normal(nq).astype(np.float32)
    dkv0 = r.standard_normal(nkv).astype(np.float32)
    dtau0 = r.standard_normal(h).astype(np.float32)
    drel0 = r.standard_normal(h * cs["nrel"]).astype(np.float32)
    with orc.threads(8):
        dq_w, dkv_w, dtau_w, drel_w = orc.attn_backward(d, n, cs["q"], cs["kv"], cs["tau"], p_want,
                                                        cs["dout"], dq0, dkv0, dtau0, drel0)
    dq, dkv = to_dev(dq0.copy()), to_dev(dkv0.copy())
    dtau, drel = to_dev(dtau0.copy()), to_dev(drel0.copy())
    core.backward(n, Q, g["qstride"], g["qoff"], KV, g["kvstride"], g["koff"], g["voff"], TAU,
                  to_dev(p_want), to_dev(cs["dout"]), dq, dkv, dtau, drel)
    assert rel_frob(to_host(dq) - dq0, dq_w - dq0) < TOL, "dq"
    assert rel_frob(to_host(dkv) - dkv0, dkv_w - dkv0) < TOL, "dkv"
    assert rel_frob(to_host(dtau) - dtau0, dtau_w - dtau0) < TOL, "dtau"
    assert rel_frob(to_host(drel) - drel0, drel_w - drel0) < TOL, "drel"


def _cols(size, stride, offs, width):
    """Mask of the columns [off, off + width) of every row, for each off."""
    m = np.zeros((size // stride, stride), bool)
    for off in offs:
        m[:, off:off + width] = True
    return m.ravel()


SET_CASES = [c for c in CASES if c[0] in ("cfg2_lsa", "gc_cross", "dh64_t16", "cross_tk256",
                                          "self_t100")]


@pytest.mark.parametrize("flags", [1, 2, 3])
@pytest.mark.parametrize("name,n,h,dh,th,tw,mh,mw,variant", SET_CASES,
                         ids=[c[0] for c in SET_CASES])
def test_attn_backward_set(rnn, orc, flags, name, n, h, dh, th, tw, mh, mw, variant):
    """rnn_attn_backward_ex: an operand flagged for overwriting receives what
    accumulating into a zeroed buffer gives (bit for bit), and its old
    contents (NaN here) are never read; an unflagged one accumulates."""
    cs = make_case(orc, n, h, dh, th, tw, mh, mw, variant, seed=11)
    g = cs["geo"]
    d = orc.attn_desc(h, dh, cs["tq"], cs["tk"], g["qstride"], g["qoff"], g["kvstride"],
                      g["koff"], g["voff"], cs["relidx"], cs["nrel"], cs["mask"])
    with orc.threads(8):
        p_w, _ = orc.attn_forward(d, n, cs["q"], cs["kv"], cs["tau"], cs["rel"])
    core = rnn.Core(h, dh, cs["tq"], cs["tk"], cs["relidx"], cs["nrel"], cs["mask"])
    Q = to_dev(cs["q"])
    KV = Q if cs["selfattn"] else to_dev(cs["kv"])
    TAU, P, DO = to_dev(cs["tau"]), to_dev(p_w), to_dev(cs["dout"])
    nq, nkv = cs["q"].size, cs["kv"].size
    r = np.random.default_rng(5)
    set_q, set_kv = bool(flags & 1), bool(flags & 2)
    dq0 = np.zeros(nq, np.float32) if set_q else r.standard_normal(nq).astype(np.float32)
    dkv0 = np.zeros(nkv, np.float32) if set_kv else r.standard_normal(nkv).astype(np.float32)
    dtau0 = r.standard_normal(h).astype(np.float32)
    drel0 = r.standard_normal(h * cs["nrel"]).astype(np.float32)
    # the accumulating call into zeroed buffers, then the flagged call into NaN
    want = [to_dev(a.copy()) for a in (dq0, dkv0, dtau0, drel0)]
    core.backward(n, Q, g["qstride"], g["qoff"], KV, g["kvstride"], g["koff"], g["voff"], TAU, P,
                  DO, *want)
    nan = np.float32(np.nan)
    got = [to_dev(np.full(nq, nan) if set_q else dq0.copy()),
           to_dev(np.full(nkv, nan) if set_kv else dkv0.copy()),
           to_dev(dtau0.copy()), to_dev(drel0.copy())]
    core.backward(n, Q, g["qstride"], g["qoff"], KV, g["kvstride"], g["koff"], g["voff"], TAU, P,
                  DO, *got, set_dq=set_q, set_dkv=set_kv)
    width = h * dh
    mq = _cols(nq, g["qstride"], [g["qoff"]], width)
    mkv = _cols(nkv, g["kvstride"], [g["koff"], g["voff"]], width)
    for nm, a, b, m in (("dq", got[0], want[0], mq), ("dkv", got[1], want[1], mkv),
                        ("dtau", got[2], want[2], None), ("drel", got[3], want[3], None)):
        a, b = to_host(a), to_host(b)
        if m is not None:
            a, b = a[m], b[m]
        assert np.isfinite(a).all() and np.array_equal(a, b), nm
    with orc.threads(8):
        dq_w, dkv_w, _, _ = orc.attn_backward(d, n, cs["q"], cs["kv"], cs["tau"], p_w, cs["dout"],
                                              dq0, dkv0, dtau0, drel0)
    assert rel_frob(to_host(got[0])[mq] - dq0[mq], dq_w[mq] - dq0[mq]) < TOL
    assert rel_frob(to_host(got[1])[mkv] - dkv0[mkv], dkv_w[mkv] - dkv0[mkv]) < TOL


@pytest.mark.parametrize("n,h,dh,t", [(32, 4, 32, 8), (4, 2, 48, 10)])
def test_attn_aliased_dq_dkv(rnn, orc, n, h, dh, t):
    """SelfAttn accumulates dq and dk/dv into one fused-QKV gradient buffer
    (attn.rs:418-438); the device path may take them aliased (both the
    register-resident kernels and, at 100 tokens, the composed path)."""
    cs = make_case(orc, n, h, dh, t, t, t, t, "lsa", seed=13)
    g = cs["geo"]
    T = t * t
    d = orc.attn_desc(h, dh, T, T, g["qstride"], 0, g["kvstride"], g["koff"], g["voff"],
                      cs["relidx"], cs["nrel"], True)
    p_w, _ = orc.attn_forward(d, n, cs["q"], cs["kv"], cs["tau"], cs["rel"])
    z = np.zeros(cs["q"].size, np.float32)
    dq_w, dkv_w, _, _ = orc.attn_backward(d, n, cs["q"], cs["kv"], cs["tau"], p_w, cs["dout"], z, z,
                                          np.zeros(h, np.float32),
                                          np.zeros(h * cs["nrel"], np.float32))
    want = dq_w + dkv_w  # attn.rs:438
    core = rnn.Core(h, dh, T, T, cs["relidx"], cs["nrel"], True)
    Q = to_dev(cs["q"])
    dab = to_dev(z.copy())
    dtau = to_dev(np.zeros(h, np.float32))
    drel = to_dev(np.zeros(h * cs["nrel"], np.float32))
    core.backward(n, Q, g["qstride"], 0, Q, g["kvstride"], g["koff"], g["voff"], to_dev(cs["tau"]),
                  to_dev(p_w), to_dev(cs["dout"]), dab, dab, dtau, drel)
    assert rel_frob(to_host(dab), want) < TOL


@pytest.mark.parametrize("th,tw,mh,mw", [(8, 8, 8, 8), (8, 8, 16, 16), (4, 4, 4, 4), (3, 3, 6, 6),
                                         (3, 3, 3, 3), (2, 5, 4, 10)])
def test_rel_index_bit_exact(rnn, orc, th, tw, mh, mw):
    want, nrel_w = orc.rel_index(th, tw, mh, mw)
    got, nrel = rnn.rel_index(th, tw, mh, mw)
    assert nrel == nrel_w and np.array_equal(got, want)
    dev = to_host(rnn.dbg_rel_index(th, tw, mh, mw)).view(np.uint32)
    assert np.array_equal(dev, want)


def test_attn_unsupported_shape_raises(rnn, orc):
    relidx, nrel = orc.rel_index(8, 8, 8, 8)  # dh = 80 at tq = tk = 64: beyond the kernel
    core = rnn.Core(1, 80, 64, 64, relidx, nrel, False)
    q = to_dev(np.zeros(64 * 80, np.float32))
    kv = to_dev(np.zeros(64 * 160, np.float32))
    with pytest.raises(rnn.RnnError):
        core.forward(1, q, 80, 0, kv, 160, 0, 80, to_dev(np.ones(1, np.float32)),
                     to_dev(np.zeros(nrel, np.float32)))
