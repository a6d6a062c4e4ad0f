"""Oracle pins for optim.rs (oracle/orc_optim.c): each function against an
independent statement of the same mathematics (float64 numpy, torch's AdamW),
plus properties a plausible slip would break."""
import numpy as np
import pytest

NS = (3.4445, -4.7750, 2.0315)


def ns_f64(g, rows, cols, steps, coef=NS):
    """newton_schulz (optim.rs:124-145) in float64 with numpy matmuls."""
    x = g.astype(np.float64).reshape(rows, cols)
    tr = rows > cols
    if tr:
        x = x.T
    x = x / (np.sqrt((x * x).sum()) + 1e-7)
    a_, b_, c_ = coef
    for _ in range(steps):
        a = x @ x.T
        x = a_ * x + (b_ * a + c_ * (a @ a)) @ x
    return (x.T if tr else x).ravel()


def test_powi_matches_repeated_products(orc):
    for base in (0.9, 0.999, 1.5, 0.5):
        for n in (0, 1, 2, 3, 7, 64, 1000, 4097):
            with np.errstate(over="ignore"):
                want = float(np.float64(np.float32(base)) ** n)
            got = orc.powi(base, n)
            if want > 3.4e38:  # past float32: the f32 product overflows
                assert got == float("inf")
                continue
            # square-and-multiply: each squaring doubles the relative error, so
            # the bound grows like n rounding errors
            assert abs(got - want) <= (2 * n + 2) * 2.0 ** -24 * abs(want) + 1e-30, (base, n)
    assert orc.powi(0.9, 0) == 1.0 and orc.powi(0.9, 1) == np.float32(0.9)
    assert orc.powi(0.9, 2) == np.float32(0.9) * np.float32(0.9)
    assert orc.powi(2.0, -3) == 0.125


@pytest.mark.parametrize("rows,cols", [(8, 16), (16, 8), (33, 70), (70, 33), (64, 64), (12, 300)])
def test_newton_schulz_matches_f64(orc, rows, cols):
    g = np.random.default_rng(rows * 100 + cols).standard_normal(rows * cols).astype(np.float32)
    got = orc.newton_schulz(g, rows, cols, 3)
    want = ns_f64(g, rows, cols, 3)
    err = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert err < 2e-5, err
    # a planted slip in the restatement (b and c swapped) is far outside that
    bad = ns_f64(g, rows, cols, 3, (NS[0], NS[2], NS[1]))
    assert np.linalg.norm(bad - want) / np.linalg.norm(want) > 1e-2


def test_newton_schulz_transpose_symmetry_and_spectrum(orc):
    g = np.random.default_rng(5).standard_normal(24 * 40).astype(np.float32)
    a = orc.newton_schulz(g, 24, 40, 5).reshape(24, 40)
    b = orc.newton_schulz(g.reshape(24, 40).T.copy(), 40, 24, 5).reshape(40, 24)
    assert np.array_equal(a, b.T)  # the tall path is the wide path on G^T
    s = np.linalg.svd(a.astype(np.float64), compute_uv=False)
    # the quintic drives every singular value into a band around 1
    assert s.min() > 0.6 and s.max() < 1.25, s


def test_muon_step_matches_f64(orc):
    rng = np.random.default_rng(11)
    rows, cols = 20, 36
    v = rng.standard_normal(rows * cols).astype(np.float32)
    g = rng.standard_normal(rows * cols).astype(np.float32)
    m = rng.standard_normal(rows * cols).astype(np.float32)
    lr, wd, mom = 0.02, 0.05, 0.95
    v64, g64, m64 = v.astype(np.float64), g.astype(np.float64), m.astype(np.float64)
    m64 = mom * m64 + g64
    g64 = g64 + mom * m64
    o = ns_f64(g64, rows, cols, 3)
    want_v = v64 - lr * (0.2 * np.sqrt(max(rows, cols)) * o + wd * v64)
    orc.muon_step(v, g, m, rows, cols, True, lr, wd, mom, 3)
    assert np.linalg.norm(v - want_v) / np.linalg.norm(want_v) < 1e-6
    assert np.linalg.norm(m - m64) / np.linalg.norm(m64) < 1e-6
    assert not g.any()


def test_muon_steps_equals_per_matrix(orc):
    """The OpenMP loop over matrices (the CPU baseline's form) gives exactly
    what muon_step gives per matrix, on shapes both sides of the transpose."""
    rng = np.random.default_rng(12)
    shapes = [(48, 20, True), (20, 48, False), (33, 33, True), (64, 8, True), (5, 70, False)]
    one, many = [], []
    for r, c, d in shapes:
        arrs = [rng.standard_normal(r * c).astype(np.float32) for _ in range(3)]
        one.append([a.copy() for a in arrs] + [r, c, d])
        many.append([a.copy() for a in arrs] + [r, c, d])
    for v, g, m, r, c, d in one:
        orc.muon_step(v, g, m, r, c, d, 0.02, 0.05, 0.95, 3)
    orc.muon_steps(many, 0.02, 0.05, 0.95, 3, threads=4)
    for a, b in zip(one, many):
        for k in range(3):
            assert np.array_equal(a[k], b[k])


def test_adam_matches_torch_adamw(orc):
    import torch
    rng = np.random.default_rng(3)
    n = 1000
    v = rng.standard_normal(n).astype(np.float32)
    m = np.zeros(n, np.float32)
    v2 = np.zeros(n, np.float32)
    p = torch.tensor(v.astype(np.float64), requires_grad=True)
    opt = torch.optim.AdamW([p], lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.05)
    for t in range(5):
        g = rng.standard_normal(n).astype(np.float32)
        gg = g.copy()
        orc.adam_step(v, gg, m, v2, True, 1e-3, 0.05, t)
        assert not gg.any()
        p.grad = torch.tensor(g.astype(np.float64))
        opt.step()
        want = p.detach().numpy()
        assert np.linalg.norm(v - want) / np.linalg.norm(want) < 1e-6, t
    # no decay: the weight-decay term is dropped
    v0 = v.copy()
    gz = np.zeros(n, np.float32)
    orc.adam_step(v, gz, np.zeros(n, np.float32), np.zeros(n, np.float32), False, 1e-3, 0.05, 0)
    assert np.array_equal(v, v0)  # zero gradient, zero moments, no decay: unchanged


def test_clip_matches_f64(orc):
    rng = np.random.default_rng(4)
    lens = [7, 100, 3, 250]
    g = (rng.standard_normal(sum(lens)) * 3).astype(np.float32)
    norm64 = np.sqrt((g.astype(np.float64) ** 2).sum())
    gg = g.copy()
    norm = orc.clip(gg, lens, 1.0)
    assert abs(norm - norm64) <= 1e-6 * norm64
    assert abs(np.sqrt((gg.astype(np.float64) ** 2).sum()) - 1.0) < 1e-5
    gg = g.copy()
    assert orc.clip(gg, lens, 1e9) == pytest.approx(norm64, rel=1e-6)
    assert np.array_equal(gg, g)  # under the limit: untouched


def test_ema_matches_f64(orc):
    rng = np.random.default_rng(9)
    w = rng.standard_normal(50).astype(np.float32)
    v = rng.standard_normal(50).astype(np.float32)
    for t, decay in ((1, 0.9998), (5, 0.9998), (10000, 0.9998), (3, 0.1)):
        d = min(decay, (1 + t) / (10 + t))
        want = d * w.astype(np.float64) + (1 - d) * v.astype(np.float64)
        ww = w.copy()
        orc.ema_update(ww, v, decay, t)
        assert np.abs(ww - want).max() <= 1e-6 * np.abs(want).max() + 1e-7, (t, decay)
