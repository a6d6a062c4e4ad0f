"""Restatement of the reference's gradient-check harness (check.rs), run
against a pluggable conv / attention backend (the CPU oracle or the HIP path).

* dircheck (check.rs:16-40): central difference along a random direction v
  drawn from the same Rng, relative error |num - ana| / (|num| + |ana| + 1e-6).
* conv_layercheck (check.rs:503-546): the three conv layer shapes at seed 1234
  in the reference's exact Rng draw order (Kaiming W, x, r, then one direction
  per dircheck), tolerance 5e-3, eps = GC_EPS or 3e-4 (check.rs:55-60).
"""
import os

import numpy as np

TOL = 5e-3  # check.rs:42-44
SEED = 1234  # check.rs:778
CONV_SHAPES = [  # check.rs:505-509
    (3, 4, 3, 1, 1, 6, "conv 3x3/s1"),
    (4, 6, 1, 2, 0, 8, "conv 1x1/s2"),
    (4, 5, 3, 2, 1, 7, "conv 3x3/s2"),
]


def gc_eps():
    try:
        return float(os.environ.get("GC_EPS", "3e-4"))
    except ValueError:
        return 3e-4


def dircheck(base, grad, eps, rng, lossf):
    """check.rs:19-40 (f32 perturbation, as the reference)."""
    n = base.size
    v = rng.rand_vec(n)
    e = np.float32(eps)
    lp = np.float32(lossf((base + e * v).astype(np.float32)))
    lm = np.float32(lossf((base - e * v).astype(np.float32)))
    num = (lp - lm) / (np.float32(2.0) * e)
    ana = np.float32(np.dot(grad.astype(np.float64), v.astype(np.float64)))
    return float(abs(num - ana) / (abs(num) + abs(ana) + 1e-6))


def dot32(a, b):
    return np.float32(np.dot(np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()))


class OracleConv:
    """Conv backend on the CPU oracle."""

    def __init__(self, orc):
        self.o = orc

    def spec(self, cin, cout, k, s, p, h):
        return self.o.ConvSpec.make(cin, cout, k, s, p, h, h)

    def forward(self, sp, n, x, w):
        return self.o.conv2d_forward(sp, n, x, w).ravel()

    def backward(self, sp, n, dy, x, w, dw):
        dw = self.o.conv2d_backward_w(sp, n, dy, x, dw).ravel()
        return self.o.conv2d_backward_x(sp, n, dy, w).ravel(), dw


class GpuConv:
    """Conv backend on the HIP path (C ABI through rustnn_amd)."""

    def __init__(self, rnn):
        import torch
        self.r = rnn
        self.t = torch

    def _d(self, a):
        return self.t.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()

    def _h(self, t):
        self.t.cuda.synchronize()
        return t.cpu().numpy().ravel()

    def spec(self, cin, cout, k, s, p, h):
        return self.r.ConvSpec.make(cin, cout, k, s, p, h, h)

    def forward(self, sp, n, x, w):
        return self._h(self.r.conv2d_forward(sp, n, self._d(x), self._d(w)))

    def backward(self, sp, n, dy, x, w, dw):
        DW = self._d(dw)
        self.r.conv2d_backward_w(sp, n, self._d(dy), self._d(x), DW)
        dx = self.r.conv2d_backward_x(sp, n, self._d(dy), self._d(w))
        return self._h(dx), self._h(DW)


def conv_layercheck(rng_cls, backend):
    """Returns [(tag, err)] for dx and dw of each conv shape (check.rs:510-546)."""
    rng = rng_cls(SEED)
    eps = gc_eps()
    out = []
    for cin, cout, k, s, p, hh, tag in CONV_SHAPES:
        fan_in = cin * k * k
        sc = np.float32(np.sqrt(np.float32(2.0) / np.float32(fan_in)))  # nn.rs:95-100
        w = (rng.rand_vec(cout * fan_in) * sc).astype(np.float32)
        x = rng.rand_vec(2 * cin * hh * hh)
        sp = backend.spec(cin, cout, k, s, p, hh)
        y0 = backend.forward(sp, 2, x, w)
        r = rng.rand_vec(y0.size)
        dx, dw = backend.backward(sp, 2, r, x, w, np.zeros(w.size, np.float32))
        e = dircheck(x, dx, eps, rng, lambda c: dot32(backend.forward(sp, 2, c, w), r))
        out.append((f"{tag} dx", e))
        e = dircheck(w, dw, eps, rng, lambda c: dot32(backend.forward(sp, 2, x, c), r))
        out.append((f"{tag} dw", e))
    return out
