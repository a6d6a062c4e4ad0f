"""Writes the golden fixtures under tests/golden/ (run in the build container).

The reference ships no golden vectors for this path, so these are produced by an
independent library -- PyTorch on the CPU in float64 -- from seeded numpy
inputs:

* conv_*.npz: F.conv2d forward, torch.nn.grad.conv2d_input (dX) and
  conv2d_weight (dW) at the reference's gradcheck conv shapes
  (check.rs:505-509) plus one stage-1 shape on a small batch.
* attn_*.npz: the Core semantics (attn.rs:148-343: tau*QK^T + rel[idx],
  diagonal mask, row softmax, PV) evaluated with torch autograd for the
  gradients dQ, dK, dV, dtau, drel at the attention gradcheck shapes
  (check.rs:294-358: c=8, h=2, 3x3 grid, cross memory 6x6).

Inputs are float32 (stored); outputs are the float64 results (stored as f64).
Usage: python tests/golden/make_golden.py
"""
import os
import zlib

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))

CONV = [
    # name, n, cin, cout, k, stride, pad, h
    ("conv_gc_3x3s1", 2, 3, 4, 3, 1, 1, 6),
    ("conv_gc_1x1s2", 2, 4, 6, 1, 2, 0, 8),
    ("conv_gc_3x3s2", 2, 4, 5, 3, 2, 1, 7),
    ("conv_s1_32x32", 1, 32, 32, 3, 1, 1, 32),
    ("conv_s2_odd", 3, 5, 7, 3, 2, 1, 9),
]


def conv_fixture(name, n, cin, cout, k, s, p, h):
    r = np.random.default_rng(zlib.crc32(name.encode()))
    x = r.standard_normal((n, cin, h, h)).astype(np.float32)
    w = (r.standard_normal((cout, cin, k, k)) * np.sqrt(2.0 / (cin * k * k))).astype(np.float32)
    X, W = torch.from_numpy(x).double(), torch.from_numpy(w).double()
    y = F.conv2d(X, W, stride=s, padding=p)
    dy = r.standard_normal(tuple(y.shape)).astype(np.float32)
    DY = torch.from_numpy(dy).double()
    dx = torch.nn.grad.conv2d_input(X.shape, W, DY, stride=s, padding=p)
    dw = torch.nn.grad.conv2d_weight(X, W.shape, DY, stride=s, padding=p)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), spec=np.array([n, cin, cout, k, s, p, h]),
                        x=x, w=w, dy=dy, y=y.numpy(), dx=dx.numpy(), dw=dw.numpy())


def rel_index_def(th, tw, mh, mw):
    """rel_index written from attn.rs:21-72 (the torch fixture needs a table;
    the tests also pin the oracle's and the device's tables against this)."""
    if mh == th:
        sy, sx, scale, oy, ox = 2 * th - 1, 2 * tw - 1, 1, th - 1, tw - 1
    else:
        sy, sx, scale, oy, ox = 2 * (th - 1) + mh, 2 * (tw - 1) + mw, 2, mh - 1, mw - 1
    idx = [(scale * qy - my + oy) * sx + (scale * qx - mx + ox)
           for qy in range(th) for qx in range(tw) for my in range(mh) for mx in range(mw)]
    return np.array(idx, np.uint32), sy * sx


def attn_fixture(name, n, h, dh, th, tw, mh, mw, mask):
    r = np.random.default_rng(zlib.crc32(name.encode()))
    tq, tk = th * tw, mh * mw
    idx, nrel = rel_index_def(th, tw, mh, mw)
    q = (r.standard_normal((n, h, tq, dh)) / np.sqrt(dh)).astype(np.float32)
    k = (r.standard_normal((n, h, tk, dh)) / np.sqrt(dh)).astype(np.float32)
    v = (r.standard_normal((n, h, tk, dh)) / np.sqrt(dh)).astype(np.float32)
    tau = (np.full(h, 1 / np.sqrt(dh)) * (1 + 0.1 * r.standard_normal(h))).astype(np.float32)
    rel = r.standard_normal((h, nrel)).astype(np.float32)
    dout = r.standard_normal((n, h, tq, dh)).astype(np.float32)
    Q, K, V = (torch.from_numpy(a).double().requires_grad_() for a in (q, k, v))
    T = torch.from_numpy(tau).double().requires_grad_()
    R = torch.from_numpy(rel).double().requires_grad_()
    S = Q @ K.transpose(-1, -2)
    bias = R[:, torch.from_numpy(idx.astype(np.int64)).view(tq, tk)]  # [h, tq, tk]
    X = T.view(1, h, 1, 1) * S + bias.unsqueeze(0)
    if mask:
        X = X.masked_fill(torch.eye(tq, tk, dtype=torch.bool), float("-inf"))
    P = torch.softmax(X, dim=-1)
    O = P @ V
    O.backward(torch.from_numpy(dout).double())
    np.savez_compressed(
        os.path.join(HERE, name + ".npz"),
        dims=np.array([n, h, dh, th, tw, mh, mw, int(mask)]), relidx=idx, nrel=np.array(nrel),
        q=q, k=k, v=v, tau=tau, rel=rel, dout=dout, p=P.detach().numpy(), o=O.detach().numpy(),
        dq=Q.grad.numpy(), dk=K.grad.numpy(), dv=V.grad.numpy(), dtau=T.grad.numpy(),
        drel=R.grad.numpy())


def main():
    for c in CONV:
        conv_fixture(*c)
    attn_fixture("attn_gc_self", 3, 2, 4, 3, 3, 3, 3, True)
    attn_fixture("attn_gc_cross", 3, 2, 4, 3, 3, 6, 6, False)
    attn_fixture("attn_cfg2_small", 2, 2, 32, 8, 8, 8, 8, True)


if __name__ == "__main__":
    main()
