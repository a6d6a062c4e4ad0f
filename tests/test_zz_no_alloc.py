"""GPU: rnn_conv2d_backward_w_noalloc (no counterpart in the reference; for
callers that cannot allocate device memory) against rnn_conv2d_backward_w,
the entry point it mirrors (Conv2d::backward_w, nn.rs:193-227).

Both run the same dW kernel and slab reduction, so the results must agree bit
for bit; the oracle checks the values themselves at the parity tolerance.  Two
calls in a row, the second on a smaller input, through the C ABI; the context
of the no-allocation calls must end with no workspace at all."""
import ctypes as C

import numpy as np
import pytest

from conftest import TOL, rel_frob, to_dev, to_host

pytestmark = pytest.mark.gpu

# (n, cin, cout, k, stride, pad, h): BASELINE config 0, then a smaller
# stride-2 shape and the few-input-channel stem (its own dW kernel).
CALLS = [(128, 32, 32, 3, 1, 1, 32), (16, 32, 64, 3, 2, 1, 16), (8, 3, 32, 3, 1, 1, 32)]


def _inputs(orc, sp, n, seed):
    rng = orc.Rng(seed)
    x = rng.rand_vec(n * sp.cin * sp.h * sp.w)
    dy = rng.rand_vec(n * sp.cout * sp.hw)
    dw0 = rng.rand_vec(sp.cout * sp.ckk)
    return x, dy, dw0


def test_noalloc_matches_backward_w(rnn, orc):
    L = rnn.lib()
    ctx_na = rnn.Context(0)   # only no-allocation calls
    ctx_ref = rnn.Context(0)  # the existing entry point (grows its workspace)
    for i, (n, cin, cout, k, s, p, h) in enumerate(CALLS):
        print(f"noalloc call {i}: n={n} {cin}->{cout} k{k} s{s} {h}x{h}", flush=True)
        sp = orc.ConvSpec.make(cin, cout, k, s, p, h, h)
        gsp = rnn.ConvSpec.make(cin, cout, k, s, p, h, h)
        x, dy, dw0 = _inputs(orc, sp, n, 100 + i)
        X, DY = to_dev(x), to_dev(dy)
        dw_na, dw_ref = to_dev(dw0.copy()), to_dev(dw0.copy())
        ctx_na.check(L.rnn_conv2d_backward_w_noalloc(ctx_na.h, C.byref(gsp), n,
                                                     C.c_void_p(DY.data_ptr()),
                                                     C.c_void_p(X.data_ptr()),
                                                     C.c_void_p(dw_na.data_ptr())))
        ctx_ref.check(L.rnn_conv2d_backward_w(ctx_ref.h, C.byref(gsp), n,
                                              C.c_void_p(DY.data_ptr()),
                                              C.c_void_p(X.data_ptr()),
                                              C.c_void_p(dw_ref.data_ptr())))
        ctx_na.synchronize()
        ctx_ref.synchronize()
        got, want = to_host(dw_na), to_host(dw_ref)
        assert np.array_equal(got, want), f"call {i}: differs from rnn_conv2d_backward_w"
        with orc.threads(8):
            orc_dw = orc.conv2d_backward_w(sp, n, dy, x, dw0).ravel()
        assert rel_frob(got - dw0, orc_dw - dw0) < TOL, f"call {i}: oracle"
    assert ctx_na.workspace_bytes() == 0, "the no-allocation calls grew a workspace"
    ctx_na.close()
    ctx_ref.close()


def test_noalloc_rejects_oversize(rnn):
    """A shape whose partial slabs exceed the fixed scratch is refused on the
    host before anything is launched (1024 -> 1024 3x3: one slab alone is
    37.7 MB)."""
    L = rnn.lib()
    ctx = rnn.Context(0)
    gsp = rnn.ConvSpec.make(1024, 1024, 3, 1, 1, 4, 4)
    n = 1
    x = to_dev(np.zeros(n * 1024 * 16, np.float32))
    dy = to_dev(np.zeros(n * 1024 * 16, np.float32))
    dw = to_dev(np.zeros(1024 * 1024 * 9, np.float32))
    rc = L.rnn_conv2d_backward_w_noalloc(ctx.h, C.byref(gsp), n, C.c_void_p(dy.data_ptr()),
                                         C.c_void_p(x.data_ptr()), C.c_void_p(dw.data_ptr()))
    assert rc == rnn.RNN_E_UNSUPPORTED
    assert b"scratch" in L.rnn_ctx_last_error(ctx.h)
    assert ctx.workspace_bytes() == 0
    ctx.close()


def test_noalloc_calls_on_two_streams(rnn, orc):
    """Two contexts on two streams of one GPU call the no-allocation entry
    point back to back with no synchronisation between them: the library
    orders them on the shared scratch, so each result equals
    rnn_conv2d_backward_w's bit for bit."""
    import torch
    L = rnn.lib()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    ca, cb, cref = rnn.Context(0, stream=s1), rnn.Context(0, stream=s2), rnn.Context(0)
    jobs = []
    for i, (ctx, (n, cin, cout, k, s, p, h)) in enumerate(zip((ca, cb), CALLS[:2])):
        sp = orc.ConvSpec.make(cin, cout, k, s, p, h, h)
        gsp = rnn.ConvSpec.make(cin, cout, k, s, p, h, h)
        x, dy, dw0 = _inputs(orc, sp, n, 300 + i)
        X, DY = to_dev(x), to_dev(dy)
        torch.cuda.synchronize()
        jobs.append((ctx, gsp, n, X, DY, to_dev(dw0.copy()), to_dev(dw0.copy())))
    for ctx, gsp, n, X, DY, dw_na, _ in jobs:
        print(f"noalloc on stream {ctx.stream_ptr():#x}: n={n}", flush=True)
        ctx.check(L.rnn_conv2d_backward_w_noalloc(ctx.h, C.byref(gsp), n,
                                                  C.c_void_p(DY.data_ptr()),
                                                  C.c_void_p(X.data_ptr()),
                                                  C.c_void_p(dw_na.data_ptr())))
    for ctx, gsp, n, X, DY, _, dw_ref in jobs:
        cref.check(L.rnn_conv2d_backward_w(cref.h, C.byref(gsp), n, C.c_void_p(DY.data_ptr()),
                                           C.c_void_p(X.data_ptr()),
                                           C.c_void_p(dw_ref.data_ptr())))
    torch.cuda.synchronize()
    for i, (ctx, gsp, n, X, DY, dw_na, dw_ref) in enumerate(jobs):
        assert np.array_equal(to_host(dw_na), to_host(dw_ref)), f"call {i}"
    for c in (ca, cb, cref):
        c.close()
