"""numpy front end of the CPU oracle (liborc.so).

TEST INFRASTRUCTURE ONLY: a restatement of the reference's CPU algorithm
(lsiddd/rustnn) used to check the HIP product path and to time the
reference-style CPU baseline.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s cpu_baseline leg may import this module; nothing under
``rustnn_amd/`` does.

Each wrapper names the reference function (file:line) the C code restates.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liborc.so")

MR, NR, KC = 6, 16, 256  # gemm.rs:11-13

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
_sz = C.c_size_t


def build(force: bool = False) -> str:
    """Compile liborc.so with the committed Makefile."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-C", HERE, "-B" if force else "all"], check=True,
                       stdout=subprocess.DEVNULL)
    return LIB_PATH


class ConvSpec(C.Structure):
    """ConvSpec (conv.rs:9-20) with oh/ow as Conv2d::out_dim (nn.rs:147-150)."""
    _fields_ = [(n, C.c_uint32) for n in
                ("cin", "cout", "k", "stride", "pad", "h", "w", "oh", "ow")]

    @classmethod
    def make(cls, cin, cout, k, stride, pad, h, w):
        return cls(cin, cout, k, stride, pad, h, w,
                   (h + 2 * pad - k) // stride + 1, (w + 2 * pad - k) // stride + 1)

    @property
    def ckk(self):
        return self.cin * self.k * self.k

    @property
    def hw(self):
        return self.oh * self.ow


class AttnDesc(C.Structure):
    """Core (attn.rs:74-84) plus the stride/offset arguments of forward/backward."""
    _fields_ = [("h", _sz), ("dh", _sz), ("tq", _sz), ("tk", _sz),
                ("qstride", _sz), ("qoff", _sz), ("kvstride", _sz), ("koff", _sz),
                ("voff", _sz), ("nrel", _sz), ("relidx", C.POINTER(C.c_uint32)),
                ("mask_diag", C.c_int)]


class RngState(C.Structure):
    _fields_ = [("s", C.c_uint64 * 4)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        build()
        L = C.CDLL(LIB_PATH)
        P = C.POINTER
        L.orc_rng_new.argtypes = [P(RngState), C.c_uint64]
        L.orc_rng_next_u64.argtypes = [P(RngState)]
        L.orc_rng_next_u64.restype = C.c_uint64
        L.orc_rng_below.argtypes = [P(RngState), _sz]
        L.orc_rng_below.restype = _sz
        L.orc_rng_uniform.argtypes = [P(RngState)]
        L.orc_rng_uniform.restype = C.c_float
        L.orc_rng_normal.argtypes = [P(RngState)]
        L.orc_rng_normal.restype = C.c_float
        L.orc_rand_vec.argtypes = [P(RngState), _f32p, _sz]
        L.orc_rand_uniform_vec.argtypes = [P(RngState), _f32p, _sz]
        L.orc_trunc_normal.argtypes = [P(RngState), _f32p, _sz, C.c_float]
        L.orc_set_threads.argtypes = [C.c_int]
        L.orc_set_threads.restype = C.c_int
        L.orc_get_threads.restype = C.c_int
        L.orc_set_simd.argtypes = [C.c_int]
        L.orc_set_simd.restype = C.c_int
        L.orc_packed_a_len.argtypes = [_sz, _sz]
        L.orc_packed_a_len.restype = _sz
        L.orc_packed_b_len.argtypes = [_sz, _sz]
        L.orc_packed_b_len.restype = _sz
        L.orc_pack_a.argtypes = [_f32p, _sz, _sz, C.c_int, _f32p]
        L.orc_pack_b.argtypes = [_f32p, _sz, _sz, C.c_int, _f32p]
        L.orc_transpose_to_panel.argtypes = [_f32p, _sz, _sz, _f32p]
        L.orc_micro_kernel.argtypes = [_sz, _f32p, _f32p, _f32p, _sz, _sz, _sz, C.c_int]
        L.orc_matmul.argtypes = [_sz, _sz, _sz, _f32p, C.c_int, _f32p, C.c_int, _f32p, C.c_int]
        L.orc_gemm_small.argtypes = L.orc_matmul.argtypes
        L.orc_matmul_dw.argtypes = [_sz, _sz, _sz, _f32p, _f32p, _f32p]
        L.orc_fold_leaves.argtypes = [_sz, C.c_int, P(_sz), P(_sz), _sz]
        L.orc_fold_leaves.restype = _sz
        sp = P(ConvSpec)
        L.orc_rowmap.argtypes = [sp, _u32p]
        L.orc_im2col.argtypes = [sp, _f32p, _f32p]
        L.orc_conv_forward_image.argtypes = [sp, _f32p, _f32p, _f32p]
        L.orc_conv_dx_image.argtypes = [sp, _f32p, _f32p, _f32p]
        L.orc_conv_dw_image.argtypes = [sp, _f32p, _f32p, _f32p]
        L.orc_conv2d_forward.argtypes = [sp, _sz, _f32p, _f32p, _f32p]
        L.orc_conv2d_backward_w.argtypes = [sp, _sz, _f32p, _f32p, _f32p]
        L.orc_conv2d_backward_x.argtypes = [sp, _sz, _f32p, _f32p, _f32p]
        L.orc_rel_index.argtypes = [_sz, _sz, _sz, _sz, _u32p]
        L.orc_rel_index.restype = _sz
        ad = P(AttnDesc)
        L.orc_attn_forward.argtypes = [ad, _sz, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p]
        L.orc_attn_backward.argtypes = [ad, _sz, _f32p, _f32p, _f32p, _f32p, _f32p,
                                        _f32p, _f32p, _f32p, _f32p]
        L.orc_linear_forward.argtypes = [_sz, _sz, _sz, _f32p, _f32p, C.c_void_p, _f32p]
        L.orc_linear_backward.argtypes = [_sz, _sz, _sz, _f32p, _f32p, _f32p, _f32p,
                                          C.c_void_p, _f32p]
        L.orc_bn_train_forward.argtypes = [_sz, _sz, _sz, _f32p, _f32p, _f32p, _f32p, _f32p,
                                           _f32p, C.c_void_p, _f32p, C.c_float, C.c_float,
                                           C.c_int]
        L.orc_bn_eval_forward.argtypes = [_sz, _sz, _sz, _f32p, _f32p, _f32p, _f32p, _f32p,
                                          C.c_float, C.c_int]
        L.orc_bn_backward.argtypes = [_sz, _sz, _sz, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p,
                                      _f32p]
        L.orc_relu_back.argtypes = [_sz, _f32p, _f32p]
        L.orc_add.argtypes = [_sz, _f32p, _f32p]
        L.orc_add_relu.argtypes = [_sz, _f32p, _f32p]
        L.orc_gap_forward.argtypes = [_sz, _sz, _f32p, _f32p]
        L.orc_gap_backward.argtypes = [_sz, _sz, _f32p, _f32p]
        L.orc_fc_forward.argtypes = [_sz, _sz, _sz, _f32p, _f32p, _f32p, _f32p]
        L.orc_fc_backward.argtypes = [_sz, _sz, _sz, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p]
        L.orc_softmax_ce.argtypes = [_sz, _sz, _f32p, _u32p, C.c_float, _f32p, P(_sz)]
        L.orc_softmax_ce.restype = C.c_float
        L.orc_sgd_step.argtypes = [_sz, _f32p, _f32p, _f32p, C.c_float, C.c_float, C.c_float]
        L.orc_powi.argtypes = [C.c_float, C.c_int]
        L.orc_powi.restype = C.c_float
        L.orc_newton_schulz.argtypes = [_f32p, _sz, _sz, _sz]
        L.orc_muon_step.argtypes = [_f32p, _f32p, _f32p, _sz, _sz, C.c_int, C.c_float,
                                    C.c_float, C.c_float, _sz]
        _pp = P(C.POINTER(C.c_float))
        L.orc_muon_steps.argtypes = [_sz, _pp, _pp, _pp, P(_sz), P(_sz), P(C.c_int), C.c_float,
                                     C.c_float, C.c_float, _sz, C.c_int]
        L.orc_adam_step.argtypes = [_sz, _f32p, _f32p, _f32p, _f32p, C.c_int, C.c_float,
                                    C.c_float, C.c_float, C.c_float, C.c_float, _sz]
        L.orc_clip.argtypes = [_f32p, P(_sz), _sz, C.c_float]
        L.orc_clip.restype = C.c_float
        L.orc_ema_update.argtypes = [_sz, _f32p, _f32p, C.c_float, _sz]
        L.orc_lr_at.argtypes = [C.c_float, C.c_float, _sz, _sz, _sz]
        L.orc_lr_at.restype = C.c_float
        vp = C.c_void_p
        L.orc_ln_forward.argtypes = [_sz, _sz, _f32p, _f32p, _f32p, C.c_float, _f32p, vp, vp]
        L.orc_ln_backward.argtypes = [_sz, _sz, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p]
        L.orc_layerscale_forward.argtypes = [_sz, _sz, _f32p, _f32p, _f32p]
        L.orc_layerscale_backward.argtypes = [_sz, _sz, _f32p, _f32p, _f32p, _f32p, _f32p]
        L.orc_swiglu_forward.argtypes = [_sz, _sz, _f32p, _f32p]
        L.orc_swiglu_backward.argtypes = [_sz, _sz, _f32p, _f32p, _f32p]
        L.orc_dwconv3_forward.argtypes = [_sz, _sz, _sz, _sz, _f32p, _f32p, _f32p, _f32p]
        L.orc_dwconv3_backward.argtypes = [_sz, _sz, _sz, _sz, _f32p, _f32p, _f32p, _f32p,
                                           _f32p, _f32p]
        L.orc_seqpool_forward.argtypes = [_sz, _sz, _sz, _f32p, _f32p, _f32p, _f32p]
        L.orc_seqpool_backward.argtypes = [_sz, _sz, _sz, _f32p, _f32p, _f32p, _f32p, _f32p,
                                           _f32p]
        L.orc_taxo_target.argtypes = [_sz, _u32p, _sz, C.c_float, C.c_float, _f32p]
        L.orc_uniform_target.argtypes = [_sz, _sz, C.c_float, _f32p]
        L.orc_soft_targets.argtypes = [_sz, _sz, _sz, _u32p, vp, vp, vp, vp, C.c_int, C.c_float,
                                       C.c_float, _f32p, vp]
        L.orc_ce_soft.argtypes = [_sz, _sz, _f32p, _f32p, _u32p, C.c_float, _f32p, P(_sz)]
        L.orc_ce_soft.restype = C.c_float
        L.orc_kl_distill.argtypes = [_sz, _sz, _f32p, _f32p, C.c_float, C.c_float, _f32p]
        L.orc_kl_distill.restype = C.c_float
        L.orc_hint_mse.argtypes = [_sz, _sz, _f32p, _f32p, C.c_float, _f32p]
        L.orc_hint_mse.restype = C.c_float
        L.orc_drop_path.argtypes = [_sz, _sz, _f32p, C.c_float, C.c_uint64, _f32p]
        L.orc_token_merge.argtypes = [_sz, _sz, _sz, _f32p, _f32p]
        L.orc_taxo_combine.argtypes = [_sz, _sz, _sz, _u32p, _f32p, _f32p]
        L.orc_taxo_combine_backward.argtypes = [_sz, _sz, _sz, _u32p, _f32p, _f32p, _f32p]
        u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
        L.orc_crop_flip_normalize.argtypes = [u8p, _f32p, C.c_long, C.c_long, C.c_int]
        L.orc_randaugment.argtypes = [u8p, C.c_float, _sz, P(RngState)]
        L.orc_ra_op.argtypes = [u8p, _sz, C.c_float, C.c_float]
        L.orc_cifar_batch_train.argtypes = [u8p, u8p, u8p, _u32p, _sz, _sz, C.c_float, _sz,
                                            C.c_float, _sz, C.c_uint64, _f32p, _u32p, _u32p]
        L.orc_mix_batch.argtypes = [_f32p, _sz, C.c_float, C.c_float, C.c_float, P(RngState),
                                    _u32p, _f32p]
        L.orc_fnv1a_bytes.argtypes = [C.c_uint64, C.c_char_p, _sz]
        L.orc_fnv1a_bytes.restype = C.c_uint64
        L.orc_fnv1a_f32.argtypes = [C.c_uint64, _f32p, _sz]
        L.orc_fnv1a_f32.restype = C.c_uint64
        _lib = L
    return _lib


def _f(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------- rng.rs
class Rng:
    """Rng (rng.rs:3-66): xoshiro256++ seeded by splitmix64."""

    def __init__(self, seed: int):
        self.st = RngState()
        lib().orc_rng_new(C.byref(self.st), C.c_uint64(seed & 0xFFFFFFFFFFFFFFFF))

    def next_u64(self) -> int:
        return int(lib().orc_rng_next_u64(C.byref(self.st)))

    def below(self, n: int) -> int:
        return int(lib().orc_rng_below(C.byref(self.st), n))

    def uniform(self) -> float:
        return float(lib().orc_rng_uniform(C.byref(self.st)))

    def normal(self) -> float:
        return float(lib().orc_rng_normal(C.byref(self.st)))

    def rand_vec(self, n: int) -> np.ndarray:
        """rand_vec (rng.rs:70-72)."""
        out = np.empty(n, np.float32)
        if n:
            lib().orc_rand_vec(C.byref(self.st), out, n)
        return out

    def trunc_normal(self, n: int, std) -> np.ndarray:
        """Param::trunc_normal's values (nn.rs:77-89); std is an f32."""
        out = np.empty(n, np.float32)
        if n:
            lib().orc_trunc_normal(C.byref(self.st), out, n, float(np.float32(std)))
        return out

    def uniform_vec(self, n: int) -> np.ndarray:
        out = np.empty(n, np.float32)
        if n:
            lib().orc_rand_uniform_vec(C.byref(self.st), out, n)
        return out


class threads:
    """Context manager: number of OpenMP workers of the parallel drivers."""

    def __init__(self, n: int):
        self.n = n

    def __enter__(self):
        self.old = lib().orc_set_threads(self.n)
        return self

    def __exit__(self, *a):
        lib().orc_set_threads(self.old)


def set_simd(on: bool) -> bool:
    return bool(lib().orc_set_simd(1 if on else 0))


# ---------------------------------------------------------------- gemm.rs
def pack_a(a, m, k, transposed=False):
    """PackedA::pack / pack_t (gemm.rs:54-113); zero where never written."""
    out = np.zeros(lib().orc_packed_a_len(m, k), np.float32)
    if out.size:
        lib().orc_pack_a(_f(a).ravel(), m, k, int(transposed), out)
    return out


def pack_b(b, n, k, transposed=False):
    """PackedB::pack / pack_t (gemm.rs:340-400); zero where never written."""
    out = np.zeros(lib().orc_packed_b_len(n, k), np.float32)
    if out.size:
        lib().orc_pack_b(_f(b).ravel(), n, k, int(transposed), out)
    return out


def transpose_to_panel(src, lds, kc):
    out = np.zeros(kc * NR, np.float32)
    lib().orc_transpose_to_panel(_f(src).ravel(), lds, kc, out)
    return out


def matmul(m, n, k, a, at, b, bt, c=None, acc=False):
    """matmul (gemm.rs:434-493).  Returns C [m*n] (flat)."""
    c = np.zeros(m * n, np.float32) if c is None else _f(c).ravel().copy()
    if m and n:
        lib().orc_matmul(m, n, k, _f(a).ravel() if a.size else np.zeros(1, np.float32), int(at),
                         _f(b).ravel() if b.size else np.zeros(1, np.float32), int(bt), c, int(acc))
    return c


def gemm_small(m, n, k, a, at, b, bt, c=None, acc=False):
    """gemm_small (gemm.rs:500-545): k == 0 leaves C untouched."""
    c = np.zeros(m * n, np.float32) if c is None else _f(c).ravel().copy()
    one = np.zeros(1, np.float32)
    lib().orc_gemm_small(m, n, k, _f(a).ravel() if a.size else one, int(at),
                         _f(b).ravel() if b.size else one, int(bt),
                         c if c.size else one, int(acc))
    return c


def matmul_dw(m, n, k, a, b, c):
    """matmul_dw (gemm.rs:555-598): returns C + A^T B."""
    c = _f(c).ravel().copy()
    one = np.zeros(1, np.float32)
    lib().orc_matmul_dw(m, n, k, _f(a).ravel() if a.size else one,
                        _f(b).ravel() if b.size else one, c if c.size else one)
    return c


def fold_leaves(length, nthreads):
    lo = (_sz * 256)()
    hi = (_sz * 256)()
    nl = lib().orc_fold_leaves(length, nthreads, lo, hi, 256)
    return [(lo[i], hi[i]) for i in range(nl)]


# ---------------------------------------------------------------- conv.rs
def rowmap(sp: ConvSpec):
    out = np.zeros(3 * sp.ckk, np.uint32)
    lib().orc_rowmap(C.byref(sp), out)
    return out.reshape(-1, 3)


def im2col(sp: ConvSpec, x_img):
    col = np.zeros(sp.ckk * sp.hw, np.float32)
    lib().orc_im2col(C.byref(sp), _f(x_img).ravel(), col)
    return col.reshape(sp.ckk, sp.hw)


def conv2d_forward(sp: ConvSpec, n, x, w):
    """Conv2d::forward (nn.rs:166-185) -> y [n, cout, oh, ow]."""
    y = np.empty(n * sp.cout * sp.hw, np.float32)
    lib().orc_conv2d_forward(C.byref(sp), n, _f(x).ravel(), _f(w).ravel(), y)
    return y.reshape(n, sp.cout, sp.oh, sp.ow)


def conv2d_backward_w(sp: ConvSpec, n, dy, x, dw=None):
    """Conv2d::backward_w (nn.rs:193-227): returns dw + sum_i dW_i."""
    dw = np.zeros(sp.cout * sp.ckk, np.float32) if dw is None else _f(dw).ravel().copy()
    lib().orc_conv2d_backward_w(C.byref(sp), n, _f(dy).ravel(), _f(x).ravel(), dw)
    return dw.reshape(sp.cout, sp.ckk)


def conv2d_backward_x(sp: ConvSpec, n, dy, w):
    """dX half of Conv2d::backward (nn.rs:230-250) -> dx [n, cin, h, w]."""
    dx = np.empty(n * sp.cin * sp.h * sp.w, np.float32)
    lib().orc_conv2d_backward_x(C.byref(sp), n, _f(dy).ravel(), _f(w).ravel(), dx)
    return dx.reshape(n, sp.cin, sp.h, sp.w)


# ---------------------------------------------------------------- attn.rs
def rel_index(th, tw, mh, mw):
    """rel_index (attn.rs:53-72) -> (idx [th*tw*mh*mw] u32, nrel)."""
    idx = np.zeros(th * tw * mh * mw, np.uint32)
    nrel = lib().orc_rel_index(th, tw, mh, mw, idx)
    return idx, int(nrel)


def attn_desc(h, dh, tq, tk, qstride, qoff, kvstride, koff, voff, relidx, nrel, mask_diag):
    relidx = np.ascontiguousarray(relidx, np.uint32)
    d = AttnDesc(h, dh, tq, tk, qstride, qoff, kvstride, koff, voff, nrel,
                 relidx.ctypes.data_as(C.POINTER(C.c_uint32)), int(mask_diag))
    d._keep = relidx
    return d


def attn_forward(d: AttnDesc, n, q, kv, tau, rel):
    """Core::forward (attn.rs:148-223) -> (p [n,h,tq,tk], o [n,tq,h*dh])."""
    p = np.empty(n * d.h * d.tq * d.tk, np.float32)
    o = np.empty(n * d.tq * d.h * d.dh, np.float32)
    lib().orc_attn_forward(C.byref(d), n, _f(q).ravel(), _f(kv).ravel(), _f(tau).ravel(),
                           _f(rel).ravel(), p, o)
    return p, o


def attn_backward(d: AttnDesc, n, q, kv, tau, p, dout, dq, dkv, dtau, drel):
    """Core::backward (attn.rs:226-343): returns updated (dq, dkv, dtau, drel)."""
    dq, dkv = _f(dq).ravel().copy(), _f(dkv).ravel().copy()
    dtau, drel = _f(dtau).ravel().copy(), _f(drel).ravel().copy()
    lib().orc_attn_backward(C.byref(d), n, _f(q).ravel(), _f(kv).ravel(), _f(tau).ravel(),
                            _f(p).ravel(), _f(dout).ravel(), dq, dkv, dtau, drel)
    return dq, dkv, dtau, drel


# ---------------------------------------------------------------- linear.rs
def linear_forward(rows, fin, fout, x, w, b=None):
    y = np.empty(rows * fout, np.float32)
    bb = _f(b).ravel() if b is not None else None
    lib().orc_linear_forward(rows, fin, fout, _f(x).ravel(), _f(w).ravel(),
                             bb.ctypes.data if bb is not None else None, y)
    return y


def linear_backward(rows, fin, fout, dy, x, w, dw, db=None):
    """Returns (dw', db', dx)."""
    dw = _f(dw).ravel().copy()
    db = _f(db).ravel().copy() if db is not None else None
    dx = np.empty(rows * fin, np.float32)
    lib().orc_linear_backward(rows, fin, fout, _f(dy).ravel(), _f(x).ravel(), _f(w).ravel(), dw,
                              db.ctypes.data if db is not None else None, dx)
    return dw, db, dx


# ---------------------------------------------------------------- nn.rs
# These wrappers work in place on C-contiguous float32 arrays, like the
# reference's &mut Tensor functions.
def _chk(*arrs):
    for a in arrs:
        assert a.dtype == np.float32 and a.flags.c_contiguous, "float32 C-contiguous array required"


def bn_train_forward(y, gamma, beta, rm, rv, mom=0.1, eps=1e-5, relu=False):
    """BatchNorm2d run_train (nn.rs:297-348) on y [n, c, h, w] in place.
    Returns (xhat, mean, invstd); rm / rv are updated in place."""
    _chk(y, gamma, beta, rm, rv)
    n, c = y.shape[0], y.shape[1]
    hw = y.size // max(n * c, 1)
    xhat = np.empty_like(y)
    mean = np.empty(c, np.float32)
    invstd = np.empty(c, np.float32)
    lib().orc_bn_train_forward(n, c, hw, y.reshape(-1), gamma, beta, rm, rv, xhat.reshape(-1),
                               mean.ctypes.data, invstd, mom, eps, int(relu))
    return xhat, mean, invstd


def bn_eval_forward(y, gamma, beta, rm, rv, eps=1e-5, relu=False):
    """BatchNorm2d run_eval (nn.rs:350-365) on y in place."""
    _chk(y, gamma, beta, rm, rv)
    n, c = y.shape[0], y.shape[1]
    lib().orc_bn_eval_forward(n, c, y.size // max(n * c, 1), y.reshape(-1), gamma, beta, rm, rv,
                              eps, int(relu))


def bn_backward(dy, xhat, gamma, invstd, dgamma, dbeta):
    """BatchNorm2d::backward (nn.rs:379-425): returns dx; dgamma / dbeta +=."""
    _chk(dy, xhat, gamma, invstd, dgamma, dbeta)
    n, c = dy.shape[0], dy.shape[1]
    dx = np.empty_like(dy)
    lib().orc_bn_backward(n, c, dy.size // max(n * c, 1), dy.reshape(-1), xhat.reshape(-1),
                          gamma, invstd, dx.reshape(-1), dgamma, dbeta)
    return dx


def relu_back(d, y):
    _chk(d, y)
    lib().orc_relu_back(d.size, d.reshape(-1), y.reshape(-1))


def add_(a, b):
    _chk(a, b)
    lib().orc_add(a.size, a.reshape(-1), b.reshape(-1))


def add_relu(a, b):
    _chk(a, b)
    lib().orc_add_relu(a.size, a.reshape(-1), b.reshape(-1))


def gap_forward(x):
    """gap_forward (nn.rs:455-463): [n, c, h, w] -> [n, c]."""
    _chk(x)
    n, c = x.shape[0], x.shape[1]
    y = np.empty((n, c), np.float32)
    lib().orc_gap_forward(n * c, x.size // max(n * c, 1), x.reshape(-1), y.reshape(-1))
    return y


def gap_backward(dy, h, w):
    _chk(dy)
    n, c = dy.shape[0], dy.shape[1]
    dx = np.empty((n, c, h, w), np.float32)
    lib().orc_gap_backward(n * c, h * w, dy.reshape(-1), dx.reshape(-1))
    return dx


def fc_forward(x, w, b, fout):
    """nn.rs Linear::forward (nn.rs:500-517): x [rows, fin] -> [rows, fout]."""
    x = _f(x)
    rows = x.shape[0]
    fin = x.size // rows
    y = np.empty((rows, fout), np.float32)
    lib().orc_fc_forward(rows, fin, fout, x.reshape(-1), _f(w).ravel(), _f(b).ravel(),
                         y.reshape(-1))
    return y


def fc_backward(dy, x, w, dw, db):
    """nn.rs Linear::backward (nn.rs:519-564): dw / db += in place; returns dx."""
    _chk(dw, db)
    dy, x = _f(dy), _f(x)
    rows, fout = dy.shape[0], dy.size // dy.shape[0]
    fin = x.size // rows
    dx = np.empty((rows, fin), np.float32)
    lib().orc_fc_backward(rows, fin, fout, dy.reshape(-1), x.reshape(-1), _f(w).ravel(), dw, db,
                          dx.reshape(-1))
    return dx


def softmax_ce(logits, labels, smooth):
    """softmax_ce (nn.rs:620-637) -> (mean loss, correct, dlogits)."""
    logits = _f(logits)
    rows = logits.shape[0]
    nclass = logits.size // rows
    d = np.empty((rows, nclass), np.float32)
    corr = _sz(0)
    loss = lib().orc_softmax_ce(rows, nclass, logits.reshape(-1),
                                np.ascontiguousarray(labels, np.uint32), smooth, d.reshape(-1),
                                C.byref(corr))
    return float(np.float32(loss)), int(corr.value), d


def sgd_step(v, g, m, lr, mom, wd):
    """Param::step (nn.rs:102-110) in place."""
    _chk(v, g, m)
    lib().orc_sgd_step(v.size, v, g, m, lr, mom, wd)


# ---------------------------------------------------------------- optim.rs
def powi(a, b):
    """f32::powi with a run-time exponent (compiler-rt __powisf2)."""
    return float(lib().orc_powi(a, int(b)))


def newton_schulz(g, rows, cols, steps):
    """newton_schulz (optim.rs:124-145); returns the orthogonalised copy."""
    g = _f(g).ravel().copy()
    lib().orc_newton_schulz(g, rows, cols, steps)
    return g


def muon_step(v, g, m, rows, cols, decay, lr, wd, mom=0.95, ns_steps=3):
    """The Muon branch of Optim::step_all (optim.rs:182-195), in place."""
    _chk(v, g, m)
    lib().orc_muon_step(v, g, m, rows, cols, int(decay), lr, wd, mom, ns_steps)


def muon_steps(params, lr, wd, mom=0.95, ns_steps=3, threads=1):
    """The Muon branch of Optim::step_all over a list of (v, g, m, rows,
    cols, decay) parameters, on an OpenMP loop over the matrices (the
    reference's par_iter over parameters, optim.rs:177-196); in place, equal
    to muon_step per parameter."""
    n = len(params)
    fp = C.POINTER(C.c_float)
    ptrs = []
    for k in range(3):
        arr = (fp * n)()
        for i, p in enumerate(params):
            _chk(p[k])
            arr[i] = p[k].ctypes.data_as(fp)
        ptrs.append(arr)
    for p in params:
        assert p[0].size == p[1].size == p[2].size == p[3] * p[4]
    rows = (_sz * n)(*[p[3] for p in params])
    cols = (_sz * n)(*[p[4] for p in params])
    dec = (C.c_int * n)(*[int(p[5]) for p in params])
    lib().orc_muon_steps(n, ptrs[0], ptrs[1], ptrs[2], rows, cols, dec, lr, wd, mom, ns_steps,
                         int(threads))


def adam_step(v, g, m, v2, decay, lr, wd, t, b1=0.9, b2=0.999, eps=1e-8):
    """Optim::step_adam (optim.rs:207-235) at step count t, in place."""
    _chk(v, g, m, v2)
    lib().orc_adam_step(v.size, v, g, m, v2, int(decay), lr, wd, b1, b2, eps, t)


def clip(g, lens, max_norm):
    """clip_ (optim.rs:237-251) over tensors laid end to end in g (in place);
    returns the global norm."""
    _chk(g)
    ls = (_sz * len(lens))(*lens)
    return float(lib().orc_clip(g, ls, len(lens), max_norm))


def ema_update(w, v, decay, t):
    """Ema::update (optim.rs:270-288) after the first call, in place on w."""
    _chk(w)
    lib().orc_ema_update(w.size, w, _f(v).ravel(), decay, t)


def lr_at(peak, lo, step, total, warm):
    """lr_at (train.rs:21-28)."""
    return float(lib().orc_lr_at(peak, lo, step, total, warm))


# ---------------------------------------------------------------- norm.rs
# Token tensors [rows, c] (or [n, t, c]) as float32 arrays; new outputs are
# returned, parameter gradients (dg, db, dl, dw, dp) are accumulated in place.
def ln_forward(x, g, b, eps=1e-5, train=True):
    """LayerNorm::forward (norm.rs:38-85): returns y, and xhat, invstd when
    training."""
    x, g, b = _f(x), _f(g), _f(b)
    c = g.size
    rows = x.size // c
    y = np.empty_like(x)
    if train:
        xhat = np.empty_like(x)
        invstd = np.empty(rows, np.float32)
        lib().orc_ln_forward(rows, c, x.ravel(), g, b, eps, y.ravel(), xhat.ctypes.data,
                             invstd.ctypes.data)
        return y, xhat, invstd
    lib().orc_ln_forward(rows, c, x.ravel(), g, b, eps, y.ravel(), None, None)
    return y


def ln_backward(dy, xhat, invstd, g, dg, db):
    """LayerNorm::backward (norm.rs:87-137): returns dx; dg / db +=."""
    _chk(dg, db)
    dy, xhat = _f(dy), _f(xhat)
    c = g.size
    dx = np.empty_like(dy)
    lib().orc_ln_backward(dy.size // c, c, dy.ravel(), xhat.ravel(), _f(invstd), _f(g),
                          dx.ravel(), dg, db)
    return dx


def layerscale_forward(x, l):
    x = _f(x)
    y = np.empty_like(x)
    lib().orc_layerscale_forward(x.size // l.size, l.size, x.ravel(), _f(l), y.ravel())
    return y


def layerscale_backward(dy, x, l, dl):
    _chk(dl)
    dy = _f(dy)
    dx = np.empty_like(dy)
    lib().orc_layerscale_backward(dy.size // l.size, l.size, dy.ravel(), _f(x).ravel(), _f(l),
                                  dx.ravel(), dl)
    return dx


def swiglu_forward(ab, h):
    ab = _f(ab)
    rows = ab.size // (2 * h)
    u = np.empty(rows * h, np.float32)
    lib().orc_swiglu_forward(rows, h, ab.ravel(), u)
    return u


def swiglu_backward(du, ab, h):
    ab = _f(ab)
    rows = ab.size // (2 * h)
    dab = np.empty(rows * 2 * h, np.float32)
    lib().orc_swiglu_backward(rows, h, _f(du).ravel(), ab.ravel(), dab)
    return dab


def dwconv3_forward(x, w, b, n, th, tw):
    """DwConv3::forward (norm.rs:338-375); x [n, th*tw, c], w [9, c]."""
    x = _f(x)
    c = b.size
    y = np.empty_like(x)
    lib().orc_dwconv3_forward(n, th, tw, c, x.ravel(), _f(w).ravel(), _f(b), y.ravel())
    return y


def dwconv3_backward(dy, x, w, n, th, tw, dw, db):
    """DwConv3::backward (norm.rs:377-452): returns dx; dw / db +=."""
    _chk(dw, db)
    dy = _f(dy)
    c = db.size
    dx = np.empty_like(dy)
    lib().orc_dwconv3_backward(n, th, tw, c, dy.ravel(), _f(x).ravel(), _f(w).ravel(),
                               dx.ravel(), dw.reshape(-1), db)
    return dx


def seqpool_forward(x, p, n, t):
    """SeqPool::forward (norm.rs:487-528): returns (z [n, c], w [n, t])."""
    x = _f(x)
    c = p.size
    z = np.empty(n * c, np.float32)
    w = np.empty(n * t, np.float32)
    lib().orc_seqpool_forward(n, t, c, x.ravel(), _f(p), z, w)
    return z, w


def seqpool_backward(dz, w, x, p, n, t, dp):
    """SeqPool::backward (norm.rs:530-580): returns dx; dp +=."""
    _chk(dp)
    c = p.size
    dx = np.empty(n * t * c, np.float32)
    lib().orc_seqpool_backward(n, t, c, _f(dz).ravel(), _f(w).ravel(), _f(x).ravel(), _f(p),
                               dx, dp)
    return dx


# ---------------------------------------------------------------- loss.rs
def _u32(a):
    return np.ascontiguousarray(a, dtype=np.uint32)


def _addr(a):
    return a.ctypes.data if a is not None else None


def taxo_target(y, parent, eps, sib):
    parent = _u32(parent)
    out = np.empty(parent.size, np.float32)
    lib().orc_taxo_target(y, parent, parent.size, eps, sib, out)
    return out


def uniform_target(y, k, eps):
    out = np.empty(k, np.float32)
    lib().orc_uniform_target(y, k, eps, out)
    return out


def soft_targets(labels, nf, eps, parent=None, sib=0.0, coarse=None, nc=0, perm=None, lam=None):
    """targets (train.rs:121-155): returns (tf [n, nf], tc [n, nc] or None)."""
    labels = _u32(labels)
    n = labels.size
    coarse = _u32(coarse) if coarse is not None else None
    perm = _u32(perm) if perm is not None else None
    lam = _f(lam) if lam is not None else None
    parent = _u32(parent) if parent is not None else None
    tf = np.empty((n, nf), np.float32)
    tc = np.empty((n, nc), np.float32) if coarse is not None else None
    lib().orc_soft_targets(n, nf, nc, labels, _addr(coarse), _addr(perm), _addr(lam),
                           _addr(parent), int(parent is not None), eps, sib, tf.reshape(-1),
                           _addr(tc))
    return tf, tc


def ce_soft(logits, target, hard, scale):
    """ce_soft (loss.rs:39-83): returns (loss, correct, dz)."""
    logits, target = _f(logits), _f(target)
    n, nc = logits.shape
    dz = np.empty_like(logits)
    cor = _sz(0)
    loss = lib().orc_ce_soft(n, nc, logits.reshape(-1), target.reshape(-1), _u32(hard), scale,
                             dz.reshape(-1), C.byref(cor))
    return float(loss), cor.value, dz


def kl_distill(student, teacher, temp, scale, dz):
    """kl_distill (loss.rs:87-130): dz += ...; returns the loss."""
    _chk(dz)
    student = _f(student)
    n, nc = student.shape
    return float(lib().orc_kl_distill(n, nc, student.reshape(-1), _f(teacher).reshape(-1), temp,
                                      scale, dz.reshape(-1)))


def hint_mse(pred, target, scale, dz):
    """hint_mse (loss.rs:133-151): dz += ...; returns the loss."""
    _chk(dz)
    pred = _f(pred)
    n, c = pred.shape
    return float(lib().orc_hint_mse(n, c, pred.reshape(-1), _f(target).reshape(-1), scale,
                                    dz.reshape(-1)))


# ---------------------------------------------------------------- vit.rs
def drop_path(x, n, p, seed):
    """DropPath::forward (vit.rs:39-59): returns (scaled copy, mask [n])."""
    x = _f(x).ravel().copy()
    mask = np.empty(n, np.float32)
    lib().orc_drop_path(n, x.size // n, x, p, C.c_uint64(seed & 0xFFFFFFFFFFFFFFFF), mask)
    return x, mask


def token_merge(z, n, th, c):
    y = np.empty(z.size, np.float32)
    lib().orc_token_merge(n, th, c, _f(z).ravel(), y)
    return y


def taxo_combine(zf, zc, parent):
    zf = _f(zf).copy()
    n, nf = zf.shape
    nc = zc.shape[1]
    lib().orc_taxo_combine(n, nf, nc, _u32(parent), zf.reshape(-1), _f(zc).reshape(-1))
    return zf


def taxo_combine_backward(dzf, dzc, parent):
    n, nf = dzf.shape
    nc = dzc.shape[1]
    dc = np.empty((n, nc), np.float32)
    lib().orc_taxo_combine_backward(n, nf, nc, _u32(parent), _f(dzf).reshape(-1),
                                    _f(dzc).reshape(-1), dc.reshape(-1))
    return dc


# ---------------------------------------------------------------- data.rs
def crop_flip_normalize(src, dy, dx, flip):
    """crop_flip_normalize (data.rs:331-362) of one u8 image [3*32*32]."""
    out = np.empty(3 * 32 * 32, np.float32)
    lib().orc_crop_flip_normalize(np.ascontiguousarray(src, np.uint8), out, dy, dx, int(flip))
    return out


def randaugment(img, ra_mag, ra_n, rng):
    """randaugment (data.rs:303-314) on a copy of one u8 image [3*32*32]."""
    im = np.ascontiguousarray(img, np.uint8).ravel().copy()
    lib().orc_randaugment(im, ra_mag, ra_n, C.byref(rng.st))
    return im


def ra_op(img, op, v, sign):
    """apply_op (data.rs:255-278) with the sign given: returns a new image."""
    im = np.ascontiguousarray(img, np.uint8).ravel().copy()
    lib().orc_ra_op(im, op, v, sign)
    return im.reshape(np.shape(img))


def cifar_batch_train(images, fine, coarse, idx, pad, erase, erase_side, seed, ra_mag=0.0,
                      ra_n=2):
    """make_batch_train (data.rs:384-416): returns (x [bs, 3, 32, 32], labels,
    coarse)."""
    idx = _u32(idx)
    bs = idx.size
    out = np.empty((bs, 3, 32, 32), np.float32)
    lab, co = np.empty(bs, np.uint32), np.empty(bs, np.uint32)
    lib().orc_cifar_batch_train(np.ascontiguousarray(images, np.uint8).reshape(-1),
                                np.ascontiguousarray(fine, np.uint8),
                                np.ascontiguousarray(coarse, np.uint8), idx, bs, pad, ra_mag,
                                ra_n, erase, erase_side, C.c_uint64(seed & 0xFFFFFFFFFFFFFFFF),
                                out.reshape(-1), lab, co)
    return out, lab, co


def mix_batch(x, alpha_mix, alpha_cut, sw, rng):
    """mix_batch (data.rs:469-492) in place on x [bs, ...] with the oracle
    Rng `rng` (advanced); returns (perm, lam)."""
    _chk(x)
    bs = x.shape[0]
    perm, lam = np.empty(bs, np.uint32), np.empty(bs, np.float32)
    lib().orc_mix_batch(x.reshape(-1), bs, alpha_mix, alpha_cut, sw, C.byref(rng.st), perm, lam)
    return perm, lam


# ---------------------------------------------------------------- train.rs
FNV_OFFSET = 0xCBF29CE484222325  # train.rs:474


def fnv1a_bytes(h, data):
    """FNV-1a 64 over bytes, continuing from hash h (train.rs:476-484)."""
    data = bytes(data)
    return int(lib().orc_fnv1a_bytes(C.c_uint64(h), data, len(data)))


def fnv1a_f32(h, values):
    """fnv_f32 (train.rs:479-484) over every value of `values` in order: each
    float as the 4 little-endian bytes of its bit pattern."""
    v = np.ascontiguousarray(np.asarray(values, np.float32).ravel())
    return int(lib().orc_fnv1a_f32(C.c_uint64(h), v, v.size))
