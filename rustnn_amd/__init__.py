"""rustnn_amd -- MI355X (gfx950) GEMM core of rustnn behind a C ABI.

The product is ``librnn.so`` (HIP kernels + C ABI, ``include/rnn.h``).  This
module binds it with ctypes for Python callers (tests, bench) and mirrors the
reference's host interface for the hot path:

* ``matmul`` / ``gemm_small_batched`` / ``matmul_dw``  -- gemm.rs:434, 500, 555
* ``Conv2d`` (forward / backward_w / backward)          -- nn.rs:115-250
* ``Linear`` (forward / backward)                       -- linear.rs:14-104
* ``Core`` (forward / backward), ``rel_index``          -- attn.rs:21-343
* ``rustnn_amd.nn``: BatchNorm2d, the classifier Linear, gap, softmax_ce,
  Param::step                                           -- nn.rs:37-637
* ``rustnn_amd.model.ResNet``: the device-resident train step -- model.rs

Device memory and streams come from PyTorch (plumbing only): every array
argument is a float32 CUDA tensor, passed to the library as a raw device
pointer.  There is no CPU fallback: without a built ``librnn.so`` or without a
GPU every call raises.
"""
from __future__ import annotations

import ctypes as C
import math
import os
import threading

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "librnn.so")
HEADER = os.path.join(HERE, "..", "include", "rnn.h")

RNN_OK, RNN_E_INVALID, RNN_E_NULL, RNN_E_HIP, RNN_E_NOMEM, RNN_E_UNSUPPORTED = 0, -1, -2, -3, -4, -5
RNN_LINEAR_ACC_DX = 1  # rnn_linear_backward_ex
RNN_DW3_ACC_DX = 1  # rnn_dwconv3_backward_ex

_sz = C.c_size_t
_vp = C.c_void_p
_i = C.c_int
_u32 = C.c_uint32


class RnnError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"rnn status {status}: {msg}")
        self.status = status


class ConvSpec(C.Structure):
    """rnn_conv_spec = ConvSpec (conv.rs:9-20)."""
    _fields_ = [(n, _u32) for n in ("cin", "cout", "k", "stride", "pad", "h", "w", "oh", "ow")]

    @classmethod
    def make(cls, cin, cout, k, stride, pad, h, w):
        sp = cls()
        rc = lib().rnn_conv_spec_init(C.byref(sp), cin, cout, k, stride, pad, h, w)
        if rc:
            raise ValueError(f"invalid conv spec cin={cin} cout={cout} k={k} s={stride} "
                             f"p={pad} {h}x{w}")
        return sp

    @property
    def ckk(self):
        return self.cin * self.k * self.k

    @property
    def hw(self):
        return self.oh * self.ow


class LossCfg(C.Structure):
    """rnn_loss_cfg: build_loss's weights (train.rs:70-118, cli.rs defaults)."""
    _fields_ = [(n, C.c_float) for n in ("coarse_w", "exit_w1", "exit_w2", "alpha", "temp",
                                         "beta")] + [("taxo", C.c_int)]


class LossIO(C.Structure):
    """rnn_loss_io: the heads build_loss reads and the gradients it writes."""
    _fields_ = [(n, C.c_void_p) for n in ("logits", "coarse", "e1", "e2", "h1", "h2", "feat",
                                          "dlogits", "dcoarse", "de1", "de2", "dh1", "dh2")]


class AttnDesc(C.Structure):
    """rnn_attn_desc = Core (attn.rs:74-84) + forward/backward strides."""
    _fields_ = [("h", _u32), ("dh", _u32), ("tq", _u32), ("tk", _u32),
                ("qstride", _sz), ("qoff", _sz), ("kvstride", _sz), ("koff", _sz),
                ("voff", _sz), ("nrel", _u32), ("relidx", C.POINTER(_u32)), ("mask_diag", _i)]


_lib = None
_lib_lock = threading.Lock()


def lib():
    """Loads librnn.so.  Raises if it has not been built (no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lib_lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m rustnn_amd.build`")
        L = C.CDLL(LIB_PATH)
        P = C.POINTER
        sigs = {
            "rnn_ctx_create": (_i, [_i, P(_vp)]),
            "rnn_ctx_destroy": (_i, [_vp]),
            "rnn_ctx_set_stream": (_i, [_vp, _vp]),
            "rnn_ctx_stream": (_vp, [_vp]),
            "rnn_ctx_synchronize": (_i, [_vp]),
            "rnn_ctx_set_defer": (_i, [_vp, _i]),
            "rnn_ctx_flush": (_i, [_vp]),
            "rnn_ctx_last_error": (C.c_char_p, [_vp]),
            "rnn_status_string": (C.c_char_p, [_i]),
            "rnn_ctx_workspace_bytes": (_sz, [_vp]),
            "rnn_dev_alloc": (_i, [_vp, _sz, P(_vp)]),
            "rnn_dev_free": (_i, [_vp, _vp]),
            "rnn_copy_to_device": (_i, [_vp, _vp, _vp, _sz]),
            "rnn_copy_to_host": (_i, [_vp, _vp, _vp, _sz]),
            "rnn_matmul": (_i, [_vp, _sz, _sz, _sz, _vp, _i, _vp, _i, _vp, _i]),
            "rnn_gemm_small_batched": (_i, [_vp, _sz, _sz, _sz, _sz, _vp, _sz, _i, _vp, _sz, _i,
                                            _vp, _sz, _i]),
            "rnn_matmul_dw": (_i, [_vp, _sz, _sz, _sz, _vp, _vp, _vp]),
            "rnn_conv_spec_init": (_i, [P(ConvSpec), _u32, _u32, _u32, _u32, _u32, _u32, _u32]),
            "rnn_conv_packed_floats": (_i, [P(ConvSpec), _i, P(_sz)]),
            "rnn_conv_pack_weights": (_i, [_vp, P(ConvSpec), _i, _vp, _vp]),
            "rnn_conv2d_forward_packed": (_i, [_vp, P(ConvSpec), _sz, _vp, _vp, _vp, _vp]),
            "rnn_conv2d_backward_x_packed": (_i, [_vp, P(ConvSpec), _sz, _vp, _vp, _vp, _vp]),
            "rnn_conv2d_forward": (_i, [_vp, P(ConvSpec), _sz, _vp, _vp, _vp]),
            "rnn_conv2d_backward_w": (_i, [_vp, P(ConvSpec), _sz, _vp, _vp, _vp]),
            "rnn_conv2d_backward_x": (_i, [_vp, P(ConvSpec), _sz, _vp, _vp, _vp]),
            "rnn_rel_index": (_i, [_u32, _u32, _u32, _u32, P(_u32), P(_u32)]),
            "rnn_attn_forward": (_i, [_vp, P(AttnDesc), _sz, _vp, _vp, _vp, _vp, _vp, _vp]),
            "rnn_attn_backward": (_i, [_vp, P(AttnDesc), _sz, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                       _vp, _vp]),
            "rnn_attn_backward_ex": (_i, [_vp, P(AttnDesc), _sz, _vp, _vp, _vp, _vp, _vp, _vp,
                                          _vp, _vp, _vp, _u32]),
            "rnn_linear_forward": (_i, [_vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp]),
            "rnn_linear_forward_residual": (_i, [_vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp,
                                                 _vp, _sz, _vp]),
            "rnn_linear_backward": (_i, [_vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _vp]),
            "rnn_linear_backward_ex": (_i, [_vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _vp,
                                            _u32]),
            "rnn_matmul_host": (_i, [_vp, _sz, _sz, _sz, _vp, _i, _vp, _i, _vp, _i]),
            "rnn_gemm_small_batched_host": (_i, [_vp, _sz, _sz, _sz, _sz, _vp, _sz, _i, _vp,
                                                 _sz, _i, _vp, _sz, _i]),
            "rnn_matmul_dw_host": (_i, [_vp, _sz, _sz, _sz, _vp, _vp, _vp]),
            "rnn_conv2d_forward_host": (_i, [_vp, P(ConvSpec), _sz, _vp, _vp, _vp]),
            "rnn_conv2d_backward_w_host": (_i, [_vp, P(ConvSpec), _sz, _vp, _vp, _vp]),
            "rnn_conv2d_backward_x_host": (_i, [_vp, P(ConvSpec), _sz, _vp, _vp, _vp]),
            "rnn_attn_forward_host": (_i, [_vp, P(AttnDesc), _sz, _vp, _vp, _vp, _vp, _vp,
                                           _vp]),
            "rnn_attn_backward_host": (_i, [_vp, P(AttnDesc), _sz, _vp, _vp, _vp, _vp, _vp,
                                            _vp, _vp, _vp, _vp]),
            "rnn_linear_forward_host": (_i, [_vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp]),
            "rnn_linear_backward_host": (_i, [_vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp,
                                              _vp]),
            "rnn_dbg_resnet_buffer": (_i, [_vp, _sz, _i, P(_vp), P(_sz)]),
            "rnn_dbg_resnet_dw_group": (_i, [_vp, _i, P(C.c_double)]),
            "rnn_dbg_im2col": (_i, [_vp, P(ConvSpec), _vp, _vp]),
            "rnn_dbg_pack_a": (_i, [_vp, _vp, _sz, _sz, _i, _vp]),
            "rnn_dbg_pack_b": (_i, [_vp, _vp, _sz, _sz, _i, _vp]),
            "rnn_dbg_rel_index": (_i, [_vp, _u32, _u32, _u32, _u32, _vp]),
            "rnn_bn_forward_train": (_i, [_vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                          _vp, C.c_float, C.c_float, _i]),
            "rnn_bn_forward_eval": (_i, [_vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _vp,
                                         C.c_float, _i]),
            "rnn_bn_backward": (_i, [_vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                     _vp]),
            "rnn_relu_back": (_i, [_vp, _sz, _vp, _vp]),
            "rnn_add": (_i, [_vp, _sz, _vp, _vp]),
            "rnn_add_relu_back": (_i, [_vp, _sz, _vp, _vp, _vp]),
            "rnn_add_relu": (_i, [_vp, _sz, _vp, _vp]),
            "rnn_gap_forward": (_i, [_vp, _sz, _sz, _sz, _vp, _vp]),
            "rnn_gap_backward": (_i, [_vp, _sz, _sz, _sz, _vp, _vp]),
            "rnn_fc_forward": (_i, [_vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp]),
            "rnn_fc_backward": (_i, [_vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _vp]),
            "rnn_softmax_ce": (_i, [_vp, _sz, _sz, _vp, _vp, C.c_float, _vp, _vp, _vp]),
            "rnn_sgd_step": (_i, [_vp, _sz, _vp, _vp, _vp, C.c_float, C.c_float, C.c_float]),
            "rnn_resnet_create": (_i, [_vp, _sz, _sz, _sz, C.c_uint64, P(_vp)]),
            "rnn_resnet_destroy": (_i, [_vp]),
            "rnn_resnet_num_params": (_sz, [_vp]),
            "rnn_resnet_num_buffers": (_sz, [_vp]),
            "rnn_resnet_num_tensors": (_sz, [_vp]),
            "rnn_resnet_tensor_len": (_i, [_vp, _sz, P(_sz), P(_i)]),
            "rnn_resnet_copy": (_i, [_vp, _i, _vp, _vp]),
            "rnn_resnet_forward": (_i, [_vp, _sz, _sz, _sz, _vp, _i, _vp]),
            "rnn_resnet_backward": (_i, [_vp, _vp]),
            "rnn_resnet_step": (_i, [_vp, C.c_float, C.c_float, C.c_float]),
            "rnn_resnet_train_step": (_i, [_vp, _sz, _sz, _sz, _vp, _vp, C.c_float, C.c_float,
                                           C.c_float, C.c_float, _vp, _vp]),
            "rnn_resnet_inputs": (_i, [_vp, _sz, _sz, _sz, P(_vp), P(_vp)]),
            "rnn_newton_schulz": (_i, [_vp, _sz, _sz, _sz, _sz, _vp, _sz]),
            "rnn_optim_create": (_i, [_vp, _i, _sz, P(_vp)]),
            "rnn_optim_destroy": (_i, [_vp]),
            "rnn_optim_set": (_i, [_vp, C.c_float, C.c_float, C.c_float, C.c_float, _sz]),
            "rnn_optim_t": (_sz, [_vp]),
            "rnn_optim_step": (_i, [_vp, _sz, _vp, C.c_float, C.c_float]),
            "rnn_clip_grad_norm": (_i, [_vp, _sz, _vp, C.c_float, _vp]),
            "rnn_ema_update": (_i, [_vp, _sz, _vp, _vp, C.c_float]),
            "rnn_clip_params": (_i, [_vp, _sz, _vp, C.c_float, _vp]),
            "rnn_cifar_batch_train": (_i, [_vp, _vp, _vp, _vp, _sz, _vp, _sz, _sz, C.c_float,
                                           _sz, C.c_float, _sz, C.c_uint64, _vp, _vp, _vp]),
            "rnn_cifar_batch_eval": (_i, [_vp, _vp, _vp, _sz, _sz, _sz, C.c_int, _vp, _vp]),
            "rnn_rng_seed": (_i, [C.c_uint64, _vp]),
            "rnn_fnv1a_bytes": (C.c_uint64, [C.c_uint64, _vp, _sz]),
            "rnn_fnv1a_f32": (C.c_uint64, [C.c_uint64, _vp, _sz]),
            "rnn_rng_next_u64": (C.c_uint64, [_vp]),
            "rnn_rng_normal_vec": (_i, [_vp, _sz, C.c_float, _vp]),
            "rnn_rng_trunc_normal": (_i, [_vp, _sz, C.c_float, _vp]),
            "rnn_mix_plan": (_i, [_vp, _sz, C.c_float, C.c_float, C.c_float, _vp, _vp, _vp, _vp,
                                  _vp]),
            "rnn_mix_apply": (_i, [_vp, _vp, _vp, _sz, _vp, C.c_int, C.c_float, _vp]),
            "rnn_drop_path_forward": (_i, [_vp, _sz, _sz, _vp, C.c_float, C.c_uint64, _vp]),
            "rnn_drop_path_backward": (_i, [_vp, _sz, _sz, _vp, _vp]),
            "rnn_drop_path_masks": (_i, [_vp, _sz, _sz, _vp, _vp, _vp]),
            "rnn_residual_add_scaled": (_i, [_vp, _sz, _sz, _vp, _vp, _vp, _vp, _sz, _vp]),
            "rnn_ln_backward_add": (_i, [_vp, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
            "rnn_ln_backward_add_ls": (_i, [_vp, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                            _vp, _vp, _vp, _vp, _sz, _vp, _vp]),
            "rnn_axpy_cols": (_i, [_vp, _sz, _sz, _vp, _vp, _vp]),
            "rnn_token_merge": (_i, [_vp, _sz, _sz, _sz, _vp, _vp]),
            "rnn_token_merge_backward": (_i, [_vp, _sz, _sz, _sz, _vp, _vp]),
            "rnn_taxo_head_combine": (_i, [_vp, _sz, _sz, _sz, _vp, _vp, _vp]),
            "rnn_taxo_head_combine_backward": (_i, [_vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp]),
            "rnn_nchw_to_tokens": (_i, [_vp, _sz, _sz, _sz, _vp, _vp]),
            "rnn_tokens_to_nchw": (_i, [_vp, _sz, _sz, _sz, _vp, _vp]),
            "rnn_soft_targets": (_i, [_vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp, C.c_int,
                                      C.c_float, C.c_float, _vp, _vp]),
            "rnn_mix_dominant": (_i, [_vp, _sz, _vp, _vp, _vp, _vp]),
            "rnn_ce_soft": (_i, [_vp, _sz, _sz, _vp, _vp, _vp, C.c_float, _vp, _vp, _vp]),
            "rnn_kl_distill": (_i, [_vp, _sz, _sz, _vp, _vp, C.c_float, C.c_float, _vp, _vp]),
            "rnn_hint_mse": (_i, [_vp, _sz, _sz, _vp, _vp, C.c_float, _vp, _vp]),
            "rnn_build_loss": (_i, [_vp, _sz, _sz, _sz, _sz, _vp, _vp, _vp, _vp, P(LossCfg),
                                    P(LossIO), _vp, _vp, _vp]),
            "rnn_ln_forward": (_i, [_vp, _sz, _sz, _vp, _vp, _vp, C.c_float, _vp, _vp, _vp]),
            "rnn_ln_backward": (_i, [_vp, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
            "rnn_layerscale_forward": (_i, [_vp, _sz, _sz, _vp, _vp, _vp]),
            "rnn_layerscale_backward": (_i, [_vp, _sz, _sz, _vp, _vp, _vp, _vp, _vp]),
            "rnn_block_branch_backward": (_i, [_vp, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _vp,
                                               _vp, _vp, _vp, _sz, _vp, _vp, _vp, _vp, _vp,
                                               _vp]),
            "rnn_drop_layerscale_backward": (_i, [_vp, _sz, _sz, _vp, _vp, _vp, _vp, _sz, _vp,
                                                  _vp]),
            "rnn_swiglu_forward": (_i, [_vp, _sz, _sz, _vp, _vp]),
            "rnn_swiglu_backward": (_i, [_vp, _sz, _sz, _vp, _vp, _vp]),
            "rnn_dwconv3_forward": (_i, [_vp, _sz, _sz, _sz, _sz, _vp, _vp, _vp, _vp]),
            "rnn_dwconv3_backward": (_i, [_vp, _sz, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp,
                                          _vp]),
            "rnn_conv_packs_create": (_i, [_vp, _sz, P(ConvSpec), P(_vp), P(_vp)]),
            "rnn_conv_packs_update": (_i, [_vp, _vp]),
            "rnn_conv_packs_get": (_vp, [_vp, _sz, _i]),
            "rnn_conv_packs_destroy": (None, [_vp]),
            "rnn_dwconv3_backward_ex": (_i, [_vp, _sz, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp,
                                             _vp, _u32]),
            "rnn_dwconv3_branch_forward": (_i, [_vp, _sz, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp,
                                                _vp, _vp, _vp, _vp, _vp]),
            "rnn_seqpool_forward": (_i, [_vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp]),
            "rnn_seqpool_backward": (_i, [_vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _vp]),
            "rnn_ema_update_params": (_i, [_vp, _sz, _vp, _vp, C.c_float]),
            "rnn_powi_f32": (C.c_float, [C.c_float, _i]),
            "rnn_lr_at": (C.c_float, [C.c_float, C.c_float, _sz, _sz, _sz]),
            "rnn_resnet_logits": (_i, [_vp, _vp]),
            "rnn_resnet_set_graph": (_i, [_vp, _i]),
            "rnn_resnet_graph_state": (_i, [_vp, P(C.c_char_p)]),
            "rnn_resnet_flops": (C.c_uint64, [_vp, _sz, _sz]),
            "rnn_conv2d_backward_w_slab_floats": (_sz, [_vp, _vp, _sz]),
            "rnn_conv2d_backward_w_slabs": (_i, [_vp, _vp, _sz, _vp, _vp, _vp, P(C.c_int)]),
            "rnn_conv2d_backward_w_noalloc": (_i, [_vp, P(ConvSpec), _sz, _vp, _vp, _vp]),
        }
        for name, (res, args) in sigs.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
        return _lib


def declared_symbols(header: str = HEADER):
    """Names of the functions include/rnn.h declares."""
    import re
    txt = open(header).read()
    return sorted(set(re.findall(r"^\s*(?:int|void \*|const char \*|size_t|uint64_t|float)\s+(rnn_\w+)\s*\(",
                                 txt, re.M)))


# ------------------------------------------------------------------ context
class Context:
    """One device, one stream, one growing workspace (rnn_ctx)."""

    def __init__(self, device: int = 0, stream=None):
        import torch
        if not torch.cuda.is_available():
            raise RuntimeError("rustnn_amd needs a ROCm GPU (torch.cuda.is_available() is False)")
        self.device = device
        h = _vp()
        rc = lib().rnn_ctx_create(device, C.byref(h))
        if rc:
            raise RnnError(rc, lib().rnn_status_string(rc).decode())
        self.h = h
        if stream is None:
            with torch.cuda.device(device):
                stream = torch.cuda.current_stream()
        self.set_stream(stream)

    def set_stream(self, stream):
        ptr = stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream or 0)
        self.check(lib().rnn_ctx_set_stream(self.h, _vp(ptr)))

    def stream_ptr(self) -> int:
        return lib().rnn_ctx_stream(self.h) or 0

    def check(self, rc: int):
        if rc != RNN_OK:
            raise RnnError(rc, lib().rnn_ctx_last_error(self.h).decode() or
                           lib().rnn_status_string(rc).decode())

    def synchronize(self):
        self.check(lib().rnn_ctx_synchronize(self.h))

    def set_defer(self, on):
        """Deferred parameter-gradient reductions on / off (off flushes)."""
        self.check(lib().rnn_ctx_set_defer(self.h, 1 if on else 0))

    def flush(self):
        """Runs the queued parameter-gradient reductions (one launch)."""
        self.check(lib().rnn_ctx_flush(self.h))

    def workspace_bytes(self) -> int:
        return int(lib().rnn_ctx_workspace_bytes(self.h))

    def close(self):
        """rnn_ctx_destroy: runs the reductions a deferral still holds, then
        frees the context; raises if that flush failed."""
        if getattr(self, "h", None):
            h, self.h = self.h, None
            rc = lib().rnn_ctx_destroy(h)
            if rc != RNN_OK:
                raise RnnError(rc, lib().rnn_status_string(rc).decode())

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


_ctx = {}


def default_ctx(device: int = 0) -> Context:
    c = _ctx.get(device)
    if c is None:
        c = _ctx[device] = Context(device)
    return c


def _ptr(t, need: int, name: str):
    """Device pointer of a float32/uint32 CUDA tensor holding >= need elements."""
    if t is None:
        return None
    import torch
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{name} must be a CUDA tensor")
    if t.dtype not in (torch.float32, torch.uint32, torch.int32):
        raise TypeError(f"{name} must be float32 (got {t.dtype})")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.numel() < need:
        raise ValueError(f"{name} has {t.numel()} elements, needs {need}")
    return _vp(t.data_ptr()) if t.numel() else None


def _new(n, like=None, device=0):
    import torch
    dev = like.device if like is not None else torch.device("cuda", device)
    return torch.empty(n, dtype=torch.float32, device=dev)


# ------------------------------------------------------------------ gemm.rs
def matmul(m, n, k, a, at, b, bt, c, acc=False, ctx=None):
    """matmul (gemm.rs:434-493): c[m*n] = op(a) op(b) (+ c)."""
    ctx = ctx or default_ctx()
    if m == 0 or n == 0:
        return c
    ctx.check(lib().rnn_matmul(ctx.h, m, n, k, _ptr(a, m * k, "a"), int(at),
                               _ptr(b, k * n, "b"), int(bt), _ptr(c, m * n, "c"), int(acc)))
    return c


def gemm_small_batched(count, m, n, k, a, stride_a, at, b, stride_b, bt, c, stride_c, acc=False,
                       ctx=None):
    """gemm_small (gemm.rs:500-545) over `count` strided problems in one launch."""
    ctx = ctx or default_ctx()
    if count == 0 or m == 0 or n == 0 or k == 0:
        return c
    need = lambda s, e: (count - 1) * s + e
    ctx.check(lib().rnn_gemm_small_batched(
        ctx.h, count, m, n, k, _ptr(a, need(stride_a, m * k), "a"), stride_a, int(at),
        _ptr(b, need(stride_b, k * n), "b"), stride_b, int(bt),
        _ptr(c, need(stride_c, m * n), "c"), stride_c, int(acc)))
    return c


def matmul_dw(m, n, k, a, b, c, ctx=None):
    """matmul_dw (gemm.rs:555-598): c[m*n] += a^T b with a [k x m], b [k x n]."""
    ctx = ctx or default_ctx()
    if m == 0 or n == 0 or k == 0:
        return c
    ctx.check(lib().rnn_matmul_dw(ctx.h, m, n, k, _ptr(a, k * m, "a"), _ptr(b, k * n, "b"),
                                  _ptr(c, m * n, "c")))
    return c


# ------------------------------------------------------------------ conv.rs
def conv2d_forward(sp: ConvSpec, n, x, w, y=None, ctx=None):
    ctx = ctx or default_ctx()
    y = _new(n * sp.cout * sp.hw, x) if y is None else y
    ctx.check(lib().rnn_conv2d_forward(ctx.h, C.byref(sp), n, _ptr(x, n * sp.cin * sp.h * sp.w, "x"),
                                       _ptr(w, sp.cout * sp.ckk, "w"),
                                       _ptr(y, n * sp.cout * sp.hw, "y")))
    return y


def conv2d_backward_w(sp: ConvSpec, n, dy, x, dw, ctx=None):
    ctx = ctx or default_ctx()
    ctx.check(lib().rnn_conv2d_backward_w(ctx.h, C.byref(sp), n,
                                          _ptr(dy, n * sp.cout * sp.hw, "dy"),
                                          _ptr(x, n * sp.cin * sp.h * sp.w, "x"),
                                          _ptr(dw, sp.cout * sp.ckk, "dw")))
    return dw


def conv2d_backward_w_noalloc(sp: ConvSpec, n, dy, x, dw, ctx=None):
    """conv2d_backward_w with its partial slabs in the library's fixed device
    scratch (no device allocation; calls overlapping on one GPU race)."""
    ctx = ctx or default_ctx()
    ctx.check(lib().rnn_conv2d_backward_w_noalloc(ctx.h, C.byref(sp), n,
                                                  _ptr(dy, n * sp.cout * sp.hw, "dy"),
                                                  _ptr(x, n * sp.cin * sp.h * sp.w, "x"),
                                                  _ptr(dw, sp.cout * sp.ckk, "dw")))
    return dw


def conv2d_backward_w_slab_floats(sp: ConvSpec, n, ctx=None):
    """Floats of the slab buffer rnn_conv2d_backward_w_slabs fills (0: no
    slab plan for the shape)."""
    ctx = ctx or default_ctx()
    return int(lib().rnn_conv2d_backward_w_slab_floats(ctx.h, C.byref(sp), n))


def conv2d_backward_w_slabs(sp: ConvSpec, n, dy, x, slabs, ctx=None):
    """dW of the batch as partial slabs (nn.rs:201-219 per-worker folds):
    returns the slab count nz; slabs[z*cout*ckk:(z+1)*cout*ckk] is slab z and
    their in-order sum is the gradient rnn_conv2d_backward_w adds."""
    ctx = ctx or default_ctx()
    nz = C.c_int(0)
    ctx.check(lib().rnn_conv2d_backward_w_slabs(
        ctx.h, C.byref(sp), n, _ptr(dy, n * sp.cout * sp.hw, "dy"),
        _ptr(x, n * sp.cin * sp.h * sp.w, "x"),
        _ptr(slabs, conv2d_backward_w_slab_floats(sp, n, ctx), "slabs"), C.byref(nz)))
    return nz.value


def conv2d_backward_x(sp: ConvSpec, n, dy, w, dx=None, ctx=None):
    ctx = ctx or default_ctx()
    dx = _new(n * sp.cin * sp.h * sp.w, dy) if dx is None else dx
    ctx.check(lib().rnn_conv2d_backward_x(ctx.h, C.byref(sp), n,
                                          _ptr(dy, n * sp.cout * sp.hw, "dy"),
                                          _ptr(w, sp.cout * sp.ckk, "w"),
                                          _ptr(dx, n * sp.cin * sp.h * sp.w, "dx")))
    return dx


def conv_packed_floats(sp: ConvSpec, dx):
    """Size of the packed copy of W for direction dx, or None (no packed form)."""
    nf = _sz()
    if lib().rnn_conv_packed_floats(C.byref(sp), int(dx), C.byref(nf)) != 0:
        return None
    return int(nf.value)


def conv_pack_weights(sp: ConvSpec, dx, w, wp=None, ctx=None):
    """Packed copy of W for the forward (dx=0) or dX (dx=1) kernel (into wp
    when given), or None when the shape has no packed form."""
    import torch
    ctx = ctx or default_ctx()
    nf = conv_packed_floats(sp, dx)
    if nf is None:
        return None
    if wp is None:
        wp = torch.empty(nf, dtype=torch.float32, device=w.device)
    ctx.check(lib().rnn_conv_pack_weights(ctx.h, C.byref(sp), int(dx),
                                          _ptr(w, sp.cout * sp.ckk, "w"), _ptr(wp, nf, "wp")))
    return wp


def conv2d_forward_packed(sp: ConvSpec, n, x, w, wp, y=None, ctx=None):
    ctx = ctx or default_ctx()
    y = _new(n * sp.cout * sp.hw, x) if y is None else y
    ctx.check(lib().rnn_conv2d_forward_packed(ctx.h, C.byref(sp), n,
                                              _ptr(x, n * sp.cin * sp.h * sp.w, "x"),
                                              _ptr(w, sp.cout * sp.ckk, "w"), _ptr(wp, 0, "wp"),
                                              _ptr(y, n * sp.cout * sp.hw, "y")))
    return y


def conv2d_backward_x_packed(sp: ConvSpec, n, dy, w, wp, dx=None, ctx=None):
    ctx = ctx or default_ctx()
    dx = _new(n * sp.cin * sp.h * sp.w, dy) if dx is None else dx
    ctx.check(lib().rnn_conv2d_backward_x_packed(ctx.h, C.byref(sp), n,
                                                 _ptr(dy, n * sp.cout * sp.hw, "dy"),
                                                 _ptr(w, sp.cout * sp.ckk, "w"), _ptr(wp, 0, "wp"),
                                                 _ptr(dx, n * sp.cin * sp.h * sp.w, "dx")))
    return dx


class Conv2d:
    """Conv2d (nn.rs:115-250) on the device: w is [cout, cin*k*k] (RowMap order),
    Kaiming-initialised as nn.rs:95-100 when an Rng-compatible generator is
    given.  forward caches x for the backward (nn.rs:181-183)."""

    def __init__(self, cin, cout, k, stride, pad, w=None, device=0, ctx=None):
        import torch
        self.cin, self.cout, self.k, self.stride, self.pad = cin, cout, k, stride, pad
        self.ctx = ctx or default_ctx(device)
        fan_in = cin * k * k
        if w is None:
            w = torch.randn(cout * fan_in, device=f"cuda:{device}") * math.sqrt(2.0 / fan_in)
        self.w = w.contiguous()
        self.g = torch.zeros_like(self.w)
        self.x = None
        self.xshape = None
        # ((h, w), forward copy, dX copy) from a ConvPacks kept current with w
        self.packed = None

    def spec(self, h, w):
        """Conv2d::spec (nn.rs:152-164)."""
        return ConvSpec.make(self.cin, self.cout, self.k, self.stride, self.pad, h, w)

    def _wp(self, h, w, dx):
        """This input size's packed weights for the forward / dX, or None."""
        pk = self.packed
        return pk[1 + dx] if pk is not None and pk[0] == (h, w) and pk[1 + dx] else None

    def forward(self, x, n, h, w, train=True):
        sp = self.spec(h, w)
        wp = self._wp(h, w, 0)
        if wp is None:
            y = conv2d_forward(sp, n, x, self.w, ctx=self.ctx)
        else:
            y = _new(n * sp.cout * sp.hw, x)
            self.ctx.check(lib().rnn_conv2d_forward_packed(
                self.ctx.h, C.byref(sp), n, _ptr(x, n * sp.cin * sp.h * sp.w, "x"),
                _ptr(self.w, sp.cout * sp.ckk, "w"), wp, _ptr(y, n * sp.cout * sp.hw, "y")))
        if train:
            self.x, self.xshape = x, (n, h, w)
        return y

    def backward_w(self, dy):
        n, h, w = self.xshape
        conv2d_backward_w(self.spec(h, w), n, dy, self.x, self.g, ctx=self.ctx)

    def backward(self, dy):
        """Returns dX and accumulates dW (nn.rs:230-250)."""
        self.backward_w(dy)
        n, h, w = self.xshape
        sp = self.spec(h, w)
        wp = self._wp(h, w, 1)
        if wp is None:
            return conv2d_backward_x(sp, n, dy, self.w, ctx=self.ctx)
        dx = _new(n * sp.cin * sp.h * sp.w, dy)
        self.ctx.check(lib().rnn_conv2d_backward_x_packed(
            self.ctx.h, C.byref(sp), n, _ptr(dy, n * sp.cout * sp.hw, "dy"),
            _ptr(self.w, sp.cout * sp.ckk, "w"), wp, _ptr(dx, n * sp.cin * sp.h * sp.w, "dx")))
        return dx


class ConvPacks:
    """Packed weights of several Conv2d layers (rnn_conv_packs_*), re-packed
    together in one launch by update(); convs: [(Conv2d, h, w)], the input
    size each runs at.  Each layer then runs its forward / dX at that size on
    the packed copies (results identical to the unpacked calls) until
    close(); update() after every change of the weights (in place: the
    copies are tied to the weight tensors' addresses)."""

    def __init__(self, convs, ctx=None):
        self.ctx = ctx or default_ctx()
        self.h = None
        k = len(convs)
        specs = (ConvSpec * k)(*[c.spec(h, w) for c, h, w in convs])
        ws = (C.c_void_p * k)(*[c.w.data_ptr() for c, _, _ in convs])
        out = C.c_void_p()
        self.ctx.check(lib().rnn_conv_packs_create(self.ctx.h, k, specs, ws, C.byref(out)))
        self.h = out.value
        self._w = [c.w for c, _, _ in convs]  # the addresses the copies are tied to
        self.convs = [c for c, _, _ in convs]
        for i, (c, h, w) in enumerate(convs):
            c.packed = ((h, w), lib().rnn_conv_packs_get(self.h, i, 0),
                        lib().rnn_conv_packs_get(self.h, i, 1))

    def update(self):
        for c, w in zip(self.convs, self._w):
            if c.w.data_ptr() != w.data_ptr():
                raise RuntimeError("ConvPacks: a layer's weights moved; build a new ConvPacks")
        self.ctx.check(lib().rnn_conv_packs_update(self.ctx.h, self.h))

    def close(self):
        if self.h:
            for c in self.convs:
                c.packed = None
            self.ctx.synchronize()
            lib().rnn_conv_packs_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown: the library may be gone
            pass


# ------------------------------------------------------------------ attn.rs
def rel_index(th, tw, mh, mw):
    """rel_index (attn.rs:53-72) -> (np.uint32 [th*tw*mh*mw], nrel)."""
    idx = np.zeros(th * tw * mh * mw, np.uint32)
    nrel = _u32()
    rc = lib().rnn_rel_index(th, tw, mh, mw, idx.ctypes.data_as(C.POINTER(_u32)), C.byref(nrel))
    if rc:
        raise ValueError("rel_index: invalid grid")
    return idx, int(nrel.value)


class Core:
    """Core (attn.rs:74-343): per (image, head) attention with LSA temperature,
    2-D relative bias and optional diagonal mask."""

    def __init__(self, h, dh, tq, tk, relidx, nrel, mask_diag, ctx=None):
        self.h, self.dh, self.tq, self.tk = h, dh, tq, tk
        self.relidx = np.ascontiguousarray(relidx, np.uint32)
        self.nrel, self.mask_diag = nrel, bool(mask_diag)
        self.ctx = ctx or default_ctx()

    def desc(self, qstride, qoff, kvstride, koff, voff):
        d = AttnDesc(self.h, self.dh, self.tq, self.tk, qstride, qoff, kvstride, koff, voff,
                     self.nrel, self.relidx.ctypes.data_as(C.POINTER(_u32)), int(self.mask_diag))
        d._keep = self.relidx
        return d

    def forward(self, n, q, qstride, qoff, kv, kvstride, koff, voff, tau, rel, p=None, o=None):
        """Core::forward (attn.rs:148-223) -> (p [n,h,tq,tk], o [n,tq,h*dh])."""
        d = self.desc(qstride, qoff, kvstride, koff, voff)
        p = _new(n * self.h * self.tq * self.tk, q) if p is None else p
        o = _new(n * self.tq * self.h * self.dh, q) if o is None else o
        nq = (n * self.tq - 1) * qstride + qoff + self.h * self.dh if n else 0
        nkv = (n * self.tk - 1) * kvstride + max(koff, voff) + self.h * self.dh if n else 0
        self.ctx.check(lib().rnn_attn_forward(
            self.ctx.h, C.byref(d), n, _ptr(q, nq, "q"), _ptr(kv, nkv, "kv"),
            _ptr(tau, self.h, "tau"), _ptr(rel, self.h * self.nrel, "rel"),
            _ptr(p, n * self.h * self.tq * self.tk, "p"), _ptr(o, n * self.tq * self.h * self.dh, "o")))
        return p, o

    def backward(self, n, q, qstride, qoff, kv, kvstride, koff, voff, tau, p, dout, dq, dkv, dtau,
                 drel, set_dq=False, set_dkv=False):
        """Core::backward (attn.rs:226-343): accumulates into dq, dkv, dtau, drel;
        set_dq / set_dkv overwrite dq / dkv instead (the values zeroed buffers
        would receive)."""
        d = self.desc(qstride, qoff, kvstride, koff, voff)
        nq = (n * self.tq - 1) * qstride + qoff + self.h * self.dh if n else 0
        nkv = (n * self.tk - 1) * kvstride + max(koff, voff) + self.h * self.dh if n else 0
        flags = (1 if set_dq else 0) | (2 if set_dkv else 0)
        self.ctx.check(lib().rnn_attn_backward_ex(
            self.ctx.h, C.byref(d), n, _ptr(q, nq, "q"), _ptr(kv, nkv, "kv"),
            _ptr(tau, self.h, "tau"), _ptr(p, n * self.h * self.tq * self.tk, "p"),
            _ptr(dout, n * self.tq * self.h * self.dh, "dout"), _ptr(dq, nq, "dq"),
            _ptr(dkv, nkv, "dkv"), _ptr(dtau, self.h, "dtau"),
            _ptr(drel, self.h * self.nrel, "drel"), flags))


# ------------------------------------------------------------------ linear.rs
def linear_forward(rows, fin, fout, x, w, b=None, y=None, ctx=None):
    ctx = ctx or default_ctx()
    y = _new(rows * fout, x) if y is None else y
    ctx.check(lib().rnn_linear_forward(ctx.h, rows, fin, fout, _ptr(x, rows * fin, "x"),
                                       _ptr(w, fout * fin, "w"), _ptr(b, fout, "b"),
                                       _ptr(y, rows * fout, "y")))
    return y


def linear_forward_residual(rows, fin, fout, x, w, b, out, l, mask, rpi, y=None, ctx=None):
    """y = x W^T + b, and out += (y l) mask[r / rpi] (a residual branch's
    LayerScale and DropPath) in the GEMM's epilogue; returns y."""
    ctx = ctx or default_ctx()
    y = _new(rows * fout, x) if y is None else y
    ctx.check(lib().rnn_linear_forward_residual(
        ctx.h, rows, fin, fout, _ptr(x, rows * fin, "x"), _ptr(w, fout * fin, "w"),
        _ptr(b, fout, "b"), _ptr(y, rows * fout, "y"), _ptr(l, fout, "l"),
        _ptr(mask, rows // rpi, "mask") if mask is not None else None, rpi,
        _ptr(out, rows * fout, "out")))
    return y


def linear_backward(rows, fin, fout, dy, x, w, dw, db=None, dx=None, ctx=None, acc_dx=False):
    """Linear::backward (linear.rs:66-96); acc_dx: dx (given) += dy W."""
    ctx = ctx or default_ctx()
    if acc_dx and dx is None:
        raise ValueError("linear_backward: acc_dx needs dx")
    dx = _new(rows * fin, dy) if dx is None else dx
    ctx.check(lib().rnn_linear_backward_ex(ctx.h, rows, fin, fout, _ptr(dy, rows * fout, "dy"),
                                           _ptr(x, rows * fin, "x"), _ptr(w, fout * fin, "w"),
                                           _ptr(dw, fout * fin, "dw"), _ptr(db, fout, "db"),
                                           _ptr(dx, rows * fin, "dx"),
                                           RNN_LINEAR_ACC_DX if acc_dx else 0))
    return dx


class Linear:
    """Linear (linear.rs:14-104): w [fout, fin], optional bias; forward caches x."""

    def __init__(self, fin, fout, bias=True, w=None, b=None, device=0, ctx=None):
        import torch
        self.fin, self.fout = fin, fout
        self.ctx = ctx or default_ctx(device)
        dev = f"cuda:{device}"
        self.w = (w if w is not None else torch.randn(fout * fin, device=dev) * 0.02).contiguous()
        self.b = (b if b is not None else torch.zeros(fout, device=dev)) if bias else None
        self.gw = torch.zeros_like(self.w)
        self.gb = torch.zeros_like(self.b) if bias else None
        self.x, self.rows = None, 0

    def forward(self, x, rows, train=True, residual=None):
        """y = x W^T + b; residual = (out, l, mask, rows per image): also
        out += (y l) mask[image] in the same launch."""
        if residual is None:
            y = linear_forward(rows, self.fin, self.fout, x, self.w, self.b, ctx=self.ctx)
        else:
            out, l, mask, rpi = residual
            y = linear_forward_residual(rows, self.fin, self.fout, x, self.w, self.b, out, l,
                                        mask, rpi, ctx=self.ctx)
        if train:
            self.x, self.rows = x, rows
        return y

    def backward(self, dy, acc_dx=None):
        """dx, or acc_dx += dx (returned) when given."""
        return linear_backward(self.rows, self.fin, self.fout, dy, self.x, self.w, self.gw, self.gb,
                               dx=acc_dx, ctx=self.ctx, acc_dx=acc_dx is not None)


# ------------------------------------------------------------------ debug exports
def dbg_im2col(sp: ConvSpec, x_img, ctx=None):
    ctx = ctx or default_ctx()
    col = _new(sp.ckk * sp.hw, x_img)
    ctx.check(lib().rnn_dbg_im2col(ctx.h, C.byref(sp), _ptr(x_img, sp.cin * sp.h * sp.w, "x"),
                                   _ptr(col, sp.ckk * sp.hw, "col")))
    return col


def packed_len(rows, k, r):
    return ((k + 255) // 256) * 256 * ((rows + r - 1) // r) * r


def dbg_pack_a(a, m, k, transposed=False, ctx=None):
    import torch
    ctx = ctx or default_ctx()
    out = torch.zeros(packed_len(m, k, 6), dtype=torch.float32, device=a.device)
    ctx.check(lib().rnn_dbg_pack_a(ctx.h, _ptr(a, m * k, "a"), m, k, int(transposed),
                                   _ptr(out, out.numel(), "out")))
    return out


def dbg_pack_b(b, n, k, transposed=False, ctx=None):
    import torch
    ctx = ctx or default_ctx()
    out = torch.zeros(packed_len(n, k, 16), dtype=torch.float32, device=b.device)
    ctx.check(lib().rnn_dbg_pack_b(ctx.h, _ptr(b, n * k, "b"), n, k, int(transposed),
                                   _ptr(out, out.numel(), "out")))
    return out


def dbg_rel_index(th, tw, mh, mw, ctx=None):
    import torch
    ctx = ctx or default_ctx()
    out = torch.zeros(th * tw * mh * mw, dtype=torch.int32, device="cuda")
    ctx.check(lib().rnn_dbg_rel_index(ctx.h, th, tw, mh, mw, _ptr(out, out.numel(), "idx")))
    return out
