"""loss.rs on the device: soft targets, soft-target cross-entropy, the
distillation KL and the hint MSE (loss.rs:11-151, targets train.rs:121-155).

Float32 / uint32 (or int32) CUDA tensors in, gradients written on the device;
the losses come back as 1-element device tensors, so a training step never
waits on the host.  Every call goes through librnn.so.
"""
from __future__ import annotations

from . import _ptr, default_ctx, lib


def soft_targets(labels, nf, eps, parent=None, sib=0.0, coarse=None, nc=0, perm=None, lam=None,
                 ctx=None):
    """targets (train.rs:121-155): returns (tf [n, nf], tc [n, nc] or None).
    parent (the superclass of each fine class) selects taxo_target; without
    it the fine targets use uniform_target."""
    import torch
    ctx = ctx or default_ctx()
    n = labels.numel()
    tf = torch.empty(n, nf, device=labels.device)
    tc = torch.empty(n, nc, device=labels.device) if coarse is not None else None
    ctx.check(lib().rnn_soft_targets(
        ctx.h, n, nf, nc, _ptr(labels, n, "labels"), _ptr(coarse, n, "coarse"),
        _ptr(perm, n, "perm"), _ptr(lam, n, "lam"), _ptr(parent, nf, "parent"),
        int(parent is not None), float(eps), float(sib), _ptr(tf, n * nf, "tf"),
        _ptr(tc, n * nc, "tc")))
    return tf, tc


def mix_dominant(labels, perm, lam, ctx=None):
    """The dominant label of each mixed image (train.rs:313-320): labels[i]
    when lam[i] >= 0.5, else labels[perm[i]] (CUDA int32)."""
    import torch
    ctx = ctx or default_ctx()
    n = labels.numel()
    dom = torch.empty(n, dtype=torch.int32, device=labels.device)
    ctx.check(lib().rnn_mix_dominant(ctx.h, n, _ptr(labels, n, "labels"), _ptr(perm, n, "perm"),
                                     _ptr(lam, n, "lam"), _ptr(dom, n, "dom")))
    return dom


def ce_soft(logits, target, hard, scale, dz=None, ctx=None):
    """ce_soft (loss.rs:39-83): returns (loss, correct, dz) with loss and
    correct as 1-element device tensors; dz [n, nclass] overwritten."""
    import torch
    ctx = ctx or default_ctx()
    n, nc = logits.shape
    dz = torch.empty_like(logits) if dz is None else dz
    loss = torch.zeros(1, device=logits.device)
    correct = torch.zeros(1, dtype=torch.int32, device=logits.device)
    ctx.check(lib().rnn_ce_soft(ctx.h, n, nc, _ptr(logits, n * nc, "logits"),
                                _ptr(target, n * nc, "target"), _ptr(hard, n, "hard"),
                                float(scale), _ptr(dz, n * nc, "dz"), _ptr(loss, 1, "loss"),
                                _ptr(correct, 1, "correct")))
    return loss, correct, dz


def kl_distill(student, teacher, temp, scale, dz, ctx=None):
    """kl_distill (loss.rs:87-130): dz += ...; returns the loss (device)."""
    import torch
    ctx = ctx or default_ctx()
    n, nc = student.shape
    loss = torch.zeros(1, device=student.device)
    ctx.check(lib().rnn_kl_distill(ctx.h, n, nc, _ptr(student, n * nc, "student"),
                                   _ptr(teacher, n * nc, "teacher"), float(temp), float(scale),
                                   _ptr(dz, n * nc, "dz"), _ptr(loss, 1, "loss")))
    return loss


def hint_mse(pred, target, scale, dz, ctx=None):
    """hint_mse (loss.rs:133-151): dz += ...; returns the loss (device)."""
    import torch
    ctx = ctx or default_ctx()
    n, c = pred.shape
    loss = torch.zeros(1, device=pred.device)
    ctx.check(lib().rnn_hint_mse(ctx.h, n, c, _ptr(pred, n * c, "pred"),
                                 _ptr(target, n * c, "target"), float(scale),
                                 _ptr(dz, n * c, "dz"), _ptr(loss, 1, "loss")))
    return loss


def build_loss(out, tf, tc, hard, hardc, nf, nc, hp, ctx=None):
    """build_loss (train.rs:70-118) in one library call (rnn_build_loss):
    returns (grads, total, ce, correct) -- grads the dict of gradients the
    backward takes (logits, coarse and, with exits, e1, e2, h1, h2), written
    by the library; total / ce / correct 1-element device tensors."""
    import ctypes as C

    import torch

    from . import LossCfg, LossIO
    ctx = ctx or default_ctx()
    n = hard.numel()
    dev = out["logits"].device
    g = {"logits": torch.empty_like(out["logits"]),
         "coarse": torch.empty(n, nc, device=dev) if nc else None}
    exits = "e1" in out
    if exits:
        g.update(e1=torch.empty_like(out["e1"]), e2=torch.empty_like(out["e2"]),
                 h1=torch.empty_like(out["h1"]), h2=torch.empty_like(out["h2"]))
    d4 = out["h1"].shape[-1] if exits else 0
    cfg = LossCfg(float(hp["coarse_w"]), float(hp["exit_w"][0]), float(hp["exit_w"][1]),
                  float(hp["alpha"]), float(hp["temp"]), float(hp["beta"]),
                  int(not hp["no_taxo"]))
    p = lambda t: t.data_ptr() if t is not None else None
    io = LossIO(p(out["logits"]), p(out.get("coarse")), p(out.get("e1")), p(out.get("e2")),
                p(out.get("h1")), p(out.get("h2")), p(out.get("feat")), p(g["logits"]),
                p(g["coarse"]), p(g.get("e1")), p(g.get("e2")), p(g.get("h1")), p(g.get("h2")))
    total = torch.empty(1, device=dev)
    ce = torch.empty(1, device=dev)
    correct = torch.empty(1, dtype=torch.int32, device=dev)
    ctx.check(lib().rnn_build_loss(
        ctx.h, n, nf, nc, d4, _ptr(tf, n * nf, "tf"), _ptr(tc, n * nc, "tc") if tc is not None
        else None, _ptr(hard, n, "hard"), _ptr(hardc, n, "hardc") if hardc is not None else None,
        C.byref(cfg), C.byref(io), _ptr(total, 1, "total"), _ptr(ce, 1, "ce"),
        _ptr(correct, 1, "correct")))
    return g, total, ce, correct
