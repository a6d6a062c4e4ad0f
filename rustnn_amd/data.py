"""data.rs on the device: the CIFAR-100 binary reader, the taxonomy, and batch
assembly from images resident in HBM.

* ``load(dir)`` / ``Dataset.from_bin(path)``: the binary version's records
  (coarse label byte, fine label byte, 3072 CHW pixel bytes; data.rs:25-53),
  read on the host once and kept on the device as u8;
* ``taxonomy(ds)``: parent superclass per fine class and the groups
  (data.rs:72-93);
* ``make_batch_train`` / ``make_batch_eval``: data.rs:384-416 / 494-512 on
  the device (RandAugment, crop, flip, normalise, random erasing);
* ``Rng`` (the trainer's generator, rng.rs, state on the host) and
  ``mix_batch`` (data.rs:469-492): the draws on the host, the blend on the
  device.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import RnnError, _ptr, _vp, default_ctx, lib

IMG, CH = 32, 3
PIX = CH * IMG * IMG
NCLASS = 100


def _u8ptr(t, need, name):
    import torch
    if not isinstance(t, torch.Tensor) or not t.is_cuda or t.dtype != torch.uint8:
        raise TypeError(f"{name} must be a uint8 CUDA tensor")
    if not t.is_contiguous() or t.numel() < need:
        raise ValueError(f"{name}: contiguous with at least {need} elements required")
    return _vp(t.data_ptr())


class Dataset:
    """Dataset (data.rs:16-53): images [len, 3, 32, 32] u8, fine and coarse
    labels u8, all on the device."""

    def __init__(self, images, labels, coarse):
        self.images, self.labels, self.coarse = images, labels, coarse
        self.len = int(labels.numel())

    @staticmethod
    def from_arrays(images, labels, coarse, device=0):
        import torch
        dev = f"cuda:{device}"
        images = np.ascontiguousarray(images, np.uint8).reshape(-1, CH, IMG, IMG)
        return Dataset(torch.from_numpy(images).to(dev),
                       torch.from_numpy(np.ascontiguousarray(labels, np.uint8)).to(dev),
                       torch.from_numpy(np.ascontiguousarray(coarse, np.uint8)).to(dev))

    @staticmethod
    def from_bin(path, device=0):
        """Dataset::from_bin (data.rs:26-52)."""
        raw = np.fromfile(path, dtype=np.uint8)
        rec = 2 + PIX
        if raw.size % rec:
            raise ValueError(f"{path}: unexpected size ({raw.size} bytes)")
        raw = raw.reshape(-1, rec)
        return Dataset.from_arrays(raw[:, 2:], raw[:, 1], raw[:, 0], device)


def load(dirname, device=0):
    """data::load (data.rs:55-60): train.bin and test.bin of the binary version."""
    return (Dataset.from_bin(os.path.join(dirname, "train.bin"), device),
            Dataset.from_bin(os.path.join(dirname, "test.bin"), device))


def taxonomy(ds):
    """taxonomy (data.rs:72-93): (parent [100], groups, ncoarse); a fine class
    with two superclasses or none is an error."""
    fine = ds.labels.cpu().numpy()
    coarse = ds.coarse.cpu().numpy()
    parent = np.full(NCLASS, -1, np.int64)
    for f, c in zip(fine, coarse):
        if parent[f] == -1:
            parent[f] = c
        elif parent[f] != c:
            raise ValueError(f"fine class {f} with two superclasses")
    if (parent < 0).any():
        raise ValueError("fine class without a superclass")
    ncoarse = int(parent.max()) + 1
    groups = [[int(f) for f in np.nonzero(parent == p)[0]] for p in range(ncoarse)]
    return parent.astype(np.uint32), groups, ncoarse


def make_batch_train(ds, idx, seed, pad=4, erase=0.0, erase_side=8, ra_mag=0.0, ra_n=2,
                     ctx=None):
    """make_batch_train (data.rs:384-416) on the device: idx (CUDA int32) picks
    the images; returns (x [bs, 3, 32, 32], labels, coarse) as CUDA tensors
    (int32 labels)."""
    import torch
    ctx = ctx or default_ctx()
    bs = idx.numel()
    out = torch.empty(bs, CH, IMG, IMG, device=ds.images.device)
    labels = torch.empty(bs, dtype=torch.int32, device=out.device)
    coarse = torch.empty(bs, dtype=torch.int32, device=out.device)
    ctx.check(lib().rnn_cifar_batch_train(
        ctx.h, _u8ptr(ds.images, ds.len * PIX, "images"), _u8ptr(ds.labels, ds.len, "labels"),
        _u8ptr(ds.coarse, ds.len, "coarse"), ds.len, _ptr(idx, bs, "idx"), bs, pad,
        float(ra_mag), ra_n, float(erase), erase_side, seed & 0xFFFFFFFFFFFFFFFF,
        _ptr(out, bs * PIX, "out"), _ptr(labels, bs, "labels"), _ptr(coarse, bs, "coarse")))
    return out, labels, coarse


def make_batch_eval(ds, start, bs, flip=False, ctx=None):
    """make_batch_eval (data.rs:494-512): (x, labels)."""
    import torch
    ctx = ctx or default_ctx()
    out = torch.empty(bs, CH, IMG, IMG, device=ds.images.device)
    labels = torch.empty(bs, dtype=torch.int32, device=out.device)
    ctx.check(lib().rnn_cifar_batch_eval(
        ctx.h, _u8ptr(ds.images, ds.len * PIX, "images"), _u8ptr(ds.labels, ds.len, "labels"),
        ds.len, start, bs, int(bool(flip)), _ptr(out, bs * PIX, "out"),
        _ptr(labels, bs, "labels")))
    return out, labels


class Rng:
    """The trainer's generator (rng.rs Rng::new / next_u64) with its state on
    the host, as the reference keeps it."""

    def __init__(self, seed):
        self.state = (C.c_uint64 * 4)()
        lib().rnn_rng_seed(C.c_uint64(seed & 0xFFFFFFFFFFFFFFFF), C.cast(self.state, _vp))

    def next_u64(self):
        return int(lib().rnn_rng_next_u64(C.cast(self.state, _vp)))

    def normal_vec(self, n, scale=1.0):
        """rand_vec (rng.rs:70-72) times an f32 scale (Param::kaiming with
        scale = sqrt(2 / fan_in), nn.rs:95-100), drawn on the host."""
        out = np.empty(n, np.float32)
        rc = lib().rnn_rng_normal_vec(C.cast(self.state, _vp), n, float(np.float32(scale)),
                                      out.ctypes.data)
        if rc:
            raise RnnError(rc, "rng normal_vec failed")
        return out

    def trunc_normal(self, n, std):
        """Param::trunc_normal's values (nn.rs:77-89), drawn on the host."""
        out = np.empty(n, np.float32)
        rc = lib().rnn_rng_trunc_normal(C.cast(self.state, _vp), n, float(np.float32(std)),
                                        out.ctypes.data)
        if rc:
            raise RnnError(rc, "rng trunc_normal failed")
        return out


def mix_batch(x, alpha_mix, alpha_cut, switch, rng, ctx=None):
    """mix_batch (data.rs:469-492): the permutation, lambda and cutmix box
    drawn from `rng` on the host, the blend on the device.  Returns
    (mixed x, perm (CUDA int32), lam (CUDA float32)); x is left as it was."""
    import torch
    ctx = ctx or default_ctx()
    bs = x.shape[0]
    perm = np.empty(bs, np.uint32)
    lam = np.empty(bs, np.float32)
    cut, l, rect = C.c_int(), C.c_float(), (C.c_int * 4)()
    rc = lib().rnn_mix_plan(C.cast(rng.state, _vp), bs, float(alpha_mix), float(alpha_cut),
                            float(switch), perm.ctypes.data, lam.ctypes.data, C.byref(cut),
                            C.byref(l), C.cast(rect, _vp))
    if rc:
        raise RnnError(rc, "mix_plan failed")
    dperm = torch.from_numpy(perm.view(np.int32)).to(x.device)
    dlam = torch.from_numpy(lam).to(x.device)
    if alpha_mix <= 0.0 and alpha_cut <= 0.0:
        return x, dperm, dlam
    out = torch.empty_like(x)
    ctx.check(lib().rnn_mix_apply(ctx.h, _ptr(x, bs * PIX, "x"), _ptr(out, bs * PIX, "out"), bs,
                                  _ptr(dperm, bs, "perm"), cut.value, l.value, C.cast(rect, _vp)))
    return out, dperm, dlam
