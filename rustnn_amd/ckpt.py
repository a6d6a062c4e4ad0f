"""ckpt.rs: the reference's checkpoint format, read and written by the host
around the device-resident models.

File layout (ckpt.rs:8-12, 99-120): the magic ``RUSTNN\\0``, u32 tensor
count, u64 scalar count, u64 configuration hash (all little-endian), then
every parameter value and every buffer as little-endian f32 in the model's
for_each_param / for_each_buffer order.  A headerless file whose size is
exactly the payload is a legacy checkpoint and loads with a warning
(ckpt.rs:164-171).  Saving writes ``path.tmp`` and renames it, so a failed
save leaves the previous file untouched (ckpt.rs:99-127).  The configuration
hash is FNV-1a over a kind tag and u64 fields (ckpt.rs:84-97); a checkpoint
of another configuration, tensor count or size is refused.
"""
from __future__ import annotations

import os
import struct
import sys

import numpy as np

MAGIC = b"RUSTNN\0"
HEADER_LEN = len(MAGIC) + 4 + 8 + 8
FNV_OFFSET = 0xCBF29CE484222325
FNV_PRIME = 0x00000100000001B3
_M64 = (1 << 64) - 1


class CheckpointError(ValueError):
    """A checkpoint that cannot be loaded into this model."""


def config_hash(kind: bytes, values) -> int:
    """config_hash (ckpt.rs:84-97): FNV-1a 64 over the kind bytes, then each
    value as 8 little-endian bytes."""
    h = FNV_OFFSET
    for b in kind:
        h = ((h ^ b) * FNV_PRIME) & _M64
    for v in values:
        for b in struct.pack("<Q", int(v) & _M64):
            h = ((h ^ b) * FNV_PRIME) & _M64
    return h


def resnet_config_hash(depth_n, width, nclass):
    """ResNet's Checkpointed::config_hash (model.rs:220-229)."""
    return config_hash(b"resnet", [depth_n, width, nclass])


def rustvit_config_hash(cfg, nclass, ncoarse, use_exits, parent):
    """RustViT's Checkpointed::config_hash (vit.rs:780-801); droppath enters
    as its f32 bit pattern."""
    dp_bits = struct.unpack("<I", struct.pack("<f", float(cfg["droppath"])))[0]
    mem_at = list(cfg["mem_at"])
    fields = [cfg["width"], cfg["cmid"], cfg["dim"], cfg["heads"], cfg["depth3"], cfg["dim4"],
              cfg["heads4"], cfg["depth4"], dp_bits, cfg["img"], nclass, ncoarse,
              int(bool(use_exits)), len(mem_at)]
    fields += mem_at
    parent = [int(p) for p in parent]
    fields.append(len(parent))
    fields += parent
    return config_hash(b"rustvit", fields)


def save(path, tensors, chash):
    """Writes the host float32 arrays `tensors` (parameters, then buffers)."""
    tmp = f"{path}.tmp"
    scalars = sum(int(np.asarray(t).size) for t in tensors)
    if len(tensors) > 0xFFFFFFFF:
        raise CheckpointError("checkpoint has more tensors than the format holds")
    try:
        with open(tmp, "wb") as f:
            f.write(MAGIC)
            f.write(struct.pack("<IQQ", len(tensors), scalars, chash & _M64))
            for t in tensors:
                f.write(np.ascontiguousarray(t, dtype="<f4").tobytes())
            f.flush()
            os.fsync(f.fileno())
    except BaseException:
        try:
            os.remove(tmp)
        except OSError:
            pass
        raise
    os.replace(tmp, path)


def load(path, lens, chash):
    """Reads a checkpoint for a model whose tensors have the lengths `lens`
    (parameters, then buffers) and configuration hash `chash`; returns the
    float32 arrays.  Raises CheckpointError on any mismatch."""
    with open(path, "rb") as f:
        data = f.read()
    expected = 4 * sum(lens)
    if data.startswith(MAGIC):
        if len(data) < HEADER_LEN:
            raise CheckpointError("checkpoint truncated before the end of the header")
        tensors, scalars, h = struct.unpack_from("<IQQ", data, len(MAGIC))
        if tensors != len(lens):
            raise CheckpointError(f"checkpoint has {tensors} tensors; the model expects "
                                  f"{len(lens)}")
        if scalars != sum(lens):
            raise CheckpointError(f"checkpoint has {scalars} scalars; the model expects "
                                  f"{sum(lens)}")
        if h != (chash & _M64):
            raise CheckpointError(f"checkpoint of another configuration (hash {h:016x}, "
                                  f"expected {chash & _M64:016x})")
        payload = memoryview(data)[HEADER_LEN:]
        if len(payload) != expected:
            raise CheckpointError(f"payload has {len(payload)} bytes; expected {expected}")
    elif len(data) == expected:
        print(f"warning: legacy checkpoint without a header: {path}", file=sys.stderr)
        payload = memoryview(data)
    else:
        raise CheckpointError(f"no magic and not a legacy size: {len(data)} bytes; expected "
                              f"{expected}")
    out, off = [], 0
    for n in lens:
        out.append(np.frombuffer(payload[off:off + 4 * n], dtype="<f4").astype(np.float32))
        off += 4 * n
    return out


# ------------------------------------------------------------------ models
def _resnet_buffer_lens(net):
    """BN running mean / var per BatchNorm2d in for_each_buffer order
    (model.rs:177-184): the stem, then per block b1, b2 and the shortcut's."""
    widths = [net.width, 2 * net.width, 4 * net.width]
    lens = [net.width, net.width]
    cin = net.width
    for stage, w in enumerate(widths):
        for i in range(net.depth_n):
            lens += [w, w, w, w]
            if i == 0 and (stage > 0 or cin != w):
                lens += [w, w]
            cin = w
    return lens


def save_resnet(net, path):
    """Checkpointed::save for the device-resident ResNet (rustnn_amd.model)."""
    import torch
    torch.cuda.synchronize()
    v = net.params().cpu().numpy()
    b = net.buffers().cpu().numpy()
    plens = [n for n, _ in net.tensor_lens()]
    blens = _resnet_buffer_lens(net)
    assert sum(blens) == b.size, "buffer layout"
    tensors = np.split(v, np.cumsum(plens)[:-1]) + np.split(b, np.cumsum(blens)[:-1])
    save(path, tensors, resnet_config_hash(net.depth_n, net.width, net.nclass))


def load_resnet(net, path):
    """Checkpointed::load for the device-resident ResNet."""
    import torch
    plens = [n for n, _ in net.tensor_lens()]
    blens = _resnet_buffer_lens(net)
    arrs = load(path, plens + blens, resnet_config_hash(net.depth_n, net.width, net.nclass))
    dev = f"cuda:{net.device}"
    net.set_params(torch.from_numpy(np.concatenate(arrs[:len(plens)])).to(dev))
    net.set_buffers(torch.from_numpy(np.concatenate(arrs[len(plens):])).to(dev))


def _vit_buffers(net):
    """RustViT::for_each_buffer (vit.rs:719-726): BN running mean / var of the
    stem, the two trunk blocks and the token conv."""
    bns = [net.stem.bn]
    for blk in (net.c1, net.c2):
        bns += [blk.a.bn, blk.b.bn] + ([blk.down.bn] if blk.down else [])
    bns.append(net.tok.bn)
    out = []
    for bn in bns:
        out += [bn.rm, bn.rv]
    return out


def _vit_hash(net):
    return rustvit_config_hash(net.cfg, net.nclass, net.head.nc, net.use_exits,
                               net.parent_host)


def save_rustvit(net, path):
    """Checkpointed::save for rustnn_amd.vit.RustViT."""
    import torch
    torch.cuda.synchronize()
    tensors = [p.v.detach().cpu().numpy() for p in net.params()]
    tensors += [b.detach().cpu().numpy() for b in _vit_buffers(net)]
    save(path, tensors, _vit_hash(net))


def load_rustvit(net, path):
    """Checkpointed::load for rustnn_amd.vit.RustViT."""
    import torch
    ps, bs = net.params(), _vit_buffers(net)
    arrs = load(path, [p.v.numel() for p in ps] + [b.numel() for b in bs], _vit_hash(net))
    for t, a in zip([p.v for p in ps] + bs, arrs):
        t.copy_(torch.from_numpy(a).to(t.device).view_as(t))
