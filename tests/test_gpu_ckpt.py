"""Checkpoints of the device-resident models (rustnn_amd/ckpt.py): a trained
ResNet-20 and a small RustViT saved, loaded into fresh models of other seeds,
and compared value for value (parameters and BN running statistics), then
through an eval forward; a checkpoint of another configuration is refused."""
import numpy as np
import pytest

from conftest import to_dev, to_host

pytestmark = pytest.mark.gpu


def test_resnet_checkpoint_round_trip(rnn, tmp_path):
    import torch
    from rustnn_amd import ckpt
    from rustnn_amd.model import ResNet
    g = torch.Generator(device="cuda").manual_seed(3)
    a = ResNet(3, 32, 100, seed=7)
    x = torch.randn(16, 3, 32, 32, device="cuda", generator=g)
    labels = torch.randint(0, 100, (16,), device="cuda", generator=g, dtype=torch.int32)
    a.train_step(x, labels, 0.1, 0.1, 0.9, 5e-4)  # weights and running stats move
    path = str(tmp_path / "resnet.ckpt")
    ckpt.save_resnet(a, path)
    b = ResNet(3, 32, 100, seed=99)
    ckpt.load_resnet(b, path)
    assert torch.equal(a.params(), b.params())
    assert torch.equal(a.buffers(), b.buffers())
    assert torch.equal(a.forward(x, train=False), b.forward(x, train=False))
    c = ResNet(3, 16, 100, seed=1)
    with pytest.raises(ckpt.CheckpointError):
        ckpt.load_resnet(c, path)
    a.close(), b.close(), c.close()


def test_rustvit_checkpoint_round_trip(rnn, tmp_path):
    import torch
    from rustnn_amd import ckpt
    from rustnn_amd.vit import RustViT
    cfg = dict(width=4, cmid=6, dim=8, heads=2, depth3=2, dim4=12, heads4=2, depth4=1,
               mem_at=(1,), droppath=0.2, img=16)
    parent = to_dev(np.array([0, 0, 1, 1, 2, 2], np.int32))
    a = RustViT(cfg, parent, 3, seed=1)
    x = torch.randn(3, 3, 16, 16, device="cuda")
    for p in a.params():
        p.v.add_(0.1)
    a.forward(x, True)  # BN running statistics move
    path = str(tmp_path / "vit.ckpt")
    ckpt.save_rustvit(a, path)
    b = RustViT(cfg, parent, 3, seed=2)
    ckpt.load_rustvit(b, path)
    for p, q in zip(a.params(), b.params()):
        assert torch.equal(p.v, q.v)
    for p, q in zip(ckpt._vit_buffers(a), ckpt._vit_buffers(b)):
        assert torch.equal(p, q)
    assert torch.equal(a.forward(x, False)["logits"], b.forward(x, False)["logits"])
    other = dict(cfg, droppath=0.1)  # part of the configuration hash
    c = RustViT(other, parent, 3, seed=3)
    with pytest.raises(ckpt.CheckpointError):
        ckpt.load_rustvit(c, path)
