"""An independent float64 statement of the reference CIFAR ResNet train
forward and loss in torch (CPU autograd), for the parity tests.

Written from the reference's definitions (model.rs:10-150, nn.rs): the stem
conv + BatchNorm2d (training mode: batch mean, biased variance, eps 1e-5) +
ReLU; BasicBlocks (conv-BN-ReLU, conv-BN, a 1x1 conv-BN shortcut when the
shape changes, add, ReLU); global average pooling; the classifier Linear
(w [nclass, fin], bias); softmax cross-entropy with label smoothing
(nn.rs:566-637: on = 1 - s on the label plus s / nclass everywhere, mean over
the batch).  ``resnet_f64(arrays, depth_n, width, nclass)`` takes the
parameters in for_each_param order (model.rs:159-175) and returns the
gradient of the loss with respect to each, plus the logits and the loss.
"""
from __future__ import annotations

import numpy as np
import torch

F = torch.nn.functional
D = torch.float64


def _bn(x, g, b):
    m = x.mean(dim=(0, 2, 3), keepdim=True)
    v = ((x - m) ** 2).mean(dim=(0, 2, 3), keepdim=True)
    return (x - m) / torch.sqrt(v + 1e-5) * g.view(1, -1, 1, 1) + b.view(1, -1, 1, 1)


def resnet_f64(arrays, depth_n, width, nclass, x, labels, smooth):
    """Returns (logits, loss, [gradient per parameter]) in float64."""
    ps = [torch.tensor(np.asarray(a, np.float64).ravel(), dtype=D, requires_grad=True)
          for a in arrays]
    it = iter(ps)
    nxt = lambda: next(it)

    def conv_bn(h, cin, cout, k, s, p):
        w = nxt().view(cout, cin, k, k)
        y = F.conv2d(h, w, stride=s, padding=p)
        return _bn(y, nxt(), nxt())

    h = torch.tensor(np.asarray(x, np.float64), dtype=D)
    h = torch.relu(conv_bn(h, 3, width, 3, 1, 1))
    cin = width
    for stage, w in enumerate((width, 2 * width, 4 * width)):
        for b in range(depth_n):
            s = 2 if stage > 0 and b == 0 else 1
            a = torch.relu(conv_bn(h, cin, w, 3, s, 1))
            y = conv_bn(a, w, w, 3, 1, 1)
            sc = conv_bn(h, cin, w, 1, s, 0) if (s != 1 or cin != w) else h
            h = torch.relu(y + sc)
            cin = w
    feat = h.mean(dim=(2, 3))
    fw, fb = nxt().view(nclass, cin), nxt()
    z = feat @ fw.T + fb
    lse = torch.logsumexp(z, 1)
    lab = torch.tensor(np.asarray(labels, np.int64))
    on, off = 1.0 - smooth, smooth / nclass
    loss = (on * (lse - z[torch.arange(z.shape[0]), lab]) +
            off * (lse.unsqueeze(1) - z).sum(1)).mean()
    loss.backward()
    return z.detach().numpy(), float(loss.item()), [p.grad.numpy() for p in ps]
