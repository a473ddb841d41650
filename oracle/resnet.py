"""ResNet18 train-step forward + backward restated in float64 on the CPU
(TEST INFRASTRUCTURE ONLY).

The forward follows the reference's module tree (src/wxx/nn/resnet.py:14-80)
with the semantics of the kernels it calls:

* conv2d NCHW, no bias, Ho = (H + 2p - d(k - 1) - 1) // s + 1
  (functional/convolution.py:658-729);
* training BatchNorm over (B, H, W): mu = E[x], var = max(0, E[x^2] - mu^2),
  y = (x - mu) / sqrt(var + 1e-5) gamma + beta, running stats
  r <- 0.9 r + 0.1 stat with the unbiased variance var M / (M - 1)
  (batchnorm.wgsl:60-95, normalization.py:148-206).  A block's bn1 runs twice
  per forward (resnet.py:33 evaluates it once inside its hasattr test), so
  its running statistics take two updates; the output is the same both times;
* max pooling 3x3 stride 2 padding 1 whose gradient goes to the window's
  first strict maximum in row-major order (maxpool2d.wgsl: init -1e38, '>');
* adaptive average pooling to 1x1, Linear with W stored (in, out)
  (module.py:154-169), CCELoss mean over rows.

Gradients are torch's float64 autograd of that forward; torch's max-pool
gradient also goes to the first maximum of the window in row-major order.

``forced`` replays another evaluation's discrete decisions: the ReLU masks
(in call order) and the max-pool indices (flat input indices, the
reference's u32 index format).  An fp32 evaluation can see a ReLU input or a
max-pool near-tie on the other side of 0 / of the tie than float64 does; at
batch 128 one such flip moves a whole batch element's gradient.  With the
decisions fixed the remaining differences are rounding alone, and the
decisions themselves are compared with the oracle's own separately.
Pinned in tests/test_oracle_models.py against the numpy per-op oracles
(oracle/conv.py, oracle/norms.py) and finite differences of the loss.
"""

import numpy as np
import torch

F64 = torch.float64
TF = torch.nn.functional


def batchnorm_train(x, gamma, beta, rm, rv, eps=1e-5, momentum=0.1):
    """(y, new running mean, new running var) of one training forward."""
    M = x.shape[0] * x.shape[2] * x.shape[3]
    mu = x.mean(dim=(0, 2, 3))
    var = torch.clamp((x * x).mean(dim=(0, 2, 3)) - mu * mu, min=0.0)
    inv = 1.0 / torch.sqrt(var + eps)
    y = (x - mu[None, :, None, None]) * inv[None, :, None, None] * gamma[None, :, None, None] \
        + beta[None, :, None, None]
    with torch.no_grad():
        unb = var * (M / (M - 1.0)) if M > 1 else var
        rm = (1 - momentum) * rm + momentum * mu
        rv = (1 - momentum) * rv + momentum * unb
    return y, rm, rv


class _Decisions:
    """The ReLU inputs / max-pool inputs seen (``seen``) and, when replaying
    (``forced``), the masks and indices to use instead of the oracle's own."""

    def __init__(self, forced=None):
        self.relu_masks = list(forced["relu"]) if forced else None
        self.pool_idx = forced["pool"] if forced else None
        self.relu_inputs = []
        self.pool_inputs = []

    def relu(self, x):
        self.relu_inputs.append(x.detach())
        if self.relu_masks is None:
            return TF.relu(x)
        mask = torch.as_tensor(np.asarray(self.relu_masks.pop(0)), dtype=x.dtype)
        return x * mask

    def maxpool(self, x):
        self.pool_inputs.append(x.detach())
        if self.pool_idx is None:
            return TF.max_pool2d(x, 3, stride=2, padding=1)
        idx = torch.as_tensor(np.asarray(self.pool_idx, np.int64))
        return torch.take(x, idx)


def _block(P, S, p, x, stride, has_shortcut, D):
    out = TF.conv2d(x, P[p + "conv1.W"], stride=stride, padding=1)
    y, rm, rv = batchnorm_train(out, P[p + "bn1.weight"], P[p + "bn1.bias"],
                                S[p + "bn1.running_mean"], S[p + "bn1.running_std"])
    # second evaluation of bn1 on the same input (reference resnet.py:33)
    y, rm, rv = batchnorm_train(out, P[p + "bn1.weight"], P[p + "bn1.bias"], rm, rv)
    S[p + "bn1.running_mean"], S[p + "bn1.running_std"] = rm, rv
    out = D.relu(y)
    out = TF.conv2d(out, P[p + "conv2.W"], stride=1, padding=1)
    out, S[p + "bn2.running_mean"], S[p + "bn2.running_std"] = batchnorm_train(
        out, P[p + "bn2.weight"], P[p + "bn2.bias"], S[p + "bn2.running_mean"],
        S[p + "bn2.running_std"])
    if has_shortcut:
        sc = TF.conv2d(x, P[p + "shortcut.0.W"], stride=stride)
        sc, S[p + "shortcut.1.running_mean"], S[p + "shortcut.1.running_std"] = batchnorm_train(
            sc, P[p + "shortcut.1.weight"], P[p + "shortcut.1.bias"],
            S[p + "shortcut.1.running_mean"], S[p + "shortcut.1.running_std"])
    else:
        sc = x
    return D.relu(out + sc)


def resnet18_forward(P, S, x, D=None):
    """Logits of ResNet18 on x (B, 3, H, W); ``S`` (running statistics,
    name -> float64 tensor) is updated in place as the train forward does;
    ``D`` (a _Decisions) records, or replays, the ReLU and max-pool choices."""
    D = D or _Decisions()
    out, S["bn1.running_mean"], S["bn1.running_std"] = batchnorm_train(
        TF.conv2d(x, P["conv1.W"], stride=2, padding=3), P["bn1.weight"], P["bn1.bias"],
        S["bn1.running_mean"], S["bn1.running_std"])
    out = D.maxpool(D.relu(out))
    cin = 64
    for li, cout in enumerate((64, 128, 256, 512), start=1):
        for bi in range(2):
            stride = 2 if (bi == 0 and li > 1) else 1
            has_sc = bi == 0 and (stride != 1 or cin != cout)
            out = _block(P, S, f"layer{li}.{bi}.", out, stride, has_sc, D)
            cin = cout
    out = TF.adaptive_avg_pool2d(out, 1).reshape(out.shape[0], -1)
    return out @ P["fc.weight"] + P["fc.bias"]


def resnet18_loss_and_grads(params, stats, x, labels, dtype=np.float64, forced=None,
                            record=None):
    """(loss, {name: grad}, {name: new running stat}, logits) of one train
    step.  ``dtype=np.float32`` runs the same restatement in single
    precision.  ``forced`` = {"relu": masks, "pool": indices} replays those
    decisions; ``record`` (a dict) receives the ReLU and max-pool inputs this
    evaluation saw ("relu_inputs", "pool_input")."""
    torch.set_num_threads(max(1, min(16, torch.get_num_threads())))
    P = {k: torch.tensor(np.asarray(v, dtype), requires_grad=True) for k, v in params.items()}
    S = {k: torch.tensor(np.asarray(v, dtype)) for k, v in stats.items()}
    D = _Decisions(forced)
    logits = resnet18_forward(P, S, torch.tensor(np.asarray(x, dtype)), D)
    if record is not None:
        record["relu_inputs"] = [t.numpy() for t in D.relu_inputs]
        record["pool_input"] = D.pool_inputs[0].numpy()
    tg = torch.as_tensor(np.asarray(labels, np.int64))
    loss = (torch.logsumexp(logits, 1) - logits[torch.arange(logits.shape[0]), tg]).mean()
    loss.backward()
    return (float(loss.detach()), {k: v.grad.numpy() for k, v in P.items()},
            {k: v.numpy() for k, v in S.items()}, logits.detach().numpy())
