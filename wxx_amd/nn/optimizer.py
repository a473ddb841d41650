"""Optimizers (reference src/wxx/nn/optimizer.py:1-84).

``AdamW.step`` applies the reference's per-parameter update (adamw.wgsl) to
the whole parameter list with one multi-tensor launch instead of one launch
per parameter.  A parameter that appears twice in the list (the reference
registers aliases such as ``LayerNorm.weight`` next to ``weightg``) is
stepped twice, in list order, with its own moment buffers each time, exactly
as the reference's sequential loop does: the list is split into rounds in
which every storage appears once, and the rounds run in order.
"""

from .. import functional
from ..backend.device import get_cmd_buffer
from ..Tensor import Tensor

cmd_encoder = get_cmd_buffer()


class Optimizer:
    def __init__(self, parameters):
        self.parameters = list(parameters)

    def step(self):
        pass

    def zero_grad(self, wait=False):
        for _, w in self.parameters:
            if w.grad is not None:
                w.grad = None
        cmd_encoder.flush(wait=wait)


class SGD(Optimizer):
    def __init__(self, parameters, lr=0.01):
        super().__init__(parameters)
        self.lr = lr

    def step(self):
        for _, w in self.parameters:
            functional._pointwise(w, -self.lr * w.grad, 0)


def _rounds(items, key):
    """Split ``items`` into consecutive-order rounds with unique ``key`` per round."""
    rounds, seen_in = [], {}
    for it in items:
        k = key(it)
        r = seen_in.get(k, -1) + 1
        seen_in[k] = r
        while len(rounds) <= r:
            rounds.append([])
        rounds[r].append(it)
    return rounds


class AdamW(Optimizer):
    def __init__(self, parameters, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-7, weight_decay=1e-4):
        super().__init__(parameters)
        self.params = self.parameters
        self.lr = lr
        self.beta1, self.beta2 = float(beta1), float(beta2)
        self.eps = float(eps)
        self.weight_decay = float(weight_decay)
        self.step_count = 0
        self.state = [{"exp_avg": Tensor(p.shape, value=0), "exp_avg_sq": Tensor(p.shape, value=0)}
                      for _, p in self.params]

    def step(self):
        self.step_count += 1
        bc1 = 1.0 - self.beta1 ** self.step_count
        bc2 = 1.0 - self.beta2 ** self.step_count
        live = [(w, st) for (_, w), st in zip(self.params, self.state) if w.grad is not None]
        for rnd in _rounds(live, key=lambda ws: (ws[0].buffer.ptr, ws[0].offset)):
            ps, gs, ms, vs = [], [], [], []
            for w, st in rnd:
                g = w.grad if w.grad.is_contiguous() else w.grad.contiguous()
                ps.append(w)
                gs.append(g)
                ms.append(st["exp_avg"])
                vs.append(st["exp_avg_sq"])
            if all(p.is_contiguous() for p in ps):
                functional.adamw_multi(ps, gs, ms, vs, float(self.lr), self.beta1, self.beta2,
                                       self.eps, self.weight_decay, bc1, bc2)
            else:
                for p, g, m, v in zip(ps, gs, ms, vs):
                    functional.adamw(p, g, m, v, self.step_count, self.lr, self.beta1,
                                     self.beta2, self.eps, self.weight_decay, bc1, bc2)
