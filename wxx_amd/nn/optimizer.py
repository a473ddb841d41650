"""Optimizers (reference src/wxx/nn/optimizer.py:1-84).

``AdamW.step`` applies the reference's per-parameter update (adamw.wgsl) to
the whole parameter list with one multi-tensor launch instead of one launch
per parameter.  A parameter that appears twice in the list (the reference
registers aliases such as ``LayerNorm.weight`` next to ``weightg``) is
stepped twice, in list order, with its own moment buffers each time, exactly
as the reference's sequential loop does: the list is split into rounds in
which every storage appears once, and the rounds run in order.
"""

import numpy as np

from .. import functional, graphs
from ..backend.device import get_cmd_buffer
from ..Tensor import Tensor

cmd_encoder = get_cmd_buffer()


class Optimizer:
    def __init__(self, parameters):
        self.parameters = list(parameters)

    def step(self):
        pass

    def state_dict(self):
        """Hyper-parameters only (a stateless optimizer)."""
        return {"lr": np.float64(self.lr)} if hasattr(self, "lr") else {}

    def load_state_dict(self, state):
        if "lr" in state:
            self.lr = float(state["lr"])

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
        if graphs.capturing():
            # the rate is a kernel argument of the recorded update: a replay
            # with another rate would silently apply the recorded one
            recorded = self.lr

            def same_rate():
                if self.lr != recorded:
                    raise RuntimeError(f"SGD's learning rate {recorded} is recorded in this "
                                       f"step graph; record it again to use {self.lr}")

            graphs.on_replay(same_rate)
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

    # The reference keeps the moments only in memory (nn/optimizer.py:50-57);
    # these two make them part of a checkpoint.  Entries are keyed by the
    # position in the parameter list (a parameter listed twice has two
    # moment pairs); the names are stored to check the list on load.
    def state_dict(self):
        """The step count, hyper-parameters and both moments of every entry,
        as numpy arrays (an ``.npz``-ready dict)."""
        sd = {
            "step_count": np.int64(self.step_count),
            "lr": np.float64(self.lr),
            "betas": np.array([self.beta1, self.beta2], np.float64),
            "eps": np.float64(self.eps),
            "weight_decay": np.float64(self.weight_decay),
            "param_names": np.array([str(n) for n, _ in self.params]),
        }
        for i, st in enumerate(self.state):
            sd[f"exp_avg.{i}"] = st["exp_avg"].numpy()
            sd[f"exp_avg_sq.{i}"] = st["exp_avg_sq"].numpy()
        return sd

    def load_state_dict(self, state):
        """Restore what :meth:`state_dict` saved into this optimizer's moment
        buffers; the parameter list must have the same names and shapes."""
        names = [str(n) for n in np.asarray(state["param_names"]).tolist()]
        mine = [str(n) for n, _ in self.params]
        if names != mine:
            raise ValueError(f"optimizer state is for parameters {names[:4]}..., "
                             f"this optimizer holds {mine[:4]}...")
        for i, st in enumerate(self.state):
            for key in ("exp_avg", "exp_avg_sq"):
                arr = np.asarray(state[f"{key}.{i}"], np.float32)
                if list(arr.shape) != list(st[key].shape):
                    raise ValueError(f"{key}.{i}: shape {arr.shape} != {tuple(st[key].shape)}")
                functional.assign(st[key], functional.from_numpy(arr))
        self.step_count = int(state["step_count"])
        self.lr = float(state["lr"])
        self.beta1, self.beta2 = (float(b) for b in np.asarray(state["betas"]))
        self.eps = float(state["eps"])
        self.weight_decay = float(state["weight_decay"])

    def _advance(self):
        """Host half of a step: the step count and its bias corrections."""
        self.step_count += 1
        return 1.0 - self.beta1 ** self.step_count, 1.0 - self.beta2 ** self.step_count

    def _replay_words(self, words):
        bc1, bc2 = self._advance()
        words.view(np.float32)[:] = (self.lr, self.beta1, self.beta2, self.eps,
                                     self.weight_decay, bc1, bc2)

    def _record_step(self):
        """The step inside a step graph: the update kernels read this step's
        hyper-parameters from per-replay device words, which each replay
        fills from the host state (step count, current learning rate)."""
        hyper = graphs.per_replay(7, self._replay_words)
        live = [(w, st) for (_, w), st in zip(self.params, self.state) if w.grad is not None]
        for rnd in _rounds(live, key=lambda ws: (ws[0].buffer.ptr, ws[0].offset)):
            ps = [w for w, _ in rnd]
            if not all(p.is_contiguous() for p in ps):
                raise RuntimeError("a step graph needs contiguous parameters for AdamW")
            gs = [w.grad if w.grad.is_contiguous() else w.grad.contiguous() for w, _ in rnd]
            functional.adamw_multi_dev(ps, gs, [st["exp_avg"] for _, st in rnd],
                                       [st["exp_avg_sq"] for _, st in rnd], hyper)

    def step(self):
        if graphs.capturing():
            return self._record_step()
        bc1, bc2 = self._advance()
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
