"""Learning-rate schedules that write ``optimizer.lr`` (reference
src/wxx/nn/scheduler.py:1-165).

Every schedule here is a pure function of the step counter ``last_epoch``:
``lr(step) = floor + (base_lr - floor) * shape(step)``, where ``floor`` is
the schedule's lower bound (0 unless it anneals towards a minimum) and
``shape`` is a factor in [0, 1] for the decaying schedules.  A scheduler
object only holds that counter and the last rate it wrote, so its state is
``{"base_lr", "last_epoch", "_last_lr"}`` (the keys torch and the reference
use).  Building one writes the rate of step 0, and ``step()`` advances the
counter by one (or sets it), as torch.optim.lr_scheduler does; the
WarmupCosineLR warm-up is the one phase that is not of the floor + shape
form, since it climbs from base_lr / warmup to base_lr.
"""

import math

from .. import graphs


def _half_cosine(done, span=1.0):
    """1 at done = 0, 0 at done = span, along half a cosine period."""
    return 0.5 * (1.0 + math.cos(math.pi * done / span))


def _require(ok, message):
    if not ok:
        raise ValueError(message)


class LRScheduler:
    """Constant schedule; subclasses supply :meth:`_shape` (and a floor)."""

    floor = 0.0

    def __init__(self, optimizer, last_epoch=-1):
        self.optimizer = optimizer
        self.base_lr = float(optimizer.lr)
        self.last_epoch = last_epoch
        self._last_lr = self.base_lr
        self.step()

    def _shape(self, step):
        return 1.0

    def get_lr(self):
        """The rate of step ``last_epoch``."""
        span = self.base_lr - self.floor
        return self.floor + span * self._shape(self.last_epoch)

    def _write(self, lr):
        self._last_lr = float(lr)
        self.optimizer.lr = self._last_lr
        return self._last_lr

    def step(self, epoch=None):
        """Advance to the next step (or to ``epoch``) and write its rate.
        Inside a step graph recording the advance runs before every replay
        instead (the optimizer's recorded update reads the rate then)."""
        if graphs.capturing():
            graphs.on_replay(lambda: self._advance(epoch))
            return self._last_lr
        return self._advance(epoch)

    def _advance(self, epoch):
        self.last_epoch = self.last_epoch + 1 if epoch is None else int(epoch)
        return self._write(self.get_lr())

    def get_last_lr(self):
        return self._last_lr

    def state_dict(self):
        return dict(base_lr=self.base_lr, last_epoch=self.last_epoch, _last_lr=self._last_lr)

    def load_state_dict(self, state):
        self.base_lr = float(state["base_lr"])
        self.last_epoch = int(state["last_epoch"])
        self._write(float(state["_last_lr"]))


class LambdaLR(LRScheduler):
    """lr = base_lr * lr_lambda(step)."""

    def __init__(self, optimizer, lr_lambda, last_epoch=-1):
        if not callable(lr_lambda):
            raise TypeError(f"lr_lambda must be a callable of the step, got {type(lr_lambda)}")
        self.lr_lambda = lr_lambda
        super().__init__(optimizer, last_epoch)

    def _shape(self, step):
        return float(self.lr_lambda(step))


class StepLR(LRScheduler):
    """lr = base_lr * gamma ** (step // step_size)."""

    def __init__(self, optimizer, step_size, gamma=0.1, last_epoch=-1):
        _require(step_size >= 1, f"StepLR step_size must be at least 1 (got {step_size})")
        self.step_size = int(step_size)
        self.gamma = float(gamma)
        super().__init__(optimizer, last_epoch)

    def _shape(self, step):
        return self.gamma ** (step // self.step_size)


class ExponentialLR(LRScheduler):
    """lr = base_lr * gamma ** step."""

    def __init__(self, optimizer, gamma, last_epoch=-1):
        self.gamma = float(gamma)
        super().__init__(optimizer, last_epoch)

    def _shape(self, step):
        return self.gamma ** step


class CosineAnnealingLR(LRScheduler):
    """Half a cosine from base_lr down to eta_min over T_max steps, then flat."""

    def __init__(self, optimizer, T_max, eta_min=0.0, last_epoch=-1):
        _require(T_max >= 1, f"CosineAnnealingLR T_max must be at least 1 (got {T_max})")
        self.T_max = int(T_max)
        self.eta_min = float(eta_min)
        self.floor = self.eta_min
        super().__init__(optimizer, last_epoch)

    def _shape(self, step):
        return _half_cosine(min(step, self.T_max), self.T_max)


class WarmupCosineLR(LRScheduler):
    """Linear warm-up over ``warmup_steps`` (step s runs at base_lr (s + 1) /
    warmup_steps, so the last warm-up step reaches base_lr), then half a
    cosine down to ``min_lr`` at ``total_steps``, then flat at min_lr."""

    def __init__(self, optimizer, warmup_steps, total_steps, min_lr=0.0, last_epoch=-1):
        _require(warmup_steps >= 0, f"warmup_steps must be non-negative (got {warmup_steps})")
        _require(total_steps >= 1, f"total_steps must be at least 1 (got {total_steps})")
        _require(total_steps > warmup_steps,
                 f"total_steps ({total_steps}) must exceed warmup_steps ({warmup_steps})")
        self.warmup_steps = int(warmup_steps)
        self.total_steps = int(total_steps)
        self.min_lr = float(min_lr)
        self.floor = self.min_lr
        super().__init__(optimizer, last_epoch)

    def _decay_progress(self, step):
        # with a warm-up the decay starts one step after its end and spans the
        # remaining steps; without one it spans steps 0 .. total_steps - 1
        if self.warmup_steps:
            done, span = step - self.warmup_steps + 1, self.total_steps - self.warmup_steps
        else:
            done, span = step, self.total_steps - 1
        return min(1.0, done / max(1, span))

    def _shape(self, step):
        return _half_cosine(self._decay_progress(step))

    def get_lr(self):
        step = self.last_epoch
        if step < self.warmup_steps:
            return self.base_lr * (step + 1) / self.warmup_steps
        return super().get_lr()


__all__ = ["LRScheduler", "LambdaLR", "StepLR", "ExponentialLR", "CosineAnnealingLR",
           "WarmupCosineLR"]
