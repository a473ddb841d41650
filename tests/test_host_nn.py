"""Host-only nn logic: learning-rate schedules (ports of the reference's
tests/test_scheduler.py exact values) and the optimizer's alias rounds."""

import math

import pytest

from wxx_amd.nn.optimizer import _rounds
from wxx_amd.nn.scheduler import (
    CosineAnnealingLR,
    ExponentialLR,
    LambdaLR,
    StepLR,
    WarmupCosineLR,
)


class DummyOptimizer:
    def __init__(self, lr):
        self.lr = lr


def test_warmup_cosine():
    opt = DummyOptimizer(1e-3)
    sched = WarmupCosineLR(opt, warmup_steps=4, total_steps=10, min_lr=1e-5)
    assert abs(opt.lr - 1e-3 / 4) < 1e-12
    for _ in range(3):
        sched.step()
    assert abs(opt.lr - 1e-3) < 1e-12
    while sched.last_epoch < 9:
        sched.step()
    assert abs(opt.lr - 1e-5) < 1e-9
    assert abs(sched.get_last_lr() - 1e-5) < 1e-9
    sched.step()
    assert abs(opt.lr - 1e-5) < 1e-9


def test_warmup_cosine_zero_warmup_and_midpoint():
    opt = DummyOptimizer(1e-3)
    sched = WarmupCosineLR(opt, warmup_steps=0, total_steps=5, min_lr=0.0)
    assert abs(opt.lr - 1e-3) < 1e-12
    sched.step()
    sched.step()  # progress 2/4: half way down the cosine
    assert abs(opt.lr - 1e-3 * 0.5 * (1 + math.cos(math.pi * 0.5))) < 1e-15
    while sched.last_epoch < 4:
        sched.step()
    assert abs(opt.lr) < 1e-9
    with pytest.raises(ValueError):
        WarmupCosineLR(DummyOptimizer(1.0), warmup_steps=5, total_steps=5)


def test_cosine_step_exponential_lambda():
    opt = DummyOptimizer(1.0)
    sched = CosineAnnealingLR(opt, T_max=4, eta_min=0.1)
    for _ in range(4):
        sched.step()
    assert abs(opt.lr - 0.1) < 1e-9
    opt = DummyOptimizer(1.0)
    sched = StepLR(opt, step_size=2, gamma=0.5)
    for _ in range(4):
        sched.step()
    assert abs(opt.lr - 0.25) < 1e-12
    opt = DummyOptimizer(1.0)
    sched = ExponentialLR(opt, gamma=0.5)
    for _ in range(3):
        sched.step()
    assert abs(opt.lr - 0.125) < 1e-12
    opt = DummyOptimizer(2.0)
    sched = LambdaLR(opt, lambda step: 1.0 / (step + 1))
    sched.step()
    assert abs(opt.lr - 1.0) < 1e-12
    restored = LambdaLR(DummyOptimizer(2.0), lambda step: 1.0 / (step + 1))
    restored.load_state_dict(sched.state_dict())
    assert restored.last_epoch == sched.last_epoch
    assert abs(restored.get_last_lr() - sched.get_last_lr()) < 1e-12


def test_alias_rounds_keep_list_order():
    items = ["a", "b", "a", "c", "a", "b"]
    rounds = _rounds(items, key=lambda x: x)
    assert rounds == [["a", "b", "c"], ["a", "b"], ["a"]]
