"""GPU: step graphs (wxx_amd.graphs) replay what the eager step computes.

A step recorded once and replayed must give the same bits as running the
step eagerly every time: the same kernels on the same inputs, with the
optimizer's step count / bias corrections, the scheduler's rate and the
dropout seeds advanced on the host before each replay in the eager order.
Each test runs an eager copy of the model beside the replayed one (same
seeds, same batches) and compares losses and weights exactly, with eager
work and host reads between the replays.
"""

import random

import numpy as np
import pytest

from conftest import rng

pytestmark = pytest.mark.gpu


def W():
    import wxx_amd

    return wxx_amd


def _gpt2(seed, V, dropout):
    nn = W().nn
    m = nn.GPT2(V, d_model=32, n_heads=4, n_layers=2, max_len=16, dropout=dropout)
    r = np.random.default_rng(seed)
    state = {k: (r.normal(0, 0.02, v.shape).astype(np.float32) if v.ndim >= 2 else v)
             for k, v in m.state_dict().items()}
    m.load_state_dict(state)
    opt = nn.AdamW(m.named_parameters(), lr=3e-3, weight_decay=0.01)
    sched = nn.WarmupCosineLR(opt, warmup_steps=2, total_steps=12, min_lr=1e-4)
    return m, opt, sched


def _batches(V, n, B=2, S=12, seed=5):
    r = rng(seed)
    return [(r.integers(0, V, (B, S)).astype(np.uint32), r.integers(0, V, (B, S)).astype(np.uint32))
            for _ in range(n)]


def _train_step(m, opt, sched, x, y, V, clip=True):
    nn = W().nn
    loss = nn.CCELoss()(m(x).reshape(-1, V), y.reshape(-1))
    opt.zero_grad()
    loss.backward()
    if clip:
        nn.clip_grad_norm_(m.parameters(), 0.05)  # small enough to clip every step
    opt.step()
    sched.step()
    return loss


@pytest.mark.parametrize("dropout", [0.0, 0.1])
def test_replayed_train_step_equals_eager_steps(device, dropout):
    wxx = W()
    F = wxx.functional
    V, steps = 40, 6
    batches = _batches(V, steps)

    random.seed(11)
    m1, o1, s1 = _gpt2(3, V, dropout)
    eager = []
    for x, y in batches:
        loss = _train_step(m1, o1, s1, F.from_numpy(x, np.uint32), F.from_numpy(y, np.uint32), V)
        eager.append(float(loss.numpy().reshape(-1)[0]))

    random.seed(11)
    m2, o2, s2 = _gpt2(3, V, dropout)
    xd = F.from_numpy(batches[0][0], np.uint32)
    yd = F.from_numpy(batches[0][1], np.uint32)
    replayed = [float(_train_step(m2, o2, s2, xd, yd, V).numpy().reshape(-1)[0])]
    g = wxx.StepGraph(lambda: _train_step(m2, o2, s2, xd, yd, V)).capture()
    assert g.nodes > 50
    assert o2.step_count == 1 and s2.last_epoch == 1  # recording advanced nothing
    for x, y in batches[1:]:
        F.assign(xd, F.from_numpy(x, np.uint32))
        F.assign(yd, F.from_numpy(y, np.uint32))
        loss = g.replay()
        replayed.append(float(loss.numpy().reshape(-1)[0]))
    assert replayed == eager
    assert o2.step_count == o1.step_count == steps and s2.last_epoch == s1.last_epoch
    assert o2.lr == o1.lr
    a, b = m1.state_dict(), m2.state_dict()
    for k in a:
        assert np.array_equal(a[k], b[k]), k
    for st1, st2 in zip(o1.state, o2.state):
        assert np.array_equal(st1["exp_avg"].numpy(), st2["exp_avg"].numpy())
    g.close()


def test_replay_leaves_eager_tensors_alone(device):
    # blocks the recording used stay with the graph: tensors made between
    # replays (same sizes as the step's activations) keep their values
    wxx = W()
    F = wxx.functional
    V = 40
    (x, y), = _batches(V, 1)
    m, opt, sched = _gpt2(4, V, 0.0)
    xd, yd = F.from_numpy(x, np.uint32), F.from_numpy(y, np.uint32)
    _train_step(m, opt, sched, xd, yd, V, clip=False)
    g = wxx.StepGraph(lambda: _train_step(m, opt, sched, xd, yd, V, clip=False)).capture()
    r = rng(9)
    keep = []
    for _ in range(3):
        vals = [r.standard_normal(shape).astype(np.float32)
                for shape in [(24, 32), (24, 96), (24, V), (2, 4, 12, 12), (24, 128)]]
        keep.append([(v, F.from_numpy(v)) for v in vals])
        g.replay()
        for batch in keep:
            for v, t in batch:
                assert np.array_equal(t.numpy(), v)
    g.close()


def test_recording_refuses_readback_and_recovers(device):
    wxx = W()
    F = wxx.functional
    a = F.from_numpy(np.arange(8, dtype=np.float32))

    def bad():
        b = a * 2.0
        return b.numpy()  # waits for the device: not allowed while recording

    g = wxx.StepGraph(bad)
    with pytest.raises(wxx.backend.lib.HIPError, match="captured"):
        g.capture()
    assert not wxx.graphs.capturing()
    np.testing.assert_array_equal((a * 3.0).numpy(), np.arange(8) * 3.0)


def test_replay_checks_cross_entropy_targets(device):
    wxx = W()
    F = wxx.functional
    V = 40
    (x, y), = _batches(V, 1)
    m, opt, sched = _gpt2(6, V, 0.0)
    xd, yd = F.from_numpy(x, np.uint32), F.from_numpy(y, np.uint32)
    _train_step(m, opt, sched, xd, yd, V)
    g = wxx.StepGraph(lambda: _train_step(m, opt, sched, xd, yd, V)).capture()
    g.replay()
    bad = y.copy()
    bad[1, 3] = V + 5
    F.assign(yd, F.from_numpy(bad, np.uint32))
    with pytest.raises(ValueError, match=f"max target {V + 5}"):
        g.replay()
    F.assign(yd, F.from_numpy(y, np.uint32))
    g.replay()
    g.close()


def test_clip_inside_recording_returns_device_norm(device):
    # the device decision and rescale equal the host path's on the same grads
    wxx = W()
    F = wxx.functional
    r = rng(2)
    vals = [r.standard_normal(s).astype(np.float32) for s in [(33, 7), (5,), (128, 64)]]
    ps = [wxx.Parameter(F.from_numpy(v)) for v in vals]
    qs = [wxx.Parameter(F.from_numpy(v)) for v in vals]
    for p, q, v in zip(ps, qs, vals):
        p.grad = F.from_numpy(v * 3)
        q.grad = F.from_numpy(v * 3)
    host = wxx.nn.clip_grad_norm_(qs, 2.5)
    g = wxx.StepGraph(lambda: wxx.nn.clip_grad_norm_(ps, 2.5)).capture()
    norm = g.replay()
    assert float(norm.numpy()[0]) == np.float32(host)
    for p, q in zip(ps, qs):
        assert np.array_equal(p.grad.numpy(), q.grad.numpy())
    g.close()
