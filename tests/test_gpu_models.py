"""GPU: the nn models end to end.

* BASELINE config 1 (toy GPT-2 1024/256/8/6, batch 4 x 128, dropout 0): loss,
  every parameter gradient and one AdamW step against the float64 oracle
  (oracle/models.py), with weights injected through load_state_dict.
* Ports of the reference's model tests (tests/test_gpt.py, test_resnet.py,
  test_hyena.py, test_clip_grad.py): shapes, gradients reaching every
  parameter, causality, state_dict round trips, generation, parameter counts.
"""

import numpy as np
import pytest

from conftest import rng
from oracle import conv as oc
from oracle import models as om

pytestmark = pytest.mark.gpu


def W():
    import wxx_amd

    return wxx_amd


def up(a):
    return W().functional.from_numpy(np.asarray(a, np.float32))


def up_u32(a):
    return W().functional.from_numpy(np.asarray(a), np.uint32)


def _close_to_scale(got, want, rel, name):
    """|got - want| <= rel * max|want| for the whole tensor (fp32 sums over long
    reductions against a float64 oracle)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = max(np.abs(want).max(), 1e-30)
    err = np.abs(got - want).max()
    assert err <= rel * scale, f"{name}: max err {err:.3g} vs scale {scale:.3g} (rel {err / scale:.3g})"
    return err / scale


def _gpt2_state(model, seed=1234):
    """Config-1 weights: N(0, 0.02) for >= 2-D parameters, biases 0, LayerNorm
    gamma 1 / beta 0 (nn/gpt.py:66-73), drawn from a seeded generator."""
    r = np.random.default_rng(seed)
    state = {}
    for name, arr in model.state_dict().items():
        if arr.ndim >= 2:
            state[name] = r.normal(0, 0.02, arr.shape).astype(np.float32)
        elif name.endswith(("weightg", "ln1.weight", "ln2.weight", "ln_f.weight")):
            state[name] = np.ones(arr.shape, np.float32)
        else:
            state[name] = np.zeros(arr.shape, np.float32)
    for name in list(state):  # LayerNorm aliases share their tensor
        if name.endswith(".weight") and name[:-7] + ".weightg" in state:
            state[name] = state[name[:-7] + ".weightg"]
        if name.endswith(".bias") and name[:-5] + ".weightb" in state:
            state[name] = state[name[:-5] + ".weightb"]
    return state


def _alias_free(state):
    """Drop LayerNorm's alias names (weight/bias of a module that has weightg/weightb)."""
    out = {}
    for k, v in state.items():
        if k.endswith(".weight") and k[:-7] + ".weightg" in state:
            continue
        if k.endswith(".bias") and k[:-5] + ".weightb" in state:
            continue
        out[k] = v
    return out


def _elementwise(got, want, name, rtol=1e-4, atol=1e-5):
    """The north star's fp32 bar, element by element: |got - want| <= atol + rtol |want|."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    bad = err > atol + rtol * np.abs(want)
    assert not bad.any(), (f"{name}: {int(bad.sum())} of {bad.size} elements outside "
                           f"rtol {rtol} atol {atol}; max err {err.max():.3g}")
    return err.max() / max(np.abs(want).max(), 1e-30)


def _gpt2_step_vs_oracle(V, D, H, L, B, S, max_len):
    """One GPT-2 forward + CCELoss + backward + AdamW step on the GPU from
    seeded weights, against the float64 restatement oracle/models.py: the
    loss, every parameter gradient and every updated parameter, each element
    within rtol 1e-4 / atol 1e-5.  Returns the largest gradient error
    relative to its tensor's scale (reported, and bounded by the caller)."""
    wxx = W()
    model = wxx.nn.GPT2(V, D, H, L, max_len=max_len, dropout=0.0)
    state = _gpt2_state(model)
    model.load_state_dict(state)
    x = rng(0).integers(0, V, (B, S)).astype(np.uint32)
    y = rng(1).integers(0, V, (B, S)).astype(np.uint32)
    opt = wxx.nn.AdamW(model.parameters(), lr=1e-3)

    logits = model(up_u32(x))
    loss = wxx.nn.CCELoss()(logits.reshape((B * S, V)), up_u32(y.reshape(-1)))
    loss.backward()

    params = {k: v.astype(np.float64) for k, v in _alias_free(state).items()}
    ol, og = om.gpt2_loss_and_grads(params, x, y, H, L)
    got_loss = float(loss.numpy().reshape(-1)[0])
    assert abs(got_loss - ol) <= 1e-5 * abs(ol), (got_loss, ol)
    gpu_grads, worst = {}, 0.0
    for name, p in model.named_parameters():
        assert p.grad is not None, name
        if name in og:  # aliases are the same tensors as their first names
            gpu_grads[name] = p.grad.numpy().astype(np.float64)
            worst = max(worst, _elementwise(gpu_grads[name], og[name], name))

    # One AdamW step: the device update of every parameter (aliases stepped
    # twice, in list order) against the oracle's update from the same
    # gradients (a gradient's sign decides the first step's direction, so the
    # update is checked on the gradients the device holds).
    order, first = [], {}
    for name, p in model.named_parameters():
        order.append(first.setdefault((p.buffer.ptr, p.offset), name))
    opt.step()
    states = [(np.zeros_like(params[k]), np.zeros_like(params[k])) for k in order]
    want = om.adamw_sequence(params, gpu_grads, order, states, 1, 1e-3)
    for name, p in model.named_parameters():
        if name in want:
            _elementwise(p.numpy(), want[name], "adamw " + name, rtol=1e-5, atol=2e-6)
    return worst


def test_gpt2_config1_train_step_matches_oracle(device):
    # GPT2(1024, 256, 8 heads, 6 layers), batch 4 x 128
    worst = _gpt2_step_vs_oracle(1024, 256, 8, 6, 4, 128, 256)
    assert worst < 2e-5, worst


def test_gpt2_config5_slice_matches_oracle(device):
    # BASELINE config 5's layer shapes at full width and length: GPT2(50304,
    # 768, 12 heads, max_len 1024), 2 of its 12 layers, batch 2 x 1024 (the
    # 50304-wide tied head, its CCE rows and the 12 x 1024 x 1024 causal
    # attention of every layer), against the float64 oracle
    worst = _gpt2_step_vs_oracle(50304, 768, 12, 2, 2, 1024, 1024)
    assert worst < 2e-5, worst


def test_gpt2_config5_full_step_properties(device):
    # the whole BASELINE config-5 train step (12 layers, batch 8 x 1024):
    # size-independent properties, since the float64 oracle of the full step
    # is too slow for a test
    import math

    wxx = W()
    V, D, H, L, B, S = 50304, 768, 12, 12, 8, 1024
    model = wxx.nn.GPT2(V, D, H, L, max_len=S, dropout=0.0)
    x = up_u32(rng(50).integers(0, V, (B, S)))
    y = up_u32(rng(51).integers(0, V, (B * S,)))
    i = np.arange(S)
    plain_mask = W().functional.from_numpy(
        np.where(i[None, :] <= i[:, None], 0.0, -1e9).astype(np.float32))

    def loss_and_grads(mask=None):
        model.zero_grad()
        loss = wxx.nn.CCELoss()(model(x, mask).reshape((B * S, V)), y)
        loss.backward()
        return (float(loss.numpy().reshape(-1)[0]),
                {n: p.grad.numpy() for n, p in model.named_parameters()})

    l1, g1 = loss_and_grads()
    # random init: logits ~ N(0, ~0.5^2), so the loss is close to ln V
    assert abs(l1 - math.log(V)) < 0.5, l1
    assert all(np.isfinite(g).all() for g in g1.values())
    # deterministic: a second identical step gives the same bits
    l2, g2 = loss_and_grads()
    assert l1 == l2
    assert all(np.array_equal(g1[n], g2[n]) for n in g1)
    # the marked causal path (triangles skipped) equals the plain masked path
    l3, g3 = loss_and_grads(plain_mask)
    assert abs(l3 - l1) <= 1e-6 * l1
    for n in g1:
        np.testing.assert_allclose(g3[n], g1[n], rtol=1e-4, atol=1e-7, err_msg=n)
    # then the optimizer half of the step: the clip's norm is the float64
    # norm of these gradients, and AdamW + WarmupCosineLR move every weight
    opt = wxx.nn.AdamW(model.parameters(), lr=1e-3)
    sched = wxx.nn.WarmupCosineLR(opt, warmup_steps=100, total_steps=5000, min_lr=1e-5)
    l4, g4 = loss_and_grads()
    # (LayerNorm's aliased parameters are listed twice and count twice, as
    # in the reference's loop over parameters())
    want = math.sqrt(sum(float((g.astype(np.float64) ** 2).sum()) for g in g4.values()))
    before = {n: p.numpy() for n, p in model.named_parameters()}
    total = wxx.nn.clip_grad_norm_(model.parameters(), 1.0)
    assert abs(total - want) <= 1e-4 * want, (total, want)
    opt.step()
    sched.step()
    after = {n: p.numpy() for n, p in model.named_parameters()}
    assert all(np.isfinite(a).all() for a in after.values())
    assert all(not np.array_equal(after[n], before[n]) for n in after)


def test_gpt2_all_parameters_receive_grad(device):
    wxx = W()
    m = wxx.nn.GPT2(64, d_model=32, n_heads=4, n_layers=2, max_len=16, dropout=0.0)
    x = up_u32(rng(2).integers(0, 64, (2, 6)))
    out = m(x)
    assert out.shape == [2, 6, 64]
    assert np.isfinite(out.numpy()).all()
    out.sum().backward()
    missing = [n for n, p in m.named_parameters() if p.grad is None]
    assert not missing, missing


def test_gpt2_shape_error_and_state_dict_roundtrip(device, tmp_path):
    wxx = W()
    m = wxx.nn.GPT2(32, d_model=16, n_heads=2, n_layers=1, max_len=8)
    with pytest.raises(ValueError):
        m(up_u32(np.zeros((1, 9))))
    state = m.state_dict()
    path = wxx.save(m, tmp_path / "m")
    m2 = wxx.nn.GPT2(32, d_model=16, n_heads=2, n_layers=1, max_len=8)
    wxx.load(path, m2)
    restored = m2.state_dict()
    assert set(restored) == set(state)
    for k, v in state.items():
        assert np.array_equal(restored[k], v), k


def test_checkpoint_resume_equals_continuous_training(device, tmp_path):
    # weights + AdamW moments/step count + WarmupCosineLR position in one
    # archive: 2 steps, save, 2 more steps == a fresh model restored from the
    # archive running the same 2 steps, bit for bit (the reference loses the
    # moments, nn/optimizer.py:50-57)
    wxx = W()
    nn = wxx.nn

    def make():
        m = nn.GPT2(48, d_model=32, n_heads=4, n_layers=2, max_len=16, dropout=0.0)
        m.load_state_dict(_gpt2_state(m, seed=7))
        opt = nn.AdamW(m.named_parameters(), lr=3e-3)  # names checked on load
        sched = nn.WarmupCosineLR(opt, warmup_steps=2, total_steps=10, min_lr=1e-4)
        return m, opt, sched

    r = rng(21)
    batches = [(r.integers(0, 48, (2, 12)), r.integers(0, 48, (2, 12))) for _ in range(4)]

    def step(m, opt, sched, xy):
        x, y = xy
        loss = nn.CCELoss()(m(up_u32(x)).reshape(-1, 48), up_u32(y.reshape(-1)))
        opt.zero_grad()
        loss.backward()
        nn.clip_grad_norm_(m.parameters(), 1.0)
        opt.step()
        sched.step()
        return float(loss.numpy().reshape(-1)[0])

    m, opt, sched = make()
    for xy in batches[:2]:
        step(m, opt, sched, xy)
    path = wxx.serialization.save_checkpoint(tmp_path / "ck", m, opt, sched)
    cont = [step(m, opt, sched, xy) for xy in batches[2:]]
    m2, opt2, sched2 = make()
    wxx.serialization.load_checkpoint(path, m2, opt2, sched2)
    assert opt2.step_count == 2 and sched2.last_epoch == sched.last_epoch - 2
    resumed = [step(m2, opt2, sched2, xy) for xy in batches[2:]]
    assert cont == resumed
    a, b = m.state_dict(), m2.state_dict()
    for k in a:
        assert np.array_equal(a[k], b[k]), k
    for s1, s2 in zip(opt.state, opt2.state):
        assert np.array_equal(s1["exp_avg_sq"].numpy(), s2["exp_avg_sq"].numpy())
    # without the moments (weights only) the next step differs
    m3, opt3, sched3 = make()
    wxx.serialization.load_checkpoint(path, m3, None, sched3)
    step(m3, opt3, sched3, batches[2])
    assert any(not np.array_equal(m3.state_dict()[k], m2.state_dict()[k]) for k in a)
    with pytest.raises(ValueError):
        other = nn.AdamW(nn.GPT2(48, d_model=32, n_heads=4, n_layers=1, max_len=16)
                         .named_parameters())
        other.load_state_dict({k[6:]: v for k, v in wxx.load(path).items()
                               if k.startswith("optim.")})


def test_gpt2_is_causal_and_mask(device):
    wxx = W()
    from wxx_amd.backend.context import inferenceMode

    m = wxx.nn.GPT2(40, d_model=16, n_heads=2, n_layers=2, max_len=8)
    ids = rng(3).integers(0, 40, (1, 6)).astype(np.uint32)
    with inferenceMode():
        before = m(up_u32(ids)).numpy()
        ids2 = ids.copy()
        ids2[0, -1] = (ids2[0, -1] + 1) % 40
        after = m(up_u32(ids2)).numpy()
    assert np.allclose(before[0, :-1], after[0, :-1], atol=1e-5)
    assert not np.allclose(before[0, -1], after[0, -1])
    mask = m.causal_mask(4).numpy()
    assert mask.shape == (4, 4)
    assert not np.any(np.tril(mask))
    assert np.all(mask[np.triu_indices(4, k=1)] < -1e8)


def test_gpt2_generate(device):
    wxx = W()
    from wxx_amd.backend import context

    m = wxx.nn.GPT2(30, d_model=16, n_heads=2, n_layers=1, max_len=10)
    prompt = rng(4).integers(0, 30, (2, 3)).astype(np.uint32)
    out = m.generate(prompt, max_new_tokens=4, temperature=0.0)
    assert out.shape == (2, 7) and out.dtype == np.uint32
    assert np.array_equal(out[:, :3], prompt)
    assert np.array_equal(out, m.generate(prompt, max_new_tokens=4, temperature=0.0))
    assert m.generate(prompt, max_new_tokens=100, temperature=1.0).shape == (2, 10)
    assert m.generate(prompt[0], max_new_tokens=2, temperature=1.0).shape == (1, 5)
    assert context.MODE == 0


def test_resnet18_forward_backward_and_bn_double_update(device):
    wxx = W()
    m = wxx.nn.ResNet18(num_classes=5)
    x = up(rng(5).standard_normal((2, 3, 32, 32)))
    out = m(x)
    assert out.shape == [2, 5]
    assert np.isfinite(out.numpy()).all()
    out.sum().backward()
    assert all(p.grad is not None for _, p in m.named_parameters())
    # bn1 of each block runs twice per forward: two EMA updates from 0
    rm = m.layer1._modules["0"].bn1.running_mean.numpy()
    assert np.abs(rm).max() > 0
    state = m.state_dict()
    m2 = wxx.nn.ResNet18(num_classes=5)
    m2.load_state_dict(state)
    assert all(np.array_equal(m2.state_dict()[k], v) for k, v in state.items())


def _hyena_expected(V, D, N, order, k=3, h=64, mlp_ratio=4, pe=8):
    # structural count of reference tests/test_hyena.py:83-113
    ffn = int(2 * (mlp_ratio * D) / 3)
    fin = 2 * pe + 1
    block = (D + (2 + order) * D * D + (k * D + D) + order * (fin * h + h + h * D + D)
             + order * D + D + 3 * D * ffn)
    return N * block + V * D + D


def test_hyena_parameter_counts_and_tying(device):
    wxx = W()
    for order in (1, 2, 3, 4):
        m = wxx.nn.Hyena(32, d_model=16, n_layers=2, order=order)
        total = sum(int(np.prod(p.shape)) for _, p in m.parameters())
        assert total == _hyena_expected(32, 16, 2, order)
    m = wxx.nn.Hyena(2048, d_model=256, n_layers=6, order=4)
    total = sum(int(np.prod(p.shape)) for _, p in m.parameters())
    assert total == 6_444_288 + 6 * 4 * 2 * 8 * 64 == 6_468_864
    assert m.head._embedding.weight is m.embed.weight
    names = [n for n, _ in m.named_parameters()]
    assert names.count("embed.weight") == 1 and not any(n.startswith("head.") for n in names)


def test_hyena_forward_backward_causal(device):
    wxx = W()
    from wxx_amd.backend.context import inferenceMode

    V, B, L = 40, 2, 32
    m = wxx.nn.Hyena(V, d_model=16, n_layers=2, order=3)
    ids = rng(6).integers(0, V, (B, L)).astype(np.uint32)
    out = m(up_u32(ids))
    assert out.shape == [B, L, V]
    assert np.isfinite(out.numpy()).all()
    out.sum().backward()
    grads = [p.grad for _, p in m.named_parameters()]
    assert all(g is not None for g in grads)
    assert any(np.any(g.numpy() != 0) for g in grads)
    with inferenceMode():
        a = m(up_u32(ids)).numpy()
        ids2 = ids.copy()
        ids2[:, 16:] = (ids2[:, 16:] + 7) % V
        b = m(up_u32(ids2)).numpy()
    assert np.allclose(a[:, :16], b[:, :16], atol=1e-3)
    assert not np.allclose(a[:, 16:], b[:, 16:])


def test_clip_grad_norm_device_path_matches_host_path(device):
    # reference tests/test_clip_grad.py: the fast path against the CPU formula
    wxx = W()
    m = wxx.nn.GPT2(50, d_model=16, n_heads=2, n_layers=2, max_len=8, dropout=0.0)
    out = m(up_u32(rng(7).integers(0, 50, (2, 8))))
    (out * 100.0).sum().backward()
    grads = [(n, p.grad.numpy().astype(np.float64)) for n, p in m.named_parameters()]
    want = np.sqrt(sum((g ** 2).sum() for _, g in grads))
    total = wxx.nn.clip_grad_norm_(m.parameters(), 1.0)
    assert abs(total - want) <= 1e-5 * want
    coef = 1.0 / (want + 1e-6)
    for (n, g0), (_, p) in zip(grads, m.named_parameters()):
        np.testing.assert_allclose(p.grad.numpy(), g0 * coef, rtol=1e-5, atol=1e-9, err_msg=n)


@pytest.mark.parametrize("S", [16, 130])
def test_causal_attention_skips_match_plain_masked_attention(device, S):
    # GPT-2's marked causal mask lets attention skip the masked triangles;
    # the same mask without the mark takes the full products: same numbers
    wxx = W()
    from wxx_amd.functional import from_numpy

    D, H, B = 32, 4, 2
    mha = wxx.nn.MultiHeadAttention(D, H)
    X = rng(80).standard_normal((B, S, D)).astype(np.float32)
    G = rng(81).standard_normal((B, S, D)).astype(np.float32)
    i = np.arange(S)
    data = np.where(i[None, :] <= i[:, None], 0.0, -1e9).astype(np.float32)
    res = []
    for marked in (True, False):
        mask = from_numpy(data)
        if marked:
            mask._causal = True
        x = up(X)
        x.requires_grad = True
        for _, p in mha.named_parameters():
            p.grad = None
        y = mha(x, mask)
        (y * up(G)).sum().backward()
        res.append([y.numpy(), x.grad.numpy()] + [p.grad.numpy() for _, p in mha.named_parameters()])
    for a, b in zip(*res):
        np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-7)


def test_causal_attention_with_dropout_matches_plain(device):
    # attention dropout > 0 takes the zero-writing causal path; same seeds,
    # same numbers as the unmarked mask
    import random

    wxx = W()
    from wxx_amd.functional import from_numpy

    S, D, H, B = 40, 16, 2, 2
    mha = wxx.nn.MultiHeadAttention(D, H, dropout=0.3)
    X = rng(82).standard_normal((B, S, D)).astype(np.float32)
    i = np.arange(S)
    data = np.where(i[None, :] <= i[:, None], 0.0, -1e9).astype(np.float32)
    res = []
    for marked in (True, False):
        mask = from_numpy(data)
        if marked:
            mask._causal = True
        random.seed(5)
        x = up(X)
        x.requires_grad = True
        for _, p in mha.named_parameters():
            p.grad = None
        y = mha(x, mask)
        y.sum().backward()
        res.append([y.numpy(), x.grad.numpy()] + [p.grad.numpy() for _, p in mha.named_parameters()])
    for a, b in zip(*res):
        np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-7)


def _walk(module, prefix=""):
    """(name, module) pairs of a module tree, depth first."""
    yield prefix.rstrip("."), module
    for name, m in module._modules.items():
        if m is not None:
            yield from _walk(m, prefix + name + ".")


def _within_error_floor(got, want64, ref32, name, c=4.0, rtol=1e-4, atol=1e-5):
    """|got - want64| <= atol + rtol |want64| + c max(|ref32 - want64|, rms)
    element by element, where ref32 is the same restated computation in
    float32 (same discrete decisions) and rms is the root mean square of
    |ref32 - want64| over the tensor: the device may miss the float64 value
    by the north star's bar plus c times what single precision itself misses
    by.  The rms term is there because the device adds in another order: two
    independent float32 evaluations miss by similar amounts overall, but not
    element by element (where ref32 happens to land almost exactly, another
    order does not), so a purely elementwise floor fails by chance on large
    tensors.  A dropped or wrong term misses by orders of magnitude more."""
    got, w, f = (np.asarray(a, np.float64) for a in (got, want64, ref32))
    err, floor = np.abs(got - w), np.abs(f - w)
    rms = float(np.sqrt(np.mean(floor ** 2))) if floor.size else 0.0
    bad = err > atol + rtol * np.abs(w) + c * np.maximum(floor, rms)
    assert not bad.any(), (f"{name}: {int(bad.sum())} of {bad.size} elements beyond the fp32 "
                           f"error floor; max err {err.max():.3g}, fp32 max err {floor.max():.3g}")
    return err.max(), floor.max()


def test_resnet18_config3_train_step_matches_oracle(device, monkeypatch):
    # ResNet18(10), batch 128 x 3 x 32 x 32, CCELoss;
    # logits, loss, every gradient and every BatchNorm running statistic after
    # the training forward, against the float64 restatement oracle/resnet.py,
    # element by element at rtol 1e-4 / atol 1e-5.
    # The oracle replays the device's discrete decisions (ReLU masks, max-pool
    # indices): an fp32 ReLU input or max-pool near-tie within rounding of the
    # other side flips between single and double precision and, at batch 128
    # with layer4 at 1 x 1, moves a whole batch element's gradient.  Those
    # decisions are checked on their own: each one that differs from the
    # oracle's own float64 choice must be a near-tie.
    from oracle import resnet as orn
    from wxx_amd import functional as wf
    from wxx_amd.autograd import convolution as ac
    from wxx_amd.autograd import normalization as an
    from wxx_amd.autograd import pointwise as ap

    wxx = W()
    relu_in, pool = [], {}
    relu_fwd = ap.relu.forward
    bn_act_fwd = an.batchnorm_act.forward

    def recording_relu(self, t):
        relu_in.append(t.numpy())
        return relu_fwd(self, t)

    def recording_bn_act(self, t, gamma, beta, res, rm, rv, updates=1, relu=True):
        if relu:  # the same kernel without the ReLU (on copies of the running statistics)
            pre, _, _ = wf.batchnorm_act(t, gamma, beta, res, wf.from_numpy(rm.numpy()),
                                         wf.from_numpy(rv.numpy()), 1, False)
            relu_in.append(pre.numpy())
        return bn_act_fwd(self, t, gamma, beta, res, rm, rv, updates, relu)

    pool_fwd = ac.maxpooling2d._fwd

    def recording_pool(*args):
        out, idx = pool_fwd(*args)
        pool["idx"] = idx.numpy()
        return out, idx

    monkeypatch.setattr(ap.relu, "forward", recording_relu)
    monkeypatch.setattr(an.batchnorm_act, "forward", recording_bn_act)
    monkeypatch.setattr(ac.maxpooling2d, "_fwd", staticmethod(recording_pool))

    model = wxx.nn.ResNet18(num_classes=10)
    r = rng(32)
    state = {n: (r.normal(0, np.sqrt(2.0 / (np.prod(a.shape[1:]))), a.shape) if a.ndim == 4
                 else (1.0 + r.normal(0, 0.1, a.shape) if n.endswith("weight") and a.ndim == 1
                       else r.normal(0, 0.1, a.shape))).astype(np.float32)
             for n, a in model.state_dict().items()}
    model.load_state_dict(state)
    params = {n: p.numpy().astype(np.float64) for n, p in model.named_parameters()}
    stats = {}
    for name, m in _walk(model):
        if hasattr(m, "running_mean"):
            stats[name + ".running_mean"] = m.running_mean.numpy().astype(np.float64)
            stats[name + ".running_std"] = m.running_std.numpy().astype(np.float64)
    x = rng(30).standard_normal((128, 3, 32, 32)).astype(np.float32)
    y = rng(31).integers(0, 10, 128)
    logits = model(up(x))
    loss = wxx.nn.CCELoss()(logits, up_u32(y))
    loss.backward()
    assert len(relu_in) == 17 and "idx" in pool

    forced = {"relu": [a > 0 for a in relu_in], "pool": pool["idx"]}
    seen = {}
    ol, og, ostats, ologits = orn.resnet18_loss_and_grads(params, stats, x, y, forced=forced,
                                                          record=seen)
    fl, fg, fstats, flogits = orn.resnet18_loss_and_grads(params, stats, x, y, np.float32,
                                                          forced=forced)
    # the device's decisions against the oracle's own float64 ones
    for k, (pre64, mask) in enumerate(zip(seen["relu_inputs"], forced["relu"])):
        differ = (pre64 > 0) != mask
        scale = np.abs(pre64).max()
        assert np.all(np.abs(pre64[differ]) <= 1e-5 * scale), f"relu {k}: a decision far from 0"
        assert differ.sum() <= 4, f"relu {k}: {int(differ.sum())} flipped decisions"
    xin = seen["pool_input"].reshape(-1)
    _, own_idx = oc.pool2d(seen["pool_input"], (3, 3), (2, 2), (1, 1), False)
    differ = own_idx != pool["idx"]
    assert differ.sum() <= 4
    assert np.all(np.abs(xin[own_idx[differ]] - xin[pool["idx"][differ]])
                  <= 1e-5 * np.abs(xin).max())

    # values: through 20 layers of fp32 arithmetic and batch statistics some
    # elements sit at the single-precision floor rather than inside the bar,
    # so the bar is widened by what the float32 restatement itself misses by
    _within_error_floor(logits.numpy(), ologits, flogits, "logits")
    assert abs(float(loss.numpy().reshape(-1)[0]) - ol) <= 1e-5 * abs(ol)
    for n, p in model.named_parameters():
        _within_error_floor(p.grad.numpy(), og[n], fg[n], n)
    for name, m in _walk(model):
        if hasattr(m, "running_mean"):
            _elementwise(m.running_mean.numpy(), ostats[name + ".running_mean"], name + " mean")
            _elementwise(m.running_std.numpy(), ostats[name + ".running_std"], name + " var")


def _hyena_slice_vs_oracle(row_cap_mode):
    from oracle import hyena as oh
    from wxx_amd.backend import compat

    wxx = W()
    V, D, L, order, B, S = 1024, 256, 1, 4, 8, 8192
    prev = compat.REFERENCE_ROW_CAP
    compat.REFERENCE_ROW_CAP = row_cap_mode
    try:
        model = wxx.nn.Hyena(V, d_model=D, n_layers=L, order=order)
        params = {n: p.numpy().astype(np.float64) for n, p in model.named_parameters()}
        ids = rng(40).integers(0, V, (B, S))
        tg = rng(41).integers(0, V, (B, S))
        logits = model(up_u32(ids))
        loss = wxx.nn.CCELoss()(logits.reshape((B * S, V)), up_u32(tg.reshape(-1)))
        loss.backward()
        got_loss = float(loss.numpy().reshape(-1)[0])
        grads = {n: p.grad.numpy() for n, p in model.named_parameters()}
        lg = logits.numpy()
    finally:
        compat.REFERENCE_ROW_CAP = prev
    cap = compat.ROW_CAP if row_cap_mode else 0
    ol, og = oh.hyena_loss_and_grads(params, ids, tg, L, order, row_cap=cap)
    assert abs(got_loss - ol) <= 1e-5 * abs(ol), (got_loss, ol)
    for n, g in grads.items():
        _elementwise(g, og[n], n)
    return lg


def test_hyena_config4_slice_matches_oracle(device):
    # BASELINE config 4 at full batch and length: Hyena(1024, 256, order 4),
    # 1 of its 6 layers, batch 8 x 8192 (FFT length 16384, 65 536 RMSNorm
    # rows), against the float64 oracle: loss and every gradient
    _hyena_slice_vs_oracle(False)


def test_hyena_config4_slice_reference_row_cap(device):
    # the same with the reference's 65 535-row cap reproduced: row 65 535 of
    # every RMSNorm (the last token of the last sequence) is zero, so its
    # logits are zero, and the oracle with the same cap agrees everywhere
    lg = _hyena_slice_vs_oracle(True)
    assert np.all(lg.reshape(-1, lg.shape[-1])[65535] == 0)
    assert np.any(lg.reshape(-1, lg.shape[-1])[65534] != 0)
