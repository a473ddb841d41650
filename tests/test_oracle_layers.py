"""Pin the oracle's loss / optimizer / embedding / dropout restatements (CPU-only).

Each check is independent of the oracle's own formula: torch's CPU
implementations of the same textbook operations (cross-entropy, AdamW with
decoupled weight decay, clip_grad_norm_), the reference's own test loops
(tests/test_embedding.py, tests/test_dropout.py, tests/test_clip_grad.py),
a scalar pure-Python restatement of the dropout hash, and finite differences.
"""

import math

import numpy as np
import pytest

from conftest import assert_close, rng
from oracle import layers as ol


def _torch():
    return pytest.importorskip("torch")


# ------------------------------------------------------------------ cceloss


def test_cceloss_matches_torch_cross_entropy():
    torch = _torch()
    z = rng(0).standard_normal((37, 101)) * 3.0
    t = rng(1).integers(0, 101, 37)
    loss, dz = ol.cceloss(z, t)
    zt = torch.tensor(z, dtype=torch.float64, requires_grad=True)
    ref = torch.nn.functional.cross_entropy(zt, torch.tensor(t), reduction="none")
    ref.sum().backward()
    assert_close(loss[:, 0], ref.detach().numpy().astype(np.float32), rtol=1e-6, atol=1e-6)
    assert_close(dz, zt.grad.numpy().astype(np.float32), rtol=1e-6, atol=1e-7)


def test_cceloss_gradient_by_finite_differences():
    z = rng(2).standard_normal((3, 9))
    t = np.array([0, 8, 4])
    _, dz = ol.cceloss(z, t)
    h = 1e-6
    for r in range(3):
        for j in range(9):
            zp, zm = z.copy(), z.copy()
            zp[r, j] += h
            zm[r, j] -= h
            def L(zz):
                m = zz[r].max()
                return math.log(np.exp(zz[r] - m).sum()) + m - zz[r, t[r]]
            fd = (L(zp) - L(zm)) / (2 * h)
            assert abs(fd - dz[r, j]) < 1e-5


def test_cceloss_rejects_out_of_range_target():
    with pytest.raises(ValueError):
        ol.cceloss(np.zeros((2, 4)), np.array([0, 4]))


# -------------------------------------------------------------------- adamw


def test_adamw_matches_torch_adamw_three_steps():
    torch = _torch()
    p0 = rng(3).standard_normal(1000).astype(np.float32)
    grads = [rng(4 + s).standard_normal(1000).astype(np.float32) for s in range(3)]
    lr, b1, b2, eps, wd = 1e-3, 0.9, 0.999, 1e-7, 1e-4  # reference defaults, nn/optimizer.py:39
    tp = torch.nn.Parameter(torch.tensor(p0.astype(np.float64)))
    opt = torch.optim.AdamW([tp], lr=lr, betas=(b1, b2), eps=eps, weight_decay=wd)
    p, m, v = p0, np.zeros_like(p0), np.zeros_like(p0)
    for s, g in enumerate(grads, start=1):
        tp.grad = torch.tensor(g.astype(np.float64))
        opt.step()
        bc1, bc2 = ol.bias_corrections(s, b1, b2)
        p, m, v = ol.adamw(p, g, m, v, lr, b1, b2, eps, wd, bc1, bc2)
    assert_close(p, tp.detach().numpy().astype(np.float32), rtol=1e-5, atol=1e-6)


def test_adamw_first_step_is_signed_lr():
    # With m = v = 0 the first bias-corrected step is g / (|g| + eps) ~= sign(g).
    g = np.array([0.5, -2.0, 3.0], np.float32)
    p = np.zeros(3, np.float32)
    bc1, bc2 = ol.bias_corrections(1, 0.9, 0.999)
    p1, _, _ = ol.adamw(p, g, np.zeros(3), np.zeros(3), 0.1, 0.9, 0.999, 1e-7, 0.0, bc1, bc2)
    assert_close(p1, -0.1 * np.sign(g), rtol=1e-5, atol=1e-6)


# ----------------------------------------------------------- clip_grad_norm


def test_clip_grad_norm_matches_torch():
    torch = _torch()
    gs = [rng(10 + i).standard_normal(s) for i, s in enumerate([(7, 3), (11,), (2, 2, 5)])]
    norm, clipped = ol.clip_grad_norm(gs, 1.0)
    ps = [torch.nn.Parameter(torch.zeros(g.shape, dtype=torch.float64)) for g in gs]
    for p, g in zip(ps, gs):
        p.grad = torch.tensor(g)
    tnorm = torch.nn.utils.clip_grad_norm_(ps, 1.0)
    assert abs(norm - float(tnorm)) < 1e-9
    for c, p in zip(clipped, ps):
        assert_close(c, p.grad.numpy(), rtol=1e-6, atol=1e-9)


def test_clip_grad_norm_leaves_small_grads():
    g = [np.full(4, 0.1)]
    norm, clipped = ol.clip_grad_norm(g, 10.0)
    assert abs(norm - 0.2) < 1e-12
    assert np.array_equal(clipped[0], g[0])


# ---------------------------------------------------------------- embedding


def test_embed_and_embeddx_match_reference_test_loops():
    # reference tests/test_embedding.py:50-60 (backward loop)
    V, D, B, L = 7, 3, 2, 5
    ids = rng(1).integers(0, V, size=(B, L)).astype(np.uint32)
    g = rng(2).standard_normal((B, L, D)).astype(np.float32)
    W = rng(3).standard_normal((V, D)).astype(np.float32)
    out = ol.embed(ids, W)
    for b in range(B):
        for l in range(L):
            assert np.array_equal(out[b, l], W[ids[b, l]])
    ref = np.zeros((V, D), dtype=np.float64)
    for b in range(B):
        for l in range(L):
            ref[ids[b, l]] += g[b, l]
    assert_close(ol.embeddx(g, ids, V), ref, atol=1e-12)


def test_embeddx_skips_out_of_range_ids():
    g = np.ones((1, 3, 2))
    ids = np.array([[0, 5, 1]], np.uint32)
    out = ol.embeddx(g, ids, 2)
    assert np.array_equal(out, np.array([[1.0, 1.0], [1.0, 1.0]]))


# ------------------------------------------------------------------ dropout


def _hash_scalar(x):
    x &= 0xFFFFFFFF
    x = (((x >> 16) ^ x) * 0x45D9F3B) & 0xFFFFFFFF
    x = (((x >> 16) ^ x) * 0x45D9F3B) & 0xFFFFFFFF
    return ((x >> 16) ^ x) & 0xFFFFFFFF


def test_dropout_hash_matches_scalar_restatement():
    xs = np.concatenate([np.arange(0, 300), rng(5).integers(0, 2**32, 300)]).astype(np.uint64)
    got = ol.dropout_hash(xs.astype(np.uint32))
    want = np.array([_hash_scalar(int(x)) for x in xs], np.uint32)
    assert np.array_equal(got, want)
    assert _hash_scalar(0) == 0


def test_dropout_mask_properties():
    # reference tests/test_dropout.py:10-30: kept values are x / (1 - p), the rest 0
    x = np.ones(20000, np.float32)
    for p in (0.1, 0.25, 0.5):
        y = ol.dropout(x, 123456789, p)
        assert set(np.unique(y).tolist()) <= {0.0, float(np.float32(1.0 / (1.0 - p)))}
        frac = np.count_nonzero(y) / y.size
        assert abs(frac - (1.0 - p)) < 0.02
    assert np.array_equal(ol.dropout(x, 7, 0.0), x)


def test_dropout_keep_is_literal_threshold():
    seed, p = 0xDEADBEEF, 0.3
    keep = ol.dropout_keep(500, seed, p)
    for i in range(500):
        r = np.float32(_hash_scalar(i ^ seed) >> 8) * np.float32(1.0 / 16777216.0)
        assert keep[i] == (r >= np.float32(p))


# ------------------------------------------------------------- decay window


def test_decay_window_closed_form_and_backward_fd():
    decay = rng(6).standard_normal((3, 4))
    stage, L = 1, 9
    w = ol.decay_window(decay, stage, L)
    assert_close(w[:, 0], np.ones(4))
    assert_close(w[2, 3], math.exp(-abs(decay[1, 2]) * 3))
    g = rng(7).standard_normal((4, L))
    d = ol.decay_window_backward(g, decay, stage, L)
    assert np.all(d[0] == 0) and np.all(d[2] == 0)
    h = 1e-6
    for c in range(4):
        dp, dm = decay.copy(), decay.copy()
        dp[stage, c] += h
        dm[stage, c] -= h
        fd = ((g * ol.decay_window(dp, stage, L)).sum() - (g * ol.decay_window(dm, stage, L)).sum()) / (2 * h)
        assert abs(fd - d[stage, c]) < 1e-6
