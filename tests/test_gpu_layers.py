"""GPU parity: cross-entropy, AdamW (single and multi-tensor), gradient-norm
clipping, embedding gather / scatter-add, dropout and the decay window."""

import ctypes as C

import numpy as np
import pytest

from conftest import assert_close, rng
from oracle import layers as ol

pytestmark = pytest.mark.gpu


def F():
    from wxx_amd import functional

    return functional


def up(a):
    return F().from_numpy(np.asarray(a, np.float32))


def up_u32(a):
    return F().from_numpy(np.asarray(a), np.uint32)


# ------------------------------------------------------------------ cceloss


@pytest.mark.parametrize("B,K,scale", [(4, 10, 1.0), (128, 10, 3.0), (512, 1024, 1.0),
                                       (33, 1023, 5.0), (7, 4097, 1.0), (64, 50304, 2.0),
                                       (3, 70001, 1.0)])
def test_cceloss(device, B, K, scale):
    z = (rng(B).standard_normal((B, K)) * scale).astype(np.float32)
    t = rng(K).integers(0, K, B).astype(np.uint32)
    t[0] = K - 1
    loss, dz = F().cceloss(up(z), up_u32(t))
    el, edz = ol.cceloss(z, t)
    assert loss.shape == [B, 1]
    assert_close(loss.numpy(), el, rtol=1e-4, atol=1e-5, msg="loss")
    assert_close(dz.numpy(), edz, rtol=1e-4, atol=1e-6, msg="dlogits")


@pytest.mark.parametrize("B,K", [(5, 10), (64, 1000), (8, 50304), (3, 70001)])
def test_cceloss_autograd_deferred_gradient(device, B, K):
    # the autograd path defers dlogits to the backward (rows <= 65536); the
    # loss and the gradient equal cceloss's, times the mean's 1/B, bit for bit
    import wxx_amd as wxx

    z = (rng(B + K).standard_normal((B, K)) * 3).astype(np.float32)
    t = rng(K).integers(0, K, B).astype(np.uint32)
    t[-1] = K - 1
    loss_e, dz_e = F().cceloss(up(z), up_u32(t))
    want = (dz_e * F().from_numpy(np.full((B, 1), 1.0 / B, np.float32))).numpy()
    x = up(z)
    x.requires_grad = True
    rows = wxx.autograd.CrossEntropyLoss(x).forward(x, up_u32(t))  # per-row losses
    assert np.array_equal(rows.numpy(), loss_e.numpy())
    loss = rows.mean()
    loss.backward()
    assert np.array_equal(x.grad.numpy(), want)
    with pytest.raises(ValueError):  # out-of-range target, autograd path
        wxx.nn.CCELoss()(x, up_u32(np.full(B, K, np.uint32)))


def test_cceloss_rejects_out_of_range_target(device):
    z = np.zeros((3, 5), np.float32)
    with pytest.raises(ValueError):
        F().cceloss(up(z), up_u32([0, 5, 1]))
    # the flag is cleared for the next call
    loss, _ = F().cceloss(up(z), up_u32([0, 4, 1]))
    assert_close(loss.numpy(), np.full((3, 1), np.log(5.0), np.float32))


# -------------------------------------------------------------------- adamw


def test_adamw_single(device):
    n = 10007
    p, g, m, v = (rng(i).standard_normal(n).astype(np.float32) for i in range(4))
    v = np.abs(v)
    tp, tm, tv = up(p), up(m), up(v)
    bc1, bc2 = ol.bias_corrections(3, 0.9, 0.999)
    F().adamw(tp, up(g), tm, tv, 3, 1e-3, 0.9, 0.999, 1e-7, 1e-4, bc1, bc2)
    ep, em, ev = ol.adamw(p, g, m, v, 1e-3, 0.9, 0.999, 1e-7, 1e-4, bc1, bc2)
    assert_close(tm.numpy(), em, rtol=1e-6, atol=1e-7)
    assert_close(tv.numpy(), ev, rtol=1e-6, atol=1e-7)
    assert_close(tp.numpy(), ep, rtol=1e-6, atol=1e-6)


def test_adamw_multi_matches_per_tensor(device):
    sizes = [1, 3, 4096, 4097, 768 * 3, 50304 * 7 + 5]
    ps = [rng(10 + i).standard_normal(s).astype(np.float32) for i, s in enumerate(sizes)]
    gs = [rng(20 + i).standard_normal(s).astype(np.float32) for i, s in enumerate(sizes)]
    tps = [up(p) for p in ps]
    tgs = [up(g) for g in gs]
    tms = [up(np.zeros(s)) for s in sizes]
    tvs = [up(np.zeros(s)) for s in sizes]
    ms = [np.zeros(s, np.float32) for s in sizes]
    vs = [np.zeros(s, np.float32) for s in sizes]
    for step in (1, 2):
        bc1, bc2 = ol.bias_corrections(step, 0.9, 0.999)
        F().adamw_multi(tps, tgs, tms, tvs, 1e-3, 0.9, 0.999, 1e-7, 1e-4, bc1, bc2)
        for i in range(len(sizes)):
            ps[i], ms[i], vs[i] = ol.adamw(ps[i], gs[i], ms[i], vs[i], 1e-3, 0.9, 0.999, 1e-7,
                                           1e-4, bc1, bc2)
    for i in range(len(sizes)):
        assert_close(tps[i].numpy(), ps[i], rtol=1e-6, atol=1e-6, msg=f"param {i}")
        assert_close(tms[i].numpy(), ms[i], rtol=1e-6, atol=1e-7, msg=f"m {i}")
        assert_close(tvs[i].numpy(), vs[i], rtol=1e-6, atol=1e-7, msg=f"v {i}")


# --------------------------------------------------------- gradient norm


def test_sumsq_multi_and_scale(device):
    sizes = [5, 4096, 123457, 768 * 768]
    gs = [rng(30 + i).standard_normal(s).astype(np.float32) for i, s in enumerate(sizes)]
    tgs = [up(g) for g in gs]
    total = F().sumsq_multi(tgs).numpy()[0]
    norm, clipped = ol.clip_grad_norm(gs, 1.0)
    assert abs(float(total) ** 0.5 - norm) / norm < 1e-5
    coef = 1.0 / (norm + 1e-6)
    F().scale_multi(tgs + [tgs[0]], coef)  # a repeated tensor is scaled once
    for t, c in zip(tgs, clipped):
        assert_close(t.numpy(), c.astype(np.float32), rtol=1e-5, atol=1e-8)


def test_sumsq_multi_empty_list(device):
    assert F().sumsq_multi([]).numpy()[0] == 0.0


# ---------------------------------------------------------------- embedding


@pytest.mark.parametrize("V,D,B,L", [(64, 32, 8, 300), (7, 3, 2, 5), (50304, 768, 2, 1024),
                                     (1024, 256, 8, 257)])
def test_embed_bit_exact_and_embeddx(device, V, D, B, L):
    ids = rng(V).integers(0, V, (B, L)).astype(np.uint32)
    W = rng(D).standard_normal((V, D)).astype(np.float32)
    out = F().embed(up_u32(ids), up(W), B * L, D)
    assert out.shape == [B, L, D]
    assert np.array_equal(out.numpy(), ol.embed(ids, W)), "gather must be bit-exact"
    g = rng(L).standard_normal((B, L, D)).astype(np.float32)
    got = F().embeddx(up(g), up_u32(ids), B * L, D, V).numpy()
    assert_close(got, ol.embeddx(g, ids, V), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("V,D,ntok", [(1024, 8, 65536), (50304, 4, 8192), (3, 5, 10000),
                                      (1024, 256, 65536)])
def test_embeddx_token_order_bit_exact(device, V, D, ntok):
    # the gradient row of id v adds its tokens' rows in token order, which
    # a float32 np.add.at reproduces bit for bit (Hyena's 1024 x 65536
    # tokens, GPT-2's vocabulary, a few ids with long runs; the placement
    # cuts the token list into segments for these sizes)
    ids = rng(V + ntok).integers(0, V, ntok).astype(np.uint32)
    g = rng(D).standard_normal((ntok, D)).astype(np.float32)
    want = np.zeros((V, D), np.float32)
    np.add.at(want, ids.astype(np.int64), g)
    got = F().embeddx(up(g), up_u32(ids), ntok, D, V).numpy()
    assert np.array_equal(got, want)


def test_embeddx_repeated_and_out_of_range_ids(device):
    V, D = 5, 6
    ids = np.array([[1, 1, 1, 9, 0, 1]], np.uint32)
    g = rng(1).standard_normal((1, 6, D)).astype(np.float32)
    got = F().embeddx(up(g), up_u32(ids), 6, D, V).numpy()
    assert_close(got, ol.embeddx(g, ids, V), rtol=1e-6, atol=1e-6)
    assert np.all(got[2:] == 0)
    # deterministic: a second call returns identical bits
    again = F().embeddx(up(g), up_u32(ids), 6, D, V).numpy()
    assert np.array_equal(got, again)


# ------------------------------------------------------------------ dropout


@pytest.mark.parametrize("n,p", [(1, 0.5), (1000, 0.1), (8 * 1024 * 768 + 3, 0.1), (4096, 0.0)])
def test_dropout_bit_exact(device, n, p):
    x = rng(n % 97).standard_normal(n).astype(np.float32)
    y, seed = F().dropout(up(x), p)
    assert 0 <= seed < 2**32
    assert np.array_equal(y.numpy(), ol.dropout(x, seed, p)), "dropout mask/scale must be bit-exact"
    g = rng(5).standard_normal(n).astype(np.float32)
    dx = F().dropoutdx(up(g), p, seed).numpy()
    assert np.array_equal(dx, ol.dropout(g, seed, p))


def test_dropout_p0_fresh_buffer_and_module_sharing(device):
    # functional.dropout / dropoutdx at p == 0 return a fresh buffer (as the
    # reference does): writing into the result leaves the input unchanged.
    # The nn/autograd layer shares the input's storage at p == 0 on purpose
    # (no copy of attention's probabilities): there the write shows through.
    from wxx_amd import nn

    x = rng(3).standard_normal((4, 6)).astype(np.float32)
    tx = up(x)
    y, _ = F().dropout(tx, 0.0)
    F().assign(y, 5.0)
    assert np.array_equal(tx.numpy(), x)
    assert np.all(y.numpy() == 5.0)
    d = F().dropoutdx(tx, 0.0, 123)
    F().assign(d, 7.0)
    assert np.array_equal(tx.numpy(), x)
    ym = nn.Dropout(0.0)(tx)
    assert np.array_equal(ym.numpy(), x)
    F().assign(ym, 9.0)
    assert np.all(tx.numpy() == 9.0), "the autograd layer's p == 0 result shares storage"


# ------------------------------------------------------------- decay window


def test_decay_window(device):
    decay = rng(6).standard_normal((4, 64)).astype(np.float32)
    L = 8192
    w = F().decay_window(up(decay), 2, L).numpy()
    assert_close(w, ol.decay_window(decay, 2, L), rtol=1e-5, atol=1e-6)
    g = rng(7).standard_normal((64, L)).astype(np.float32)
    d = F().decay_window_backward(up(g), up(decay), 2, L).numpy()
    assert_close(d, ol.decay_window_backward(g, decay, 2, L), rtol=1e-4, atol=1e-4)


# ------------------------------------------------------------------- SwiGLU


@pytest.mark.parametrize("T,d,hid", [(256, 128, 170), (512, 256, 682), (128, 128, 128 + 1)])
def test_swiglu_padded_matches_composed(device, T, d, hid):
    # the SwiGLU op with its hidden width padded to a multiple of 128 (zero
    # weight columns / rows) against the composed ops (Linear, silu, product,
    # Linear) on the same weights: output and every gradient
    import wxx_amd as wxx
    from wxx_amd import nn

    r = rng(T + hid)
    x = (r.standard_normal((2, T // 2, d)) * 0.5).astype(np.float32)
    g = r.standard_normal((2, T // 2, d)).astype(np.float32)
    m = nn.SwiGLU(d, hidden_dim=hid)
    outs = []
    for padded in (True, False):
        for lin in (m.w1, m.w2, m.w3):
            lin.weight.grad = None
        tx = up(x)
        tx.requires_grad = True
        if padded:
            y = m(tx)
            assert y.creator is not None and type(y.creator).__name__ == "swiglu_padded"
        else:
            y = m.w3(m.w1(tx).silu() * m.w2(tx))
        (y * up(g)).sum().backward()
        outs.append([y.numpy(), tx.grad.numpy()] + [lin.weight.grad.numpy()
                                                     for lin in (m.w1, m.w2, m.w3)])
    for name, a, e in zip(["y", "dx", "dw1", "dw2", "dw3"], *outs):
        assert a.shape == e.shape, name
        assert_close(a, e, rtol=1e-4, atol=2e-5 * np.sqrt(max(d, hid)), msg=name)


@pytest.mark.parametrize("n", [1, 7, 4096, 65536 * 3 + 5])
def test_swiglu_gate_bit_exact_against_composed_ops(device, n):
    # silu(a) * b and its backward in one kernel each: the same roundings as
    # the sigmoid, product, product-backward and sigmoid-backward kernels
    r = rng(n)
    a = (r.standard_normal(n) * 4).astype(np.float32)
    a[: min(n, 3)] = [100.0, -100.0, 0.0][: min(n, 3)]  # the sigmoid's clamp and zero
    b = r.standard_normal(n).astype(np.float32)
    dh = r.standard_normal(n).astype(np.float32)
    ta, tb, tdh = up(a), up(b), up(dh)
    s = F().unary(ta, "sigmoid")
    g = F().pointwise(s, ta, 2)
    h = F().pointwise(g, tb, 2)
    assert np.array_equal(F().swiglu_gate(ta, tb).numpy(), h.numpy())
    db = F().pointwise(tdh, g, 2)
    dg = F().pointwise(tdh, tb, 2)
    da = F().pointwise(F().pointwise(dg, s, 2),
                       F().unary_backward(s, F().pointwise(dg, ta, 2), "sigmoid"), 0)
    gda, gdb = F().swiglu_gate_backward(tdh, ta, tb)
    assert np.array_equal(gda.numpy(), da.numpy())
    assert np.array_equal(gdb.numpy(), db.numpy())
