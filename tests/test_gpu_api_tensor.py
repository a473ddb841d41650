"""GPU: Tensor construction, views, shape errors and buffer reuse across train
steps — the behaviours of reference tests/test_tensor.py,
tests/test_validation.py and tests/test_memory.py, checked against numpy."""

import numpy as np
import pytest

from conftest import rng

pytestmark = pytest.mark.gpu


def wxx():
    import wxx_amd

    return wxx_amd


def f32(a):
    return wxx().functional.from_numpy(np.asarray(a, np.float32))


def u32_raw(a):
    """u32 tensor the way the reference's helpers build one: bytes + type tag."""
    a = np.ascontiguousarray(a, np.uint32)
    t = wxx().Tensor(list(a.shape), data=a.tobytes())
    t.type = "u32"
    t.nbytes = a.nbytes
    return t


def close(a, b, tol=1e-6):
    np.testing.assert_allclose(np.asarray(a), np.asarray(b), rtol=tol, atol=tol)


# ---- construction and round trips -------------------------------------------


def test_value_fill_and_item(device):
    t = wxx().Tensor((2, 3), value=5.0)
    assert t.shape == [2, 3] and t.type == "f32"
    np.testing.assert_array_equal(t.numpy(), np.full((2, 3), 5.0, np.float32))
    assert wxx().Tensor((1,), value=7.0).item() == 7.0


def test_numpy_round_trips(device):
    from wxx_amd.functional.fft import from_numpy_complex

    a = rng(0).standard_normal((4, 5)).astype(np.float32)
    np.testing.assert_array_equal(f32(a).numpy(), a)
    z = (rng(6).standard_normal((3, 4)) + 1j * rng(7).standard_normal((3, 4))).astype(np.complex64)
    tz = from_numpy_complex(z)
    assert tz.type == "c64" and tz.shape == [3, 4]
    np.testing.assert_array_equal(tz.numpy(), z)
    ids = u32_raw(np.arange(10))
    np.testing.assert_array_equal(ids.numpy(), np.arange(10, dtype=np.uint32))


# ---- views ------------------------------------------------------------------


def test_broadcast_add(device):
    a, b = rng(1).standard_normal((3, 4)), rng(2).standard_normal(4)
    c = f32(a) + f32(b)
    assert c.shape == [3, 4]
    close(c.numpy(), (a.astype(np.float32) + b.astype(np.float32)))
    c2 = f32(rng(11).standard_normal((3, 1))) + f32(rng(12).standard_normal((1, 4)))
    assert c2.shape == [3, 4]
    with pytest.raises(ValueError):
        f32(np.zeros((3, 2))) + f32(np.zeros((1, 4)))


def test_reshape_permute_transpose_squeeze(device):
    a = rng(3).standard_normal((2, 3, 4)).astype(np.float32)
    x = f32(a)
    np.testing.assert_array_equal(x.reshape((6, 4)).numpy(), a.reshape(6, 4))
    assert x.reshape((-1, 4)).shape == [6, 4]
    np.testing.assert_array_equal(x.permute(2, 0, 1).numpy(), a.transpose(2, 0, 1))
    assert x.view(6, 4).shape == [6, 4]
    assert x.flatten(1, 2).shape == [2, 12]
    b = f32(np.zeros((2, 1, 4)))
    assert b.transpose(0, 2).shape == [4, 1, 2]
    assert b.unsqueeze(1).shape == [2, 1, 1, 4]
    assert b.squeeze().shape == [2, 4]
    assert b.squeeze(2).shape == [2, 1, 4]


@pytest.mark.parametrize("axes", [(2, 0, 1), (-1, 0, 1)])
def test_permute_tuple_and_backward(device, axes):
    a = rng(9).standard_normal((2, 3, 4)).astype(np.float32)
    x = f32(a)
    x.requires_grad = True
    p = x.permute(axes)
    ax = tuple(i % 3 for i in axes)
    np.testing.assert_array_equal(p.numpy(), a.transpose(ax))
    w = rng(10).standard_normal(p.shape).astype(np.float32)
    (p * f32(w)).sum().backward()
    np.testing.assert_array_equal(x.grad.numpy(), w.transpose(np.argsort(ax)))


def test_slice_narrow_chunk_index(device):
    a = rng(4).standard_normal((4, 6)).astype(np.float32)
    x = f32(a)
    np.testing.assert_array_equal(x[:, 2:5].numpy(), a[:, 2:5])
    np.testing.assert_array_equal(x.narrow(1, 1, 4).numpy(), a[:, 1:5])
    for i, c in enumerate(x.chunk(3, dim=1)):
        np.testing.assert_array_equal(c.numpy(), a[:, 2 * i:2 * i + 2])
    b = rng(5).standard_normal((5, 4)).astype(np.float32)
    np.testing.assert_array_equal(f32(b)[[0, 2, 4]].numpy(), b[[0, 2, 4]])


def test_strided_views_materialise(device):
    a = rng(6).standard_normal((4, 6)).astype(np.float32)
    x = f32(a)
    v = x[:, ::2]
    assert not v.is_contiguous()
    c = v.contiguous()
    assert c.is_contiguous()
    np.testing.assert_array_equal(c.numpy(), a[:, ::2])
    close((v + 1.0).numpy(), a[:, ::2] + np.float32(1.0))
    np.testing.assert_array_equal(v.reshape((-1,)).numpy(), a[:, ::2].reshape(-1))
    np.testing.assert_array_equal(x.permute(1, 0).numpy(), a.T)


def test_unsqueeze_of_strided_view_backward(device):
    x = f32(rng(19).standard_normal((2, 3, 4)))
    x.requires_grad = True
    u = x[:, 1:, :].unsqueeze(1)
    assert u.shape == [2, 1, 2, 4]
    u.sum().backward()
    want = np.zeros((2, 3, 4), np.float32)
    want[:, 1:, :] = 1.0
    np.testing.assert_array_equal(x.grad.numpy(), want)


# ---- validation errors ------------------------------------------------------


def test_normalize_dim():
    from wxx_amd import validation

    assert validation.normalize_dim(-1, 3) == 2
    assert validation.normalize_dim(1, 3) == 1
    for dim, rank in ((5, 3), (0, 0)):
        with pytest.raises(IndexError):
            validation.normalize_dim(dim, rank)


def test_shape_errors(device):
    x = f32(np.zeros((2, 3)))
    for bad in ((7,), (2, 2)):
        with pytest.raises(ValueError):
            x.reshape(bad)
    y = f32(np.zeros((2, 3, 4)))
    for axes in ((0, 1), (0, 0, 1)):
        with pytest.raises(ValueError):
            y.permute(*axes)
    with pytest.raises(ValueError):
        y.flatten(2, 1)
    z = f32(np.zeros((4, 6)))
    with pytest.raises(IndexError):
        z.narrow(1, 5, 2)
    with pytest.raises((IndexError, ValueError, TypeError)):
        z.narrow(1, 0, -1)


def test_matmul_operator_shapes(device):
    c = f32(np.ones((2, 3, 4))) @ f32(np.ones((2, 4, 5)))
    assert c.shape == [2, 3, 5]
    np.testing.assert_array_equal(c.numpy(), np.full((2, 3, 5), 4.0, np.float32))
    with pytest.raises(ValueError):
        f32(np.ones(4)) @ f32(np.ones((4, 5)))


def test_assign_checks(device):
    a = f32(rng(15).standard_normal((2, 3)))
    with pytest.raises(ValueError):
        wxx().functional.assign(a, f32(np.zeros((2, 4))))
    wxx().functional.assign(a, 0.0)
    np.testing.assert_array_equal(a.numpy(), np.zeros((2, 3), np.float32))


def test_cceloss_argument_checks(device):
    F = wxx().functional
    logits = f32(rng(17).standard_normal((4, 5)))
    loss, grad = F.cceloss(logits, u32_raw([0, 1, 2, 3]))
    assert loss.shape == [4, 1] and grad.shape == [4, 5]
    with pytest.raises(ValueError):
        F.cceloss(logits, u32_raw([0, 1]))
    with pytest.raises(ValueError):
        F.cceloss(f32(np.zeros(5)), u32_raw([0, 1, 2, 3]))
    two = f32(rng(24).standard_normal((2, 4)))
    F.cceloss(two, u32_raw([0, 3]))  # K - 1 is the last legal target
    with pytest.raises(ValueError):
        F.cceloss(two, u32_raw([0, 4]))
    with pytest.raises(ValueError):  # hidden states mistaken for logits
        F.cceloss(f32(rng(25).standard_normal((2, 256))), u32_raw([0, 4095]))


def test_concat_checks(device):
    F = wxx().functional
    a, b = rng(20).standard_normal((2, 3)), rng(21).standard_normal((2, 4))
    c = F.concat([f32(a), f32(b)], dim=1)
    np.testing.assert_array_equal(c.numpy(), np.concatenate([a, b], 1).astype(np.float32))
    with pytest.raises(ValueError):
        F.concat([f32(a), f32(np.zeros((3, 3)))], dim=1)
    with pytest.raises(ValueError):
        F.concat([], dim=0)


# ---- buffer reuse -----------------------------------------------------------


def test_train_steps_do_not_grow_live_buffers(device):
    W = wxx()
    from wxx_amd.backend.device import get_buffer_pool

    pool = get_buffer_pool()
    V, S, B = 64, 8, 2
    model = W.nn.GPT2(V, d_model=16, n_heads=2, n_layers=2, max_len=S, tie_weights=True)
    loss_fn = W.nn.CCELoss()
    opt = W.nn.AdamW(list(model.parameters()), lr=1e-4)
    r = rng(7)
    xs, ys = r.integers(0, V, (B, S)), r.integers(0, V, (B, S))

    def step():
        out = model(u32_raw(xs))
        b, s, v = out.shape
        loss = loss_fn(out.reshape((b * s, v)), u32_raw(ys).reshape((b * s,)))
        loss.backward()
        loss.item()
        opt.step()
        opt.zero_grad()

    def live():
        snap = pool.get_memory_snapshot()
        return len(snap["active"]), snap["active_bytes"]

    for _ in range(3):
        step()
    n0, b0 = live()
    for _ in range(8):
        step()
    n1, b1 = live()
    assert n1 <= n0 + 4, (n0, n1)
    assert b1 <= b0 + 64 * 1024, (b0, b1)
