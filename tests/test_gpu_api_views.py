"""GPU: Tensor view semantics of the reference API — ``detach``/``detach_`` and
``diagonal`` (behaviours of reference tests/test_detach.py and
tests/test_diagonal.py, re-derived here against numpy)."""

import gc

import numpy as np
import pytest

from conftest import rng

pytestmark = pytest.mark.gpu


def wxx():
    import wxx_amd

    return wxx_amd


def f32(a):
    return wxx().functional.from_numpy(np.asarray(a, np.float32))


def u32(a):
    return wxx().functional.from_numpy(np.asarray(a), np.uint32)


# ---- detach (Tensor.py detach / detach_) ------------------------------------


def test_detach_is_a_gradless_view(device):
    a = rng(0).standard_normal((3, 4)).astype(np.float32)
    x = f32(a)
    x.requires_grad = True
    d = x.detach()
    assert (d.shape, d.type, d.requires_grad, d.creator, d.grad) == ([3, 4], "f32", False, None,
                                                                     None)
    assert d.buffer is x.buffer
    np.testing.assert_array_equal(d.numpy(), a)


def test_backward_through_detached_only_tensor_raises(device):
    x = f32(np.ones((2, 3)))
    x.requires_grad = True
    y = (x.detach() * 3.0).sum()
    assert y.requires_grad is False
    with pytest.raises(RuntimeError):
        y.backward()
    assert x.grad is None


def test_detach_cuts_one_branch_only(device):
    x = f32(np.ones((2, 3)))
    x.requires_grad = True
    z = (x.detach() + x).sum()
    assert z.requires_grad
    z.backward()
    np.testing.assert_array_equal(x.grad.numpy(), np.ones((2, 3), np.float32))


@pytest.mark.parametrize("view", ["whole", "column_slice"])
def test_detach_writes_through_to_the_source(device, view):
    a = rng(1).standard_normal((4, 6)).astype(np.float32)
    x = f32(a)
    src = x if view == "whole" else x[:, 1:5]
    d = src.detach()
    if view == "column_slice":
        assert d.shape == [4, 4] and not d.is_contiguous()
        np.testing.assert_array_equal(d.numpy(), a[:, 1:5])
    wxx().functional.assign(d, -1.0)
    want = a.copy()
    if view == "whole":
        want[:] = -1.0
    else:
        want[:, 1:5] = -1.0
    np.testing.assert_array_equal(x.numpy(), want)


def test_detached_view_keeps_its_storage(device):
    a = rng(3).standard_normal((2, 3)).astype(np.float32)
    d = f32(a).detach()
    gc.collect()
    np.testing.assert_array_equal(d.numpy(), a)


def test_detach_in_place(device):
    x = f32(np.ones((2, 2)))
    x.requires_grad = True
    y = x * 2.0
    assert y.creator is not None
    assert y.detach_() is y
    assert (y.requires_grad, y.creator, y.grad) == (False, None, None)


def test_detach_of_parameter_is_plain_tensor(device):
    W = wxx()
    p = W.Parameter(W.Tensor((3,), value=2.0))
    d = p.detach()
    assert isinstance(d, W.Tensor) and not isinstance(d, W.Parameter)
    assert d.requires_grad is False and d.buffer is p.buffer
    np.testing.assert_array_equal(d.numpy(), np.full(3, 2.0, np.float32))


def test_detach_keeps_dtype(device):
    from wxx_amd.functional.fft import from_numpy_complex

    ids = u32(np.arange(6).reshape(2, 3))
    assert ids.detach().type == "u32"
    np.testing.assert_array_equal(ids.detach().numpy(), np.arange(6).reshape(2, 3))
    z = np.full((2, 2), 1 + 2j, np.complex64)
    dz = from_numpy_complex(z).detach()
    assert dz.type == "c64"
    np.testing.assert_array_equal(dz.numpy(), z)


def test_module_on_detached_input_trains_only_the_module(device):
    from wxx_amd.nn.module import LayerNorm

    x = f32(np.ones((2, 4)))
    x.requires_grad = True
    ln = LayerNorm(4)
    out = ln(x.detach()).sum()
    assert out.requires_grad
    out.backward()
    assert x.grad is None
    assert ln.weight.grad is not None


# ---- diagonal (Tensor.diagonal, functional/utils.py diagonal) ----------------


def _diag_grad(shape, w, offset, d1, d2):
    """Gradient of sum(diagonal(x) * w): w placed on the diagonal, built with
    numpy's own diagonal as a writable view of a zero array."""
    out = np.zeros(shape, np.float32)
    view = np.diagonal(out, offset, axis1=d1, axis2=d2)
    view.setflags(write=True)
    view[...] = w
    return out


@pytest.mark.parametrize("offset", list(range(-5, 6)))
def test_diagonal_2d_offsets(device, offset):
    a = rng(0).standard_normal((3, 4)).astype(np.float32)
    d = f32(a).diagonal(offset)
    want = np.diagonal(a, offset)
    assert d.shape == list(want.shape)
    np.testing.assert_array_equal(d.numpy().reshape(want.shape), want)


def test_diagonal_default_main(device):
    a = rng(1).standard_normal((4, 4)).astype(np.float32)
    np.testing.assert_array_equal(f32(a).diagonal().numpy(), np.diag(a))


@pytest.mark.parametrize("d1,d2", [(i, j) for i in range(4) for j in range(4) if i != j])
def test_diagonal_every_dim_pair(device, d1, d2):
    a = rng(2).standard_normal((2, 3, 4, 5)).astype(np.float32)
    x = f32(a)
    for offset in (-2, 0, 1):
        d = x.diagonal(offset, d1, d2)
        want = np.diagonal(a, offset, axis1=d1, axis2=d2)
        assert d.shape == list(want.shape)
        np.testing.assert_array_equal(d.numpy().reshape(want.shape), want)


def test_diagonal_negative_dims(device):
    a = rng(3).standard_normal((2, 3, 4)).astype(np.float32)
    x = f32(a)
    np.testing.assert_array_equal(x.diagonal(0, -1, -2).numpy(), np.diagonal(a, 0, 2, 1))
    np.testing.assert_array_equal(x.diagonal(1, -3, -1).numpy(), np.diagonal(a, 1, 0, 2))


def test_diagonal_out_of_range_offsets_are_empty(device):
    x = f32(rng(4).standard_normal((2, 5)))
    for offset in (5, 100, -2, -50):
        d = x.diagonal(offset)
        assert d.shape == [0] and d.numpy().shape == (0,)
    y = f32(rng(5).standard_normal((2, 3, 4)))
    assert y.diagonal(9, 0, 2).shape == [3, 0]
    assert y.diagonal(-9, 1, 2).shape == [2, 0]


def test_diagonal_is_a_strided_view(device):
    a = rng(6).standard_normal((4, 6)).astype(np.float32)
    x = f32(a)
    d = x.diagonal(-1)
    assert d.buffer is x.buffer and d._base is x
    assert list(d.stride) == [x.stride[0] + x.stride[1]]
    assert d.offset == x.offset + x.stride[0]
    wxx().functional.assign(d, -1.0)
    want = a.copy()
    np.fill_diagonal(want[1:], -1.0)
    np.testing.assert_array_equal(x.numpy(), want)


def test_diagonal_view_of_3d(device):
    a = rng(7).standard_normal((2, 3, 4)).astype(np.float32)
    x = f32(a)
    d = x.diagonal(1, 1, 2)
    assert d.shape == [2, 3]
    assert list(d.stride) == [x.stride[0], x.stride[1] + x.stride[2]]
    wxx().functional.assign(d, -2.0)
    want = a.copy()
    i, j = np.meshgrid(np.arange(2), np.arange(3), indexing="ij")
    want[i, j, j + 1] = -2.0
    np.testing.assert_array_equal(x.numpy(), want)


def test_diagonal_of_strided_inputs(device):
    a = rng(8).standard_normal((4, 6)).astype(np.float32)
    x = f32(a)
    s = x[:, 1:5]
    assert not s.is_contiguous()
    np.testing.assert_array_equal(s.diagonal(1).numpy(), np.diagonal(a[:, 1:5], 1))
    np.testing.assert_array_equal(x.permute(1, 0).diagonal(-1).numpy(), np.diagonal(a.T, -1))


@pytest.mark.parametrize("shape,offset,d1,d2", [((3, 4), -1, 0, 1), ((3, 4), 0, 0, 1),
                                                ((3, 4), 2, 0, 1), ((2, 3, 4), 1, 0, 2),
                                                ((2, 3, 4), -1, 2, 0), ((2, 3, 4), 0, 1, 2)])
def test_diagonal_backward(device, shape, offset, d1, d2):
    a = rng(9).standard_normal(shape).astype(np.float32)
    x = f32(a)
    x.requires_grad = True
    d = x.diagonal(offset, d1, d2)
    w = rng(10 + offset).standard_normal(tuple(d.shape)).astype(np.float32)
    (d * f32(w)).sum().backward()
    np.testing.assert_array_equal(x.grad.numpy(), _diag_grad(shape, w, offset, d1, d2))


def test_diagonal_backward_through_permute(device):
    a = rng(30).standard_normal((4, 5)).astype(np.float32)
    base = f32(a)
    base.requires_grad = True
    x = base.permute(1, 0)
    assert not x.is_contiguous()
    d = x.diagonal(-1)
    w = rng(31).standard_normal(tuple(d.shape)).astype(np.float32)
    (d * f32(w)).sum().backward()
    np.testing.assert_array_equal(base.grad.numpy(), _diag_grad((5, 4), w, -1, 0, 1).T)


def test_diagonal_keeps_dtype(device):
    ids = u32(np.arange(24).reshape(2, 3, 4))
    d = ids.diagonal(1, 1, 2)
    assert d.type == "u32"
    np.testing.assert_array_equal(d.numpy(), np.diagonal(np.arange(24).reshape(2, 3, 4), 1, 1, 2))


def test_diagonal_argument_errors(device):
    with pytest.raises(ValueError):
        f32(np.zeros(4)).diagonal()
    x = f32(np.zeros((3, 3, 3)))
    for bad in (1.5, "1", True, None):
        with pytest.raises(TypeError):
            x.diagonal(bad)
    with pytest.raises(ValueError):
        x.diagonal(0, 1, 1)
    for dims in ((0, 3), (-4, 0)):
        with pytest.raises((IndexError, ValueError)):
            x.diagonal(0, *dims)
